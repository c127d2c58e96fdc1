/*
 * Sweep of binary32 inputs through the sampler's correctly rounded math
 * (g4s_crmath.h, host build) against long double evaluations.  Reports how
 * many inputs took the double-double fallback and lists every input where
 * the result differs from fl32(long double); the Python test resolves those
 * with 60-digit mpmath.  Inputs: positive finite binary32 bit patterns
 * [lo, hi) with stride `stride`.
 *   fn 0: exp(x)                     (exp_cr32, x = binary32)
 *   fn 1: 30*tanh(x/30)              (softcap_topk_cr32)
 *   fn 2: tanh(x*fl32(1/30))*30      (softcap_full_cr32)
 */
#include <cmath>
#include <cstdio>
#include <thread>
#include <vector>

#include "../../gemma4.pas_amd/csrc/g4s_crmath.h"

using namespace g4s::cr;

extern "C" long crmath_sweep(int fn, unsigned lo, unsigned hi, unsigned stride, int threads,
                             unsigned* out_bad, long max_bad, long* out_slow)
{
    std::vector<std::vector<unsigned>> bad(threads);
    std::vector<long> slow(threads, 0);
    const float cap = 30.0f;
    const float inv = (float)(1.0 / 30.0);
    auto work = [&](int t) {
        for (unsigned long b = (unsigned long)lo + (unsigned long)t * stride; b < hi;
             b += (unsigned long)stride * threads) {
            float x = u2f((unsigned)b);
            float got, ref;
            double y;
            if (fn == 0) {
                if (!(x <= 89.0f)) continue;
                got = exp_cr32((double)x, 0.0);
                ref = (float)expl((long double)x);
                y = exp_fast_d((double)x);
                if (!rounding_safe(y, 8, 0x1p-50)) slow[t]++;
                /* negative arguments too: the sweep runs x and -x */
                float gotn = exp_cr32(-(double)x, 0.0);
                float refn = (float)expl(-(long double)x);
                double yn = exp_fast_d(-(double)x);
                if (-(double)x >= -104.0 && !rounding_safe(yn, 8, 0x1p-50)) slow[t]++;
                if (f2u(gotn) != f2u(refn)) bad[t].push_back((unsigned)b | 0x80000000u);
            } else if (fn == 1) {
                got = softcap_topk_cr32(x, cap);
                ref = (float)((long double)cap * tanhl((long double)x / (long double)cap));
                double xd = x, wh = xd / cap;
                double wl = fma_d(-wh, (double)cap, xd) / cap;
                double tt = tanh_fast_d(wh);
                y = (double)cap * fma_d(wl, fma_d(-tt, tt, 1.0), tt);
                if (!rounding_safe(y, 16, 0x1p-49)) slow[t]++;
            } else {
                got = softcap_full_cr32(x, inv, cap);
                ref = (float)(tanhl((long double)x * (long double)inv) * (long double)cap);
                y = tanh_fast_d((double)x * (double)inv) * (double)cap;
                if (!rounding_safe(y, 16, 0x1p-49)) slow[t]++;
            }
            if (f2u(got) != f2u(ref)) bad[t].push_back((unsigned)b);
        }
    };
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t) pool.emplace_back(work, t);
    for (auto& th : pool) th.join();
    long n = 0, ns = 0;
    for (int t = 0; t < threads; ++t) {
        ns += slow[t];
        for (unsigned v : bad[t])
            if (n < max_bad) out_bad[n++] = v;
    }
    *out_slow = ns;
    return n;
}
