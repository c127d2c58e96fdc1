/*
 * seqsum_check.cpp -- CPU proof of g4s_seqsum.h against the literal
 * left-to-right binary32 loop (test code; built by tests/native/Makefile).
 *
 * The sequence checks evaluate the running sum the way the sampler's
 * kernels do: terms are cut into chunks of `chunk` terms and threads of
 * `per_thread` terms; every chunk gets the map of its terms in the binade
 * predicted from double-precision prefix sums; a chain walks the chunks,
 * accepting a chunk's map only when the sum entering it is in the predicted
 * binade and the map's result stays in it; any other chunk is re-evaluated
 * thread by thread (thread maps in the current binade, plain binary32 steps
 * inside the thread where the sum leaves its binade).  The result and the
 * first index whose running sum reaches a threshold must equal the literal
 * loop's, bit for bit.
 */
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "../../gemma4.pas_amd/csrc/g4s_seqsum.h"

using namespace g4s::ss;

namespace {

uint64_t mix(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
struct Rng {
    uint64_t s;
    uint64_t next() { return mix(s += 0x9E3779B97F4A7C15ull); }
    double unif() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
    double normal()
    {
        double u1 = 1.0 - unif(), u2 = unif();
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    }
};

/* term generators */
float gen_term(Rng& r, int kind)
{
    switch (kind) {
    case 0: return (float)std::exp(0.5 * r.normal() - 2.5);          /* softmax-like e_i */
    case 1: return (float)(std::exp(0.5 * r.normal() - 2.5) * 3.8e-6); /* probabilities */
    case 2: {                                                         /* few mantissa bits: ties */
        float v = (float)std::exp(r.normal() - 2.0);
        uint32_t b;
        std::memcpy(&b, &v, 4);
        b &= 0xFFFF0000u;
        std::memcpy(&v, &b, 4);
        return v;
    }
    case 3: return (r.next() & 7) == 0 ? 0.0f : (float)std::ldexp(1.0, -(int)(r.next() % 40)); /* powers of two */
    case 4: return (float)std::exp(8.0 * r.normal());                 /* huge dynamic range */
    case 5: {                                                         /* subnormal and tiny */
        uint32_t b = (uint32_t)(r.next() % 0x01000000u);
        float v;
        std::memcpy(&v, &b, 4);
        return v;
    }
    default: return (float)r.unif();
    }
}

State apply_map_state(State st, PMap f) { return State{st.e, map_apply(f, st.m)}; }

/* Evaluate terms[lo, hi) from `st`, thread by thread (`pt` terms per
 * thread), as the chain's re-evaluation of a chunk does; tracks the first
 * index whose running sum reaches thr. */
State resolve(State st, const float* a, int64_t lo, int64_t hi, int pt, float thr, int64_t& hit,
              int64_t& rounds)
{
    int64_t pos = lo;
    while (pos < hi) {
        ++rounds;
        /* thread maps in the current binade, composed in order; find the
         * first thread whose exit leaves the binade or reaches thr */
        State cur = st;
        int64_t t0 = pos;
        bool moved = false;
        for (; t0 < hi; t0 += (t0 == pos ? pt - ((pos - lo) % pt) : pt)) {
            const int64_t t1 = std::min(hi, t0 + (t0 == pos ? pt - ((pos - lo) % pt) : pt));
            PMap f = map_identity();
            for (int64_t i = t0; i < t1; ++i) f = map_sat(map_then(f, map_of_ct(term_ct(a[i], cur.e))));
            const int32_t m_exit = map_apply(f, cur.m);
            const bool leaves = m_exit >= kTop;
            const bool reaches = hit < 0 && !leaves && value_of(State{cur.e, m_exit}) >= thr;
            if (leaves || reaches) {
                /* plain binary32 steps through this thread's terms */
                State s2 = cur;
                for (int64_t i = t0; i < t1; ++i) {
                    s2 = step_add(s2, a[i]);
                    if (hit < 0 && value_of(s2) >= thr) hit = i;
                }
                st = s2;
                pos = t1;
                moved = true;
                break;
            }
            cur.m = m_exit;
        }
        if (!moved) {
            st = cur;
            pos = hi;
        }
    }
    return st;
}

}  // namespace

extern "C" {

/* Single steps: for random S and a, the map step equals RN32(S + a) whenever
 * it stays in the binade, and says "left" exactly when the sum leaves it. */
int64_t ss_check_steps(uint64_t seed, int64_t n)
{
    Rng r{seed};
    int64_t bad = 0;
    for (int64_t i = 0; i < n; ++i) {
        float s = gen_term(r, (int)(r.next() % 7));
        float a = gen_term(r, (int)(r.next() % 7));
        if ((r.next() & 3) == 0) {
            /* a close to S: same or adjacent binade */
            a = s * (float)(0.25 + r.unif());
        }
        if (!(s >= 0.0f) || !(a >= 0.0f) || std::isinf(s) || std::isinf(a)) continue;
        const float ref = s + a;
        State st = state_of(s);
        const int32_t m2 = map_apply(map_of_ct(term_ct(a, st.e)), st.m);
        if (m2 < kTop) {
            if (fbits(value_of(State{st.e, m2})) != fbits(ref)) ++bad;
        } else {
            /* left the binade: the exact sum must be >= 2^(E-126) or round up to it */
            if (!(ref >= value_of(State{st.e, kTop}))) ++bad;
        }
    }
    return bad;
}

/* term_ct_f == term_ct over random terms (all classes, subnormals
 * included) and binades 1..254. */
int64_t ss_check_term_ct_f(uint64_t seed, int64_t n)
{
    Rng r{seed};
    int64_t bad = 0;
    for (int64_t i = 0; i < n; ++i) {
        float a;
        if ((r.next() & 3) == 0) {
            const uint32_t b = (uint32_t)(r.next() & 0x7F7FFFFFu); /* any finite a >= 0 */
            std::memcpy(&a, &b, 4);
        } else {
            a = gen_term(r, (int)(r.next() % 7));
        }
        const int32_t e = 1 + (int32_t)(r.next() % 254);
        if (term_ct_f(a, e) != term_ct(a, e)) ++bad;
        /* and the binades around a's own */
        const int32_t ea = (int32_t)(fbits(a) >> 23);
        for (int32_t d = -2; d <= 26; ++d) {
            const int32_t e2 = ea + d;
            if (e2 >= 1 && e2 <= 254 && term_ct_f(a, e2) != term_ct(a, e2)) ++bad;
        }
    }
    return bad;
}

/* lane_map against the literal loop: runs of 16 terms in binade e (unit
 * fractions with few bits, forced half-unit ties, zeros, terms that alone
 * leave the binade), each applied literally from an even and an odd entering
 * significand.  Where the literal sum stays in the binade the map must give
 * its significand exactly; where it leaves, the map's result must be >= 2^24.
 * Also against the composition of per-term maps. */
int64_t ss_check_lane_map(uint64_t seed, int64_t n)
{
    Rng r{seed};
    int64_t bad = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int32_t e = 30 + (int32_t)(r.next() % 170);
        const int len = 1 + (int)(r.next() % 16);
        float t[16];
        const int mode = (int)(r.next() % 4);
        for (int j = 0; j < len; ++j) {
            double q;
            const uint64_t z = r.next();
            if ((z & 7) == 0) {
                q = 0.0;
            } else if ((z & 7) == 1) {
                q = (double)(r.next() % 4096) + 0.5;                 /* a tie */
            } else if (mode == 3 && (z & 15) == 2) {
                q = 16777216.0 + (double)(r.next() % 1000);          /* leaves alone */
            } else {
                const int bits = 1 + (int)(r.next() % 12);           /* fraction bits */
                const double scale = mode == 0 ? 4096.0 : (mode == 1 ? 64.0 : 1048576.0);
                q = std::floor(r.unif() * scale * (double)(1 << bits)) / (double)(1 << bits);
            }
            t[j] = (float)std::ldexp(q, e - 150);
        }
        const PMap f = lane_map(t, len, e);
        PMap g = map_identity();
        for (int j = 0; j < len; ++j) g = map_sat(map_then(g, map_of_ct(term_ct(t[j], e))));
        for (int p = 0; p < 2; ++p) {
            const int32_t gd = p ? g.d1 : g.d0, fd = p ? f.d1 : f.d0;
            if ((gd < kTop || fd < kTop) && gd != fd) ++bad;
            /* literal from M = 2^23 + something of parity p */
            const int32_t m0 = (int32_t)((0x800000u + (uint32_t)(r.next() % 0x7FFFFEu)) & ~1u) | p;
            float sum = value_of(State{e, m0});
            for (int j = 0; j < len; ++j) sum = sum + t[j];
            const State s2 = state_of(sum);
            const int32_t got = m0 + fd;
            if (s2.e == e) {
                if (got != s2.m) ++bad;
            } else if (got < kTop) {
                ++bad;
            }
        }
    }
    return bad;
}

/* lane_map_fma against lane_map: runs of 1-16 terms below 2^22 units (none,
 * one or several forced half-unit ties, zeros, terms of few fraction bits);
 * both maps must be equal. */
int64_t ss_check_lane_map_fma(uint64_t seed, int64_t n)
{
    Rng r{seed};
    int64_t bad = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int32_t e = 30 + (int32_t)(r.next() % 170);
        const int len = 1 + (int)(r.next() % 16);
        float t[16];
        const int mode = (int)(r.next() % 4);
        for (int j = 0; j < len; ++j) {
            double q;
            const uint64_t z = r.next();
            const uint64_t tie_rate = mode == 3 ? 3 : 31; /* mode 3: several ties a lane */
            if ((z & 7) == 0) {
                q = 0.0;
            } else if (((z >> 3) & tie_rate) == 1) {
                q = (double)(r.next() % 4194303) + 0.5;             /* a tie */
            } else {
                const int bits = 1 + (int)(r.next() % 12);           /* fraction bits */
                const double scale = mode == 0 ? 4096.0 : (mode == 1 ? 64.0 : 4194000.0);
                q = std::floor(r.unif() * scale * (double)(1 << bits)) / (double)(1 << bits);
            }
            t[j] = (float)std::ldexp(q, e - 150);
        }
        const PMap f = lane_map_fma(t, len, e), g = lane_map(t, len, e);
        if (f.d0 != g.d0 || f.d1 != g.d1) ++bad;
    }
    return bad;
}

/* Associativity of map composition over random term maps. */
int64_t ss_check_assoc(uint64_t seed, int64_t n)
{
    Rng r{seed};
    int64_t bad = 0;
    for (int64_t i = 0; i < n; ++i) {
        PMap f{(int32_t)(r.next() % 1000), (int32_t)(r.next() % 1000)};
        PMap g{(int32_t)(r.next() % 1000), (int32_t)(r.next() % 1000)};
        PMap h{(int32_t)(r.next() % 1000), (int32_t)(r.next() % 1000)};
        PMap a1 = map_then(map_then(f, g), h), a2 = map_then(f, map_then(g, h));
        if (a1.d0 != a2.d0 || a1.d1 != a2.d1) ++bad;
        for (int32_t m = 0; m < 4; ++m)
            if (map_apply(map_then(f, g), m) != map_apply(g, map_apply(f, m))) ++bad;
    }
    return bad;
}

/* A full sequence: chunked evaluation with predicted binades vs the literal
 * loop.  out[0] = mismatch flags (bit 0: final sum, bit 1: first reach),
 * out[1] = chunks accepted from their map, out[2] = chunks re-evaluated,
 * out[3] = re-evaluation rounds, out[4] = literal first-reach index. */
void ss_check_sequence(uint64_t seed, int kind, int64_t n, int chunk, int per_thread,
                       double thr_frac, int64_t* out)
{
    Rng r{seed};
    std::vector<float> a((size_t)n);
    for (auto& v : a) v = gen_term(r, kind);
    /* literal loop */
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) s = s + a[(size_t)i];
    const float thr = (float)(thr_frac * (double)s);
    float c = 0.0f;
    int64_t hit_ref = -1;
    for (int64_t i = 0; i < n; ++i) {
        c = c + a[(size_t)i];
        if (c >= thr) {
            hit_ref = i;
            break;
        }
    }
    /* per-chunk double sums and predicted binade at each chunk start */
    const int64_t nch = (n + chunk - 1) / chunk;
    std::vector<double> pre((size_t)nch + 1, 0.0);
    for (int64_t b = 0; b < nch; ++b) {
        double d = 0.0;
        for (int64_t i = b * chunk; i < std::min(n, (b + 1) * chunk); ++i) d += a[(size_t)i];
        pre[(size_t)b + 1] = pre[(size_t)b] + d;
    }
    std::vector<PMap> cmap((size_t)nch);
    std::vector<int32_t> cbin((size_t)nch);
    for (int64_t b = 0; b < nch; ++b) {
        const int32_t e = state_of((float)pre[(size_t)b]).e;
        cbin[(size_t)b] = e;
        PMap f = map_identity();
        for (int64_t i = b * chunk; i < std::min(n, (b + 1) * chunk); ++i)
            f = map_sat(map_then(f, map_of_ct(term_ct(a[(size_t)i], e))));
        cmap[(size_t)b] = f;
    }
    /* chain */
    State st = state_of(0.0f);
    int64_t hit = -1, acc = 0, reev = 0, rounds = 0;
    for (int64_t b = 0; b < nch; ++b) {
        const int64_t lo = b * chunk, hi = std::min(n, (b + 1) * chunk);
        if (st.e == cbin[(size_t)b]) {
            const int32_t m2 = map_apply(cmap[(size_t)b], st.m);
            if (m2 < kTop && !(hit < 0 && value_of(State{st.e, m2}) >= thr)) {
                st.m = m2;
                ++acc;
                continue;
            }
        }
        ++reev;
        st = resolve(st, a.data(), lo, hi, per_thread, hit < 0 ? thr : INFINITY, hit, rounds);
    }
    const float s2 = value_of(st);
    out[0] = (fbits(s2) != fbits(s) ? 1 : 0) | (hit != hit_ref ? 2 : 0);
    out[1] = acc;
    out[2] = reev;
    out[3] = rounds;
    out[4] = hit_ref;
}

}  // extern "C"
