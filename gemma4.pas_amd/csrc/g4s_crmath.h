/*
 * g4s_crmath.h -- correctly rounded binary32 results of the sampler's
 * transcendental steps, identical on the host and on gfx950.
 *
 * The reference evaluates Exp / Tanh and compound Single expressions in
 * Extended precision and rounds once on assignment to a Single
 * (src/Gemma4.Tensors.pas:660, src/Gemma4.Model.pas:2776,2797,
 * src/Gemma4.Layers.pas:314).  The sampler therefore needs the correctly
 * rounded (RN) binary32 value of
 *     exp(a - b)                 a, b binary32 (difference taken exactly)
 *     cap * tanh(x / cap)        top-k softcap form, quotient exact
 *     tanh(x * c) * cap          full-vocabulary form, c = fl32(1/cap)
 *     u * P                      u binary64, P binary32
 * Method (Ziv's strategy): evaluate in binary64 with a proven relative error
 * bound eps, accept fl32(y) when y is farther than eps*y from every binary32
 * rounding midpoint, otherwise re-evaluate in double-double (~2^-100) and
 * round that.  The accept test reads the 29 discarded mantissa bits of y.
 * Constants (ln 2 split, 1/n!, tanh Taylor coefficients) were computed with
 * 80-digit arithmetic; no vendor math library is used.
 *
 * Build with -ffp-contract=off: every fused operation below is an explicit
 * fma().
 */
#ifndef G4S_CRMATH_H
#define G4S_CRMATH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define G4S_HD __host__ __device__ __forceinline__
#define G4S_HD_COLD static __host__ __device__ __attribute__((noinline, cold))
#else
#define G4S_HD static inline
#define G4S_HD_COLD static __attribute__((noinline, cold))
#endif

namespace g4s {
namespace cr {

G4S_HD uint64_t d2u(double x) { return __builtin_bit_cast(uint64_t, x); }
G4S_HD double u2d(uint64_t u) { return __builtin_bit_cast(double, u); }
G4S_HD uint32_t f2u(float x) { return __builtin_bit_cast(uint32_t, x); }
G4S_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
G4S_HD double fma_d(double a, double b, double c) { return __builtin_fma(a, b, c); }
G4S_HD double fabs_d(double x) { return __builtin_fabs(x); }
G4S_HD bool isnan_d(double x) { return x != x; }

/* 2^k for k in [-1022, 1023] */
G4S_HD double pow2i(int k) { return u2d((uint64_t)(k + 1023) << 52); }

/* ------------------------------------------------------- double-double */

struct dd {
    double hi, lo;
};

G4S_HD dd two_sum(double a, double b)
{
    double s = a + b;
    double bb = s - a;
    double e = (a - (s - bb)) + (b - bb);
    return {s, e};
}
G4S_HD dd fast_two_sum(double a, double b) /* |a| >= |b| or a == 0 */
{
    double s = a + b;
    double e = b - (s - a);
    return {s, e};
}
G4S_HD dd two_prod(double a, double b)
{
    double p = a * b;
    return {p, fma_d(a, b, -p)};
}
G4S_HD dd dd_add(dd a, dd b)
{
    dd s = two_sum(a.hi, b.hi);
    dd t = two_sum(a.lo, b.lo);
    s.lo += t.hi;
    s = fast_two_sum(s.hi, s.lo);
    s.lo += t.lo;
    return fast_two_sum(s.hi, s.lo);
}
G4S_HD dd dd_neg(dd a) { return {-a.hi, -a.lo}; }
G4S_HD dd dd_sub(dd a, dd b) { return dd_add(a, dd_neg(b)); }
G4S_HD dd dd_mul(dd a, dd b)
{
    dd p = two_prod(a.hi, b.hi);
    p.lo = fma_d(a.hi, b.lo, p.lo);
    p.lo = fma_d(a.lo, b.hi, p.lo);
    return fast_two_sum(p.hi, p.lo);
}
G4S_HD dd dd_mul_d(dd a, double b)
{
    dd p = two_prod(a.hi, b);
    p.lo = fma_d(a.lo, b, p.lo);
    return fast_two_sum(p.hi, p.lo);
}
G4S_HD dd dd_div(dd a, dd b)
{
    double q1 = a.hi / b.hi;
    dd r = dd_sub(a, dd_mul_d(b, q1));
    double q2 = r.hi / b.hi;
    r = dd_sub(r, dd_mul_d(b, q2));
    double q3 = r.hi / b.hi;
    dd q = fast_two_sum(q1, q2);
    return dd_add(q, dd{q3, 0.0});
}

/* ------------------------------------------------------ binary32 rounding */

G4S_HD float f32_next_up(float f)
{
    uint32_t b = f2u(f);
    if (b == 0x80000000u) b = 0;
    return ((int32_t)b >= 0) ? u2f(b + 1) : u2f(b - 1);
}
G4S_HD float f32_next_down(float f) { return -f32_next_up(-f); }

/* RN32(hi + lo) for a normalised double-double (|lo| <= ulp(hi)/2).
 * fl32(hi) is already right unless hi sits exactly on a binary32 midpoint,
 * in which case the sign of lo decides. */
G4S_HD float round_dd_f32(double hi, double lo)
{
    float f = (float)hi;
    double fd = (double)f;
    if (lo == 0.0 || fd == hi || isnan_d(hi)) return f;
    if (fabs_d(fd) == __builtin_inf()) {
        /* beyond FLT_MAX: the only midpoint is +-(2^128 - 2^103) */
        double m = 0x1.fffffep+127 + 0x1p+103;
        if (fabs_d(hi) != m) return f;
        float fmax = u2f(0x7F7FFFFFu);
        if (hi > 0) return lo > 0.0 ? f : fmax;
        return lo < 0.0 ? f : -fmax;
    }
    float g = hi > fd ? f32_next_up(f) : f32_next_down(f);
    double mid = 0.5 * (fd + (double)g);
    if (hi != mid) return f;
    /* hi is exactly the midpoint of f and g: lo's sign decides */
    float upper = hi > fd ? g : f;
    float lower = hi > fd ? f : g;
    return lo > 0.0 ? upper : lower;
}

/* Is fl32(y) guaranteed to be RN32(Y) for any Y with |Y - y| <= tol_ulps
 * binary64 ulps of y (normal binary32 range) or eps_rel*y (subnormal range)? */
G4S_HD bool rounding_safe(double y, int tol_ulps, double eps_rel)
{
    /* both tests evaluated and one selected (no branch: callers evaluate
     * several of these side by side) */
    double a = fabs_d(y);
    int32_t low = (int32_t)(d2u(a) & 0x1FFFFFFFu);
    int32_t dist = low - 0x10000000;
    dist = dist < 0 ? -dist : dist;
    double z = a * 0x1p149; /* exact below 2^-126: units of the binary32 subnormal grid */
    double frac = z - __builtin_floor(z);
    const bool sub = fabs_d(frac - 0.5) > z * eps_rel + 0x1p-60;
    return a >= 0x1p-126 ? dist > tol_ulps : sub;
}

/* -------------------------------------------------------------- constants */

#define G4S_LOG2E 0x1.71547652b82fep+0
/* ln 2 = LN2_HI32 + LN2_LO32 (+ ~2^-86); LN2_HI32 has 32 fraction bits */
#define G4S_LN2_HI32 0x1.62e42fee00000p-1
#define G4S_LN2_LO32 0x1.a39ef35793c76p-33
/* ln 2 = LN2_1 + LN2_2 + LN2_3 (+ ~2^-155); LN2_1 has 42 significant bits */
#define G4S_LN2_1 0x1.62e42fefa3800p-1
#define G4S_LN2_2 0x1.ef35793c76730p-45
#define G4S_LN2_3 0x1.f97b57a079a19p-103

/* 1/n! as double-double, n = 0..31 */
G4S_HD dd inv_fact(int n)
{
    switch (n) {
    case 0: return {0x1.0000000000000p+0, 0.0};
    case 1: return {0x1.0000000000000p+0, 0.0};
    case 2: return {0x1.0000000000000p-1, 0.0};
    case 3: return {0x1.5555555555555p-3, 0x1.5555555555555p-57};
    case 4: return {0x1.5555555555555p-5, 0x1.5555555555555p-59};
    case 5: return {0x1.1111111111111p-7, 0x1.1111111111111p-63};
    case 6: return {0x1.6c16c16c16c17p-10, -0x1.f49f49f49f49fp-65};
    case 7: return {0x1.a01a01a01a01ap-13, 0x1.a01a01a01a01ap-73};
    case 8: return {0x1.a01a01a01a01ap-16, 0x1.a01a01a01a01ap-76};
    case 9: return {0x1.71de3a556c734p-19, -0x1.c154f8ddc6c00p-73};
    case 10: return {0x1.27e4fb7789f5cp-22, 0x1.cbbc05b4fa99ap-76};
    case 11: return {0x1.ae64567f544e4p-26, -0x1.c062e06d1f209p-80};
    case 12: return {0x1.1eed8eff8d898p-29, -0x1.2aec959e14c06p-83};
    case 13: return {0x1.6124613a86d09p-33, 0x1.f28e0cc748ebep-87};
    case 14: return {0x1.93974a8c07c9dp-37, 0x1.05d6f8a2efd1fp-92};
    case 15: return {0x1.ae7f3e733b81fp-41, 0x1.1d8656b0ee8cbp-97};
    case 16: return {0x1.ae7f3e733b81fp-45, 0x1.1d8656b0ee8cbp-101};
    case 17: return {0x1.952c77030ad4ap-49, 0x1.ac981465ddc6cp-103};
    case 18: return {0x1.6827863b97d97p-53, 0x1.eec01221a8b0bp-107};
    case 19: return {0x1.2f49b46814157p-57, 0x1.2650f61dbdcb4p-112};
    case 20: return {0x1.e542ba4020225p-62, 0x1.ea72b4afe3c2fp-120};
    case 21: return {0x1.71b8ef6dcf572p-66, -0x1.d043ae40c4647p-120};
    case 22: return {0x1.0ce396db7f853p-70, -0x1.aebcdbd20331cp-124};
    case 23: return {0x1.761b41316381ap-75, -0x1.3423c7d91404fp-130};
    case 24: return {0x1.f2cf01972f578p-80, -0x1.9ada5fcc1ab14p-135};
    case 25: return {0x1.3f3ccdd165fa9p-84, -0x1.58ddadf344487p-139};
    case 26: return {0x1.88e85fc6a4e5ap-89, -0x1.71c37ebd16540p-143};
    case 27: return {0x1.d1ab1c2dccea3p-94, 0x1.054d0c78aea14p-149};
    case 28: return {0x1.0a18a2635085dp-98, 0x1.b9e2e28e1aa54p-153};
    case 29: return {0x1.259f98b4358adp-103, 0x1.eaf8c39dd9bc5p-157};
    case 30: return {0x1.3932c5047d60ep-108, 0x1.832b7b530a627p-162};
    default: return {0x1.434d2e783f5bcp-113, 0x1.0b87b91be9affp-167};
    }
}

/* ------------------------------------------------------------------- exp */

/* e^x = 2^k * exp_fast_poly(x): r = x - k ln2, |r| <= 0.347, degree-13
 * Taylor polynomial (truncation < 2^-57). */
G4S_HD double exp_fast_poly(double x, int* kout)
{
    double k = __builtin_rint(x * G4S_LOG2E);
    double r = fma_d(-k, G4S_LN2_HI32, x); /* exact */
    r = fma_d(-k, G4S_LN2_LO32, r);
    double q = 0x1.6124613a86d09p-33;            /* 1/13! */
    q = fma_d(q, r, 0x1.1eed8eff8d898p-29);      /* 1/12! */
    q = fma_d(q, r, 0x1.ae64567f544e4p-26);      /* 1/11! */
    q = fma_d(q, r, 0x1.27e4fb7789f5cp-22);      /* 1/10! */
    q = fma_d(q, r, 0x1.71de3a556c734p-19);      /* 1/9!  */
    q = fma_d(q, r, 0x1.a01a01a01a01ap-16);      /* 1/8!  */
    q = fma_d(q, r, 0x1.a01a01a01a01ap-13);      /* 1/7!  */
    q = fma_d(q, r, 0x1.6c16c16c16c17p-10);      /* 1/6!  */
    q = fma_d(q, r, 0x1.1111111111111p-7);       /* 1/5!  */
    q = fma_d(q, r, 0x1.5555555555555p-5);       /* 1/4!  */
    q = fma_d(q, r, 0x1.5555555555555p-3);       /* 1/3!  */
    q = fma_d(q, r, 0.5);
    q = fma_d(q, r, 1.0);
    *kout = (int)k;
    return fma_d(q, r, 1.0);
}
/* e^x in binary64 for x in [-750, 710]; relative error < 2^-51.5 when the
 * result is a normal binary64 (x > -708). */
G4S_HD double exp_fast_d(double x)
{
    int ki;
    const double y = exp_fast_poly(x, &ki);
    if (ki < -1000) return y * pow2i(-1000) * pow2i(ki + 1000);
    if (ki > 1000) return y * pow2i(1000) * pow2i(ki - 1000);
    return y * pow2i(ki);
}

/* e^(xh + xl) in double-double, relative error ~2^-100. */
G4S_HD dd exp_dd(double xh, double xl)
{
    double k = __builtin_rint(xh * G4S_LOG2E);
    dd r = two_sum(fma_d(-k, G4S_LN2_1, xh), xl); /* k*LN2_1 exact, difference exact */
    r = dd_sub(r, two_prod(k, G4S_LN2_2));
    r = dd_sub(r, dd{k * G4S_LN2_3, 0.0});
    dd s = inv_fact(24);
    for (int n = 23; n >= 0; --n) s = dd_add(dd_mul(s, r), inv_fact(n));
    int ki = (int)k;
    double sc1 = ki < -1000 ? pow2i(-1000) : (ki > 1000 ? pow2i(1000) : 1.0);
    int rest = ki < -1000 ? ki + 1000 : (ki > 1000 ? ki - 1000 : ki);
    double sc2 = pow2i(rest);
    return {s.hi * sc1 * sc2, s.lo * sc1 * sc2};
}

/* e^x - 1 in double-double for |x| <= 1.1, relative error ~2^-100. */
G4S_HD dd expm1_dd(dd x)
{
    dd s = inv_fact(31);
    for (int n = 30; n >= 1; --n) s = dd_add(dd_mul(s, x), inv_fact(n));
    return dd_mul(s, x);
}

/* The double-double evaluations below run only when the binary64 result
 * lies too close to a binary32 rounding midpoint (a few times in 2^20): they
 * are kept out of line so the fast paths stay small. */
G4S_HD_COLD float exp_cr32_slow(double xh, double xl)
{
    dd e = exp_dd(xh, xl);
    return round_dd_f32(e.hi, e.lo);
}

/* RN32(e^(xh + xl)), |xl| <= ulp(xh). */
G4S_HD float exp_cr32(double xh, double xl)
{
    if (isnan_d(xh)) return (float)xh;
    if (xh > 89.0) return __builtin_inff();
    if (xh < -104.0) return 0.0f; /* e^-104 < 2^-150: rounds to +0 */
    double y = exp_fast_d(xh);
    y = fma_d(y, xl, y);
    if (rounding_safe(y, 8, 0x1p-50)) return (float)y; /* eps = 2^-50 */
    return exp_cr32_slow(xh, xl);
}

/* RN32(e^(a - b)) for binary32 a, b with the difference taken exactly
 * (`Exp(LVals[LI] - LMax)`, Model.pas:2797; Tensors.pas:660). */
G4S_HD float exp_diff_cr32(float a, float b)
{
    dd d = two_sum((double)a, -(double)b);
    return exp_cr32(d.hi, d.lo);
}

/* exp_cr32 without its double-double route and without branches, so that
 * several evaluations interleave: *r = exp_cr32(xh, xl) whenever it returns
 * true (the same binary64 evaluation and the same rounding test, the special
 * cases selected); false (rarely) when that route is needed. */
G4S_HD bool exp_cr32_try(double xh, double xl, float* r)
{
    const bool nan = isnan_d(xh), over = xh > 89.0, under = xh < -104.0;
    const bool special = nan || over || under;
    int ki;
    /* |x| <= 104: k within +-151, so the scale needs no split */
    double y = exp_fast_poly(special ? 0.0 : xh, &ki) * pow2i(ki);
    y = fma_d(y, xl, y);
    *r = nan ? (float)xh : (over ? __builtin_inff() : (under ? 0.0f : (float)y));
    return special || rounding_safe(y, 8, 0x1p-50);
}
G4S_HD bool exp_diff_cr32_try(float a, float b, float* r)
{
    dd d = two_sum((double)a, -(double)b);
    return exp_cr32_try(d.hi, d.lo, r);
}

/* ------------------------------------------------------------------ tanh */

/* tanh(w) in binary64 with relative error < 2^-50.5. */
G4S_HD double tanh_fast_d(double w)
{
    double a = fabs_d(w);
    double t;
    if (a < 0.55) {
        double a2 = a * a;
        double q = 0x1.2efe8db3aff1fp-24;        /* x^37 */
        q = fma_d(q, a2, -0x1.75cde6563fed9p-23); /* x^35 */
        q = fma_d(q, a2, 0x1.cd299de4ae6bbp-22); /* x^33 */
        q = fma_d(q, a2, -0x1.1c77df95c1c0dp-20); /* x^31 */
        q = fma_d(q, a2, 0x1.5ef2da474e5b7p-19); /* x^29 */
        q = fma_d(q, a2, -0x1.b0f72d3ee24e9p-18);
        q = fma_d(q, a2, 0x1.0b132d39a6050p-16);
        q = fma_d(q, a2, -0x1.497d8eea25259p-15);
        q = fma_d(q, a2, 0x1.967e18afcafadp-14);
        q = fma_d(q, a2, -0x1.f57d7734d1664p-13);
        q = fma_d(q, a2, 0x1.3558248036744p-11);
        q = fma_d(q, a2, -0x1.7da36452b75e3p-10);
        q = fma_d(q, a2, 0x1.d6d3d0e157de0p-9);
        q = fma_d(q, a2, -0x1.226e355e6c23dp-7);
        q = fma_d(q, a2, 0x1.664f4882c10fap-6);
        q = fma_d(q, a2, -0x1.ba1ba1ba1ba1cp-5);
        q = fma_d(q, a2, 0x1.1111111111111p-3);
        q = fma_d(q, a2, -0x1.5555555555555p-2);
        q = q * a2;
        t = fma_d(a, q, a);
    } else if (a < 22.0) {
        double e = exp_fast_d(2.0 * a);
        t = 1.0 - 2.0 / (e + 1.0);
    } else {
        t = 1.0;
    }
    return w < 0 ? -t : t;
}

/* tanh of a double-double argument, relative error ~2^-100. */
G4S_HD dd tanh_dd(dd w)
{
    bool neg = w.hi < 0;
    dd a = neg ? dd_neg(w) : w;
    dd t;
    if (a.hi < 0.55) {
        dd e = expm1_dd(dd{2.0 * a.hi, 2.0 * a.lo});
        t = dd_div(e, dd_add(e, dd{2.0, 0.0}));
    } else if (a.hi < 350.0) {
        dd e = exp_dd(2.0 * a.hi, 2.0 * a.lo);
        t = dd_sub(dd{1.0, 0.0}, dd_div(dd{2.0, 0.0}, dd_add(e, dd{1.0, 0.0})));
    } else {
        t = dd{1.0, 0.0};
    }
    return neg ? dd_neg(t) : t;
}

/* RN32(c * tanh(wh + wl)) in double-double (out of line, rare). */
G4S_HD_COLD float tanh_scaled_cr32_slow(double wh, double wl, double c)
{
    dd tt = tanh_dd(dd{wh, wl});
    dd yy = dd_mul_d(tt, c);
    return round_dd_f32(yy.hi, yy.lo);
}

/* RN32(cap * tanh(x / cap)) with the quotient exact: the top-k softcap
 * `LCap * Tanh(LVals[LI] / LCap)` (Model.pas:2776).  cap > 0. */
G4S_HD float softcap_topk_cr32(float x, float cap)
{
    double xd = x, cd = cap;
    if (isnan_d(xd)) return x;
    if (fabs_d(xd) == __builtin_inf()) return xd > 0 ? cap : -cap;
    double wh = xd / cd;
    double wl = fma_d(-wh, cd, xd) / cd; /* exact remainder / cap */
    double t = tanh_fast_d(wh);
    double y = cd * fma_d(wl, fma_d(-t, t, 1.0), t);
    if (rounding_safe(y, 16, 0x1p-49)) return (float)y; /* eps = 2^-49 */
    return tanh_scaled_cr32_slow(wh, wl, cd);
}

/* RN32(tanh(x * inv_cap) * cap), inv_cap = fl32(1/cap): the full-vocabulary
 * softcap `Tanh(LVal * LInvCap) * ACap` (Layers.pas:309-314).  The product
 * of two binary32 values is exact in binary64. */
G4S_HD float softcap_full_cr32(float x, float inv_cap, float cap)
{
    double w = (double)x * (double)inv_cap;
    if (isnan_d(w)) return (float)w;
    if (fabs_d(w) == __builtin_inf()) return w > 0 ? cap : -cap;
    double t = tanh_fast_d(w);
    double y = t * (double)cap;
    if (rounding_safe(y, 16, 0x1p-49)) return (float)y;
    return tanh_scaled_cr32_slow(w, 0.0, (double)cap);
}

/* RN32(u * p) for binary64 u and binary32 p (`Random * TopP`, Model.pas:2813). */
G4S_HD float mul_u_p_cr32(double u, float p)
{
    dd prod = two_prod(u, (double)p);
    return round_dd_f32(prod.hi, prod.lo);
}

/* RN32(a / b) for binary32 a, b: the binary64 quotient never lands on a
 * binary32 midpoint unless it is exact, so one extra rounding is harmless. */
G4S_HD float div_cr32(float a, float b) { return (float)((double)a / (double)b); }

}  // namespace cr
}  // namespace g4s

#endif
