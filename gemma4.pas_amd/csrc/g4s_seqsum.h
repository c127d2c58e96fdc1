/*
 * g4s_seqsum.h -- exact parallel evaluation of a left-to-right binary32
 * running sum of non-negative terms, identical on the host and on gfx950.
 *
 * The reference accumulates LSum and the index-order running sum of the
 * sampling draw one term at a time in binary32 (src/Gemma4.Tensors.pas:657-
 * 663, src/Gemma4.Model.pas:2727-2735): S_0 = 0, S_{i+1} = RN32(S_i + a_i).
 * Summing in any other order changes the last bits, and over 262144 terms
 * that changes which token is drawn.  This header restates the recurrence so
 * that blocks of terms can be evaluated independently and chained:
 *
 *  - While S stays inside one binade of width 2^24 units u (u = 2^(E-150),
 *    E = max(exponent field of S, 1)), S = M*u for an integer M < 2^24 and
 *    RN32(M*u + a) = u * RNE(M + a/u).  With a/u = k + f (k integer,
 *    0 <= f < 1) that is M + k when f < 1/2, M + k + 1 when f > 1/2, and at
 *    f = 1/2 the even one of M + k and M + k + 1.  So every term is the map
 *    M -> M + d[M & 1] with d[p] = c + t*((p + c) & 1), where
 *    c = k + (f > 1/2) and t = (f == 1/2).
 *  - Maps of that form are closed under composition:
 *    (f then g)[p] = f[p] + g[(p + f[p]) & 1]; the composition is
 *    associative, so a block of terms reduces to one map by any tree or scan.
 *  - Applying a block's map is exact as long as no intermediate sum leaves
 *    the binade.  M only grows, so a result below 2^24 proves it; a result
 *    >= 2^24 means the block crosses (or may cross) into the next binade,
 *    and the caller re-evaluates that block at finer grain around the
 *    crossing, where one plain binary32 addition is exact by definition.
 *
 * The subnormal range and [2^-126, 2^-125) share u = 2^-149 (E = 1), so
 * S = 0 is simply M = 0 in binade E = 1; no special case is needed.
 */
#ifndef G4S_SEQSUM_H
#define G4S_SEQSUM_H

#include <stdint.h>

#if defined(__HIPCC__)
#define G4S_SS_HD __host__ __device__ __forceinline__
#else
#define G4S_SS_HD static inline
#endif

namespace g4s {
namespace ss {

constexpr int32_t kTop = 1 << 24; /* M reaching this left the binade */

/* State of a running sum: binade E (>= 1) and significand M in units of
 * 2^(E-150), 0 <= M < 2^24 (M >= 2^23 unless E == 1). */
struct State {
    int32_t e;
    int32_t m;
};

/* A block's effect: M -> M + d[M & 1]. */
struct PMap {
    int32_t d0, d1;
};

G4S_SS_HD uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }
G4S_SS_HD float bitsf(uint32_t b) { return __builtin_bit_cast(float, b); }

G4S_SS_HD State state_of(float s)
{
    const uint32_t b = fbits(s) & 0x7FFFFFFFu;
    const int32_t ef = (int32_t)(b >> 23);
    const int32_t man = (int32_t)(b & 0x7FFFFFu);
    State st;
    if (ef == 0) {
        st.e = 1;
        st.m = man; /* subnormal or zero: units of 2^-149 */
    } else {
        st.e = ef;
        st.m = man | 0x800000;
    }
    return st;
}

/* The binary32 value of a state (M < 2^24; M == 2^24 is 2^(E-126)). */
G4S_SS_HD float value_of(State st)
{
    if (st.m >= kTop) return bitsf((uint32_t)(st.e + 1) << 23);
    if (st.m < 0x800000) return bitsf((uint32_t)st.m); /* only for E == 1 */
    return bitsf(((uint32_t)st.e << 23) + (uint32_t)(st.m - 0x800000));
}

/* c and t of one term a >= 0 in binade E; c = kTop when a alone leaves the
 * binade (a >= 2^(E-126)).  Packed as c*2 + t. */
G4S_SS_HD int32_t term_ct(float a, int32_t e)
{
    /* branch-free: s = e - E(a) units of shift; s < 0: a alone leaves the
     * binade; s = 0: a is an integer number of units; s >= 25: a < u/2
     * rounds away (k = 0, rem < half); +0 gives k = rem = 0 */
    const uint32_t b = fbits(a);
    const int32_t ea = (int32_t)(b >> 23);
    const uint32_t ma = (b & 0x7FFFFFu) | (ea ? 0x800000u : 0u);
    const int32_t s = e - (ea ? ea : 1);
    const int32_t sc = s < 0 ? 0 : (s > 31 ? 31 : s);
    const uint32_t k = ma >> sc;
    const uint32_t rem = ma & ((1u << sc) - 1u);
    const uint32_t half = sc ? (1u << (sc - 1)) : 1u; /* s = 0: rem = 0 is no tie */
    const int32_t ct = (int32_t)((k + (rem > half ? 1u : 0u)) * 2u + (rem == half ? 1u : 0u));
    return s < 0 ? kTop * 2 : ct;
}

/* term_ct in binary32 arithmetic (fewer instructions on the GPU): with
 * u = 2^(E-150), q = a/u = ldexp(a, 150-E) is exact (or >= 2^24, or far
 * below 1/2 when it underflows), k = floor(q) and f = q - k are exact, and
 * c, t follow from f.  Equal to term_ct for every a >= 0 and binade E. */
G4S_SS_HD int32_t term_ct_f(float a, int32_t e)
{
    const float q = __builtin_ldexpf(a, 150 - e);
    const bool left = q >= 16777216.0f;
    const float qc = left ? 0.0f : q; /* keeps the conversion in range */
    const float k = __builtin_floorf(qc);
    const float f = qc - k;
    const int32_t ct = ((int32_t)k + (f > 0.5f ? 1 : 0)) * 2 + (f == 0.5f ? 1 : 0);
    return left ? kTop * 2 : ct;
}

G4S_SS_HD PMap map_of_ct(int32_t ct)
{
    const int32_t c = ct >> 1, t = ct & 1;
    PMap r;
    r.d0 = c + (t & c);         /* p = 0: (0 + c) & 1 */
    r.d1 = c + (t & (c + 1));   /* p = 1: (1 + c) & 1 */
    return r;
}

G4S_SS_HD PMap map_identity()
{
    PMap r;
    r.d0 = 0;
    r.d1 = 0;
    return r;
}

/* f then g */
G4S_SS_HD PMap map_then(PMap f, PMap g)
{
    PMap r;
    r.d0 = f.d0 + (((f.d0) & 1) ? g.d1 : g.d0);
    r.d1 = f.d1 + (((1 + f.d1) & 1) ? g.d1 : g.d0);
    return r;
}

/* Apply a map: the new M (may be >= kTop: the block left the binade). */
G4S_SS_HD int32_t map_apply(PMap f, int32_t m) { return m + ((m & 1) ? f.d1 : f.d0); }

/* Saturating variant for long blocks: keeps the increments below 2^30 so
 * compositions cannot overflow; any value >= kTop already means "left". */
G4S_SS_HD PMap map_sat(PMap f)
{
    const int32_t cap = 1 << 26;
    PMap r;
    r.d0 = f.d0 > cap ? cap + (f.d0 & 1) : f.d0;
    r.d1 = f.d1 > cap ? cap + (f.d1 & 1) : f.d1;
    return r;
}

/* The map of a run of n terms in binade e in one pass over the terms.
 * A term q = a/u = k + f adds k + (f > 1/2) units unless f == 1/2 (a
 * half-unit tie), where it adds k or k + 1, whichever makes the sum even.
 * The running parity chain that starts even gives d0.  The chain that starts
 * odd adds the same units up to the first tie (only ties depend on parity),
 * rounds that tie the other way, and from there on both sums are even and
 * identical: d1 = d0 + 1 when the even chain rounds its first tie down,
 * d0 - 1 when it rounds it up, d0 without a tie.  Each d_p is exact when the
 * true value is below kTop and at least kTop otherwise (q is clamped at
 * 2^25, where a term alone leaves the binade, and d0 at 2^26). */
G4S_SS_HD PMap lane_map(const float* t, int n, int32_t e)
{
    /* A tie adds fi + x, x = (P ^ fi) & 1, which leaves the sum even: the
     * parity P carried from term to term is 0 after a tie and P ^ (c & 1)
     * after any other term adding c units, so it does not wait on the
     * units a tie adds (the chain between terms is one xor and one
     * select). */
    int32_t D = 0, P = 0, delta = 0;
    bool seen = false;
    for (int j = 0; j < n; ++j) {
        float q = __builtin_ldexpf(t[j], 150 - e);
        q = q < 33554432.0f ? q : 33554432.0f;
        const float fl = __builtin_floorf(q);
        const float fr = q - fl;
        const int32_t fi = (int32_t)fl;
        const bool tie = fr == 0.5f;
        const int32_t c = fi + ((!tie && fr > 0.5f) ? 1 : 0);
        const int32_t x = (P ^ fi) & 1;
        delta = (tie && !seen) ? 1 - 2 * x : delta;
        seen = seen || tie;
        D += c + (tie ? x : 0);
        D = D > (1 << 26) ? (1 << 26) : D;
        P = tie ? 0 : (P ^ (c & 1));
    }
    PMap r;
    r.d0 = D;
    r.d1 = D + delta;
    return r;
}

/* lane_map for terms q = t * 2^(150-e) all in [0, 2^22), in one fma pass:
 * r = fl(q + 1.5 * 2^23) holds rint(q) and fma(t, 2^(150-e), 1.5 * 2^23 - r)
 * is q - rint(q) exactly, +-1/2 at a half-unit tie.  Without a tie the map is
 * the constant sum of rint(q); with one, that sum less the tie's rint plus
 * floor(q) + x, x = (units before it + floor(q)) & 1 for the even start and
 * 1 - x for the odd one (the tie makes the sum even).  Two or more ties in
 * the lane take lane_map. */
G4S_SS_HD PMap lane_map_fma(const float* t, int n, int32_t e)
{
    const float S = __builtin_ldexpf(1.0f, 150 - e);
    const float M = 12582912.0f; /* 1.5 * 2^23 */
    int32_t tot = 0, before = 0, rj = 0, fj = 0, nt = 0;
    for (int j = 0; j < n; ++j) {
        const float r = __builtin_fmaf(t[j], S, M);
        const float d = __builtin_fmaf(t[j], S, M - r);
        const int32_t ri = (int32_t)(r - M);
        if (__builtin_fabsf(d) == 0.5f) {
            before = tot;
            rj = ri;
            fj = d > 0.0f ? ri : ri - 1;
            ++nt;
        }
        tot += ri;
    }
    PMap f;
    if (nt > 1) return lane_map(t, n, e);
    if (nt == 0) {
        f.d0 = f.d1 = tot;
        return f;
    }
    const int32_t x = (before + fj) & 1;
    f.d0 = tot - rj + fj + x;
    f.d1 = f.d0 + 1 - 2 * x;
    return f;
}

/* One reference step, S <- RN32(S + a), on a state (exact by definition). */
G4S_SS_HD State step_add(State st, float a)
{
    const float s = value_of(st);
    const float r = s + a;
    return state_of(r);
}

}  // namespace ss
}  // namespace g4s

#endif
