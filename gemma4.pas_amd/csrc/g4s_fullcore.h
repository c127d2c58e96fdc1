/*
 * g4s_fullcore.h -- device helpers shared by the softmax-path kernels
 * (g4s_full.hip: every dtype, wide rows; g4s_fullbf.hip: the streaming
 * pipeline of full bf16 rows): row classes and masks, loads, the exact
 * softcap/temperature/exp forms, the e table lookups, block and wave
 * reductions, the running-sum maps (g4s_seqsum.h) composed over lanes and
 * chunks, the exact resolution rounds, and the chain helpers.
 *
 * Included inside namespace g4s by those translation units only.
 */
#ifndef G4S_FULLCORE_H
#define G4S_FULLCORE_H

#include <climits>

#include "g4s_full.h"

namespace g4s {

using namespace g4s::cr;
using ss::PMap;
using ss::State;

namespace {

constexpr int NWF = kFullBlock / 64;                 /* waves per workgroup */
constexpr int kSelCPT = kSelMaxChunks / kFullBlock;   /* select records per thread */

struct RowIn {
    g4s_params p;
    double u;
};
__device__ __forceinline__ RowIn row_in(const FullArgs& a, int row)
{
    RowIn r;
    r.p = a.params ? a.params[row] : a.p0;
    r.u = a.u ? a.u[row] : a.u0;
    return r;
}

/* DoSample's dispatch (Model.pas:2756) as this launch sees it. */
__device__ __forceinline__ int row_class(const FullArgs& a, int K)
{
    if (K <= 0 || K >= a.vocab) return kRowFull;
    if (K > kMaxTopK && a.wide_on) return kRowWide;
    return kRowTopk;
}

/* Which terms of a row take part in the softmax: all of a full row; the
 * survivors of a wide row. */
struct Mask {
    int32_t cls;
    int32_t state;
    uint32_t tau;
    int32_t idx_thr;
    const uint32_t* bits;
};

/* The row's class and mask; false when these kernels have nothing to do
 * with the row (a top-k row, or a wide row without survivors). */
__device__ __forceinline__ bool row_mask(const FullArgs& a, int row, const RowIn& ri, Mask& k)
{
    k.cls = row_class(a, ri.p.top_k);
    k.state = kSelAll;
    k.tau = 0u;
    k.idx_thr = INT_MAX;
    k.bits = nullptr;
    if (k.cls == kRowTopk) return false;
    if (k.cls == kRowWide) {
        const WideSel s = a.ws.sel[row];
        k.state = s.state;
        k.tau = s.tau;
        k.idx_thr = s.idx_thr;
        k.bits = a.ws.bits + (int64_t)row * a.ws.bits_stride;
        if (s.state == kSelEmpty) return false;
    }
    return true;
}

__device__ __forceinline__ bool takes_part(const Mask& k, float x, int64_t idx)
{
    if (k.cls == kRowFull) return true;
    const uint32_t key = cand_key(x); /* 0: at or below -1e30, never a survivor */
    if (key > k.tau) return true;
    if (key != k.tau) return false;
    if (k.state == kSelLowest) return idx <= k.idx_thr;
    if (k.state == kSelBits) return (k.bits[idx >> 5] >> (idx & 31)) & 1u;
    return true;
}

/* The 16 consecutive terms of one thread as raw bits: binary32 bits, or the
 * 16-bit bf16 code.  Terms at or beyond V are 0 and not counted. */
template <int DT>
__device__ __forceinline__ int load16(const char* rowp, int64_t e0, int V,
                                      uint32_t (&raw)[kFullPer])
{
    const int nvalid = (int)(V - e0 < 0 ? 0 : (V - e0 > kFullPer ? kFullPer : V - e0));
    if (nvalid == kFullPer) {
        if constexpr (DT == 0) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 w = reinterpret_cast<const uint4*>(rowp + e0 * 4)[q];
                raw[4 * q] = w.x;
                raw[4 * q + 1] = w.y;
                raw[4 * q + 2] = w.z;
                raw[4 * q + 3] = w.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const uint4 w = reinterpret_cast<const uint4*>(rowp + e0 * 2)[q];
                const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    raw[8 * q + 2 * i] = ww[i] & 0xFFFFu;
                    raw[8 * q + 2 * i + 1] = ww[i] >> 16;
                }
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < kFullPer; ++j) {
            raw[j] = 0u;
            if (j < nvalid) {
                if constexpr (DT == 0)
                    raw[j] = reinterpret_cast<const uint32_t*>(rowp)[e0 + j];
                else
                    raw[j] = reinterpret_cast<const uint16_t*>(rowp)[e0 + j];
            }
        }
    }
    return nvalid;
}

template <int DT>
__device__ __forceinline__ float x_of(uint32_t raw)
{
    return DT == 0 ? __uint_as_float(raw) : __uint_as_float(raw << 16);
}

template <int DT>
__device__ __forceinline__ const char* row_ptr(const FullArgs& a, int row)
{
    return reinterpret_cast<const char*>(a.logits) + (int64_t)row * a.row_stride * Elem<DT>::SIZE;
}

/* y = softcap(x) [* 1/T] exactly as the reference rounds it: the full-row
 * form Tanh(x * fl32(1/cap)) * cap (Layers.pas:309-314) or the top-k form
 * cap * Tanh(x / cap) (Model.pas:2776), then * fl32(1/T) (Model.pas:
 * 2703-2708, 2780-2785). */
__device__ __forceinline__ float y_exact(float x, int cls, float cap, float inv_cap, int scale,
                                         float inv_t)
{
    float y = x;
    if (cap > 0.0f)
        y = cls == kRowWide ? softcap_topk_cr32(x, cap) : softcap_full_cr32(x, inv_cap, cap);
    if (scale) y = y * inv_t;
    return y;
}

/* A cheap approximation of y for the binade predictions only (a few ulps
 * to ~1e-4 relative; the chains verify every step, so a poor prediction
 * only costs a re-evaluation). */
__device__ __forceinline__ float y_approx(float x, float cap, float inv_cap, int scale, float inv_t)
{
    float y = x;
    if (cap > 0.0f) {
        /* cap * tanh(w) = cap - 2 cap / (e^(2w) + 1): branch-free, absolute
         * error a few cap * 2^-24 (what the predictions need) */
        const float w = x * inv_cap;
        const float wc = __builtin_fminf(__builtin_fmaxf(w, -12.0f), 12.0f);
        const float e2 = __builtin_amdgcn_exp2f(wc * 2.8853900817779268f); /* e^(2w) */
        y = cap - (2.0f * cap) * __builtin_amdgcn_rcpf(e2 + 1.0f);
    }
    if (scale) y = y * inv_t;
    return y;
}

__device__ __forceinline__ float wave_sum_f32(float v)
{
#define G4S_FSTEP(ctrl, rmask)                                                                  \
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, rmask, 0xf, false))
    G4S_FSTEP(0x111, 0xf);
    G4S_FSTEP(0x112, 0xf);
    G4S_FSTEP(0x114, 0xf);
    G4S_FSTEP(0x118, 0xf);
    G4S_FSTEP(0x142, 0xa);
    G4S_FSTEP(0x143, 0xc);
#undef G4S_FSTEP
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

/* The table holds the codes whose |x| lies in the 16 binades from win_lo
 * up, entry (sign << 11) | (binade - win_lo) << 7 | mantissa.  With
 * d = code - (win_lo << 7) that entry is (d & 0x7FF) | ((code >> 4) & 0x800)
 * (bit 11 of code >> 4 is the sign: the exponent field shifted right by 4
 * stays below 0x800), and the code is in the window exactly when bits 11-14
 * of d are 0 (a code below the window borrows into them: win_lo <= 240). */
__device__ __forceinline__ uint32_t tab_index(uint32_t code, uint32_t base, uint32_t& d)
{
    d = code - base;
    return (d & 0x7FFu) | ((code >> 4) & 0x800u);
}
constexpr uint32_t kTabMiss = 0x7800u;

struct Ctx {
    float cap, inv_cap, inv_t, m;
    int scale, win_lo, cls;
    float inv, lsum; /* for p (after the LSum chain) */
};

/* e of one term evaluated from x (kept out of line: it is the rare case for
 * bf16 logits, whose codes are tabulated). */
__device__ __noinline__ float e_direct(float x, Ctx c)
{
    return exp_diff_cr32(y_exact(x, c.cls, c.cap, c.inv_cap, c.scale, c.inv_t), c.m);
}

/* p of one term from its e: RN32(e * fl32(1/LSum)) on a full row
 * (Tensors.pas:666-672), RN32(e / LSum) on a wide row (Model.pas:2800-2801). */
__device__ __forceinline__ float p_of(float e, int cls, float inv, float lsum)
{
    return cls == kRowWide ? div_cr32(e, lsum) : e * inv;
}

/* p of one term evaluated from x (out of line, as e_direct). */
__device__ __noinline__ float p_direct(float x, Ctx c)
{
    return p_of(e_direct(x, c), c.cls, c.inv, c.lsum);
}

/* The e of one lane's 16 terms (0 for terms that do not take part), or,
 * with P, their p (the table then holds p).  For bf16 logits every term
 * reads the table (no branch); the rare codes outside its window are
 * evaluated afterwards, behind one wave-uniform branch.  Returns true when
 * every term of the wave came from the table. */
template <int DT, bool GENERAL, bool P>
__device__ __forceinline__ bool terms_e_t(const uint32_t (&raw)[kFullPer], int nvalid,
                                          int64_t e0, const Ctx& c, const Mask& k,
                                          const float* tab, float (&t)[kFullPer])
{
    if (DT == 1 && c.win_lo >= 0) {
        const uint32_t base = (uint32_t)c.win_lo << 7;
        uint32_t anymiss = 0u;
        bool part[kFullPer];
#pragma unroll
        for (int j = 0; j < kFullPer; ++j) {
            part[j] = GENERAL ? (j < nvalid && takes_part(k, x_of<DT>(raw[j]), e0 + j)) : true;
            uint32_t d;
            const float v = tab[tab_index(raw[j], base, d)];
            t[j] = part[j] ? v : 0.0f;
            anymiss |= part[j] ? (d & kTabMiss) : 0u;
        }
        if (__ballot(anymiss != 0u) == 0) return true;
#pragma unroll
        for (int j = 0; j < kFullPer; ++j) {
            uint32_t d;
            (void)tab_index(raw[j], base, d);
            if (part[j] && (d & kTabMiss) != 0u)
                t[j] = P ? p_direct(x_of<DT>(raw[j]), c) : e_direct(x_of<DT>(raw[j]), c);
        }
        return false;
    }
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) {
        const bool part = GENERAL ? (j < nvalid && takes_part(k, x_of<DT>(raw[j]), e0 + j)) : true;
        t[j] = part ? (P ? p_direct(x_of<DT>(raw[j]), c) : e_direct(x_of<DT>(raw[j]), c)) : 0.0f;
    }
    return false;
}

/* Two 16-bit lanes of one dword, subtracted lane-wise (v_pk_sub_u16). */
__device__ __forceinline__ uint32_t pk_sub_u16(uint32_t a, uint32_t b)
{
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t,
                              __builtin_bit_cast(u16x2, a) - __builtin_bit_cast(u16x2, b));
}

/* The table terms of a whole bf16 chunk of a full row straight from its two
 * 16-byte loads: the table index of both codes of a dword at once (16-bit
 * lane arithmetic; the same index and window test as tab_index).  Returns
 * false, uniformly, when some code of the wave lies outside the table
 * window (the caller then takes the general route). */
__device__ __forceinline__ bool terms_bf16_whole(const char* rowp, int64_t e0, const Ctx& c,
                                                 const float* tab, float (&t)[kFullPer])
{
    const uint32_t base = (uint32_t)c.win_lo << 7;
    const uint32_t base2 = base | (base << 16);
    uint32_t miss = 0u;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint4 w4 = reinterpret_cast<const uint4*>(rowp + e0 * 2)[q];
        const uint32_t ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t d = pk_sub_u16(ww[i], base2);
            const uint32_t ix = (d & 0x07FF07FFu) | ((ww[i] >> 4) & 0x08000800u);
            miss |= d & (kTabMiss | (kTabMiss << 16));
            t[8 * q + 2 * i] = tab[ix & 0xFFFFu];
            t[8 * q + 2 * i + 1] = tab[ix >> 16];
        }
    }
    return __ballot(miss != 0u) == 0;
}

/* Whole chunks of full rows (the common case) skip the per-term mask. */
template <int DT, bool P = false>
__device__ __forceinline__ bool terms_e(const uint32_t (&raw)[kFullPer], int nvalid, int64_t e0,
                                        const Ctx& c, const Mask& k, const float* tab,
                                        float (&t)[kFullPer])
{
    if (k.cls == kRowWide || nvalid < kFullPer)
        return terms_e_t<DT, true, P>(raw, nvalid, e0, c, k, tab, t);
    return terms_e_t<DT, false, P>(raw, nvalid, e0, c, k, tab, t);
}

/* ------------------------------------------------------ block helpers */

struct Scratch {
    PMap wmap[NWF];
    int32_t went[NWF];
    int32_t tcand[NWF];
    uint32_t ured[3 * NWF];
    float fred[NWF];
    double dred[NWF];
    int32_t iscan[NWF];
    int32_t misc[16];
};


__device__ __forceinline__ uint32_t block_max_key(uint32_t v, Scratch& sh, int slot)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wave_max_u32(v);
    if (lane == 0) sh.ured[slot * NWF + wid] = v;
    __syncthreads();
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < NWF; ++w) r = g4s_max_u(r, sh.ured[slot * NWF + w]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint32_t block_min_u(uint32_t v, Scratch& sh)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wave_min_u32(v);
    if (lane == 0) sh.ured[wid] = v;
    __syncthreads();
    uint32_t r = 0xFFFFFFFFu;
#pragma unroll
    for (int w = 0; w < NWF; ++w) r = g4s_min_u(r, sh.ured[w]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ int block_sum_int(int v, Scratch& sh)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wave_sum_i32(v);
    if (lane == 0) sh.iscan[wid] = v;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int w = 0; w < NWF; ++w) r += sh.iscan[w];
    __syncthreads();
    return r;
}

/* One DPP step of an inclusive wave scan of doubles: both halves move
 * together; a lane without a source adds +0. */
template <int CTRL, int RMASK>
__device__ __forceinline__ double dpp_add_d(double x)
{
    const uint64_t b = (uint64_t)__double_as_longlong(x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, RMASK, 0xf, false);
    const uint32_t hi =
        (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, RMASK, 0xf, false);
    return x + __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

/* Inclusive scan of doubles over the wave in lane order (DPP, as the
 * integer scans). */
__device__ __forceinline__ double wave_incl_scan_d(double x)
{
    x = dpp_add_d<0x111, 0xf>(x);
    x = dpp_add_d<0x112, 0xf>(x);
    x = dpp_add_d<0x114, 0xf>(x);
    x = dpp_add_d<0x118, 0xf>(x);
    x = dpp_add_d<0x142, 0xa>(x);
    x = dpp_add_d<0x143, 0xc>(x);
    return x;
}

/* Exclusive prefix over the workgroup in thread order (doubles), and the
 * workgroup's total. */
__device__ __forceinline__ double block_excl_scan_d(double v, Scratch& sh, double& total)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const double x = wave_incl_scan_d(v);
    if (lane == 63) sh.dred[wid] = x;
    __syncthreads();
    double off = 0.0, tot = 0.0;
#pragma unroll
    for (int w = 0; w < NWF; ++w) {
        const double d = sh.dred[w];
        off += (w < wid) ? d : 0.0;
        tot += d;
    }
    __syncthreads();
    total = tot;
    return off + x - v;
}

/* Exclusive prefix over the workgroup in thread order (ints). */
__device__ __forceinline__ int block_excl_scan_i(int v, Scratch& sh, int& total)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int x = wave_inclusive_scan(v);
    if (lane == 63) sh.iscan[wid] = x;
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NWF; ++w) {
        off += (w < wid) ? sh.iscan[w] : 0;
        tot += sh.iscan[w];
    }
    total = tot;
    __syncthreads();
    return off + x - v;
}

/* Inclusive scan of running-sum maps over the wave, in lane order (lane i
 * gets the composition of lanes 0..i); lanes without a source add the
 * identity (0, 0). */
__device__ __forceinline__ PMap wave_scan_maps(PMap f)
{
#define G4S_MAP_STEP(ctrl, rmask)                                                      \
    do {                                                                               \
        PMap o;                                                                        \
        o.d0 = __builtin_amdgcn_update_dpp(0, f.d0, ctrl, rmask, 0xf, false);          \
        o.d1 = __builtin_amdgcn_update_dpp(0, f.d1, ctrl, rmask, 0xf, false);          \
        f = ss::map_sat(ss::map_then(o, f));                                           \
    } while (0)
    G4S_MAP_STEP(0x111, 0xf);
    G4S_MAP_STEP(0x112, 0xf);
    G4S_MAP_STEP(0x114, 0xf);
    G4S_MAP_STEP(0x118, 0xf);
    G4S_MAP_STEP(0x142, 0xa);
    G4S_MAP_STEP(0x143, 0xc);
#undef G4S_MAP_STEP
    return f;
}

/* The previous lane's value (lane 0: the identity). */
__device__ __forceinline__ PMap wave_shift_map(PMap f)
{
    PMap o;
    o.d0 = __builtin_amdgcn_update_dpp(0, f.d0, 0x138, 0xf, 0xf, false);
    o.d1 = __builtin_amdgcn_update_dpp(0, f.d1, 0x138, 0xf, 0xf, false);
    return o;
}

/* The map of one thread's terms in binade e (terms beyond the row are 0,
 * and a 0 term is the identity). */
__device__ __forceinline__ PMap thread_map(const float (&t)[kFullPer], int nvalid, int32_t e)
{
    (void)nvalid;
    /* Without a half-unit tie every term adds c = rint(q) units, q = a/u =
     * ldexp(a, 150-E) exact, whatever the parity: the map is (C, C) with C
     * the sum of the c (summed in binary32: exact below 2^24, and a sum
     * that reaches 2^24 means the thread leaves the binade either way).  A
     * tie (fract(q) == 1/2) anywhere in the wave takes the exact per-term
     * lane maps of ss::lane_map (wave-uniform branch). */
    float cs = 0.0f;
    bool tie = false;
    const int sh = 150 - e;
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) {
        const float q = __builtin_ldexpf(t[j], sh);
        cs += __builtin_rintf(q);
        tie = tie || __builtin_amdgcn_fractf(q) == 0.5f;
    }
    PMap f;
    if (__ballot(tie) == 0) {
        f.d0 = (int32_t)__builtin_fminf(cs, 67108864.0f); /* 2^26, as map_sat caps */
        f.d1 = f.d0;
        return f;
    }
    return ss::lane_map(t, kFullPer, e);
}

/* The lane map without the tie vote, for waves whose terms are known to
 * hold no half-unit tie in binade e (every term tabulated, and the row's
 * tie mask clear for e). */
__device__ __forceinline__ PMap thread_map_nt(const float (&t)[kFullPer], int32_t e)
{
    float cs = 0.0f;
    const int sh = 150 - e;
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) cs += __builtin_rintf(__builtin_ldexpf(t[j], sh));
    PMap f;
    f.d0 = f.d1 = (int32_t)__builtin_fminf(cs, 67108864.0f);
    return f;
}

/* A value v > 0 is a half-unit tie in binade E (fract(v / 2^(E-150)) ==
 * 1/2) exactly when its lowest set bit is 2^(E-151), E = (lowest set bit's
 * exponent) + 151.  A row's tie mask records, for the 64 binades from `base`
 * on, whether a value of its table is a tie there; binades outside the
 * window count as possible ties. */
constexpr int kTieBaseE = 120; /* LSum >= 1: binades 127 and up */
constexpr int kTieBaseP = 72;  /* running sums of p <= 1: binades up to 127 */

/* The 64-bit window mask of one value (0: no tie inside the window). */
__device__ __forceinline__ uint64_t tie_bits(float v, int base)
{
    const uint32_t b = __float_as_uint(v);
    const int ef = (int)(b >> 23);
    const uint32_t sig = (b & 0x7FFFFFu) | (ef ? 0x800000u : 0u);
    const int E = (ef ? ef : 1) + (int)__builtin_ctz(sig | 0x1000000u) + 1 - base;
    return (b != 0u && (unsigned)E < 64u) ? (1ull << E) : 0ull;
}

__device__ __forceinline__ bool tie_possible(uint64_t mask, int base, int32_t e)
{
    const int i = e - base;
    return (unsigned)i >= 64u || ((mask >> i) & 1ull) != 0ull;
}

/* OR over the wave of a 64-bit value (every lane gets it): DPP scans of
 * both halves, lane 63's result broadcast. */
__device__ __forceinline__ uint32_t g4s_or_u(uint32_t a, uint32_t b) { return a | b; }
__device__ __forceinline__ uint64_t wave_or64(uint64_t v)
{
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    G4S_DPP_SCAN(lo, g4s_or_u, 0u, uint32_t);
    G4S_DPP_SCAN(hi, g4s_or_u, 0u, uint32_t);
    lo = (uint32_t)__builtin_amdgcn_readlane((int)lo, 63);
    hi = (uint32_t)__builtin_amdgcn_readlane((int)hi, 63);
    return ((uint64_t)hi << 32) | lo;
}

/* ------------------------------------------------------- wave helpers */

/* The map of a wave's 1024 terms (every lane gets it): the sum of constant
 * thread maps, or the composition of the thread maps in lane order. */
__device__ __forceinline__ PMap wave_chunk_map(PMap f)
{
    PMap r;
    if (__ballot(f.d0 != f.d1) == 0) {
        /* a thread map >= 2^24 leaves the binade whatever follows: capping it
         * there keeps the sum of 64 below 2^31 */
        const int32_t c = f.d0 > ss::kTop ? ss::kTop : f.d0;
        int32_t s = wave_sum_i32(c);
        s = s > (1 << 26) ? (1 << 26) : s;
        r.d0 = r.d1 = s;
        return r;
    }
    const PMap incl = wave_scan_maps(f);
    r.d0 = __builtin_amdgcn_readlane(incl.d0, 63);
    r.d1 = __builtin_amdgcn_readlane(incl.d1, 63);
    return r;
}

/*
 * One resolution round over a chunk held by the wave (lane l holds terms
 * l*16 .. l*16+15, 0 beyond the row): `f` are this round's lane maps in the
 * binade of `st` (identity for lanes before `pos`, which are accounted for).
 * The maps are composed over the wave and applied to st; if every lane stays
 * in the binade (and below thr) st becomes the state after the chunk and the
 * round returns true.  Otherwise the first lane ls that leaves (or reaches
 * thr) enters exactly at its composed state, so it adds its terms to that
 * sum with plain binary32 additions: st becomes the state after lane ls, pos
 * ls + 1, and *hit the chunk-relative index of the first term whose running
 * sum reaches thr, if one does.  Wave-uniform control flow.
 */
__device__ __forceinline__ bool round_step(PMap f, const float (&t)[kFullPer], State& st,
                                           float thr, int& pos, int* hit)
{
    const int lane = threadIdx.x & 63;
    const int32_t e = st.e;
    int32_t m_in, m_out;
    if (__ballot(f.d0 != f.d1) == 0) {
        /* constant maps: a prefix sum (a lane's map >= 2^24 leaves anyway) */
        const int32_t c = f.d0 > ss::kTop ? ss::kTop : f.d0;
        const int32_t x = wave_inclusive_scan(c); /* <= 2^30 */
        m_in = st.m + (x - c);
        m_out = st.m + x;
    } else {
        const PMap incl = wave_scan_maps(f);
        const PMap excl = wave_shift_map(incl);
        m_in = ss::map_apply(excl, st.m);
        m_in = m_in >= ss::kTop ? ss::kTop : m_in;
        m_out = m_in >= ss::kTop ? ss::kTop : ss::map_apply(f, m_in);
    }
    const uint64_t bal =
        __ballot(lane >= pos && (m_out >= ss::kTop || ss::value_of(State{e, m_out}) >= thr));
    if (bal == 0) {
        st.m = __builtin_amdgcn_readlane(m_out, 63);
        return true;
    }
    const int ls = (int)__builtin_ctzll(bal);
    /* every lane adds its terms from its own entering sum (no divergence;
     * only lane ls's is used); terms are >= 0, so the running sum is
     * monotone and the first term reaching thr follows the count of partial
     * sums below it */
    float sum = ss::value_of(State{e, m_in < ss::kTop ? m_in : 0});
    int below = 0;
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) {
        sum = sum + t[j];
        below += sum < thr ? 1 : 0;
    }
    sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sum), ls));
    below = __builtin_amdgcn_readlane(below, ls);
    st = ss::state_of(sum);
    if (sum >= thr) *hit = ls * kFullPer + below;
    pos = ls + 1;
    return false;
}

/* Exact evaluation of one chunk held by the wave from the exact entering
 * state st, lanes from `pos` on: rounds with the lane maps in the current
 * binade.  Returns the state after the chunk, or at the term reaching thr
 * (*hit, chunk-relative; -1: none). */
__device__ State resolve_wave(const float (&t)[kFullPer], int nvalid, State st, float thr,
                              int pos, int* hit, int* rounds)
{
    const int lane = threadIdx.x & 63;
    while (pos < 64) {
        ++*rounds;
        PMap f = thread_map(t, nvalid, st.e); /* every lane: thread_map votes over the wave */
        if (lane < pos) f = ss::map_identity();
        if (round_step(f, t, st, thr, pos, hit) || *hit >= 0) break;
    }
    return st;
}

/* The first kHeadLanes lanes of a row's first chunk, one lane after the
 * other with plain binary32 additions (the running sum changes binade every
 * few terms there). */
constexpr int kHeadLanes = 8;
[[maybe_unused]] __device__ State head_walk(const float (&t)[kFullPer], float thr, int* hit)
{
    float s = 0.0f;
    for (int l = 0; l < kHeadLanes; ++l) {
        float x = s;
        int below = 0;
#pragma unroll
        for (int j = 0; j < kFullPer; ++j) {
            x = x + t[j];
            below += x < thr ? 1 : 0;
        }
        s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
        below = __builtin_amdgcn_readlane(below, l);
        if (s >= thr) {
            *hit = l * kFullPer + below;
            break;
        }
    }
    return ss::state_of(s);
}

/* The first n terms (a multiple of 64) of a staged chunk (terms in index
 * order in LDS) added term by term with plain binary32 additions from 0,
 * every lane computing the same sum from broadcast reads: the head of a
 * row's first chunk, where the running sum changes binade every few dozen
 * terms, costs less this way than round after round of lane maps.  The
 * running sum is monotone, so a 64-term block whose end reaches thr is
 * walked again to find the first term that does (*hit, chunk-relative). */
constexpr int kSeqLanes = 24; /* lanes of the first chunk walked term by term */
__device__ State seq_walk(const float* tv, int n, float thr, int* hit)
{
    float s = 0.0f;
    for (int b = 0; b < n; b += 64) {
        const float4* src = reinterpret_cast<const float4*>(tv + b);
        const float s0 = s;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const float4 x = src[q];
            s = s + x.x;
            s = s + x.y;
            s = s + x.z;
            s = s + x.w;
        }
        if (s >= thr) {
            float u = s0;
            for (int j = 0; j < 64; ++j) {
                u = u + tv[b + j];
                if (u >= thr) {
                    *hit = b + j;
                    return ss::state_of(u);
                }
            }
        }
    }
    return ss::state_of(s);
}

/*
 * Chain the chunk maps from chunk c on, 64 chunks per step: the maps are
 * composed over the wave and applied to the entering state, and accepted up
 * to the first chunk whose map does not apply -- a chunk applies when the
 * sum enters it in the predicted binade and stays in that binade (and, for
 * the draw, below thr).  Returns that chunk (nch: none) with `st` the exact
 * state entering it; cpost (when given) gets the exact running sum after
 * every accepted chunk.  One wave; wave-uniform control flow.
 */
template <bool THR>
__device__ int walk_maps(const PMap* cm, const int32_t* cb, int c, int nch, State& st, float thr,
                         float* cpost)
{
    const int lane = threadIdx.x & 63;
    for (int g = c; g < nch; g += 64) {
        const int cc = g + lane;
        const bool valid = cc < nch;
        const PMap f = valid ? cm[cc] : ss::map_identity();
        const int32_t be = valid ? cb[cc] : -1;
        int32_t m_after;
        if (__ballot(f.d0 != f.d1) == 0) {
            const int32_t x = wave_inclusive_scan(f.d0 > ss::kTop ? ss::kTop : f.d0);
            m_after = st.m + x;
        } else {
            m_after = ss::map_apply(wave_scan_maps(f), st.m);
        }
        bool bad = !valid || be != st.e || m_after >= ss::kTop;
        if (THR) bad = bad || ss::value_of(State{st.e, m_after}) >= thr;
        const uint64_t bal = __ballot(bad);
        const int l = bal ? (int)__builtin_ctzll(bal) : 64;
        if (cpost && lane < l) cpost[cc] = ss::value_of(State{st.e, m_after});
        if (l > 0) st.m = __builtin_amdgcn_readlane(m_after, l - 1);
        if (l < 64) return g + l < nch ? g + l : nch;
    }
    return nch;
}

/* 16 terms of a lane from a staged (full) chunk in LDS. */
template <int DT>
__device__ __forceinline__ void stage16(const char* src, uint32_t (&raw)[kFullPer])
{
    if constexpr (DT == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4 w = reinterpret_cast<const uint4*>(src)[q];
            raw[4 * q] = w.x;
            raw[4 * q + 1] = w.y;
            raw[4 * q + 2] = w.z;
            raw[4 * q + 3] = w.w;
        }
    } else {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint4 w = reinterpret_cast<const uint4*>(src)[q];
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                raw[8 * q + 2 * i] = ww[i] & 0xFFFFu;
                raw[8 * q + 2 * i + 1] = ww[i] >> 16;
            }
        }
    }
}

/* Most chunks a chain precomputes: the ones it is predicted to re-evaluate
 * (where the running sum changes binade, chunk 0, the draw's last chunk). */
constexpr int kStageMax = 16;

/* A staged chunk's lane maps in its predicted binade b and in b + 1. */
struct StageMaps {
    PMap lo[64];
    PMap hi[64];
    int32_t b;
    int32_t pad[3];
};

/* LDS of a chain workgroup (dynamic shared memory): the e table, the chunk
 * maps and predicted binades, the exact running sum after every chunk, the
 * staged chunk numbers, and per staged chunk its maps and its terms (lane l's
 * 16 terms at l*16). */
struct ChainLds {
    float* tab;
    PMap* cm;
    int32_t* cb;
    float* cpost;
    int32_t* sid;
    StageMaps* sm;
    float* tv;
};

__host__ __device__ __forceinline__ size_t chain_lds_layout(int dt, int nch, int nstage, size_t* off)
{
    size_t o = 0;
    off[0] = o;
    o += dt == 1 ? (size_t)kFullTab * 4 : 0;
    off[1] = o;
    o += (size_t)nch * sizeof(PMap);
    off[2] = o;
    o += (size_t)nch * 4;
    off[3] = o;
    o += (size_t)nch * 4;
    off[4] = o;
    o += (size_t)kStageMax * 4;
    o = (o + 15) & ~(size_t)15;
    off[5] = o;
    o += (size_t)nstage * sizeof(StageMaps);
    o = (o + 15) & ~(size_t)15;
    off[6] = o;
    o += (size_t)nstage * kFullChunk * 4;
    return o;
}

template <int DT>
__device__ __forceinline__ ChainLds chain_lds(char* base, int nch, int nstage)
{
    size_t off[7];
    (void)chain_lds_layout(DT, nch, nstage, off);
    ChainLds L;
    L.tab = reinterpret_cast<float*>(base + off[0]);
    L.cm = reinterpret_cast<PMap*>(base + off[1]);
    L.cb = reinterpret_cast<int32_t*>(base + off[2]);
    L.cpost = reinterpret_cast<float*>(base + off[3]);
    L.sid = reinterpret_cast<int32_t*>(base + off[4]);
    L.sm = reinterpret_cast<StageMaps*>(base + off[5]);
    L.tv = reinterpret_cast<float*>(base + off[6]);
    return L;
}

/* The 16 terms (e, or p when P) of lane `lane` in chunk c. */
template <int DT, bool P>
__device__ __forceinline__ int chain_load_terms(const FullArgs& a, const char* rowp, int c,
                                                const Ctx& ctx, const Mask& k, const FullRow& r,
                                                const float* tab, float (&t)[kFullPer])
{
    const int lane = threadIdx.x & 63;
    uint32_t raw[kFullPer];
    const int64_t e0 = (int64_t)c * kFullChunk + (int64_t)lane * kFullPer;
    const int nv = load16<DT>(rowp, e0, a.vocab, raw);
    (void)r;
    terms_e<DT, P>(raw, nv, e0, ctx, k, tab, t);
    return nv;
}

/*
 * Prologue of a chain workgroup (all threads): the row's table, the chunk
 * maps and binades of chunks 0..clast (identity and -1 beyond), the first
 * `nstage` full chunks that `pred` selects, and for each of those (one wave
 * per chunk) its terms and its lanes' constant maps in its predicted binade
 * and the next.  Ends with a barrier.
 */
/* Chain workgroups: 16 waves for the prologue (one staged chunk each), then
 * wave 0 alone. */
constexpr int kChainBlock = 1024;
constexpr int kChainWaves = kChainBlock / 64;
constexpr int kChainCPT = kFullMaxChunks / kChainBlock;
static_assert(kFullTab / 4 == kChainBlock, "one float4 of the table per thread");
static_assert(kStageMax % kChainWaves == 0, "staged chunks per wave");

struct ChainScratch {
    int32_t iscan[kChainWaves];
    uint32_t lastw[kChainWaves];
    uint32_t pm[2];
    float lsum, inv;
    int32_t argmax, reev, rounds;
};

/* Exclusive prefix over the chain workgroup in thread order (ints). */
__device__ __forceinline__ int chain_excl_scan(int v, ChainScratch& sh, int& total)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int x = wave_inclusive_scan(v);
    if (lane == 63) sh.iscan[wid] = x;
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kChainWaves; ++w) {
        off += (w < wid) ? sh.iscan[w] : 0;
        tot += sh.iscan[w];
    }
    total = tot;
    __syncthreads();
    return off + x - v;
}

template <int DT, bool P, typename Pred>
__device__ void chain_prologue(const FullArgs& a, int row, const FullRow& r, const Ctx& ctx,
                               const Mask& k, const PMap* gmap, const int32_t* gbeta, int clast,
                               Pred pred, const ChainLds& L, ChainScratch& sh)
{
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int nch = a.nch;
    const int V = a.vocab;
    const int nstage = a.nstage;
    if (DT == 1 && r.win_lo >= 0) {
        const float4* src =
            reinterpret_cast<const float4*>((P ? a.ws.ptab : a.ws.etab) + (int64_t)row * kFullTab);
        reinterpret_cast<float4*>(L.tab)[tid] = src[tid]; /* kFullTab / 4 == kChainBlock */
    }
    for (int c = tid; c < nch; c += kChainBlock) {
        L.cm[c] = c <= clast ? gmap[c] : ss::map_identity();
        L.cb[c] = c <= clast ? gbeta[c] : -1;
    }
    /* the staged chunks: the first nstage full chunks in index order that
     * pred selects (thread t looks at chunks t*cpt .. t*cpt+cpt-1) */
    const int cpt = (nch + kChainBlock - 1) / kChainBlock;
    uint32_t selm = 0u;
    int cnt = 0;
#pragma unroll
    for (int q = 0; q < kChainCPT; ++q) {
        const int c = tid * cpt + q;
        if (q < cpt && c < nch && c <= clast && (int64_t)(c + 1) * kFullChunk <= V && pred(c)) {
            selm |= 1u << q;
            ++cnt;
        }
    }
    int total;
    int pos = chain_excl_scan(cnt, sh, total);
#pragma unroll
    for (int q = 0; q < kChainCPT; ++q) {
        if (selm & (1u << q)) {
            if (pos < nstage) L.sid[pos] = tid * cpt + q;
            ++pos;
        }
    }
    if (tid < kStageMax && tid >= (total < nstage ? total : nstage)) L.sid[tid] = -1;
    __syncthreads();
    /* wave w precomputes slot w */
    constexpr int kSlots = kStageMax / kChainWaves;
    constexpr int kVec = kFullPer * Elem<DT>::SIZE / 16; /* 16-byte loads per lane per chunk */
    const char* rowp = row_ptr<DT>(a, row);
    uint4 pk[kSlots][kVec];
    int cs[kSlots];
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
        const int sl = wid + i * kChainWaves;
        cs[i] = sl < nstage ? L.sid[sl] : -1;
        if (cs[i] >= 0) {
            const uint4* src = reinterpret_cast<const uint4*>(
                rowp + ((int64_t)cs[i] * kFullChunk + (int64_t)lane * kFullPer) * Elem<DT>::SIZE);
#pragma unroll
            for (int q = 0; q < kVec; ++q) pk[i][q] = src[q];
        }
    }
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
        const int c = cs[i];
        if (c < 0) continue;
        const int sl = wid + i * kChainWaves;
        uint32_t raw[kFullPer];
#pragma unroll
        for (int q = 0; q < kVec; ++q) {
            const uint32_t w4[4] = {pk[i][q].x, pk[i][q].y, pk[i][q].z, pk[i][q].w};
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                if (DT == 0) {
                    raw[4 * q + m] = w4[m];
                } else {
                    raw[8 * q + 2 * m] = w4[m] & 0xFFFFu;
                    raw[8 * q + 2 * m + 1] = w4[m] >> 16;
                }
            }
        }
        float t[kFullPer];
        const int64_t e0 = (int64_t)c * kFullChunk + (int64_t)lane * kFullPer;
        terms_e<DT, P>(raw, kFullPer, e0, ctx, k, L.tab, t);
        float4* dst = reinterpret_cast<float4*>(L.tv + (size_t)sl * kFullChunk + lane * kFullPer);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            dst[q] = make_float4(t[4 * q], t[4 * q + 1], t[4 * q + 2], t[4 * q + 3]);
        const int32_t b = gbeta[c] < 1 ? 1 : (gbeta[c] > 253 ? 253 : gbeta[c]);
        L.sm[sl].lo[lane] = thread_map(t, kFullPer, b);
        L.sm[sl].hi[lane] = thread_map(t, kFullPer, b + 1);
        if (lane == 0) L.sm[sl].b = b;
    }
    __syncthreads();
}

/*
 * The exact running sum through chunk c from the exact entering state st,
 * by the chain wave: chunk 0 starts with the sequential head; a staged chunk
 * takes its precomputed lane maps for the predicted binade and the next (a
 * crossing into the next binade then costs two map compositions and one
 * lane's plain additions); anything else takes the general rounds.  *hit gets
 * the chunk-relative index of the first term whose running sum reaches thr
 * (-1: none).
 */
template <int DT, bool P>
__device__ State chain_chunk(const FullArgs& a, const char* rowp, int c, State st, float thr,
                             const ChainLds& L, const Ctx& ctx, const Mask& k, const FullRow& r,
                             int* hit, int* rounds)
{
    const int lane = threadIdx.x & 63;
    const int sl = lane < a.nstage ? L.sid[lane] : -1;
    const uint64_t hb = __ballot(sl == c);
    float t[kFullPer];
    int nv = kFullPer;
    int pos = 0;
    *hit = -1;
    if (hb) {
        const int s = (int)__builtin_ctzll(hb);
        const float4* src =
            reinterpret_cast<const float4*>(L.tv + (size_t)s * kFullChunk + lane * kFullPer);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = src[q];
            t[4 * q] = v.x;
            t[4 * q + 1] = v.y;
            t[4 * q + 2] = v.z;
            t[4 * q + 3] = v.w;
        }
        const StageMaps* sm = L.sm + s;
        const int32_t b = sm->b;
        if (c == 0) {
            st = seq_walk(L.tv + (size_t)s * kFullChunk, kSeqLanes * kFullPer, thr, hit);
            if (*hit >= 0) return st;
            pos = kSeqLanes;
        } else if (st.e == b) {
            ++*rounds;
            if (round_step(sm->lo[lane], t, st, thr, pos, hit) || *hit >= 0) return st;
            if (pos < 64 && st.e == b + 1) {
                ++*rounds;
                const PMap f = lane >= pos ? sm->hi[lane] : ss::map_identity();
                if (round_step(f, t, st, thr, pos, hit) || *hit >= 0) return st;
            }
        }
    } else {
        nv = chain_load_terms<DT, P>(a, rowp, c, ctx, k, r, L.tab, t);
        if (c == 0) {
            st = head_walk(t, thr, hit);
            if (*hit >= 0) return st;
            pos = kHeadLanes;
        }
    }
    if (pos < 64) st = resolve_wave(t, nv, st, thr, pos, hit, rounds);
    return st;
}

/* Final outputs of a row (called by wave 0 of the row's workgroup). */
__device__ void write_row_outputs(const FullArgs& a, int row, int32_t id, int32_t argmax, float lsum,
                                  int32_t count, uint32_t flags)
{
    if ((threadIdx.x & 63) == 0) {
        st_sys(&a.ids[row], id);
        if (a.out.count) a.out.count[row] = count;
        if (a.out.argmax) a.out.argmax[row] = argmax;
        if (a.out.lsum) a.out.lsum[row] = lsum;
        if (a.out.flags) st_sys(&a.out.flags[row], flags);
    }
    publish_done(a.done, row, a.seq);
}

__device__ __forceinline__ uint32_t row_flags(const Mask& k)
{
    if (k.cls == kRowFull) return G4S_FLAG_FULL_PATH;
    uint32_t f = G4S_FLAG_TOPK_PATH | G4S_FLAG_WIDE_K;
    if (k.state == kSelLowest) f |= G4S_FLAG_TIE_LOWEST;
    if (k.state == kSelBits) f |= G4S_FLAG_HEAP_REPLAY;
    return f;
}

/* Are outputs per term requested?  Full rows: every p when capacity >= V;
 * wide rows: the first `capacity` survivors. */
__device__ __forceinline__ bool term_outputs(const FullArgs& a, int cls)
{
    if (cls == kRowFull) return a.out.probs && a.out.capacity >= a.vocab;
    return (a.out.probs || a.out.indices) && a.out.capacity >= 1;
}

/* Context of the e evaluation: the row's formula, m and table window. */
__device__ __forceinline__ Ctx make_ctx(const FullArgs& a, const FullRow& r, int cls)
{
    Ctx c;
    c.cap = a.softcap;
    c.inv_cap = c.cap > 0.0f ? div_cr32(1.0f, c.cap) : 1.0f;
    c.inv_t = r.inv_t;
    c.m = r.m;
    c.scale = r.scale;
    c.win_lo = r.win_lo;
    c.cls = cls;
    c.inv = r.inv;
    c.lsum = r.lsum;
    return c;
}

/* Copy the row's e table into LDS (ends with a barrier). */
template <int DT>
__device__ __forceinline__ void load_tab(const float* gtab, int row, const FullRow& r, float* tab)
{
    if (DT == 1 && r.win_lo >= 0) {
        const float4* src = reinterpret_cast<const float4*>(gtab + (int64_t)row * kFullTab);
        float4 v[kFullTab / 4 / kFullBlock];
#pragma unroll
        for (int q = 0; q < kFullTab / 4 / kFullBlock; ++q) v[q] = src[threadIdx.x + q * kFullBlock];
#pragma unroll
        for (int q = 0; q < kFullTab / 4 / kFullBlock; ++q)
            reinterpret_cast<float4*>(tab)[threadIdx.x + q * kFullBlock] = v[q];
    }
    __syncthreads();
}

/* Index of the r-th (1-based) term of chunk cb, in index order, whose key
 * satisfies pred; every thread gets it. */
template <int DT, typename Pred>
__device__ int kth_in_chunk(const FullArgs& a, const char* rowp, int cb, int r, Pred pred,
                            Scratch& sh)
{
    uint32_t raw[kFullPer];
    const int64_t e0 = (int64_t)cb * kSelChunk + (int64_t)threadIdx.x * kFullPer;
    const int nv = load16<DT>(rowp, e0, a.vocab, raw);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) cnt += (j < nv && pred(cand_key(x_of<DT>(raw[j])))) ? 1 : 0;
    int total;
    const int off = block_excl_scan_i(cnt, sh, total);
    if (off < r && r <= off + cnt) {
        int seen = off;
        for (int j = 0; j < nv; ++j)
            if (pred(cand_key(x_of<DT>(raw[j]))) && ++seen == r) {
                sh.misc[13] = (int)(e0 + j);
                break;
            }
    }
    __syncthreads();
    const int res = sh.misc[13];
    __syncthreads();
    return res;
}

}  // namespace

}  // namespace g4s

#endif
