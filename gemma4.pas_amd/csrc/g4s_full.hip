/*
 * g4s_full.hip -- the softmax sampling path on gfx950: full-vocabulary rows
 * (TopK <= 0 or TopK >= V) and wide top-k rows (g4s_max_top_k() < TopK < V).
 *
 * Full rows replace the TopK <= 0 branch of DoSample with CpuLogitSoftcap,
 * DoSampleTopP and CpuSoftmaxF32 (src/Gemma4.Model.pas:2756-2763,
 * 2691-2737; src/Gemma4.Layers.pas:300-316; src/Gemma4.Tensors.pas:638-673):
 *   y_i = RN32(tanh(x_i * fl32(1/cap)) * cap)      (when cap > 0)
 *   y_i = RN32(y_i * fl32(1/T))                      (when T > 0 and T <> 1)
 *   m = max y;  e_i = RN32(exp(y_i - m));  LSum = e_0 + e_1 + ... left to
 *   right in binary32;  p_i = RN32(e_i * fl32(1/LSum));  argmax = first
 *   index of the largest p;  if T > 0: the first i whose left-to-right
 *   binary32 running sum of p reaches fl32(u * TopP), else the argmax.
 *
 * Wide top-k rows replace DoSelectTopKIndices + the top-k tail
 * (Model.pas:2615-2689, 2765-2826) when K is beyond what the single-launch
 * top-k kernel holds on chip.  The survivors are found by a three-pass
 * radix select of the K-th largest key tau over the whole row, with the
 * reference's min-heap tie semantics (lowest index when the heap layout
 * cannot matter, a replay of the heap otherwise).  The tail then runs on
 * the same machinery as a full row with every non-survivor contributing 0
 * (adding +0 leaves a binary32 running sum unchanged), the top-k forms of
 * the arithmetic (y = RN32(cap * tanh(x / cap)), p_i = RN32(e_i / LSum)),
 * and the first survivor as the draw when fl32(u * TopP) <= 0.
 *
 * Rows are cut into chunks of 1024 terms, one wave's: 16 consecutive terms
 * per lane.  The streaming passes give every wave a run of consecutive
 * chunks and use no barrier beyond loading the e table; the two chains are
 * one workgroup per row whose wave 0 walks the row.  Launches (the wide
 * ones only when wide rows can occur; they cut rows into 4096-term select
 * chunks):
 *   wide hist/find x3: 11+11+10-bit MSD radix select of tau (LDS
 *             histograms added into a per-row histogram, one workgroup per
 *             row fixes each digit);
 *   wide ties, ties-find, replay: when tau is tied beyond the slots left,
 *             per-chunk counts locate the K-th key >= tau and the last key
 *             above tau in index order; the rare heap-dependent rows replay
 *             the heap exactly;
 *   1 max:    raw-logit maximum (softcap and 1/T are monotone, so
 *             m = y(max x)) and approximate chunk sums of exp(y - m);
 *   2 row:    the row's m; for bf16 logits, e for the 4096 codes of the 16
 *             largest exponents of |x| (correctly rounded, once per row), so
 *             the streaming passes look e up; the predicted binade of LSum
 *             entering every chunk (a parallel prefix of the estimates);
 *   3 lsum:   each chunk's terms as one exact map of the running sum in its
 *             predicted binade (g4s_seqsum.h);
 *   4 chain:  LSum: the workgroup stages in LDS the chunks where the sum is
 *             predicted to change binade, then wave 0 composes the chunk
 *             maps 64 at a time, verifying every step, and re-evaluates the
 *             chunks whose map does not apply; the argmax; the predicted
 *             binades of the draw's running sum;
 *   5 cdf:    p for the outputs and the same maps for p, up to the chunk
 *             where the running sum is predicted to reach fl32(u*TopP);
 *   6 draw:   the same chain over the maps of p: the exact first index, and
 *             the token.
 * Transcendental steps are correctly rounded (g4s_crmath.h); every running
 * sum is the reference's left-to-right binary32 sum, bit for bit.
 */
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
__device__ State head_walk(const float (&t)[kFullPer], float thr, int* hit)
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
        a.ids[row] = id;
        if (a.out.count) a.out.count[row] = count;
        if (a.out.argmax) a.out.argmax[row] = argmax;
        if (a.out.lsum) a.out.lsum[row] = lsum;
        if (a.out.flags) a.out.flags[row] = flags;
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

/* ------------------------------------------------ wide rows: radix select */

/* Histogram of one digit of the keys that match the digits fixed so far
 * (pass 0: bits 31-21, pass 1: bits 20-10, pass 2: bits 9-0). */
template <int DT>
__global__ __launch_bounds__(kFullBlock) void wide_hist_kernel(FullArgs a, int pass)
{
    __shared__ uint32_t hist[kWideBins];
    const int tid = threadIdx.x;
    const int row = blockIdx.y, b = blockIdx.x;
    const RowIn ri = row_in(a, row);
    if (row_class(a, ri.p.top_k) != kRowWide) return;
    uint32_t prefix = 0u;
    if (pass > 0) {
        const WideSel s = a.ws.sel[row];
        if (s.state != kSelSearch) return;
        prefix = s.prefix;
    }
    for (int i = tid; i < kWideBins; i += kFullBlock) hist[i] = 0u;
    __syncthreads();
    uint32_t raw[kFullPer];
    const int nv = load16<DT>(row_ptr<DT>(a, row), (int64_t)b * kSelChunk + (int64_t)tid * kFullPer,
                              a.vocab, raw);
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) {
        const uint32_t key = cand_key(x_of<DT>(raw[j]));
        if (j >= nv || key == 0u) continue;
        bool match;
        uint32_t d;
        if (pass == 0) {
            match = true;
            d = key >> 21;
        } else if (pass == 1) {
            match = (key >> 21) == prefix;
            d = (key >> 10) & 0x7FFu;
        } else {
            match = (key >> 10) == prefix;
            d = key & 0x3FFu;
        }
        if (match) atomicAdd(&hist[d], 1u);
    }
    __syncthreads();
    uint32_t* gh = a.ws.hist + (int64_t)row * kWideBins;
    for (int i = tid; i < kWideBins; i += kFullBlock)
        if (hist[i]) atomicAdd(&gh[i], hist[i]);
}

/* Fix one digit: the bin holding the rank-krem key counted from the top
 * (the heap keeps the K largest as a multiset, Model.pas:2615-2664).
 * Clears the row's histogram for the next pass. */
__global__ __launch_bounds__(kFullBlock) void wide_find_kernel(FullArgs a, int pass)
{
    __shared__ Scratch sh;
    const int tid = threadIdx.x;
    const int row = blockIdx.y;
    const RowIn ri = row_in(a, row);
    if (row_class(a, ri.p.top_k) != kRowWide) return;
    const int K = ri.p.top_k;
    WideSel* sp = a.ws.sel + row;
    WideSel s;
    if (pass == 0) {
        s.prefix = 0u;
        s.krem = K;
        s.state = kSelSearch;
    } else {
        s = *sp;
        if (s.state != kSelSearch) return;
    }
    const int nb = pass == 2 ? 1024 : kWideBins;
    const int per = nb / kFullBlock;
    uint32_t* gh = a.ws.hist + (int64_t)row * kWideBins;
    /* thread t holds bins nb-1-t*per down to nb-per-t*per (highest first) */
    uint32_t c[kWideBins / kFullBlock];
    int tsum = 0;
    for (int q = 0; q < per; ++q) {
        const int bin = nb - 1 - tid * per - q;
        c[q] = gh[bin];
        gh[bin] = 0u;
        tsum += (int)c[q];
    }
    int total;
    int above = block_excl_scan_i(tsum, sh, total);
    if (pass == 0 && total <= K) {
        /* at most K logits above -1e30: every one survives (the -1e30
         * fillers are dropped, Model.pas:2668-2676) */
        if (tid == 0) {
            sp->state = total == 0 ? kSelEmpty : kSelAll;
            sp->tau = 1u;
            sp->idx_thr = INT_MAX;
            sp->count = total;
        }
        if (total == 0 && tid < 64) {
            if (tid == 0) {
                a.ids[row] = -1;
                if (a.out.count) a.out.count[row] = 0;
                if (a.out.flags)
                    a.out.flags[row] = G4S_FLAG_TOPK_PATH | G4S_FLAG_WIDE_K | G4S_FLAG_EMPTY;
            }
            publish_done(a.done, row, a.seq);
        }
        return;
    }
    const int krem = s.krem;
    for (int q = 0; q < per; ++q) {
        const int bin = nb - 1 - tid * per - q;
        if (above < krem && krem <= above + (int)c[q]) {
            const int k2 = krem - above;
            if (pass < 2) {
                sp->prefix = pass == 0 ? (uint32_t)bin : ((s.prefix << 11) | (uint32_t)bin);
                sp->krem = k2;
                sp->state = kSelSearch;
                sp->idx_thr = INT_MAX;
            } else {
                sp->tau = (s.prefix << 10) | (uint32_t)bin;
                sp->need = k2;
                sp->eq = (int)c[q];
                sp->count = K;
                sp->state = k2 == (int)c[q] ? kSelAll : kSelTies;
            }
        }
        above += (int)c[q];
    }
}

/* Per chunk: keys >= tau, keys == tau, the last index above tau. */
template <int DT>
__global__ __launch_bounds__(kFullBlock) void wide_ties_kernel(FullArgs a)
{
    __shared__ Scratch sh;
    const int tid = threadIdx.x;
    const int row = blockIdx.y, b = blockIdx.x;
    const RowIn ri = row_in(a, row);
    if (row_class(a, ri.p.top_k) != kRowWide) return;
    const WideSel s = a.ws.sel[row];
    if (s.state != kSelTies) return;
    uint32_t raw[kFullPer];
    const int64_t e0 = (int64_t)b * kSelChunk + (int64_t)tid * kFullPer;
    const int nv = load16<DT>(row_ptr<DT>(a, row), e0, a.vocab, raw);
    int ge = 0, eq = 0;
    uint32_t gt = 0u; /* last index above tau, plus one */
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) {
        const uint32_t key = cand_key(x_of<DT>(raw[j]));
        if (j >= nv) continue;
        ge += key >= s.tau;
        eq += key == s.tau;
        if (key > s.tau) gt = (uint32_t)(e0 + j) + 1u;
    }
    ge = block_sum_int(ge, sh);
    eq = block_sum_int(eq, sh);
    gt = block_max_key(gt, sh, 0);
    if (tid == 0) {
        TieRec t;
        t.cge = ge;
        t.ceq = eq;
        t.maxgt = (int32_t)gt - 1;
        t.pad = 0;
        a.ws.ties[(int64_t)row * kSelMaxChunks + b] = t;
    }
}

/* The tie rule.  t* = index of the K-th key >= tau in index order.  When
 * every key above tau precedes t*, the heap holds exactly the first K keys
 * >= tau once it has passed t*, and rejects every later copy of tau
 * (v <= root, Model.pas:2643): the survivors are the keys above tau and the
 * first `need` copies of tau.  Otherwise the heap's layout decides: replay. */
template <int DT>
__global__ __launch_bounds__(kFullBlock) void wide_ties_find_kernel(FullArgs a)
{
    __shared__ Scratch sh;
    const int tid = threadIdx.x;
    const int row = blockIdx.y;
    const RowIn ri = row_in(a, row);
    if (row_class(a, ri.p.top_k) != kRowWide) return;
    WideSel* sp = a.ws.sel + row;
    const WideSel s = *sp;
    if (s.state != kSelTies) return;
    const int nch = a.nsel;
    const int K = ri.p.top_k;
    const TieRec* tr = a.ws.ties + (int64_t)row * kSelMaxChunks;
    int ge[kSelCPT], eq[kSelCPT];
    int sge = 0, seqn = 0, mgt = -1;
#pragma unroll
    for (int q = 0; q < kSelCPT; ++q) {
        const int cb = tid * kSelCPT + q;
        ge[q] = eq[q] = 0;
        if (cb < nch) {
            const TieRec t = tr[cb];
            ge[q] = t.cge;
            eq[q] = t.ceq;
            mgt = t.maxgt > mgt ? t.maxgt : mgt;
        }
        sge += ge[q];
        seqn += eq[q];
    }
    int tot;
    int run_ge = block_excl_scan_i(sge, sh, tot);
    int run_eq = block_excl_scan_i(seqn, sh, tot);
    const int32_t max_gt = (int32_t)block_max_key((uint32_t)(mgt + 1), sh, 1) - 1;
    const int need = s.need;
    if (tid == 0) {
        sh.misc[0] = sh.misc[2] = -1;
        sh.misc[1] = sh.misc[3] = 0;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kSelCPT; ++q) {
        const int cb = tid * kSelCPT + q;
        if (run_ge < K && K <= run_ge + ge[q]) {
            sh.misc[0] = cb;
            sh.misc[1] = K - run_ge;
        }
        if (run_eq < need && need <= run_eq + eq[q]) {
            sh.misc[2] = cb;
            sh.misc[3] = need - run_eq;
        }
        run_ge += ge[q];
        run_eq += eq[q];
    }
    __syncthreads();
    const int c1 = sh.misc[0], r1 = sh.misc[1], c2 = sh.misc[2], r2 = sh.misc[3];
    __syncthreads();
    if (c1 < 0 || c1 >= nch || c2 < 0 || c2 >= nch) {
        /* counts inconsistent with the select (not expected): the replay
         * decides from the row itself */
        if (tid == 0) sp->state = kSelReplay;
        return;
    }
    const char* rowp = row_ptr<DT>(a, row);
    const uint32_t tau = s.tau;
    const int tstar = kth_in_chunk<DT>(a, rowp, c1, r1, [&](uint32_t k) { return k >= tau; }, sh);
    if (max_gt < tstar) {
        const int thr = kth_in_chunk<DT>(a, rowp, c2, r2, [&](uint32_t k) { return k == tau; }, sh);
        if (tid == 0) {
            sp->idx_thr = thr;
            sp->state = kSelLowest;
        }
    } else if (tid == 0) {
        sp->state = kSelReplay;
    }
}

/* Exact replay of the reference's min-heap pass (Model.pas:2632-2664) for
 * the rows whose tie at tau depends on the heap layout, one row at a time
 * with the heap in device memory.  One wave screens 64 logits per step
 * against the current root; lane 0 inserts the ones that pass, in index
 * order.  The surviving copies of tau are then marked in the row's bitmask.
 * Cost: about (K + K ln(V/K)) log2(K) dependent heap steps per row. */
template <int DT>
__global__ __launch_bounds__(64) void wide_replay_kernel(FullArgs a)
{
    const int lane = threadIdx.x;
    const int V = a.vocab;
    float* hv = a.ws.heap_v;
    int32_t* hi = a.ws.heap_i;
    for (int row = 0; row < a.batch; ++row) {
        const RowIn ri = row_in(a, row);
        if (row_class(a, ri.p.top_k) != kRowWide) continue;
        WideSel* sp = a.ws.sel + row;
        const WideSel s = *sp;
        if (s.state != kSelReplay) continue;
        const int K = ri.p.top_k;
        const char* rowp = row_ptr<DT>(a, row);
        if (lane == 0) {
            for (int i = 0; i < K; ++i) { /* :2634-2638 */
                hv[i] = -1e30f;
                hi[i] = -1;
            }
        }
        float root = -1e30f;
        for (int base = 0; base < V; base += 64) {
            const int e = base + lane;
            float x = 0.0f;
            if (e < V) {
                if constexpr (DT == 0)
                    x = reinterpret_cast<const float*>(rowp)[e];
                else
                    x = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(rowp)[e] << 16);
            }
            uint64_t take = __ballot(e < V && !(x <= root));
            while (take) {
                const int l = (int)__builtin_ctzll(take);
                take &= take - 1;
                const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
                if (lane == 0 && !(v <= hv[0])) { /* :2643-2644 */
                    int p = 0;
                    for (;;) { /* :2647-2661 */
                        int c = p * 2 + 1;
                        if (c >= K) break;
                        if (c + 1 < K && hv[c + 1] < hv[c]) c += 1;
                        if (hv[c] >= v) break;
                        hv[p] = hv[c];
                        hi[p] = hi[c];
                        p = c;
                    }
                    hv[p] = v;
                    hi[p] = base + l;
                }
            }
            const float r0 = lane == 0 ? hv[0] : 0.0f;
            root = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r0), 0));
        }
        if (lane == 0) {
            uint32_t* bits = a.ws.bits + (int64_t)row * a.ws.bits_stride;
            for (int w = 0; w < a.ws.bits_stride; ++w) bits[w] = 0u;
            for (int i = 0; i < K; ++i) {
                const int32_t idx = hi[i];
                if (idx >= 0 && cand_key(hv[i]) == s.tau) bits[idx >> 5] |= 1u << (idx & 31);
            }
            sp->state = kSelBits;
        }
    }
}

/* ------------------------------------------------------------ 1: max */

/* Wave w of workgroup g handles chunks (g*4 + w)*cpw .. +cpw-1 of its row;
 * every chunk gets its record. */
template <int DT>
__global__ __launch_bounds__(kFullBlock) void full_max_kernel(FullArgs a)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.y;
    const int cw = (blockIdx.x * NWF + (threadIdx.x >> 6)) * a.cpw;
    const int V = a.vocab;
    if (cw >= a.nch) return;
    const int bend = cw + a.cpw < a.nch ? cw + a.cpw : a.nch;
    const RowIn ri = row_in(a, row);
    Mask k;
    if (!row_mask(a, row, ri, k)) return;
    const float cap = a.softcap;
    const float inv_cap = cap > 0.0f ? div_cr32(1.0f, cap) : 1.0f;      /* Layers.pas:309 */
    const float T = ri.p.temperature;
    const int scale = (T > 0.0f) && (T != 1.0f);                       /* Model.pas:2703 */
    const float inv_t = scale ? div_cr32(1.0f, T) : 1.0f;              /* Model.pas:2705 */
    const char* rowp = row_ptr<DT>(a, row);
    FullChunk* rc = a.ws.chunks + (int64_t)row * a.ws.cstride;
    if (cw == 0 && lane < 2) a.ws.tmask[(int64_t)row * 2 + lane] = 0ull; /* for the row kernel */

    for (int b = cw; b < bend; ++b) {
        uint32_t raw[kFullPer];
        const int64_t e0 = (int64_t)b * kFullChunk + (int64_t)lane * kFullPer;
        const int nvalid = load16<DT>(rowp, e0, V, raw);
        /* maxima as floats (the key of a float maximum is the maximum key:
         * the order-preserving map identifies -0 and +0, as the comparisons
         * do) */
        uint32_t kmax, amax;
        float ymax, s = 0.0f;
        uint32_t fs;
        int ns;
        /* wave-uniform: the branches hold wave reductions */
        const bool whole = k.cls != kRowWide && (int64_t)(b + 1) * kFullChunk <= V;
        if (!whole) {
            float xm = -__builtin_inff(), am = 0.0f, ym = -__builtin_inff();
            float ya[kFullPer];
            bool part[kFullPer];
            fs = 0xFFFFFFFFu;
            ns = 0;
#pragma unroll
            for (int j = 0; j < kFullPer; ++j) {
                const float xj = x_of<DT>(raw[j]);
                part[j] = j < nvalid && takes_part(k, xj, e0 + j);
                ya[j] = y_approx(xj, cap, inv_cap, scale, inv_t);
                if (j < nvalid) xm = __builtin_fmaxf(xm, xj);
                am = part[j] ? __builtin_fmaxf(am, __builtin_fabsf(xj)) : am;
                ym = part[j] ? __builtin_fmaxf(ym, ya[j]) : ym;
                ns += part[j] ? 1 : 0;
                fs = part[j] ? g4s_min_u(fs, (uint32_t)(e0 + j)) : fs;
            }
            kmax = wave_max_u32(nvalid > 0 ? f2key(xm) : 0u);
            amax = wave_max_u32(__float_as_uint(am));
            ymax = key2f(wave_max_u32(f2key(ym)));
            const float lg2e_ymax = ymax * 1.4426950408889634f;
#pragma unroll
            for (int j = 0; j < kFullPer; ++j)
                if (part[j])
                    s += __builtin_amdgcn_exp2f(__builtin_fmaf(ya[j], 1.4426950408889634f, -lg2e_ymax));
            ns = wave_sum_i32(ns);
            fs = wave_min_u32(fs);
        } else {
            /* a whole chunk of a full row: every term takes part, and the
             * approximate y is monotone in x, so its maximum is y(max x) */
            float xa[kFullPer];
            float xm = -__builtin_inff(), xn = __builtin_inff();
#pragma unroll
            for (int j = 0; j < kFullPer; ++j) xa[j] = x_of<DT>(raw[j]);
#pragma unroll
            for (int j = 0; j < kFullPer; j += 2) {
                xm = __builtin_fmaxf(xm, __builtin_fmaxf(xa[j], xa[j + 1]));
                xn = __builtin_fminf(xn, __builtin_fminf(xa[j], xa[j + 1]));
            }
            kmax = wave_max_u32(f2key(xm));
            amax = wave_max_u32(__float_as_uint(__builtin_fmaxf(__builtin_fabsf(xm),
                                                                __builtin_fabsf(xn))));
            const float xmax = key2f(kmax);
            /* every |x/cap| < 0.1: cap tanh(x/cap) = x - x^3/(3 cap^2) +
             * O(x^5/cap^4), relative error < 1e-5 -- enough for predictions */
            const bool cubic = cap > 0.0f && __uint_as_float(amax) * inv_cap < 0.1f;
            const float c3 = -(inv_cap * inv_cap) * (1.0f / 3.0f);
            const auto yap = [&](float x) {
                if (cubic) {
                    const float y = __builtin_fmaf(x * (x * x), c3, x);
                    return scale ? y * inv_t : y;
                }
                return y_approx(x, cap, inv_cap, scale, inv_t);
            };
            ymax = yap(xmax);
            const float lg2e_ymax = ymax * 1.4426950408889634f;
#pragma unroll
            for (int j = 0; j < kFullPer; ++j)
                s += __builtin_amdgcn_exp2f(__builtin_fmaf(yap(xa[j]), 1.4426950408889634f, -lg2e_ymax));
            ns = kFullChunk;
            fs = (uint32_t)((int64_t)b * kFullChunk);
        }
        s = wave_sum_f32(s);
        if (lane == 0) {
            FullChunk r;
            r.maxkey = kmax;
            r.amax = amax;
            r.ymax = ymax;
            r.sapx = s;
            r.nsurv = ns;
            r.fsurv = fs == 0xFFFFFFFFu ? INT_MAX : (int32_t)fs;
            r.soff = 0;
            r.pad = 0;
            rc[b] = r;
        }
    }
}

/* ------------------------------------------------------------ 2: row */

/* Every workgroup of a row reduces the chunk records to the row's m; for
 * bf16 logits workgroup g fills entries g*1024 .. g*1024+1023 of the e
 * table (kRowPer per thread: four workgroups per row launch far faster than
 * sixteen); workgroup 0 also writes the row record, the predicted binades
 * and the survivor offsets (thread t handles chunks t*cpt .. t*cpt+cpt-1). */
constexpr int kRowPer = 4; /* e-table entries per thread of the row kernel */
static_assert(kFullTab % (kFullBlock * kRowPer) == 0, "whole workgroups of table entries");

template <int DT>
__global__ __launch_bounds__(kFullBlock) void full_row_kernel(FullArgs a)
{
    __shared__ Scratch sh;
    const int tid = threadIdx.x;
    const int row = blockIdx.y, g = blockIdx.x;
    const RowIn ri = row_in(a, row);
    Mask k;
    if (!row_mask(a, row, ri, k)) return;
    const int nch = a.nch;
    const int cpt = (nch + kFullBlock - 1) / kFullBlock;
    FullChunk* rc = a.ws.chunks + (int64_t)row * a.ws.cstride;
    uint32_t km = 0u, am = 0u;
    for (int cb = tid; cb < nch; cb += kFullBlock) {
        km = g4s_max_u(km, rc[cb].maxkey);
        am = g4s_max_u(am, rc[cb].amax);
    }
    km = block_max_key(km, sh, 0);
    am = block_max_key(am, sh, 1);
    const float cap = a.softcap;
    const float inv_cap = cap > 0.0f ? div_cr32(1.0f, cap) : 1.0f;
    const float T = ri.p.temperature;
    const int scale = (T > 0.0f) && (T != 1.0f);
    const float inv_t = scale ? div_cr32(1.0f, T) : 1.0f;
    const float m = y_exact(key2f(km), k.cls, cap, inv_cap, scale, inv_t); /* Tensors.pas:648-654 */
    /* table window: the 16 binades of |x| below and at the largest one */
    int win = -1;
    if (DT == 1) {
        const int eb = (int)((am >> 23) & 0xFFu);
        win = eb - 15 < 0 ? 0 : eb - 15;
        uint64_t tb = 0ull;
        for (int s = 0; s < kRowPer; ++s) {
            const int i = (g * kRowPer + s) * kFullBlock + tid;
            const uint32_t ebi = (uint32_t)win + (((uint32_t)i >> 7) & 15u);
            const uint32_t code = (((uint32_t)i >> 11) << 15) | (ebi << 7) | ((uint32_t)i & 0x7Fu);
            const float x = __uint_as_float(code << 16);
            const float ev = exp_diff_cr32(y_exact(x, k.cls, cap, inv_cap, scale, inv_t), m);
            a.ws.etab[(int64_t)row * kFullTab + i] = ev;
            tb |= tie_bits(ev, kTieBaseE);
        }
        /* the binades in which a table value is a half-unit tie */
        tb = wave_or64(tb);
        if ((tid & 63) == 0 && tb != 0ull)
            atomicOr((unsigned long long*)&a.ws.tmask[(int64_t)row * 2], (unsigned long long)tb);
    }
    if (g != 0) return;

    /* predicted binade of LSum entering every chunk: exclusive prefix of the
     * chunk estimates (a prediction only: non-finite estimates add 0); the
     * survivor offsets and the first survivor */
    const auto est = [&](const FullChunk& c) {
        double z = (double)c.ymax - (double)m;
        z = z > 50.0 ? 50.0 : (z < -700.0 ? -700.0 : z);
        const double v = (double)c.sapx * exp_fast_d(z);
        return (v >= 0.0 && v < 1e300) ? v : 0.0;
    };
    double tsum = 0.0;
    int tns = 0;
    uint32_t fs = 0xFFFFFFFFu;
    for (int q = 0; q < cpt; ++q) {
        const int cb = tid * cpt + q;
        if (cb < nch) {
            const FullChunk c = rc[cb];
            tsum += est(c);
            tns += c.nsurv;
            fs = g4s_min_u(fs, (uint32_t)c.fsurv);
        }
    }
    double total;
    double pre = block_excl_scan_d(tsum, sh, total);
    int count;
    int soff = block_excl_scan_i(tns, sh, count);
    fs = block_min_u(fs, sh);
    int32_t* bl = a.ws.beta_l + (int64_t)row * a.ws.cstride;
    for (int q = 0; q < cpt; ++q) {
        const int cb = tid * cpt + q;
        if (cb < nch) {
            const FullChunk c = rc[cb];
            bl[cb] = ss::state_of((float)pre).e;
            rc[cb].soff = soff;
            pre += est(c);
            soff += c.nsurv;
        }
    }
    if (tid == 0) {
        FullRow r;
        r.maxkey = km;
        r.amax = am;
        r.m = m;
        r.inv_t = inv_t;
        r.scale = scale;
        r.win_lo = win;
        r.lsum = 0.0f;
        r.inv = 0.0f;
        r.thr = 0.0f;
        r.argmax = 0;
        r.c_last = -1;
        r.nodraw = 0;
        r.count = count;
        r.first = (int32_t)fs;
        r.beta_end = ss::state_of((float)total).e;
        for (int j = 0; j < kNear; ++j) r.near[j] = INT_MAX;
        r.l_reev = r.l_rounds = r.c_reev = r.c_rounds = 0;
        a.ws.rows[row] = r;
    }
}

/* ------------------------------------------------- 3: lsum chunk maps */

template <int DT>
struct TabLds {
    float tab[DT == 1 ? kFullTab : 1];
};

/* Each chunk's terms as one map of LSum in the chunk's predicted binade,
 * one chunk per wave at a time; the first index of e == 1 and, on wide rows,
 * of its near ties. */
template <int DT>
__global__ __launch_bounds__(kFullBlock) void full_lsum_kernel(FullArgs a)
{
    __shared__ TabLds<DT> sh;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.y;
    const int V = a.vocab;
    const int nch = a.nch;
    if ((int)blockIdx.x * NWF * a.cpw >= nch) return;
    const RowIn ri = row_in(a, row);
    Mask k;
    if (!row_mask(a, row, ri, k)) return;
    const char* rowp = row_ptr<DT>(a, row);
    FullRow* rr = a.ws.rows + row;
    const FullRow r = *rr;
    const Ctx c = make_ctx(a, r, k.cls);
    load_tab<DT>(a.ws.etab, row, r, sh.tab);
    const int64_t rbase = (int64_t)row * a.ws.cstride;
    const int cw = (blockIdx.x * NWF + (threadIdx.x >> 6)) * a.cpw;
    const int bend = cw + a.cpw < nch ? cw + a.cpw : nch;
    const uint64_t tm = a.ws.tmask[(int64_t)row * 2];
    /* the predicted binades of the wave's chunks in one load (lane q: chunk
     * cw + q) */
    const int32_t betas = cw + lane < bend ? a.ws.beta_l[rbase + cw + lane] : 0;

    for (int b = cw; b < bend; ++b) {
        const int64_t e0 = (int64_t)b * kFullChunk + (int64_t)lane * kFullPer;
        float t[kFullPer];
        int nvalid = kFullPer;
        bool tabbed = DT == 1 && k.cls == kRowFull && c.win_lo >= 0 &&
                      (int64_t)(b + 1) * kFullChunk <= V &&
                      terms_bf16_whole(rowp, e0, c, sh.tab, t);                /* Tensors.pas:660 */
        if (!tabbed) {
            uint32_t raw[kFullPer];
            nvalid = load16<DT>(rowp, e0, V, raw);
            tabbed = terms_e<DT>(raw, nvalid, e0, c, k, sh.tab, t);
        }
        /* the terms with e = 1 - jj*2^-24, jj < kNear (the row maximum and
         * its near ties): looked at only in waves that hold one */
        constexpr float kNearLo = 1.0f - (float)(kNear - 1) * 0x1p-24f;
        float tmx = 0.0f;
#pragma unroll
        for (int j = 0; j < kFullPer; ++j) tmx = __builtin_fmaxf(tmx, t[j]);
        if (__ballot(tmx >= kNearLo)) {
            uint32_t first1 = 0xFFFFFFFFu;
            uint32_t nearm = 0u;
#pragma unroll
            for (int j = 0; j < kFullPer; ++j) {
                first1 = t[j] == 1.0f ? g4s_min_u(first1, (uint32_t)(e0 + j)) : first1;
                nearm |= (t[j] >= kNearLo && t[j] < 1.0f) ? (1u << j) : 0u;
            }
            if (k.cls == kRowWide && nearm != 0u) {
                for (int j = 0; j < kFullPer; ++j)
                    if (nearm & (1u << j))
                        atomicMin(&rr->near[(int)((1.0f - t[j]) * 0x1p24f)], (int32_t)(e0 + j));
            }
            first1 = wave_min_u32(first1);
            if (lane == 0 && first1 != 0xFFFFFFFFu) atomicMin(&rr->near[0], (int32_t)first1);
        }
        const int32_t beta = __builtin_amdgcn_readlane(betas, b - cw);
        const PMap cm = wave_chunk_map(tabbed && !tie_possible(tm, kTieBaseE, beta)
                                           ? thread_map_nt(t, beta)
                                           : thread_map(t, nvalid, beta));
        if (lane == 0) a.ws.lmap[rbase + b] = cm;
    }
}

/* ------------------------------------------------------- 4: LSum chain */

/* One workgroup per row: LSum by chaining the chunk maps left to right
 * (Tensors.pas:657-663; Model.pas:2794-2799), re-evaluating the chunks whose
 * map does not apply (the predicted binade crossings, staged in LDS by the
 * whole workgroup; then wave 0 alone); then the argmax and the predictions
 * for the draw. */
template <int DT>
__global__ __launch_bounds__(kChainBlock) void full_lsum_chain_kernel(FullArgs a)
{
    extern __shared__ __align__(16) char dsm[];
    __shared__ ChainScratch sh;
    const int tid = threadIdx.x, lane = tid & 63;
    const int row = blockIdx.y;
    const RowIn ri = row_in(a, row);
    Mask k;
    if (!row_mask(a, row, ri, k)) return;
    const char* rowp = row_ptr<DT>(a, row);
    const int nch = a.nch;
    const int64_t rbase = (int64_t)row * a.ws.cstride;
    const FullRow r = a.ws.rows[row];
    const ChainLds L = chain_lds<DT>(dsm, nch, a.nstage);
    const int32_t* gb = a.ws.beta_l + rbase;
    const int32_t bend = r.beta_end;
    const Ctx c = make_ctx(a, r, k.cls);
    if (tid < 2) sh.pm[tid] = 0u;
    chain_prologue<DT, false>(
        a, row, r, c, k, a.ws.lmap + rbase, gb, nch - 1,
        [&](int q) { return q == 0 || gb[q] != (q + 1 < nch ? gb[q + 1] : bend); }, L, sh);
    /* the draw's settings (every wave: they decide whether the others wait
     * for the chain) */
    const float T = ri.p.temperature;
    const bool all = term_outputs(a, k.cls);
    const bool nodraw = !(T > 0.0f);
    const float thr = nodraw ? __builtin_inff() : mul_u_p_cr32(ri.u, ri.p.top_p); /* :2726 */
    /* fl32(u*TopP) <= 0: the first term's running sum already reaches it */
    const bool direct = !nodraw && !(thr > 0.0f);
    const bool early = (nodraw || direct) && !all;
    if (tid >= 64 && early) return;

    if (tid < 64) {
        State st = ss::state_of(0.0f);
        int reev = 0, rounds = 0;
        for (int cb = 0; cb < nch;) {
            if (cb > 0) {
                cb = walk_maps<false>(L.cm, L.cb, cb, nch, st, 0.0f, L.cpost);
                if (cb >= nch) break;
            }
            ++reev;
            int h;
            st = chain_chunk<DT, false>(a, rowp, cb, st, __builtin_inff(), L, c, k, r, &h, &rounds);
            if (lane == 0) L.cpost[cb] = ss::value_of(st);
            ++cb;
        }
        const float lsum = ss::value_of(st);
        const float inv = div_cr32(1.0f, lsum);                        /* Tensors.pas:668 */
        /* argmax of p.  Full row: p = fl32(e * inv) <= inv with equality
         * exactly at e == 1 (the next float below 1 gives a p below inv), so
         * the first e == 1.  Wide row: p = fl32(e / LSum) can also equal
         * fl32(1 / LSum) for e = 1 - j*2^-24 with small j (never for j >=
         * kNear): the first index among the values whose quotient ties
         * (Model.pas:2804-2807). */
        int32_t argmax = r.near[0];
        if (k.cls == kRowWide) {
            for (int j = 1; j < kNear; ++j)
                if (r.near[j] < argmax && div_cr32(1.0f - (float)j * 0x1p-24f, lsum) == inv)
                    argmax = r.near[j];
        }
        if (early) {
            uint32_t f = row_flags(k);
            if (direct) f |= G4S_FLAG_DREW | G4S_FLAG_REACHED;
            write_row_outputs(a, row, direct ? r.first : argmax, argmax, lsum, r.count, f);
            return;
        }
        if (lane == 0) {
            sh.lsum = lsum;
            sh.inv = inv;
            sh.argmax = argmax;
            sh.reev = reev;
            sh.rounds = rounds;
        }
    }
    __syncthreads();
    const float lsum = sh.lsum, inv = sh.inv;
    /* the p table (Tensors.pas:666-672; Model.pas:2800-2801 on wide rows)
     * and the binades where one of its values is a half-unit tie */
    if (DT == 1 && r.win_lo >= 0) {
        const float4 e4 = reinterpret_cast<const float4*>(L.tab)[tid];
        float4 p4;
        p4.x = p_of(e4.x, k.cls, inv, lsum);
        p4.y = p_of(e4.y, k.cls, inv, lsum);
        p4.z = p_of(e4.z, k.cls, inv, lsum);
        p4.w = p_of(e4.w, k.cls, inv, lsum);
        reinterpret_cast<float4*>(a.ws.ptab + (int64_t)row * kFullTab)[tid] = p4;
        const uint64_t tb = wave_or64(tie_bits(p4.x, kTieBaseP) | tie_bits(p4.y, kTieBaseP) |
                                      tie_bits(p4.z, kTieBaseP) | tie_bits(p4.w, kTieBaseP));
        if (lane == 0 && tb != 0ull) {
            atomicOr(&sh.pm[0], (uint32_t)tb);
            atomicOr(&sh.pm[1], (uint32_t)(tb >> 32));
        }
    }
    /* predicted binade of the draw's running sum entering each chunk (the
     * exact LSum prefix before the chunk times 1/LSum), and the chunk where
     * it is predicted to reach thr (with margin) */
    uint32_t last = (uint32_t)(nch - 1);
    int32_t* gbc = a.ws.beta_c + rbase;
    for (int cb = tid; cb < nch; cb += kChainBlock) {
        const double pre = cb > 0 ? (double)L.cpost[cb - 1] : 0.0;
        const double post = (double)L.cpost[cb];
        gbc[cb] = ss::state_of((float)(pre * (double)inv)).e;
        if (post * (double)inv >= (double)thr * (1.0 + 0x1p-10)) last = g4s_min_u(last, (uint32_t)cb);
    }
    last = wave_min_u32(last);
    if (lane == 0) sh.lastw[tid >> 6] = last;
    __syncthreads();
    if (tid == 0) a.ws.tmask[(int64_t)row * 2 + 1] = ((uint64_t)sh.pm[1] << 32) | sh.pm[0];
    if (tid == 0) {
        for (int w = 0; w < kChainWaves; ++w) last = g4s_min_u(last, sh.lastw[w]);
        FullRow w = r;
        w.lsum = lsum;
        w.inv = inv;
        w.thr = thr;
        w.argmax = sh.argmax;
        w.c_last = (all || direct) ? nch - 1 : (int32_t)last;
        w.nodraw = nodraw ? 1 : (direct ? 2 : 0);
        w.l_reev = sh.reev;
        w.l_rounds = sh.rounds;
        w.c_reev = 0;
        w.c_rounds = 0;
        a.ws.rows[row] = w;
    }
}

/* -------------------------------------------------- 5: draw chunk maps */

template <int DT>
__global__ __launch_bounds__(kFullBlock) void full_cdf_kernel(FullArgs a)
{
    __shared__ TabLds<DT> sh;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.y;
    const int V = a.vocab;
    const RowIn ri = row_in(a, row);
    Mask k;
    if (!row_mask(a, row, ri, k)) return;
    const FullRow r = a.ws.rows[row];
    if (r.c_last < 0 || (int)blockIdx.x * NWF * a.cpw > r.c_last) return;
    const char* rowp = row_ptr<DT>(a, row);
    const int64_t rbase = (int64_t)row * a.ws.cstride;
    const FullChunk* rc = a.ws.chunks + rbase;
    const Ctx c = make_ctx(a, r, k.cls);
    load_tab<DT>(a.ws.ptab, row, r, sh.tab);
    const bool all = term_outputs(a, k.cls);
    const int cw = (blockIdx.x * NWF + (threadIdx.x >> 6)) * a.cpw;
    const int bend = cw + a.cpw <= r.c_last ? cw + a.cpw : r.c_last + 1;
    const uint64_t tm = a.ws.tmask[(int64_t)row * 2 + 1];
    /* per-chunk inputs up front (lane q: chunk cw + q) */
    const bool mine = cw + lane < bend;
    const int32_t betas = mine ? a.ws.beta_c[rbase + cw + lane] : 0;
    const int32_t soffs = (mine && all && k.cls != kRowFull) ? rc[cw + lane].soff : 0;

    for (int b = cw; b < bend; ++b) {
        uint32_t raw[kFullPer]; /* loaded on the general route only (wide rows take it) */
        const int64_t e0 = (int64_t)b * kFullChunk + (int64_t)lane * kFullPer;
        float t[kFullPer];
        int nvalid = kFullPer;
        bool tabbed = DT == 1 && k.cls == kRowFull && c.win_lo >= 0 &&
                      (int64_t)(b + 1) * kFullChunk <= V &&
                      terms_bf16_whole(rowp, e0, c, sh.tab, t);
        if (!tabbed) {
            nvalid = load16<DT>(rowp, e0, V, raw);
            tabbed = terms_e<DT, true>(raw, nvalid, e0, c, k, sh.tab, t);
        }
        if (all) {
            float* po = a.out.probs ? a.out.probs + (int64_t)row * a.out.capacity : nullptr;
            int32_t* io = a.out.indices ? a.out.indices + (int64_t)row * a.out.capacity : nullptr;
            if (k.cls == kRowFull) {
#pragma unroll
                for (int j = 0; j < kFullPer; ++j)
                    if (j < nvalid) {
                        po[e0 + j] = t[j]; /* Tensors.pas:671 */
                        if (io) io[e0 + j] = (int32_t)(e0 + j);
                    }
            } else {
                /* the survivors in index order (Model.pas:2678-2688) */
                int cnt = 0;
                bool part[kFullPer];
#pragma unroll
                for (int j = 0; j < kFullPer; ++j) {
                    part[j] = j < nvalid && takes_part(k, x_of<DT>(raw[j]), e0 + j);
                    cnt += part[j] ? 1 : 0;
                }
                int pos = __builtin_amdgcn_readlane(soffs, b - cw) + wave_inclusive_scan(cnt) - cnt;
#pragma unroll
                for (int j = 0; j < kFullPer; ++j)
                    if (part[j]) {
                        if (pos < a.out.capacity) {
                            if (po) po[pos] = t[j];
                            if (io) io[pos] = (int32_t)(e0 + j);
                        }
                        ++pos;
                    }
            }
        }
        if (r.nodraw) continue;
        const int32_t beta = __builtin_amdgcn_readlane(betas, b - cw);
        const PMap cm = wave_chunk_map(tabbed && !tie_possible(tm, kTieBaseP, beta)
                                           ? thread_map_nt(t, beta)
                                           : thread_map(t, nvalid, beta));
        if (lane == 0) a.ws.cmap[rbase + b] = cm;
    }
}

/* -------------------------------------------------------- 6: the draw */

/* One workgroup per row: the first index whose left-to-right binary32
 * running sum of p reaches thr (Model.pas:2727-2735, 2811-2824), else the
 * argmax. */
template <int DT>
__global__ __launch_bounds__(kChainBlock) void full_cdf_chain_kernel(FullArgs a)
{
    extern __shared__ __align__(16) char dsm[];
    __shared__ ChainScratch sh;
    const int tid = threadIdx.x, lane = tid & 63;
    const int row = blockIdx.y;
    const RowIn ri = row_in(a, row);
    if (!a.topk_on && row_class(a, ri.p.top_k) == kRowTopk) {
        /* no top-k launch in this call: reject the row rather than leave an
         * earlier call's id in place */
        if (tid < 64)
            write_row_outputs(a, row, -1, -1, 0.0f, 0, G4S_FLAG_ERROR | G4S_FLAG_TOPK_PATH);
        return;
    }
    Mask k;
    if (!row_mask(a, row, ri, k)) return;
    const FullRow r = a.ws.rows[row];
    if (r.c_last < 0) return;
    const uint32_t fl = row_flags(k);
    if (r.nodraw == 1) {
        if (tid < 64) write_row_outputs(a, row, r.argmax, r.argmax, r.lsum, r.count, fl);
        return;
    }
    if (r.nodraw == 2) {
        if (tid < 64)
            write_row_outputs(a, row, r.first, r.argmax, r.lsum, r.count,
                              fl | G4S_FLAG_DREW | G4S_FLAG_REACHED);
        return;
    }
    const char* rowp = row_ptr<DT>(a, row);
    const int nch = a.nch;
    const int64_t rbase = (int64_t)row * a.ws.cstride;
    const ChainLds L = chain_lds<DT>(dsm, nch, a.nstage);
    const int32_t* gb = a.ws.beta_c + rbase;
    const int cl = r.c_last;
    const Ctx c = make_ctx(a, r, k.cls);
    chain_prologue<DT, true>(a, row, r, c, k, a.ws.cmap + rbase, gb, cl,
                             [&](int q) { return q == 0 || q == cl || gb[q] != gb[q + 1]; }, L, sh);
    if (tid >= 64) return;

    const float thr = r.thr;
    State st = ss::state_of(0.0f);
    int64_t hit = -1;
    int reev = 0, rounds = 0;
    for (int cb = 0; cb < nch; ++cb) {
        if (cb > 0) {
            cb = walk_maps<true>(L.cm, L.cb, cb, nch, st, thr, nullptr);
            if (cb >= nch) break;
        }
        ++reev;
        int h;
        st = chain_chunk<DT, true>(a, rowp, cb, st, thr, L, c, k, r, &h, &rounds);
        if (h >= 0) {
            hit = (int64_t)cb * kFullChunk + h;
            break;
        }
    }
    if (lane == 0) {
        a.ws.rows[row].c_reev = reev;
        a.ws.rows[row].c_rounds = rounds;
    }
    uint32_t flags = fl | G4S_FLAG_DREW;
    int32_t id = r.argmax;
    if (hit >= 0) {
        id = (int32_t)hit;
        flags |= G4S_FLAG_REACHED;
    }
    write_row_outputs(a, row, id, r.argmax, r.lsum, r.count, flags);
}

/* ---------------------------------------------------------------- host */

bool full_supported(int32_t vocab)
{
    return (vocab + kFullChunk - 1) / kFullChunk <= kFullMaxChunks &&
           (vocab + kSelChunk - 1) / kSelChunk <= kSelMaxChunks;
}

hipError_t full_alloc(FullWorkspace& ws, int32_t vocab, int32_t max_batch)
{
    const size_t mb = (size_t)max_batch;
    ws.bits_stride = (vocab + 31) / 32;
    ws.cstride = (vocab + kFullChunk - 1) / kFullChunk;
    const size_t nc = mb * (size_t)ws.cstride;
    hipError_t e = hipMalloc((void**)&ws.rows, mb * sizeof(FullRow));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.chunks, nc * sizeof(FullChunk));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.lmap, nc * sizeof(PMap));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.cmap, nc * sizeof(PMap));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.beta_l, nc * sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.beta_c, nc * sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.etab, mb * kFullTab * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.ptab, mb * kFullTab * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.tmask, mb * 2 * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.sel, mb * sizeof(WideSel));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.hist, mb * kWideBins * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.ties, mb * kSelMaxChunks * sizeof(TieRec));
    if (e == hipSuccess)
        e = hipMalloc((void**)&ws.bits, mb * (size_t)ws.bits_stride * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.heap_v, (size_t)vocab * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.heap_i, (size_t)vocab * sizeof(int32_t));
    return e;
}

void full_free(FullWorkspace& ws)
{
    void* ptrs[] = {ws.rows, ws.chunks, ws.lmap, ws.cmap, ws.beta_l, ws.beta_c, ws.etab, ws.ptab, ws.tmask,
                    ws.sel, ws.hist, ws.ties, ws.bits, ws.heap_v, ws.heap_i};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
    ws = FullWorkspace{};
}

hipError_t full_init(FullWorkspace& ws, int32_t max_batch, hipStream_t s)
{
    hipError_t e = hipMemsetAsync(ws.hist, 0, (size_t)max_batch * kWideBins * sizeof(uint32_t), s);
    return e;
}

/* Chunks the chains precompute: kStageMax when the LDS allows, fewer on a
 * device with less LDS per workgroup (then the chains re-evaluate more from
 * the logits).  Raises the launch limit for dynamic LDS beyond 64 KiB once
 * per kernel. */
template <int DT>
static int chain_nstage(int nch, size_t* lds)
{
    static int limit = -1;    /* dynamic LDS the chain kernels may use */
    static bool raised = false;
    if (limit < 0) {
        int dev = 0, v = 65536;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
            v = 65536;
        /* less the chain kernels' static LDS (as allocated, padding included) */
        size_t st = 0;
        hipFuncAttributes fa;
        if (hipFuncGetAttributes(&fa, (const void*)full_lsum_chain_kernel<DT>) == hipSuccess)
            st = fa.sharedSizeBytes;
        if (hipFuncGetAttributes(&fa, (const void*)full_cdf_chain_kernel<DT>) == hipSuccess &&
            fa.sharedSizeBytes > st)
            st = fa.sharedSizeBytes;
        (void)hipGetLastError();
        limit = v - (int)((st + 255) & ~(size_t)255);
    }
    const auto fit = [&](int lim) {
        size_t off[7];
        int ns = kStageMax;
        for (; ns > 0; --ns)
            if (chain_lds_layout(DT, nch, ns, off) <= (size_t)lim) break;
        *lds = chain_lds_layout(DT, nch, ns, off);
        return ns;
    };
    int ns = fit(limit);
    if (*lds > 65536 && !raised) {
        hipError_t e = hipFuncSetAttribute((const void*)full_lsum_chain_kernel<DT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, limit);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)full_cdf_chain_kernel<DT>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, limit);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            limit = 65536 - 1024; /* stay within the default */
            ns = fit(limit);
        }
        raised = true;
    }
    return ns;
}

/* Chunks per wave of the streaming passes: 4 (the fastest run length on the
 * B=256 batch) unless that leaves fewer than 16384 waves, then fewer, down
 * to 1, so that small batches spread over the chip.  At most 64: a wave's
 * per-chunk inputs are read with one lane per chunk. */
static int stream_cpw(int nch, int batch)
{
    const int64_t chunks = (int64_t)nch * batch;
    int cpw = 4;
    while (cpw > 1 && chunks / cpw < 16384) cpw >>= 1;
    return cpw;
}

template <int DT>
static hipError_t launch_dt(const FullArgs& a0, hipStream_t s)
{
    FullArgs a = a0;
    size_t lds = 0;
    a.nstage = chain_nstage<DT>(a.nch, &lds);
    a.cpw = stream_cpw(a.nch, a.batch);
    const dim3 sel((unsigned)a.nsel, (unsigned)a.batch);
    const dim3 rows(1u, (unsigned)a.batch);
    const dim3 waves((unsigned)((a.nch + NWF * a.cpw - 1) / (NWF * a.cpw)), (unsigned)a.batch);
    if (a.wide_on) {
        for (int pass = 0; pass < 3; ++pass) {
            hipLaunchKernelGGL((wide_hist_kernel<DT>), sel, dim3(kFullBlock), 0, s, a, pass);
            hipLaunchKernelGGL(wide_find_kernel, rows, dim3(kFullBlock), 0, s, a, pass);
        }
        hipLaunchKernelGGL((wide_ties_kernel<DT>), sel, dim3(kFullBlock), 0, s, a);
        hipLaunchKernelGGL((wide_ties_find_kernel<DT>), rows, dim3(kFullBlock), 0, s, a);
        hipLaunchKernelGGL((wide_replay_kernel<DT>), dim3(1), dim3(64), 0, s, a);
    }
    hipLaunchKernelGGL((full_max_kernel<DT>), waves, dim3(kFullBlock), 0, s, a);
    hipLaunchKernelGGL((full_row_kernel<DT>),
                       dim3(DT == 1 ? (unsigned)(kFullTab / (kFullBlock * kRowPer)) : 1u,
                            (unsigned)a.batch),
                       dim3(kFullBlock), 0, s, a);
    hipLaunchKernelGGL((full_lsum_kernel<DT>), waves, dim3(kFullBlock), 0, s, a);
    hipLaunchKernelGGL((full_lsum_chain_kernel<DT>), rows, dim3(kChainBlock), lds, s, a);
    hipLaunchKernelGGL((full_cdf_kernel<DT>), waves, dim3(kFullBlock), 0, s, a);
    hipLaunchKernelGGL((full_cdf_chain_kernel<DT>), rows, dim3(kChainBlock), lds, s, a);
    return hipGetLastError();
}

hipError_t full_launch(const FullArgs& a, int dtype, hipStream_t s)
{
    return dtype == G4S_DTYPE_BF16 ? launch_dt<1>(a, s) : launch_dt<0>(a, s);
}

}  // namespace g4s
