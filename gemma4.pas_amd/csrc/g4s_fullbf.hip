/*
 * g4s_fullbf.hip -- the streaming pipeline of full-vocabulary bf16 rows on
 * gfx950 (TopK <= 0 or TopK >= V in a batch without wide top-k rows).
 *
 * It computes what g4s_full.hip computes for such rows -- CpuLogitSoftcap,
 * DoSampleTopP and CpuSoftmaxF32 (src/Gemma4.Layers.pas:300-316,
 * src/Gemma4.Model.pas:2691-2737, src/Gemma4.Tensors.pas:638-673) with every
 * running sum the reference's left-to-right binary32 sum -- arranged so that
 * the logits are streamed two and a half times with few instructions per
 * term and the chains find what they re-evaluate already staged:
 *
 *   max:    per run of chunks of a wave, the largest and smallest x, and per
 *           chunk the approximate sum of exp(y - y_run) with y approximated
 *           by a cubic in x (hardware exp2): predictions only;
 *   row:    m = y(max x) from the handle's table of y per bf16 code; e for
 *           the 8192 codes of the 32 largest binades of |x|, correctly
 *           rounded, eight per thread over four workgroups per row; the
 *           binades in which a table e is a half-unit tie; the smallest key
 *           whose e is 1.  Workgroup 0: the predicted binade of LSum entering
 *           every chunk and the chunks to stage (a binade crossing predicted
 *           within a relative margin);
 *   lsum:   per chunk the map of its terms in the predicted binade: a term
 *           adds rint(e / u) units, one fma into 1.5 * 2^23 and one integer
 *           add of the result's bits; staged chunks store their terms and
 *           their lane maps in b and b + 1; the argmax (the first e equal to
 *           1) in the runs that can hold one; and, on a wave the last chunks
 *           leave idle, chunk 0's e and LSum after it, exactly from 0;
 *   lchain: one workgroup per row copies the staged chunks to LDS, then
 *           wave 0 walks the chunk maps from the state after chunk 0 and
 *           resolves each crossing from the staged lane maps; LSum, 1/LSum,
 *           the draw's predicted binades, staged chunks and last chunk;
 *   cdf:    the p table from the e table, the same maps for p up to the
 *           draw's predicted last chunk (every chunk when all probabilities
 *           are requested), and on an idle wave chunk 0 exactly against
 *           thr = fl32(u * TopP);
 *   dchain: the walk against thr: the exact first index, and the token.
 *
 * Chunks are 1024 terms, one wave's (16 consecutive terms per lane), as in
 * g4s_full.hip, whose map and resolution helpers (g4s_fullcore.h) this file
 * shares.
 */
#include "g4s_fullcore.h"

#include <mutex>

namespace g4s {

namespace {

constexpr int kBfWaves = kBfBlock / 64;   /* waves of a table-lookup workgroup */
constexpr int kBfMaxCpw = 4;              /* chunks per wave of the streaming passes */
constexpr float kMagic = 12582912.0f;     /* 1.5 * 2^23 */
constexpr uint32_t kMagicBits = 0x4B400000u;
constexpr double kMargin = 0x1p-10;       /* relative margin of the binade predictions */
constexpr uint32_t kBfMiss2 = 0x70007000u;

/* Table index of the two codes of a dword: entry (sign << 12) | (binade -
 * win_lo) << 7 | mantissa.  With d = code - (win_lo << 7) per 16-bit lane,
 * the entry is (d & 0xFFF) | ((code >> 3) & 0x1000) (bit 12 of code >> 3 is
 * the sign), and a code lies in the window exactly when bits 12-14 of its d
 * are 0 (a code below the window borrows into them since win_lo <= 223). */
__device__ __forceinline__ uint32_t bf_index2(uint32_t w, uint32_t base2, uint32_t& d)
{
    d = pk_sub_u16(w, base2);
    return (d & 0x0FFF0FFFu) | ((w >> 3) & 0x10001000u);
}

/* Both 16-bit lanes shifted left by 2 (byte offsets of 4-byte entries; the
 * largest, 8191 * 4, fits 16 bits). */
__device__ __forceinline__ uint32_t pk_shl2_u16(uint32_t a)
{
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const u16x2 two = {2, 2};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) << two);
}

__device__ __forceinline__ float lds_at(const float* tab, uint32_t byte_off)
{
    return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(tab) + byte_off);
}

/* The 16 terms of one lane from an LDS table, straight from its two 16-byte
 * loads.  Returns the OR of the lane's d words: kBfMiss2 bits set when a
 * code lies outside the table. */
__device__ __forceinline__ uint32_t bf_lookup(const uint4 (&w)[2], uint32_t base2,
                                             const float* tab, float (&t)[kFullPer])
{
    uint32_t acc = 0u;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t ww[4] = {w[q].x, w[q].y, w[q].z, w[q].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t d;
            const uint32_t o = pk_shl2_u16(bf_index2(ww[i], base2, d));
            acc |= d;
            t[8 * q + 2 * i] = lds_at(tab, o & 0xFFFFu);
            t[8 * q + 2 * i + 1] = lds_at(tab, o >> 16);
        }
    }
    return acc;
}

/* The terms of codes outside the table, evaluated from x (rare; the caller
 * branches on a wave vote). */
template <bool P>
__device__ __forceinline__ void bf_fix(const uint4 (&w)[2], uint32_t base2, const Ctx& c,
                                       float (&t)[kFullPer])
{
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t ww[4] = {w[q].x, w[q].y, w[q].z, w[q].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t d;
            (void)bf_index2(ww[i], base2, d);
            if (d & 0x7000u) {
                const float x = __uint_as_float(ww[i] << 16);
                t[8 * q + 2 * i] = P ? p_direct(x, c) : e_direct(x, c);
            }
            if (d & 0x70000000u) {
                const float x = __uint_as_float(ww[i] & 0xFFFF0000u);
                t[8 * q + 2 * i + 1] = P ? p_direct(x, c) : e_direct(x, c);
            }
        }
    }
}

/* The same terms from the row's table in global memory (the chains'
 * re-evaluation of a chunk that was not staged). */
template <bool P>
__device__ __forceinline__ void bf_terms_global(const char* rowp, int c, uint32_t base2,
                                                const float* gtab, const Ctx& ctx,
                                                float (&t)[kFullPer])
{
    const int lane = threadIdx.x & 63;
    const uint4* src = reinterpret_cast<const uint4*>(
        rowp + ((int64_t)c * kFullChunk + (int64_t)lane * kFullPer) * 2);
    uint4 w[2];
    w[0] = src[0];
    w[1] = src[1];
    uint32_t acc = 0u;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t ww[4] = {w[q].x, w[q].y, w[q].z, w[q].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t d;
            const uint32_t ix = bf_index2(ww[i], base2, d);
            acc |= d;
            t[8 * q + 2 * i] = gtab[ix & 0x1FFFu];
            t[8 * q + 2 * i + 1] = gtab[(ix >> 16) & 0x1FFFu];
        }
    }
    if (__ballot((acc & kBfMiss2) != 0u)) bf_fix<P>(w, base2, ctx, t);
}

/* thread_map_nt when every term q = t * 2^(150-e) is below 2^22:
 * RN(t * 2^(150-e) + 1.5 * 2^23) = 1.5 * 2^23 + rint(q) (ties to even, as
 * rint), a binary32 in [2^23, 2^24) whose bits are bits(1.5 * 2^23) +
 * rint(q), so the bits of the 16 results add up to the map. */
__device__ __forceinline__ PMap thread_map_fma(const float (&t)[kFullPer], int32_t e)
{
    const float S = __builtin_ldexpf(1.0f, 150 - e);
    uint32_t acc = 0u;
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) acc += __float_as_uint(__builtin_fmaf(t[j], S, kMagic));
    PMap f;
    f.d0 = f.d1 = (int32_t)(acc - (uint32_t)kFullPer * kMagicBits);
    return f;
}

/* thread_map_fma with the tie vote: r = fl(q + 1.5 * 2^23) holds rint(q)
 * (every term below 2^22 units), and fma(t, S, 1.5 * 2^23 - r) is
 * q - rint(q) exactly; a term is a half-unit tie when that is +-1/2.  A tie
 * anywhere in the wave takes ss::lane_map_fma, the lane maps in the same
 * form (closed form for a lane with one tie). */
__device__ __forceinline__ PMap thread_map_fma_tie(const float (&t)[kFullPer], int32_t e)
{
    const float S = __builtin_ldexpf(1.0f, 150 - e);
    uint32_t acc = 0u;
    float dmax = 0.0f;
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) {
        const float r = __builtin_fmaf(t[j], S, kMagic);
        acc += __float_as_uint(r);
        dmax = __builtin_fmaxf(dmax, __builtin_fabsf(__builtin_fmaf(t[j], S, kMagic - r)));
    }
    if (__ballot(dmax == 0.5f) != 0) return ss::lane_map_fma(t, kFullPer, e);
    PMap f;
    f.d0 = f.d1 = (int32_t)(acc - (uint32_t)kFullPer * kMagicBits);
    return f;
}

/* The lane map of a chunk's terms in binade e: the constant map when no
 * term can be a half-unit tie (the fma form where every term is below
 * 2^(e-128), i.e. tmax * 2^(150-e) < 2^22), else with the tie vote, and the
 * exact per-term lane map where a tie is found. */
__device__ __forceinline__ PMap bf_map(const float (&t)[kFullPer], int32_t e, bool tie, float tmax)
{
    const bool small = __builtin_ldexpf(tmax, 150 - e) < 4194303.0f;
    if (tie) return small ? thread_map_fma_tie(t, e) : thread_map(t, kFullPer, e);
    if (small) return thread_map_fma(t, e);
    return thread_map_nt(t, e);
}

__device__ __forceinline__ int binade_of(double v) { return ss::state_of((float)v).e; }

__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* ------------------------------------------------------------ y table */

/* y = softcap(x) of every bf16 code in the full-row form
 * RN32(tanh(x * fl32(1/cap)) * cap) (Layers.pas:309-314), or x without a
 * softcap; temperature scaling is applied per row. */
__global__ __launch_bounds__(256) void fb_ytab_kernel(float* ytab, float cap)
{
    const uint32_t code = blockIdx.x * 256u + threadIdx.x;
    const float x = __uint_as_float(code << 16);
    ytab[code] = cap > 0.0f ? softcap_full_cr32(x, div_cr32(1.0f, cap), cap) : x;
}

/* ------------------------------------------------------------ reset */

/* The per-row words the kernels accumulate with atomics, as the next call
 * needs them: set once per row when the workspace is created, then by the
 * last kernel of every call after it has read them. */
__device__ __forceinline__ void fb_reset_row(const FullArgs& a, int row)
{
    FbRow f;
    f.kmax = 0u;
    f.amax = 0u;
    f.key1 = 0xFFFFFFFFu;
    f.amx = INT_MAX;
    f.s0 = 0.0f;
    f.c0 = 0.0f;
    f.hit0 = -1;
    f.nsl = 0;
    f.nsc = 0;
    f.e_ninf = f.e_pinf = f.e_tiny = 0.0f;
    f.p_ninf = f.p_pinf = f.p_tiny = 0.0f;
    f.pad = 0;
    a.ws.fbrow[row] = f;
    a.ws.tmask[(int64_t)row * 2] = 0ull;
    a.ws.tmask[(int64_t)row * 2 + 1] = 0ull;
}

__global__ __launch_bounds__(256) void fb_reset_kernel(FullArgs a)
{
    const int row = blockIdx.x * 256 + threadIdx.x;
    if (row < a.batch) fb_reset_row(a, row);
}

/* ------------------------------------------------------------ 1: max */

/* Wave w of workgroup g handles the run of chunks (g*4 + w)*cpw .. +cpw-1;
 * every chunk record gets the run's maxima and the chunk's sum. */
__global__ __launch_bounds__(kFullBlock) void fb_max_kernel(FullArgs a)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.y;
    const int cw = (blockIdx.x * (kFullBlock / 64) + (threadIdx.x >> 6)) * a.cpw;
    if (cw >= a.nch) return;
    const RowIn ri = row_in(a, row);
    if (row_class(a, ri.p.top_k) != kRowFull) return;
    const int n = a.nch - cw < a.cpw ? a.nch - cw : a.cpw;
    const char* rowp = row_ptr<1>(a, row);
    /* every load issued unconditionally (a run shorter than cpw reads its
     * first chunk again in the unused slots), so that each chunk's terms are
     * waited for on their own */
    uint4 w[kBfMaxCpw][2];
#pragma unroll
    for (int q = 0; q < kBfMaxCpw; ++q) {
        const int cq = q < n ? cw + q : cw;
        const uint4* src = reinterpret_cast<const uint4*>(
            rowp + ((int64_t)cq * kFullChunk + (int64_t)lane * kFullPer) * 2);
        w[q][0] = src[0];
        w[q][1] = src[1];
    }
    /* the run's largest and smallest x (the key of the float maximum is the
     * largest key: the order-preserving map identifies -0 and +0) */
    float xm = -__builtin_inff(), xn = __builtin_inff();
#pragma unroll
    for (int q = 0; q < kBfMaxCpw; ++q) {
        if (q < n) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t ww[4] = {w[q][h].x, w[q][h].y, w[q][h].z, w[q][h].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float xl = __uint_as_float(ww[i] << 16);
                    const float xh = __uint_as_float(ww[i] & 0xFFFF0000u);
                    xm = __builtin_fmaxf(xm, __builtin_fmaxf(xl, xh));
                    xn = __builtin_fminf(xn, __builtin_fminf(xl, xh));
                }
            }
        }
    }
    const uint32_t kmax = wave_max_u32(f2key(xm));
    uint32_t amax =
        wave_max_u32(__float_as_uint(__builtin_fmaxf(__builtin_fabsf(xm), __builtin_fabsf(xn))));
    if (amax >= 0x7F800000u) {
        /* an infinity (or NaN) in the run: the table window follows the largest
         * finite |x| (infinities take the row's e(-inf), e(+inf)) */
        uint32_t fa = 0u;
#pragma unroll
        for (int q = 0; q < kBfMaxCpw; ++q) {
            if (q < n) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t ww[4] = {w[q][h].x, w[q][h].y, w[q][h].z, w[q][h].w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t lo = (ww[i] << 16) & 0x7FFFFFFFu, hi = ww[i] & 0x7FFF0000u;
                        fa = lo < 0x7F800000u ? g4s_max_u(fa, lo) : fa;
                        fa = hi < 0x7F800000u ? g4s_max_u(fa, hi) : fa;
                    }
                }
            }
        }
        amax = wave_max_u32(fa);
    }
    if (lane == 0) {
        atomicMax(&a.ws.fbrow[row].kmax, kmax);
        atomicMax(&a.ws.fbrow[row].amax, amax);
    }
    const float cap = a.softcap;
    const float inv_cap = cap > 0.0f ? div_cr32(1.0f, cap) : 1.0f;
    const float T = ri.p.temperature;
    const int scale = (T > 0.0f) && (T != 1.0f);
    const float inv_t = scale ? div_cr32(1.0f, T) : 1.0f;
    const float xmax = key2f(kmax);
    constexpr float kLog2e = 1.4426950408889634f;
    /* |x/cap| < 0.1 everywhere: cap tanh(x/cap) = x - x^3/(3 cap^2) + O(x^5/cap^4),
     * relative error < 1e-5, so log2(e) * y ~ x * (A + B x^2) */
    const bool cubic = !(cap > 0.0f) || __uint_as_float(amax) * inv_cap < 0.1f;
    const float sc = scale ? inv_t : 1.0f;
    const float A = kLog2e * sc;
    const float B = cap > 0.0f ? -A * (inv_cap * inv_cap) * (1.0f / 3.0f) : 0.0f;
    const float K = cubic ? xmax * __builtin_fmaf(B, xmax * xmax, A)
                          : y_approx(xmax, cap, inv_cap, scale, inv_t) * kLog2e;
    const float ymax = K * 0.6931471805599453f;
    FullChunk* rc = a.ws.chunks + (int64_t)row * a.ws.cstride;
#pragma unroll
    for (int q = 0; q < kBfMaxCpw; ++q) {
        if (q < n) {
            float s = 0.0f;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t ww[4] = {w[q][h].x, w[q][h].y, w[q][h].z, w[q][h].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float xl = __uint_as_float(ww[i] << 16);
                    const float xh = __uint_as_float(ww[i] & 0xFFFF0000u);
                    if (cubic) {
                        s += __builtin_amdgcn_exp2f(__builtin_fmaf(xl, __builtin_fmaf(B, xl * xl, A), -K));
                        s += __builtin_amdgcn_exp2f(__builtin_fmaf(xh, __builtin_fmaf(B, xh * xh, A), -K));
                    } else {
                        s += __builtin_amdgcn_exp2f(__builtin_fmaf(
                            y_approx(xl, cap, inv_cap, scale, inv_t), kLog2e, -K));
                        s += __builtin_amdgcn_exp2f(__builtin_fmaf(
                            y_approx(xh, cap, inv_cap, scale, inv_t), kLog2e, -K));
                    }
                }
            }
            s = wave_sum_f32(s);
            if (lane == 0) {
                FullChunk r;
                r.maxkey = kmax;
                r.amax = amax;
                r.ymax = ymax;
                r.sapx = s;
                r.nsurv = kFullChunk;
                r.fsurv = (cw + q) * kFullChunk;
                r.soff = 0;
                r.pad = 0;
                rc[cw + q] = r;
            }
        }
    }
}

/* ------------------------------------------------------------ 2: row */

constexpr int kRowWG = 4;                                   /* table workgroups per row */
constexpr int kRowEnt = kBfTab / (kRowWG * kFullBlock);    /* table entries per thread */
static_assert(kRowEnt * kRowWG * kFullBlock == kBfTab, "whole workgroups of table entries");

/* e of one bf16 code: RN32(exp(y - m)), y from the handle's table scaled by
 * 1/T when the row scales (the same value e_direct computes). */
__device__ __forceinline__ float bf_e_y(float y0, int scale, float inv_t, float m)
{
    return exp_diff_cr32(scale ? y0 * inv_t : y0, m); /* Tensors.pas:660 */
}
__device__ __forceinline__ float bf_e(const float* ytab, uint32_t code, int scale, float inv_t,
                                     float m)
{
    return bf_e_y(ytab[code], scale, inv_t, m);
}

/* bf_e_y of N values side by side: the branch-free binary64 route for all
 * of them (their evaluations interleave), then the exact route for the few
 * it leaves. */
template <int N>
__device__ __forceinline__ void bf_e_many(const float (&y0)[N], int scale, float inv_t, float m,
                                          float (&ev)[N])
{
    uint32_t miss = 0u;
#pragma unroll
    for (int q = 0; q < N; ++q)
        if (!exp_diff_cr32_try(scale ? y0[q] * inv_t : y0[q], m, &ev[q])) miss |= 1u << q;
    if (miss != 0u) {
#pragma unroll
        for (int q = 0; q < N; ++q)
            if ((miss >> q) & 1u) ev[q] = bf_e_y(y0[q], scale, inv_t, m);
    }
}

/* Workgroups 1 .. kRowWG of a row: table entries ((g-1)*kRowEnt + q)*256 +
 * tid, the binades where one is a half-unit tie, the smallest key whose e
 * is 1.  Workgroup 0: the row record, the predicted binade of LSum entering
 * every chunk and the staged chunks.  (Chunk 0 is evaluated exactly by the
 * LSum map pass, beside its chunk maps.) */
__global__ __launch_bounds__(kFullBlock) void fb_row_kernel(FullArgs a)
{
    __shared__ Scratch sh;
    const int tid = threadIdx.x, lane = tid & 63;
    const int row = blockIdx.y, g = blockIdx.x;
    const RowIn ri = row_in(a, row);
    if (row_class(a, ri.p.top_k) != kRowFull) return;
    const int nch = a.nch;
    const int64_t rbase = (int64_t)row * a.ws.cstride;
    FbRow* fr = a.ws.fbrow + row;
    const uint32_t km = fr->kmax, am = fr->amax;
    const float T = ri.p.temperature;
    const int scale = (T > 0.0f) && (T != 1.0f);                       /* Model.pas:2703 */
    const float inv_t = scale ? div_cr32(1.0f, T) : 1.0f;              /* Model.pas:2705 */
    const float* ytab = a.ws.ytab;
    const float ym = ytab[__float_as_uint(key2f(km)) >> 16];
    const float m = scale ? ym * inv_t : ym;                           /* Tensors.pas:648-654 */
    int win = (int)((am >> 23) & 0xFFu) - (kBfWin - 1);
    win = win < 0 ? 0 : (win > 223 ? 223 : win);
    if (g > 0 && g <= kRowWG) {
        uint64_t tb = 0ull;
        uint32_t k1 = 0xFFFFFFFFu;
        /* every entry's y gathered before the exps, which run side by side */
        float ev[kRowEnt], y0[kRowEnt];
        uint32_t code[kRowEnt];
#pragma unroll
        for (int q = 0; q < kRowEnt; ++q) {
            const int i = ((g - 1) * kRowEnt + q) * kFullBlock + tid;
            code[q] = ((uint32_t)(i >> 12) << 15) |
                      ((uint32_t)(win + ((i >> 7) & (kBfWin - 1))) << 7) | (uint32_t)(i & 127);
            y0[q] = ytab[code[q]];
        }
        bf_e_many(y0, scale, inv_t, m, ev);
#pragma unroll
        for (int q = 0; q < kRowEnt; ++q) {
            const int i = ((g - 1) * kRowEnt + q) * kFullBlock + tid;
            a.ws.etab8[(int64_t)row * kBfTab + i] = ev[q];
            tb |= tie_bits(ev[q], kTieBaseE);
            /* the argmax is the first e == 1; e is monotone in x, so the codes
             * with e == 1 are those from key1 up -- unless the smallest
             * positive code of the window already has e == 1, when codes
             * below the window may too: then every chunk is searched */
            if (ev[q] == 1.0f) k1 = g4s_min_u(k1, i == 0 ? 0u : f2key(__uint_as_float(code[q] << 16)));
        }
        tb = wave_or64(tb);
        if (lane == 0 && tb != 0ull)
            atomicOr((unsigned long long*)&a.ws.tmask[(int64_t)row * 2], (unsigned long long)tb);
        k1 = wave_min_u32(k1);
        if (lane == 0 && k1 != 0xFFFFFFFFu) atomicMin(&fr->key1, k1);
        return;
    }

    /* the terms of codes outside the table: e(-inf), e(+inf), and the codes
     * below its binades -- e is monotone in x, so when the largest negative and
     * the largest positive one give the same e, every code between does
     * (threads 0-3, one evaluation each; combined after the barriers below) */
    __shared__ float s_out[4];
    if (tid < 4) {
        const uint32_t top = win > 0 ? ((uint32_t)win << 7) - 1u : 0u;
        const uint32_t code = tid == 0 ? 0xFF80u : (tid == 1 ? 0x7F80u : (tid == 2 ? 0x8000u | top : top));
        s_out[tid] = bf_e(ytab, code, scale, inv_t, m);
    }

    /* predicted LSum entering every chunk: exclusive prefix of the estimates
     * (non-finite estimates add 0); a chunk is staged when LSum is predicted
     * to change binade in it within the margin */
    const FullChunk* rc = a.ws.chunks + rbase;
    const auto est = [&](const FullChunk& c) {
        double z = (double)c.ymax - (double)m;
        z = z > 50.0 ? 50.0 : (z < -700.0 ? -700.0 : z);
        const double v = (double)c.sapx * exp_fast_d(z);
        return (v >= 0.0 && v < 1e300) ? v : 0.0;
    };
    constexpr int kCpt = (kBfMaxChunks + kFullBlock - 1) / kFullBlock;
    const int cpt = (nch + kFullBlock - 1) / kFullBlock;
    /* each estimate evaluated once and kept for the three passes */
    double es[kCpt];
    double tsum = 0.0;
#pragma unroll
    for (int q = 0; q < kCpt; ++q) {
        const int cb = tid * cpt + q;
        es[q] = (q < cpt && cb < nch) ? est(rc[cb]) : 0.0;
        tsum += es[q];
    }
    double total;
    const double pre0 = block_excl_scan_d(tsum, sh, total);
    int cnt = 0;
    {
        double p = pre0;
#pragma unroll
        for (int q = 0; q < kCpt; ++q) {
            const int cb = tid * cpt + q;
            if (q < cpt && cb < nch) {
                const double e = es[q];
                if (cb > 0 && binade_of(p * (1.0 - kMargin)) != binade_of((p + e) * (1.0 + kMargin)))
                    ++cnt;
                p += e;
            }
        }
    }
    int nstaged;
    int pos = block_excl_scan_i(cnt, sh, nstaged);
    int32_t* bl = a.ws.beta_l + rbase;
    BfStage* sg = a.ws.stage + (int64_t)row * kBfStage;
    {
        double p = pre0;
#pragma unroll
        for (int q = 0; q < kCpt; ++q) {
            const int cb = tid * cpt + q;
            if (q < cpt && cb < nch) {
                const double e = es[q];
                int32_t beta = -1;
                if (cb > 0) {
                    const int lo = binade_of(p * (1.0 - kMargin));
                    beta = binade_of(p);
                    if (lo != binade_of((p + e) * (1.0 + kMargin))) {
                        if (pos < kBfStage) {
                            beta = -2 - pos;
                            sg[pos].b = lo;
                            sg[pos].chunk = cb;
                            sg[pos].pad[0] = 0;
                        }
                        ++pos;
                    }
                }
                bl[cb] = beta;
                p += e;
            }
        }
    }
    if (tid == 0) {
        const float en = s_out[0], ep = s_out[1];
        fr->e_ninf = en;
        fr->e_pinf = ep;
        fr->e_tiny = (win > 0 && s_out[2] == s_out[3]) ? s_out[3] : __builtin_nanf("");
        /* infinities with e == 1 hold the argmax's value too */
        if (ep == 1.0f) atomicMin(&fr->key1, f2key(__builtin_inff()));
        if (en == 1.0f) atomicMin(&fr->key1, f2key(-__builtin_inff()));
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
        r.count = a.vocab;
        r.first = 0;
        r.beta_end = binade_of(total);
        for (int j = 0; j < kNear; ++j) r.near[j] = INT_MAX;
        r.l_reev = r.l_rounds = r.c_reev = r.c_rounds = 0;
        a.ws.rows[row] = r;
        fr->nsl = nstaged < kBfStage ? nstaged : kBfStage;
    }
}

/* Chunk 0 exactly from 0 (one wave of the LSum map pass, which has the row's
 * values in its record r): its e, kept for the draw's chunk 0, its first
 * e == 1, and LSum after it (Tensors.pas:657-663): the first kSeqLanes lanes
 * term by term (the sum changes binade every few dozen terms there), then
 * rounds of lane maps. */
__device__ void bf_head(const FullArgs& a, int row, float* hbuf)
{
    const int lane = threadIdx.x & 63;
    const FullRow r = a.ws.rows[row];
    FbRow* fr = a.ws.fbrow + row;
    const uint4* src = reinterpret_cast<const uint4*>(row_ptr<1>(a, row) + (int64_t)lane * kFullPer * 2);
    const uint4 w0 = src[0], w1 = src[1];
    const uint32_t ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    float t[kFullPer], y0[kFullPer];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        y0[2 * i] = a.ws.ytab[ww[i] & 0xFFFFu];
        y0[2 * i + 1] = a.ws.ytab[ww[i] >> 16];
    }
    /* two halves of eight: sixteen side by side would not fit this kernel's
     * registers */
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float yh[kFullPer / 2], th[kFullPer / 2];
#pragma unroll
        for (int j = 0; j < kFullPer / 2; ++j) yh[j] = y0[h * (kFullPer / 2) + j];
        bf_e_many(yh, r.scale, r.inv_t, r.m, th);
#pragma unroll
        for (int j = 0; j < kFullPer / 2; ++j) t[h * (kFullPer / 2) + j] = th[j];
    }
    float4* hd = reinterpret_cast<float4*>(a.ws.head + (int64_t)row * kFullChunk + lane * kFullPer);
    float4* hb = reinterpret_cast<float4*>(hbuf + lane * kFullPer);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 e4 = make_float4(t[4 * k], t[4 * k + 1], t[4 * k + 2], t[4 * k + 3]);
        hd[k] = e4;
        hb[k] = e4;
    }
    uint32_t f1 = 0xFFFFFFFFu;
#pragma unroll
    for (int j = kFullPer - 1; j >= 0; --j) f1 = t[j] == 1.0f ? (uint32_t)(lane * kFullPer + j) : f1;
    f1 = wave_min_u32(f1);
    if (lane == 0 && f1 != 0xFFFFFFFFu) atomicMin(&fr->amx, (int32_t)f1);
    wave_lds_sync();
    int hit = -1, rounds = 0;
    State st = seq_walk(hbuf, kSeqLanes * kFullPer, __builtin_inff(), &hit);
    /* the lane's terms again from LDS: not held in registers across the walk */
    const float4* hr = reinterpret_cast<const float4*>(hbuf + lane * kFullPer);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 e4 = hr[k];
        t[4 * k] = e4.x;
        t[4 * k + 1] = e4.y;
        t[4 * k + 2] = e4.z;
        t[4 * k + 3] = e4.w;
    }
    st = resolve_wave(t, kFullPer, st, __builtin_inff(), kSeqLanes, &hit, &rounds);
    if (lane == 0) fr->s0 = ss::value_of(st);
}

/* The draw through chunk 0 (Model.pas:2727-2735), one wave of the draw's
 * map pass: p = fl32(e * inv) of its terms, staged in index order in hbuf,
 * then as LSum's chunk 0 but against thr. */
__device__ void bf_draw0(const FullArgs& a, int row, const FullRow& r, float* hbuf)
{
    const int lane = threadIdx.x & 63;
    float t[kFullPer];
    const float4* src =
        reinterpret_cast<const float4*>(a.ws.head + (int64_t)row * kFullChunk + lane * kFullPer);
    float4* hb = reinterpret_cast<float4*>(hbuf + lane * kFullPer);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 e = src[k];
        t[4 * k] = e.x * r.inv;
        t[4 * k + 1] = e.y * r.inv;
        t[4 * k + 2] = e.z * r.inv;
        t[4 * k + 3] = e.w * r.inv;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) hb[k] = make_float4(t[4 * k], t[4 * k + 1], t[4 * k + 2], t[4 * k + 3]);
    wave_lds_sync();
    int hit = -1, rounds = 0;
    State st = seq_walk(hbuf, kSeqLanes * kFullPer, r.thr, &hit);
    if (hit < 0) {
        /* the lane's terms again from LDS, as in bf_head */
        const float4* hr = reinterpret_cast<const float4*>(hbuf + lane * kFullPer);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 p4 = hr[k];
            t[4 * k] = p4.x;
            t[4 * k + 1] = p4.y;
            t[4 * k + 2] = p4.z;
            t[4 * k + 3] = p4.w;
        }
        st = resolve_wave(t, kFullPer, st, r.thr, kSeqLanes, &hit, &rounds);
    }
    if (lane == 0) {
        a.ws.fbrow[row].hit0 = hit;
        a.ws.fbrow[row].c0 = ss::value_of(st);
    }
}

/* ------------------------------------------ 3 and 5: chunk maps (e, then p) */

constexpr int kRing = 2; /* chunks a wave keeps in flight */

/* Chunks per wave of the table-lookup passes: three times the max pass's
 * runs, so that a 256-chunk row takes three 512-thread workgroups and the
 * B=256 batch (768 workgroups) is resident at once at three per compute
 * unit (81 VGPRs, 32 KiB of LDS each). */
__host__ __device__ __forceinline__ int bf_maps_cpw(int cpw) { return 3 * cpw; }

/* A chunk whose map a chain must build itself (a code outside the table):
 * map {-1, -1}, or an invalid binade for a staged chunk. */
constexpr int32_t kDeferred = -1;

/* The per-chunk work of fb_maps_kernel (chunk cw + q * cstep of the wave,
 * its two 16-byte loads in w); the row's values arrive in MapsRow. */
struct MapsRow {
    const float* tab;
    BfStage* stg;
    PMap* gmap;
    int32_t* amxp;
    float* po_row;
    int32_t* io_row;
    uint64_t tm;
    uint64_t argm;
    Ctx ctx;
    uint32_t base, base2;
    int32_t betas;
    int cw, cstep, tbase; /* chunk q of the wave: cw + q * cstep */
    float tmax, kninf, kpinf, ktiny;
    bool maps;
};

template <bool P, bool ALL>
__device__ __forceinline__ void maps_chunk(const MapsRow& R, const uint4 (&w)[2], int q)
{
    const int lane = threadIdx.x & 63;
    const float* tab = R.tab;
    BfStage* stg = R.stg;
    PMap* gmap = R.gmap;
    int32_t* amxp = R.amxp;
    float* po_row = R.po_row;
    int32_t* io_row = R.io_row;
    const uint64_t tm = R.tm, argm = R.argm;
    const Ctx& ctx = R.ctx;
    const uint32_t base = R.base, base2 = R.base2;
    const int32_t betas = R.betas;
    const int tbase = R.tbase;
    const float tmax = R.tmax, kninf = R.kninf, kpinf = R.kpinf, ktiny = R.ktiny;
    const bool maps = R.maps;
    const int cb = R.cw + q * R.cstep;
    if (!ALL && cb == 0) return; /* chunk 0: outputs only */
    const int64_t e0 = (int64_t)cb * kFullChunk + (int64_t)lane * kFullPer;
    float t[kFullPer];
    const uint32_t acc = bf_lookup(w, base2, tab, t);          /* Tensors.pas:660, 671 */
    bool miss = __ballot((acc & kBfMiss2) != 0u) != 0;
    const int32_t beta = __builtin_amdgcn_readlane(betas, q);
    /* codes outside the table: infinities and (when they all share one
     * value) the codes below its binades take the row's constants; a NaN,
     * or codes below that differ, leave the chunk to the chain */
    const bool outside = miss;
    if (miss && !ALL) {
        bool bad = false;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t ww[4] = {w[h].x, w[h].y, w[h].z, w[h].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const uint32_t code = k ? ww[i] >> 16 : ww[i] & 0xFFFFu;
                    const uint32_t ac = code & 0x7FFFu;
                    const bool in = ac - base < 0x1000u; /* in the table */
                    const bool above = ac >= base + 0x1000u;
                    bad = bad || (!in && ((above && ac != 0x7F80u) || (!above && !(ktiny == ktiny))));
                    const float v = above ? ((code & 0x8000u) ? kninf : kpinf) : ktiny;
                    t[8 * h + 2 * i + k] = in ? t[8 * h + 2 * i + k] : v;
                }
            }
        }
        miss = __ballot(bad) != 0;
    }
    if (miss) {
        if (ALL) {
            bf_fix<P>(w, base2, ctx, t);
        } else {
            if (lane == 0) {
                if (beta <= -2)
                    stg[-2 - beta].b = kDeferred;
                else
                    gmap[cb] = PMap{kDeferred, kDeferred};
            }
            return;
        }
    }
    if (!P && ((argm >> q) & 1ull)) {
        /* the first index of the largest p: the first e == 1 (the next
         * float below 1 gives a p below 1/LSum under the reciprocal
         * multiply), Model.pas:2712-2721 */
        uint32_t f1 = 0xFFFFFFFFu;
#pragma unroll
        for (int j = 0; j < kFullPer; ++j)
            f1 = t[j] == 1.0f ? g4s_min_u(f1, (uint32_t)(e0 + j)) : f1;
        f1 = wave_min_u32(f1);
        if (lane == 0 && f1 != 0xFFFFFFFFu) atomicMin(amxp, (int32_t)f1);
    }
    if (ALL) {
        /* caller rows need not be 16-byte aligned: scalar stores */
        float* po = po_row + e0;
        int32_t* io = io_row ? io_row + e0 : nullptr;
#pragma unroll
        for (int j = 0; j < kFullPer; ++j) {
            po[j] = t[j]; /* Tensors.pas:671 */
            if (io) io[j] = (int32_t)(e0 + j);
        }
    }
    if (cb == 0 || !maps) return;
    if (beta <= -2) {
        /* a staged chunk, for the chain: its terms (pad[0]: a code outside the
         * table) and its lane maps in the predicted binade b and in b + 1
         * (ties per the row's mask), with their inclusive lane scans from an
         * even and from an odd entering significand (pad[1]: bit h set when
         * the maps in b + h are constant, bit 2 when the scans are there) */
        BfStage* sg = stg + (-2 - beta);
        if (lane == 0) sg->pad[0] = outside ? 1 : 0;
        float4* dst = reinterpret_cast<float4*>(sg->t + lane * kFullPer);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            dst[k] = make_float4(t[4 * k], t[4 * k + 1], t[4 * k + 2], t[4 * k + 3]);
        const int32_t b = __builtin_amdgcn_readfirstlane(sg->b);
        if (b >= 1) {
            int32_t flags = 4;
#pragma nounroll
            for (int h = 0; h < 2; ++h) {
                const PMap m = bf_map(t, b + h, outside || tie_possible(tm, tbase, b + h), tmax);
                (h ? sg->hi : sg->lo)[lane] = m;
                int32_t x0, x1;
                if (__ballot(m.d0 != m.d1) == 0) {
                    x0 = x1 = wave_inclusive_scan(m.d0 > ss::kTop ? ss::kTop : m.d0);
                    flags |= 1 << h;
                } else {
                    const PMap incl = wave_scan_maps(m);
                    x0 = incl.d0;
                    x1 = incl.d1;
                }
                sg->xs[128 * h + lane] = x0;
                sg->xs[128 * h + 64 + lane] = x1;
            }
            if (lane == 0) sg->pad[1] = flags;
        }
    } else if (beta >= 1) {
        const PMap cm =
            wave_chunk_map(bf_map(t, beta, outside || tie_possible(tm, tbase, beta), tmax));
        if (lane == 0) gmap[cb] = cm;
    }
}

/* One pass over the chunks 1 .. clast of every full row (chunk 0 is
 * evaluated exactly, on the last wave of the row's last workgroup): the
 * terms from the LDS table (e, or p when P, made from the e table as it is
 * copied), per chunk its map in the predicted binade (or, for a staged
 * chunk, its lane maps in b and b + 1 and its terms).  Without P: the
 * argmax in the chunks whose run can hold an e == 1.  With
 * ALL (P and every probability requested): the probabilities, including
 * those of codes outside the table; otherwise a chunk holding such a code
 * is left to the chain.  Every wave streams the chunks dealt to it (about
 * bf_maps_cpw() of them), kRing of them in flight. */
template <bool P, bool ALL>
__global__ __launch_bounds__(kBfBlock) __attribute__((amdgpu_waves_per_eu(6, 6))) void fb_maps_kernel(FullArgs a)
{
    __shared__ __align__(16) float tab[kBfTab];
    __shared__ __align__(16) float hbuf[kFullChunk];
    __shared__ uint64_t s_tmw[kBfWaves];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int row = blockIdx.y;
    const int nch = a.nch;
    const int cpw = bf_maps_cpw(a.cpw);
    const RowIn ri = row_in(a, row);
    if (row_class(a, ri.p.top_k) != kRowFull) return;
    const FullRow r = a.ws.rows[row];
    /* the draw's pass has nothing to do for a row that draws nothing (T <= 0,
     * or a threshold <= 0: its chain writes the outputs) unless every
     * probability is written */
    const int clast = P ? ((!ALL && r.nodraw != 0) ? -1 : r.c_last) : nch - 1;
    /* the wave that evaluates chunk 0 is in workgroup glast: the last one
     * with a chunk of the LSum pass, the last of the grid in the draw's pass
     * (whose last chunk varies by row); another workgroup that no chunk is
     * dealt to has nothing to do */
    const int glast = P ? (int)gridDim.x - 1 : clast / (kBfWaves * cpw);
    if (P ? (clast < 0 || ((int)blockIdx.x != glast && (int)blockIdx.x * kBfWaves > clast))
          : (int)blockIdx.x * kBfWaves * cpw > clast)
        return;
    {
        const float4* src = reinterpret_cast<const float4*>(a.ws.etab8 + (int64_t)row * kBfTab);
        float4 v[kBfTab / 4 / kBfBlock];
#pragma unroll
        for (int q = 0; q < kBfTab / 4 / kBfBlock; ++q) v[q] = src[threadIdx.x + q * kBfBlock];
        if (P) {
            /* the p table (Tensors.pas:666-672) and the binades where one of
             * its values is a half-unit tie; the first workgroup keeps the
             * table for the draw's chain (its chunks evaluated anew) */
            float4* dst = reinterpret_cast<float4*>(a.ws.ptab8 + (int64_t)row * kBfTab);
            uint64_t tb = 0ull;
#pragma unroll
            for (int q = 0; q < kBfTab / 4 / kBfBlock; ++q) {
                v[q] = make_float4(v[q].x * r.inv, v[q].y * r.inv, v[q].z * r.inv, v[q].w * r.inv);
                tb |= tie_bits(v[q].x, kTieBaseP) | tie_bits(v[q].y, kTieBaseP) |
                      tie_bits(v[q].z, kTieBaseP) | tie_bits(v[q].w, kTieBaseP);
                if (blockIdx.x == 0) dst[threadIdx.x + q * kBfBlock] = v[q];
            }
            tb = wave_or64(tb);
            if (lane == 0) s_tmw[wid] = tb;
        }
#pragma unroll
        for (int q = 0; q < kBfTab / 4 / kBfBlock; ++q)
            reinterpret_cast<float4*>(tab)[threadIdx.x + q * kBfBlock] = v[q];
    }
    __syncthreads();
    uint64_t tm = 0ull;
    if (P) {
#pragma unroll
        for (int k = 0; k < kBfWaves; ++k) tm |= s_tmw[k];
    } else {
        tm = a.ws.tmask[(int64_t)row * 2];
    }
    /* The last wave of workgroup glast evaluates chunk 0 (for LSum, or the
     * draw against thr) and takes no other chunk.  Chunks 0 .. clast are dealt
     * in turn to the row's other waves (W of them, over workgroups 0 ..
     * glast): wave g takes g, g + W, g + 2W, ...  The chunks of a binade that
     * takes the per-term tie vote, and the staged chunks, which cluster where
     * the sum is small, so spread over every wave of the row, and in the
     * draw's pass a row that stops early spreads as wide as one that does
     * not. */
    if ((int)blockIdx.x == glast && wid == kBfWaves - 1) {
        if (!P)
            bf_head(a, row, hbuf);
        else if (r.nodraw == 0)
            bf_draw0(a, row, r, hbuf);
        return;
    }
    const int W = (glast + 1) * kBfWaves - 1;
    const int cw = (int)blockIdx.x * kBfWaves + wid;
    const int cstep = W;
    if (cw > clast) return;
    const int n = (clast - cw) / W + 1; /* <= cpw * 8 / 7 + 1 */
    const char* rowp = row_ptr<1>(a, row);
    const int64_t rbase = (int64_t)row * a.ws.cstride;
    const uint32_t base = (uint32_t)r.win_lo << 7;
    const uint32_t base2 = base | (base << 16);
    const int tbase = P ? kTieBaseP : kTieBaseE;
    const int32_t betas = lane < n ? (P ? a.ws.beta_c : a.ws.beta_l)[rbase + cw + lane * cstep] : 0;
    PMap* gmap = (P ? a.ws.cmap : a.ws.lmap) + rbase;
    /* chunks whose run can hold an e == 1 (bit q: chunk cw + q * cstep) */
    uint64_t argm = 0ull;
    if (!P) {
        const uint32_t key1 = a.ws.fbrow[row].key1;
        argm = __ballot(lane < n && a.ws.chunks[rbase + cw + lane * cstep].maxkey >= key1);
    }
    const bool maps = !P || !r.nodraw;
    const float tmax = P ? r.inv : 1.0f; /* no term exceeds it: e <= 1, p <= fl32(1/LSum) */
    const FbRow* fq = a.ws.fbrow + row;
    const float kninf = P ? fq->p_ninf : fq->e_ninf;
    const float kpinf = P ? fq->p_pinf : fq->e_pinf;
    const float ktiny = P ? fq->p_tiny : fq->e_tiny;
    const Ctx ctx = make_ctx(a, r, kRowFull);

    MapsRow R;
    R.tab = tab;
    R.stg = a.ws.stage + (int64_t)row * kBfStage;
    R.gmap = gmap;
    R.amxp = &a.ws.fbrow[row].amx;
    R.po_row = ALL ? a.out.probs + (int64_t)row * a.out.capacity : nullptr;
    R.io_row = (ALL && a.out.indices) ? a.out.indices + (int64_t)row * a.out.capacity : nullptr;
    R.tm = tm;
    R.argm = argm;
    R.ctx = ctx;
    R.base = base;
    R.base2 = base2;
    R.betas = betas;
    R.cw = cw;
    R.cstep = cstep;
    R.tbase = tbase;
    R.tmax = tmax;
    R.kninf = kninf;
    R.kpinf = kpinf;
    R.ktiny = ktiny;
    R.maps = maps;
    const auto load = [rowp, lane](uint4 (&w)[2], int c) {
        const uint4* src = reinterpret_cast<const uint4*>(
            rowp + ((int64_t)c * kFullChunk + (int64_t)lane * kFullPer) * 2);
        w[0] = src[0];
        w[1] = src[1];
    };
    /* The loads are issued unconditionally (past the run's last chunk a slot
     * reads that chunk again), and the next slot's terms are waited for
     * before this slot is loaded again: the waits then never include the
     * load just issued, which stays in flight while the next chunk is
     * processed. */
    const auto ready = [](const uint4 (&v)[2]) {
        asm volatile("" ::"v"(v[0].x), "v"(v[0].y), "v"(v[0].z), "v"(v[0].w), "v"(v[1].x),
                     "v"(v[1].y), "v"(v[1].z), "v"(v[1].w));
    };
    uint4 w[kRing][2];
#pragma unroll
    for (int r = 0; r < kRing; ++r) load(w[r], cw + (r < n ? r : n - 1) * cstep);
    for (int q = 0; q < n; q += kRing) {
#pragma unroll
        for (int r = 0; r < kRing; ++r) {
            if (q + r < n) maps_chunk<P, ALL>(R, w[r], q + r);
            ready(w[(r + 1) % kRing]);
            const int nx = q + r + kRing;
            load(w[r], cw + (nx < n ? nx : n - 1) * cstep);
        }
    }
}

/* ------------------------------------------------------- 4 and 6: chains */

/* LDS of a chain workgroup: the chunk maps and predicted binades, the exact
 * LSum after every chunk, the wrapping prefix sums of the chunk increments,
 * the walk's stops and the staged chunks (with their lane maps and scans). */
struct BfChainLds {
    PMap* cm;
    int32_t* cb;
    float* cpost;
    uint64_t* pre;   /* pre[c] = sum over chunks 0..c of the capped increment, plus
                        2^40 for each map that is not constant */
    int32_t* stops;  /* chunks the walk resolves one by one, ascending, then nch */
    int32_t* nstop;
    BfStage* st;
};

__host__ __device__ __forceinline__ size_t bf_chain_lds(int nch, size_t* off)
{
    size_t o = 0;
    off[0] = o;
    o += (size_t)nch * sizeof(PMap);
    off[1] = o;
    o += (size_t)nch * 4;
    off[2] = o;
    o += (size_t)nch * 4;
    o = (o + 7) & ~(size_t)7;
    off[3] = o;
    o += (size_t)nch * 8;
    off[4] = o;
    o += (size_t)(nch + 1) * 4;
    off[5] = o;
    o += 16;
    o = (o + 15) & ~(size_t)15;
    off[6] = o;
    o += (size_t)kBfStage * sizeof(BfStage);
    return o;
}

__device__ __forceinline__ BfChainLds bf_chain_layout(char* base, int nch)
{
    size_t off[7];
    (void)bf_chain_lds(nch, off);
    BfChainLds L;
    L.cm = reinterpret_cast<PMap*>(base + off[0]);
    L.cb = reinterpret_cast<int32_t*>(base + off[1]);
    L.cpost = reinterpret_cast<float*>(base + off[2]);
    L.pre = reinterpret_cast<uint64_t*>(base + off[3]);
    L.stops = reinterpret_cast<int32_t*>(base + off[4]);
    L.nstop = reinterpret_cast<int32_t*>(base + off[5]);
    L.st = reinterpret_cast<BfStage*>(base + off[6]);
    return L;
}

/* A chunk the walk must resolve by itself: staged, deferred, beyond the last
 * chunk, or a map that alone leaves its binade. */
__device__ __forceinline__ bool bf_stop(PMap f, int32_t b) { return b < 1 || f.d0 >= ss::kTop; }

constexpr uint64_t kNonConst = 1ull << 40; /* marks a map with a half-unit tie in pre[] */

__device__ __forceinline__ uint64_t bf_pre_inc(PMap f)
{
    const uint64_t c = (uint64_t)(f.d0 < 0 ? 0 : (f.d0 > ss::kTop ? ss::kTop : f.d0));
    return c + (f.d0 != f.d1 ? kNonConst : 0ull);
}

/* Chain prologue (all threads; ends with a barrier): the maps and binades of
 * chunks 0 .. clast (a deferred map, or anything beyond clast, gets binade
 * -1) and the first `ns` staged chunks (with the lane maps and scans the map
 * pass left in them), every global load issued before the first LDS store;
 * then wave 0 lists the stops and the prefix sums of the chunk increments. */
__device__ __forceinline__ void bf_chain_prologue(const PMap* gmap, const int32_t* gbeta,
                                                  const BfStage* gst, int ns, int nch, int clast,
                                                  const BfChainLds& L)
{
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    constexpr int kPer = kBfMaxChunks / kFullBlock;
    PMap f[kPer];
    int32_t b[kPer];
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const int c = tid + q * kFullBlock;
        const bool in = c < nch && c <= clast;
        f[q] = in ? gmap[c] : ss::map_identity();
        b[q] = in ? gbeta[c] : -1;
    }
    const uint4* src = reinterpret_cast<const uint4*>(gst);
    uint4* dst = reinterpret_cast<uint4*>(L.st);
    const int nvec = ns * (int)(sizeof(BfStage) / 16);
    /* every staged chunk's 16-byte pieces loaded in batches of eight, each
     * batch's loads issued before its stores (a plain copy loop waits for
     * each load before its store) */
    constexpr int kCopy = (kBfStage * (int)(sizeof(BfStage) / 16) + kFullBlock - 1) / kFullBlock;
    static_assert(kCopy <= 32, "four batches of eight");
    for (int r0 = 0; r0 < kCopy && tid + r0 * kFullBlock < nvec; r0 += 8) {
        uint4 c0, c1, c2, c3, c4, c5, c6, c7;
        const int i0 = tid + r0 * kFullBlock;
#define G4S_LD(k) if (i0 + (k) * kFullBlock < nvec) c##k = src[i0 + (k) * kFullBlock];
#define G4S_ST(k) if (i0 + (k) * kFullBlock < nvec) dst[i0 + (k) * kFullBlock] = c##k;
        G4S_LD(0) G4S_LD(1) G4S_LD(2) G4S_LD(3) G4S_LD(4) G4S_LD(5) G4S_LD(6) G4S_LD(7)
        G4S_ST(0) G4S_ST(1) G4S_ST(2) G4S_ST(3) G4S_ST(4) G4S_ST(5) G4S_ST(6) G4S_ST(7)
#undef G4S_LD
#undef G4S_ST
    }
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const int c = tid + q * kFullBlock;
        if (c < nch) {
            L.cm[c] = f[q];
            L.cb[c] = (b[q] >= 0 && f[q].d0 < 0) ? -1 : b[q];
        }
    }
    __syncthreads();
    if (wid == 0) {
        /* prefix sums of the capped increments and the stops (lane l: chunks
         * l*cpt .. l*cpt+cpt-1) */
        const int cpt = (nch + 63) / 64;
        uint64_t sum = 0ull;
        int nst = 0;
        for (int q = 0; q < cpt; ++q) {
            const int c = lane * cpt + q;
            if (c < nch) {
                const PMap m = L.cm[c];
                sum += bf_pre_inc(m);
                nst += bf_stop(m, L.cb[c]) ? 1 : 0;
            }
        }
        /* every total stays below 2^51 (at most 1024 chunks of 2^24 + 2^40); the
         * scan over the wave runs in binary64, exact below 2^53 */
        const double incl = wave_incl_scan_d((double)sum);
        uint64_t run = (uint64_t)incl - sum;
        const int sincl = wave_inclusive_scan(nst);
        int pos = sincl - nst;
        for (int q = 0; q < cpt; ++q) {
            const int c = lane * cpt + q;
            if (c < nch) {
                const PMap m = L.cm[c];
                run += bf_pre_inc(m);
                L.pre[c] = run;
                if (bf_stop(m, L.cb[c])) L.stops[pos++] = c;
            }
        }
        if (lane == 63) {
            L.stops[sincl] = nch;
            *L.nstop = sincl;
        }
    }
    __syncthreads();
}

/* The exact running sum through chunk c from the exact entering state st
 * (wave 0 of a chain): a staged chunk takes its lane maps in b and b + 1 --
 * with constant maps one step over the precomputed lane scans: the first lane
 * that leaves b (or reaches thr) adds its terms with plain binary32
 * additions and the lanes after it apply in b + 1; any other chunk is
 * re-evaluated from the logits and the row's table in global memory and,
 * without P, searched for an e == 1 (*amx: the first index found).  *hit:
 * the chunk-relative index of the first term whose running sum reaches thr,
 * -1: none. */
template <bool P>
__device__ State bf_chain_chunk(const char* rowp, int c, State st, float thr, const BfChainLds& L,
                                uint32_t base2, const float* gtab, const Ctx& ctx, int* hit,
                                int* rounds, uint32_t* amx)
{
    const int lane = threadIdx.x & 63;
    const int32_t beta = L.cb[c];
    float t[kFullPer];
    int pos = 0;
    *hit = -1;
    const int sl = beta <= -2 ? -2 - beta : -1;
    const BfStage* sg = sl >= 0 ? L.st + sl : nullptr;
    /* every LDS read of a staged chunk issued together: its binade, its
     * terms, and the lane scans of its b maps from the parity st enters with
     * and of its b + 1 maps from either parity */
    int32_t b = -1, cst = 0, xl = 0, xh0 = 0, xh1 = 0;
    if (sg) {
        b = sg->b;
        cst = sg->pad[1];
        xl = sg->xs[64 * (st.m & 1) + lane];
        xh0 = sg->xs[128 + lane];
        xh1 = sg->xs[192 + lane];
        const float4* src = reinterpret_cast<const float4*>(sg->t + lane * kFullPer);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 v = src[k];
            t[4 * k] = v.x;
            t[4 * k + 1] = v.y;
            t[4 * k + 2] = v.z;
            t[4 * k + 3] = v.w;
        }
    }
    if (sg && b >= 1) {
        if (st.e == b && (cst & 4) != 0) {
            ++*rounds;
            const int32_t mo = st.m + xl;
            const uint64_t bal = __ballot(mo >= ss::kTop || ss::value_of(State{b, mo}) >= thr);
            if (bal == 0) {
                st.m = __builtin_amdgcn_readlane(mo, 63);
                return st;
            }
            const int ls = (int)__builtin_ctzll(bal);
            /* lanes before ls stayed in b: their scan is exact */
            const int32_t xl0 = ls == 0 ? 0 : __builtin_amdgcn_readlane(xl, ls - 1);
            const int32_t mi = st.m + xl0;
            float sum = ss::value_of(State{b, mi < ss::kTop ? mi : 0});
            int below = 0;
#pragma unroll
            for (int j = 0; j < kFullPer; ++j) {
                sum = sum + t[j];
                below += sum < thr ? 1 : 0;
            }
            sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sum), ls));
            below = __builtin_amdgcn_readlane(below, ls);
            st = ss::state_of(sum);
            if (sum >= thr) {
                *hit = ls * kFullPer + below;
                return st;
            }
            pos = ls + 1;
            if (st.e == b + 1) {
                /* lanes after ls from st: a difference of the b + 1 scans from
                 * a start whose parity after lane ls is st's (any start when
                 * the maps are constant) */
                const int32_t r0 = __builtin_amdgcn_readlane(xh0, ls);
                const int32_t r1 = __builtin_amdgcn_readlane(xh1, ls);
                const int32_t pp = st.m & 1;
                const bool use0 = (cst & 2) != 0 || (r0 < ss::kTop && (r0 & 1) == pp);
                const bool use1 = !use0 && r1 < ss::kTop && ((1 + r1) & 1) == pp;
                if (use0 || use1) {
                    const int32_t m2 = st.m + (use0 ? xh0 - r0 : xh1 - r1);
                    const uint64_t bad = __ballot(
                        lane >= pos && (m2 >= ss::kTop || ss::value_of(State{b + 1, m2}) >= thr));
                    if (bad == 0) {
                        st.m = __builtin_amdgcn_readlane(m2, 63);
                        return st;
                    }
                }
            }
        } else if (st.e == b) {
            ++*rounds;
            if (round_step(sg->lo[lane], t, st, thr, pos, hit) || *hit >= 0) return st;
        }
        if (pos < 64 && st.e == b + 1) {
            ++*rounds;
            const PMap f = lane >= pos ? sg->hi[lane] : ss::map_identity();
            if (round_step(f, t, st, thr, pos, hit) || *hit >= 0) return st;
        }
    } else {
        bf_terms_global<P>(rowp, c, base2, gtab, ctx, t);
        if (!P) {
            uint32_t f1 = 0xFFFFFFFFu;
#pragma unroll
            for (int j = 0; j < kFullPer; ++j)
                f1 = t[j] == 1.0f ? g4s_min_u(f1, (uint32_t)(c * kFullChunk + lane * kFullPer + j)) : f1;
            *amx = g4s_min_u(*amx, wave_min_u32(f1));
        }
    }
    if (pos < 64) st = resolve_wave(t, kFullPer, st, thr, pos, hit, rounds);
    return st;
}

/* The walk of a chain (wave 0) from the exact state st entering chunk c0:
 * each run of chunks between two stops applies at once (its increments are
 * a prefix-sum difference) when the sum enters it in the run's predicted
 * binade and stays there (and below thr); otherwise the run is walked
 * chunk map by chunk map.  Each stop is resolved by bf_chain_chunk.  The
 * stops and their runs' end values are read ahead, 64 at a time, one per
 * lane, so that the walk's decisions take them from registers.  Without
 * THR, cpost[c] gets the exact sum after every chunk.  Returns the absolute
 * index of the first term reaching thr (-1: none); st becomes the final
 * state. */
__device__ __forceinline__ uint64_t rl64(uint64_t v, int l)
{
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((uint64_t)hi << 32) | lo;
}

template <bool THR>
__device__ int64_t bf_walk(const char* rowp, int c0, int nch, State& st, float thr,
                           const BfChainLds& L, uint32_t base2, const float* gtab, const Ctx& ctx,
                           int* rounds, uint32_t* amx)
{
    const int lane = threadIdx.x & 63;
    const int nstop = *L.nstop;
    int cur = c0;
    for (int j0 = 0; j0 <= nstop && cur < nch; j0 += 64) {
        /* lane q: stop j0 + q and the run before it, which starts after the
         * previous stop (c0 for the first), read ahead in one batch */
        const int jq = j0 + lane;
        const int sq = jq <= nstop ? L.stops[jq] : nch; /* stops[nstop] == nch */
        const int rq = jq == 0 ? c0 : (jq <= nstop ? L.stops[jq - 1] + 1 : nch);
        const bool runq = rq < sq;
        const int32_t bq = runq ? L.cb[rq] : -1;
        const int32_t eq = runq ? L.cb[sq - 1] : -1;
        const uint64_t p0q = (runq && rq > 0) ? L.pre[rq - 1] : 0ull;
        const uint64_t peq = runq ? L.pre[sq - 1] : 0ull;
        const int jn = nstop + 1 - j0 < 64 ? nstop + 1 - j0 : 64;
        for (int q = 0; q < jn && cur < nch; ++q) {
            const int s = __builtin_amdgcn_readlane(sq, q);
            if (s < cur) continue;
            if (s > cur) {
                /* the run cur .. s-1 */
                int32_t b, be;
                uint64_t p0, pe;
                if (cur == __builtin_amdgcn_readlane(rq, q)) {
                    b = __builtin_amdgcn_readlane(bq, q);
                    be = __builtin_amdgcn_readlane(eq, q);
                    p0 = rl64(p0q, q);
                    pe = rl64(peq, q);
                } else {
                    b = L.cb[cur];
                    be = L.cb[s - 1];
                    p0 = cur > 0 ? L.pre[cur - 1] : 0ull;
                    pe = L.pre[s - 1];
                }
                const uint64_t inc = pe - p0; /* >= kNonConst: a map with a tie */
                const int32_t mend = st.m + (int32_t)(inc < (uint64_t)ss::kTop ? inc : (uint64_t)ss::kTop);
                bool ok = b == st.e && be == b && mend < ss::kTop;
                if (THR) ok = ok && ss::value_of(State{b, mend}) < thr;
                if (ok) {
                    if (!THR) /* constant maps: the sum after each chunk of the run */
                        for (int c = cur + lane; c < s; c += 64)
                            L.cpost[c] = ss::value_of(State{b, st.m + (int32_t)(L.pre[c] - p0)});
                    st.m = mend;
                    cur = s;
                } else {
                    /* chunk map by chunk map; a chunk whose map does not apply is
                     * resolved on its own */
                    while (cur < s) {
                        const int cc = walk_maps<THR>(L.cm, L.cb, cur, s, st, thr, THR ? nullptr : L.cpost);
                        if (cc >= s) {
                            cur = s;
                            break;
                        }
                        int h;
                        st = bf_chain_chunk<THR>(rowp, cc, st, thr, L, base2, gtab, ctx, &h, rounds, amx);
                        if (h >= 0) return (int64_t)cc * kFullChunk + h;
                        if (!THR && lane == 0) L.cpost[cc] = ss::value_of(st);
                        cur = cc + 1;
                    }
                }
            }
            if (s >= nch || cur != s) continue;
            int h;
            st = bf_chain_chunk<THR>(rowp, s, st, thr, L, base2, gtab, ctx, &h, rounds, amx);
            if (h >= 0) return (int64_t)s * kFullChunk + h;
            if (!THR && lane == 0) L.cpost[s] = ss::value_of(st);
            cur = s + 1;
        }
    }
    return -1;
}

/* One workgroup per row: LSum by chaining the chunk maps left to right from
 * the exact state after chunk 0 (Tensors.pas:657-663), 1/LSum
 * (Tensors.pas:668), the argmax, and the draw's predictions (the last chunk
 * it needs, the predicted binade of its running sum entering every chunk,
 * the chunks to stage). */
__global__ __launch_bounds__(kFullBlock) __attribute__((amdgpu_waves_per_eu(1, 2))) void fb_lsum_chain_kernel(FullArgs a)
{
    extern __shared__ __align__(16) char dsm[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int row = blockIdx.y;
    const RowIn ri = row_in(a, row);
    if (row_class(a, ri.p.top_k) != kRowFull) return;
    const int nch = a.nch;
    const int64_t rbase = (int64_t)row * a.ws.cstride;
    const FullRow r = a.ws.rows[row];
    const FbRow fr = a.ws.fbrow[row];
    const BfChainLds L = bf_chain_layout(dsm, nch);
    bf_chain_prologue(a.ws.lmap + rbase, a.ws.beta_l + rbase,
                      a.ws.stage + (int64_t)row * kBfStage, fr.nsl, nch, nch - 1, L);
    const float T = ri.p.temperature;
    const bool all = term_outputs(a, kRowFull);
    const bool nodraw = !(T > 0.0f);
    const float thr = nodraw ? __builtin_inff() : mul_u_p_cr32(ri.u, ri.p.top_p); /* :2726 */
    /* fl32(u*TopP) <= 0: the first term's running sum already reaches it */
    const bool direct = !nodraw && !(thr > 0.0f);
    const bool early = (nodraw || direct) && !all;
    if (tid >= 64) return; /* the rest is wave 0's */

    const Ctx c0 = make_ctx(a, r, kRowFull);
    const uint32_t base = (uint32_t)r.win_lo << 7;
    const char* rowp = row_ptr<1>(a, row);
    const float* gtab = a.ws.etab8 + (int64_t)row * kBfTab;
    State st = ss::state_of(fr.s0);
    if (lane == 0) L.cpost[0] = fr.s0;
    int rounds = 0;
    uint32_t amx = (uint32_t)fr.amx;
    (void)bf_walk<false>(rowp, 1, nch, st, __builtin_inff(), L, base | (base << 16), gtab, c0,
                         &rounds, &amx);
    const float lsum = ss::value_of(st);
    const float inv = div_cr32(1.0f, lsum);                        /* Tensors.pas:668 */
    const int32_t argmax = (int32_t)amx;
    if (early) {
        uint32_t f = G4S_FLAG_FULL_PATH;
        if (direct) f |= G4S_FLAG_DREW | G4S_FLAG_REACHED;
        write_row_outputs(a, row, direct ? 0 : argmax, argmax, lsum, a.vocab, f);
        return;
    }
    if (lane == 0) {
        a.ws.fbrow[row].p_ninf = fr.e_ninf * inv;
        a.ws.fbrow[row].p_pinf = fr.e_pinf * inv;
        a.ws.fbrow[row].p_tiny = fr.e_tiny * inv; /* NaN stays NaN */
    }
    wave_lds_sync(); /* the walk's LSum after every chunk, from every lane */
    /* the last chunk the draw needs (the first whose running sum, LSum
     * prefix times 1/LSum, surely reaches thr), the draw's predicted binades
     * and its staged chunks up to there (where the running sum is predicted
     * to change binade or reach thr); lane l: chunks l*cpt .. */
    const int cpt = (nch + 63) / 64;
    uint32_t last = (uint32_t)(nch - 1);
    for (int q = 0; q < cpt; ++q) {
        const int cb = lane * cpt + q;
        if (cb < nch && (double)L.cpost[cb] * (double)inv * (1.0 - kMargin) >= (double)thr)
            last = g4s_min_u(last, (uint32_t)cb);
    }
    last = wave_min_u32(last);
    const int clast = (all || direct || nodraw) ? nch - 1 : (int)last;
    const auto staged = [&](int cb, double& pre) {
        pre = (double)L.cpost[cb - 1] * (double)inv;
        const double post = (double)L.cpost[cb] * (double)inv;
        const double lo = pre * (1.0 - kMargin), hi = post * (1.0 + kMargin);
        return binade_of(lo) != binade_of(hi) || (lo < (double)thr && hi >= (double)thr);
    };
    int cnt = 0;
    for (int q = 0; q < cpt; ++q) {
        const int cb = lane * cpt + q;
        double pre;
        if (cb > 0 && cb <= clast && cb < nch && staged(cb, pre)) ++cnt;
    }
    const int incl = wave_inclusive_scan(cnt);
    const int nstaged = __builtin_amdgcn_readlane(incl, 63);
    int pos = incl - cnt;
    int32_t* bc = a.ws.beta_c + rbase;
    BfStage* sg = a.ws.stage + (int64_t)row * kBfStage;
    for (int q = 0; q < cpt; ++q) {
        const int cb = lane * cpt + q;
        if (cb >= nch) continue;
        int32_t beta = -1;
        if (cb > 0 && cb <= clast) {
            double pre;
            const bool stg = staged(cb, pre);
            beta = binade_of(pre);
            if (stg) {
                if (pos < kBfStage) {
                    beta = -2 - pos;
                    sg[pos].b = binade_of(pre * (1.0 - kMargin));
                    sg[pos].chunk = cb;
                    sg[pos].pad[0] = 0;
                }
                ++pos;
            }
        }
        bc[cb] = beta;
    }
    if (lane == 0) {
        /* the fields this chain decides (the record itself is not held in
         * registers through the walk) */
        FullRow* w = &a.ws.rows[row];
        w->lsum = lsum;
        w->inv = inv;
        w->thr = thr;
        w->argmax = argmax;
        w->c_last = clast;
        w->nodraw = nodraw ? 1 : (direct ? 2 : 0);
        w->l_rounds = rounds;
        a.ws.fbrow[row].nsc = nstaged < kBfStage ? nstaged : kBfStage;
    }
}

/* One workgroup per row: the first index whose left-to-right binary32
 * running sum of p reaches thr (Model.pas:2727-2735), else the argmax. */
__global__ __launch_bounds__(kFullBlock) __attribute__((amdgpu_waves_per_eu(1, 2))) void fb_cdf_chain_kernel(FullArgs a)
{
    extern __shared__ __align__(16) char dsm[];
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
    if (row_class(a, ri.p.top_k) != kRowFull) return;
    const FbRow fr = a.ws.fbrow[row];
    __syncthreads(); /* every thread has read the row's words before they are reset */
    if (tid == 0) fb_reset_row(a, row);
    const FullRow r = a.ws.rows[row];
    if (r.c_last < 0) return;
    const uint32_t fl = G4S_FLAG_FULL_PATH;
    if (r.nodraw == 1) {
        if (tid < 64) write_row_outputs(a, row, r.argmax, r.argmax, r.lsum, a.vocab, fl);
        return;
    }
    if (r.nodraw == 2) {
        if (tid < 64)
            write_row_outputs(a, row, 0, r.argmax, r.lsum, a.vocab,
                              fl | G4S_FLAG_DREW | G4S_FLAG_REACHED);
        return;
    }
    const int nch = a.nch;
    const int64_t rbase = (int64_t)row * a.ws.cstride;
    const BfChainLds L = bf_chain_layout(dsm, nch);
    bf_chain_prologue(a.ws.cmap + rbase, a.ws.beta_c + rbase,
                      a.ws.stage + (int64_t)row * kBfStage, fr.nsc, nch, r.c_last, L);
    if (tid >= 64) return;

    const float thr = r.thr;
    int64_t hit = fr.hit0;
    int rounds = 0;
    if (hit < 0) {
        const Ctx c = make_ctx(a, r, kRowFull);
        const uint32_t base = (uint32_t)r.win_lo << 7;
        const char* rowp = row_ptr<1>(a, row);
        const float* gtab = a.ws.ptab8 + (int64_t)row * kBfTab;
        State st = ss::state_of(fr.c0);
        uint32_t unused = 0u;
        hit = bf_walk<true>(rowp, 1, nch, st, thr, L, base | (base << 16), gtab, c, &rounds, &unused);
    }
    if (lane == 0) a.ws.rows[row].c_rounds = rounds;
    uint32_t flags = fl | G4S_FLAG_DREW;
    int32_t id = r.argmax;
    if (hit >= 0) {
        id = (int32_t)hit;
        flags |= G4S_FLAG_REACHED;
    }
    write_row_outputs(a, row, id, r.argmax, r.lsum, a.vocab, flags);
}

/* Chunks per wave of the streaming passes: 4 unless that leaves fewer than
 * 16384 waves, then fewer, down to 1, so that small batches spread. */
int bf_cpw(int nch, int batch)
{
    const int64_t chunks = (int64_t)nch * batch;
    int cpw = kBfMaxCpw;
    while (cpw > 1 && chunks / cpw < 16384) cpw >>= 1;
    return cpw;
}

}  // namespace

bool fb_supported(int32_t vocab)
{
    return vocab >= kFullChunk && vocab % kFullChunk == 0 && vocab / kFullChunk <= kBfMaxChunks;
}

hipError_t fb_init(FullWorkspace& ws, int32_t max_batch, float softcap, hipStream_t s)
{
    hipLaunchKernelGGL(fb_ytab_kernel, dim3(65536 / 256), dim3(256), 0, s, ws.ytab, softcap);
    FullArgs a{};
    a.ws = ws;
    a.batch = max_batch;
    hipLaunchKernelGGL(fb_reset_kernel, dim3((unsigned)((max_batch + 255) / 256)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t fb_launch(const FullArgs& a0, hipStream_t s)
{
    FullArgs a = a0;
    a.cpw = bf_cpw(a.nch, a.batch);
    size_t off[7];
    const size_t lds = bf_chain_lds(a.nch, off);
    /* the chains' dynamic LDS exceeds the default 64 KiB: raise the limit once
     * per process to what the largest supported vocabulary needs (handles on
     * several threads may make their first call together) */
    static std::once_flag raised;
    static hipError_t raise_err = hipSuccess;
    std::call_once(raised, [] {
        size_t o[7];
        const int most = (int)bf_chain_lds(kBfMaxChunks, o);
        hipError_t e = hipFuncSetAttribute((const void*)fb_lsum_chain_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, most);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)fb_cdf_chain_kernel,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, most);
        raise_err = e;
    });
    if (raise_err != hipSuccess) return raise_err;
    const unsigned B = (unsigned)a.batch;
    const dim3 gmax((unsigned)((a.nch + 4 * a.cpw - 1) / (4 * a.cpw)), B);
    const dim3 grow((unsigned)(kRowWG + 1), B);
    const int cpw2 = bf_maps_cpw(a.cpw);
    const dim3 gmaps((unsigned)((a.nch + kBfWaves * cpw2 - 1) / (kBfWaves * cpw2)), B);
    const dim3 gchain(1u, B);
    hipLaunchKernelGGL(fb_max_kernel, gmax, dim3(kFullBlock), 0, s, a);
    hipLaunchKernelGGL(fb_row_kernel, grow, dim3(kFullBlock), 0, s, a);
    hipLaunchKernelGGL((fb_maps_kernel<false, false>), gmaps, dim3(kBfBlock), 0, s, a);
    hipLaunchKernelGGL(fb_lsum_chain_kernel, gchain, dim3(kFullBlock), lds, s, a);
    if (a.out.probs && a.out.capacity >= a.vocab)
        hipLaunchKernelGGL((fb_maps_kernel<true, true>), gmaps, dim3(kBfBlock), 0, s, a);
    else
        hipLaunchKernelGGL((fb_maps_kernel<true, false>), gmaps, dim3(kBfBlock), 0, s, a);
    hipLaunchKernelGGL(fb_cdf_chain_kernel, gchain, dim3(kFullBlock), lds, s, a);
    return hipGetLastError();
}

}  // namespace g4s
