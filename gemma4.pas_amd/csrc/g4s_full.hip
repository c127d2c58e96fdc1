/*
 * g4s_full.hip -- the full-vocabulary sampling path on gfx950
 * (rows with TopK <= 0 or TopK >= V).
 *
 * Replaces the TopK <= 0 branch of DoSample with CpuLogitSoftcap,
 * DoSampleTopP and CpuSoftmaxF32 (src/Gemma4.Model.pas:2756-2763,
 * 2691-2737; src/Gemma4.Layers.pas:300-316; src/Gemma4.Tensors.pas:638-673):
 *   y_i = RN32(tanh(x_i * fl32(1/cap)) * cap)      (when cap > 0)
 *   y_i = RN32(y_i * fl32(1/T))                      (when T > 0 and T <> 1)
 *   m = max y;  e_i = RN32(exp(y_i - m));  LSum = e_0 + e_1 + ... left to
 *   right in binary32;  p_i = RN32(e_i * fl32(1/LSum));  argmax = first
 *   index of the largest p;  if T > 0: the first i whose left-to-right
 *   binary32 running sum of p reaches fl32(u * TopP), else the argmax.
 *
 * Rows are cut into chunks of 4096 terms, 16 consecutive terms per thread
 * of a 256-thread workgroup.  Six launches:
 *   1 max:    raw-logit maximum (softcap and 1/T are monotone, so
 *             m = y(max x)) and approximate chunk sums of exp(y - m); the
 *             row's last workgroup (atomic ticket) turns their prefix into
 *             the predicted binade of LSum entering every chunk;
 *   2 table:  for bf16 logits, e for the 4096 codes of the 16 largest
 *             exponents of |x| (correctly rounded, once per row), so the
 *             streaming passes look e up instead of evaluating it;
 *   3 lsum:   each chunk's terms as one exact map of the running sum in its
 *             predicted binade (g4s_seqsum.h), plus binary64 chunk sums;
 *   4 chain:  one workgroup per row chains the maps left to right,
 *             verifying every step and re-evaluating any chunk whose map
 *             does not apply: LSum, 1/LSum, the argmax, and the predicted
 *             binades of the draw's running sum;
 *   5 cdf:    the same maps for p, up to the chunk where the running sum is
 *             predicted to reach fl32(u*TopP);
 *   6 draw:   one workgroup per row finds the exact first index and writes
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

constexpr int NWF = kFullBlock / 64; /* waves per workgroup */

__device__ __forceinline__ bool is_full_row(int K, int V) { return K <= 0 || K >= V; }

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

/* y = softcap(x) [* 1/T] exactly as the reference rounds it (Layers.pas:
 * 309-314, Model.pas:2703-2708). */
__device__ __forceinline__ float y_exact(float x, float cap, float inv_cap, int scale, float inv_t)
{
    float y = (cap > 0.0f) ? softcap_full_cr32(x, inv_cap, cap) : x;
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
        const float w = x * inv_cap;
        float t;
        if (__builtin_fabsf(w) < 0.5f) {
            const float w2 = w * w; /* odd Taylor series of tanh to w^9 */
            t = w * (1.0f + w2 * (-0.33333334f + w2 * (0.13333334f + w2 * (-0.053968254f +
                                                                        w2 * 0.021869488f))));
        } else {
            const float wc = w > 12.0f ? 12.0f : (w < -12.0f ? -12.0f : w);
            const float e2 = __builtin_amdgcn_exp2f(wc * 2.8853900817779268f); /* e^(2w) */
            t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e2 + 1.0f);
        }
        y = t * cap;
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

/* Index of a bf16 code in the row's table, or -1 outside the window. */
__device__ __forceinline__ int tab_index(uint32_t code, int win_lo)
{
    const int eb = (int)((code >> 7) & 0xFFu) - win_lo;
    if ((unsigned)eb >= 16u) return -1;
    return (int)(((code >> 15) << 11) | ((uint32_t)eb << 7) | (code & 0x7Fu));
}

struct Ctx {
    float cap, inv_cap, inv_t, m;
    int scale, win_lo;
};

/* e of one term evaluated from x (kept out of line: it is the rare case for
 * bf16 logits, whose codes are tabulated). */
__device__ __noinline__ float e_direct(float x, Ctx c)
{
    return exp_diff_cr32(y_exact(x, c.cap, c.inv_cap, c.scale, c.inv_t), c.m);
}

/* e of one term: the table when the code is in the window, else evaluated. */
template <int DT>
__device__ __forceinline__ float e_of(uint32_t raw, const Ctx& c, const float* tab)
{
    if constexpr (DT == 1) {
        if (c.win_lo >= 0) {
            const int ti = tab_index(raw, c.win_lo);
            if (ti >= 0) return tab[ti];
        }
    }
    return e_direct(x_of<DT>(raw), c);
}

/* ------------------------------------------------------ block helpers */

struct FullShared {
    float tab[kFullTab];
    PMap wmap[NWF];
    int32_t went[NWF];
    int32_t tcand[NWF];
    uint32_t ured[3 * NWF];
    float fred[NWF];
    double dred[NWF];
    int32_t misc[16];
    int flag_last;
    /* chain: per-chunk records of the row */
    PMap cmap[kFullMaxChunks];
    int32_t cbeta[kFullMaxChunks];
};

__device__ __forceinline__ uint32_t block_max_key(uint32_t v, FullShared& sh, int slot)
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

__device__ __forceinline__ uint32_t block_min_u(uint32_t v, FullShared& sh)
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

__device__ __forceinline__ float block_sum_f(float v, FullShared& sh)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if (lane == 0) sh.fred[wid] = v;
    __syncthreads();
    float r = 0.0f;
#pragma unroll
    for (int w = 0; w < NWF; ++w) r += sh.fred[w];
    __syncthreads();
    return r;
}

__device__ __forceinline__ double block_sum_d(double v, FullShared& sh)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if (lane == 0) sh.dred[wid] = v;
    __syncthreads();
    double r = 0.0;
#pragma unroll
    for (int w = 0; w < NWF; ++w) r += sh.dred[w];
    __syncthreads();
    return r;
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

/* The map of one thread's terms in binade e (terms before `from` skipped). */
__device__ __forceinline__ PMap thread_map(const float (&t)[kFullPer], int nvalid, int32_t e)
{
    int32_t csum = 0, ties = 0;
    int32_t ct[kFullPer];
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) {
        ct[j] = (j < nvalid) ? ss::term_ct(t[j], e) : 0;
        csum += ct[j] >> 1;
        ties |= ct[j];
    }
    PMap f;
    if ((ties & 1) == 0) {
        /* no half-ulp tie: the map does not depend on the parity */
        f.d0 = csum > (1 << 26) ? (1 << 26) : csum;
        f.d1 = f.d0;
        return f;
    }
    f = ss::map_identity();
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) f = ss::map_sat(ss::map_then(f, ss::map_of_ct(ct[j])));
    return f;
}

/* The whole workgroup's map of a chunk (thread maps scanned over the wave,
 * wave totals composed in order); valid in thread 0. */
__device__ __forceinline__ PMap block_chunk_map(PMap f, FullShared& sh)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const PMap incl = wave_scan_maps(f);
    if (lane == 63) sh.wmap[wid] = incl;
    __syncthreads();
    PMap r = ss::map_identity();
    if (threadIdx.x == 0)
        for (int w = 0; w < NWF; ++w) r = ss::map_sat(ss::map_then(r, sh.wmap[w]));
    __syncthreads();
    return r;
}

/*
 * Exact evaluation of one chunk's running sum from the exact entering state
 * `st`, by the whole workgroup (thread t holds terms t*16 .. t*16+15 of the
 * chunk; threads before `pos` are already accounted for).  Each round maps
 * every remaining thread's terms in the current binade, finds the first
 * thread whose exit leaves the binade (or reaches `thr`), and walks that
 * thread's terms from its exact entering sum: the map step while the sum
 * stays in its binade, one plain binary32 addition where it leaves it.
 * Returns the state after the chunk or, when `thr` is reached, the index
 * (chunk-relative) of the first term whose running sum reaches it in *hit.
 * Rounds are counted in sh.misc[12].
 */
__device__ State resolve_chunk(const float (&t)[kFullPer], int nvalid, State st, float thr,
                               int pos, int* hit, FullShared& sh)
{
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    *hit = -1;
    while (pos < kFullBlock) {
        const int32_t e = st.e;
        const PMap f = (tid >= pos) ? thread_map(t, nvalid, e) : ss::map_identity();
        const PMap incl = wave_scan_maps(f);
        const PMap excl = wave_shift_map(incl);
        if (lane == 63) sh.wmap[wid] = incl;
        __syncthreads();
        if (tid == 0) {
            ++sh.misc[12];
            int32_t m = st.m;
            for (int w = 0; w < NWF; ++w) {
                sh.went[w] = m;
                m = m >= ss::kTop ? m : ss::map_apply(sh.wmap[w], m);
            }
            sh.misc[8] = m;
        }
        __syncthreads();
        const int32_t mw = sh.went[wid];
        const int32_t m_in = mw >= ss::kTop ? ss::kTop : ss::map_apply(excl, mw);
        const int32_t m_out = m_in >= ss::kTop ? ss::kTop : ss::map_apply(f, m_in);
        const bool stop = tid >= pos && (m_out >= ss::kTop ||
                                         ss::value_of(State{e, m_out}) >= thr);
        const uint64_t bal = __ballot(stop);
        if (lane == 0) sh.tcand[wid] = bal ? wid * 64 + (int)__builtin_ctzll(bal) : INT_MAX;
        __syncthreads();
        int tstar = INT_MAX;
#pragma unroll
        for (int w = 0; w < NWF; ++w) tstar = sh.tcand[w] < tstar ? sh.tcand[w] : tstar;
        if (tstar == INT_MAX) {
            st.m = sh.misc[8];
            __syncthreads();
            return st;
        }
        if (tid == tstar) {
            /* m_in is exact: every earlier thread stayed in the binade */
            State s2{e, m_in};
            int h = -1;
#pragma unroll
            for (int j = 0; j < kFullPer; ++j) {
                if (j >= nvalid) break;
                const int32_t m2 =
                    ss::map_apply(ss::map_of_ct(ss::term_ct(t[j], s2.e)), s2.m);
                if (m2 < ss::kTop)
                    s2.m = m2;
                else
                    s2 = ss::step_add(s2, t[j]);
                if (ss::value_of(s2) >= thr) {
                    h = tstar * kFullPer + j;
                    break;
                }
            }
            sh.misc[9] = s2.e;
            sh.misc[10] = s2.m;
            sh.misc[11] = h;
        }
        __syncthreads();
        st.e = sh.misc[9];
        st.m = sh.misc[10];
        const int h = sh.misc[11];
        __syncthreads();
        if (h >= 0) {
            *hit = h;
            return st;
        }
        pos = tstar + 1;
    }
    return st;
}

/* The row's first kHead terms (threads 0 .. kHead/16 - 1 of chunk 0), where
 * the running sum changes binade every few terms, summed left to right in
 * binary32 by wave 0 (one readlane per term); the result and the first index
 * reaching `thr` go to sh.misc[9..11] for the whole workgroup. */
constexpr int kHead = 256;
__device__ void head_walk(const float (&t)[kFullPer], float thr, FullShared& sh)
{
    if (threadIdx.x >= 64) return;
    float s = 0.0f;
    int h = -1;
    for (int l = 0; l < kHead / kFullPer; ++l) {
#pragma unroll
        for (int j = 0; j < kFullPer; ++j) {
            s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t[j]), l));
            if (h < 0 && s >= thr) h = l * kFullPer + j;
        }
        if (h >= 0) break;
    }
    if (threadIdx.x == 0) {
        const State st = ss::state_of(s);
        sh.misc[9] = st.e;
        sh.misc[10] = st.m;
        sh.misc[11] = h;
    }
}

__device__ __forceinline__ bool last_of_row(uint32_t* ticket, uint32_t count, FullShared& sh)
{
    return elect_last(ticket, count, &sh.flag_last);
}

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

/* Final outputs of a row (called by wave 0 of the row's last workgroup). */
__device__ void write_row_outputs(const FullArgs& a, int row, int32_t id, int32_t argmax, float lsum,
                                  uint32_t flags)
{
    if ((threadIdx.x & 63) == 0) {
        a.ids[row] = id;
        if (a.out.count) a.out.count[row] = a.vocab;
        if (a.out.argmax) a.out.argmax[row] = argmax;
        if (a.out.lsum) a.out.lsum[row] = lsum;
        if (a.out.flags) a.out.flags[row] = flags;
    }
    publish_done(a.done, row, a.seq);
}

}  // namespace

/* ------------------------------------------------------------ 1: max */

template <int DT>
__global__ __launch_bounds__(kFullBlock) void full_max_kernel(FullArgs a)
{
    __shared__ FullShared sh;
    const int tid = threadIdx.x;
    const int row = blockIdx.y, b = blockIdx.x;
    const int V = a.vocab;
    const RowIn ri = row_in(a, row);
    if (!is_full_row(ri.p.top_k, V)) return;
    const char* rowp = reinterpret_cast<const char*>(a.logits) +
                       (int64_t)row * a.row_stride * Elem<DT>::SIZE;
    const float cap = a.softcap;
    const float inv_cap = cap > 0.0f ? div_cr32(1.0f, cap) : 1.0f;      /* Layers.pas:309 */
    const float T = ri.p.temperature;
    const int scale = (T > 0.0f) && (T != 1.0f);                       /* Model.pas:2703 */
    const float inv_t = scale ? div_cr32(1.0f, T) : 1.0f;              /* Model.pas:2705 */

    uint32_t raw[kFullPer];
    const int nvalid = load16<DT>(rowp, (int64_t)b * kFullChunk + (int64_t)tid * kFullPer, V, raw);
    uint32_t kmax = 0u, amax = 0u, ymk = 0u;
    float ya[kFullPer];
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) {
        const float xj = x_of<DT>(raw[j]);
        ya[j] = y_approx(xj, cap, inv_cap, scale, inv_t);
        if (j < nvalid) {
            kmax = g4s_max_u(kmax, f2key(xj));
            amax = g4s_max_u(amax, __float_as_uint(xj) & 0x7FFFFFFFu);
            ymk = g4s_max_u(ymk, f2key(ya[j]));
        }
    }
    /* the three maxima in one LDS exchange */
    {
        const int lane = tid & 63, wid = tid >> 6;
        kmax = wave_max_u32(kmax);
        amax = wave_max_u32(amax);
        ymk = wave_max_u32(ymk);
        if (lane == 0) {
            sh.ured[wid] = kmax;
            sh.ured[NWF + wid] = amax;
            sh.ured[2 * NWF + wid] = ymk;
        }
        __syncthreads();
#pragma unroll
        for (int w = 0; w < NWF; ++w) {
            kmax = g4s_max_u(kmax, sh.ured[w]);
            amax = g4s_max_u(amax, sh.ured[NWF + w]);
            ymk = g4s_max_u(ymk, sh.ured[2 * NWF + w]);
        }
    }
    const float ymax = key2f(ymk);
    const float lg2e_ymax = ymax * 1.4426950408889634f;
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kFullPer; ++j)
        if (j < nvalid) s += __builtin_amdgcn_exp2f(ya[j] * 1.4426950408889634f - lg2e_ymax);
    s = wave_sum_f32(s);
    if ((tid & 63) == 0) sh.fred[tid >> 6] = s;
    __syncthreads();
    s = 0.0f;
#pragma unroll
    for (int w = 0; w < NWF; ++w) s += sh.fred[w];
    FullChunk* rc = a.ws.chunks + (int64_t)row * kFullMaxChunks;
    if (tid == 0) {
        uint64_t* w = reinterpret_cast<uint64_t*>(&rc[b]);
        st_dev(w, ((uint64_t)amax << 32) | kmax);
        st_dev(w + 1, ((uint64_t)__float_as_uint(s) << 32) | __float_as_uint(ymax));
    }
    if (!last_of_row(a.ws.tickets + (int64_t)row * 4 + 0, (uint32_t)a.nch, sh)) return;

    /* the row's maximum, m = y(max x), and the predicted binade of LSum
     * entering every chunk */
    const int nch = a.nch;
    uint32_t km = 0u, am = 0u;
    for (int c = tid; c < nch; c += kFullBlock) {
        const uint64_t w = ld_dev(reinterpret_cast<const uint64_t*>(&rc[c]));
        km = g4s_max_u(km, (uint32_t)w);
        am = g4s_max_u(am, (uint32_t)(w >> 32));
    }
    km = block_max_key(km, sh, 0);
    am = block_max_key(am, sh, 1);
    const float xmax = key2f(km);
    const float m = y_exact(xmax, cap, inv_cap, scale, inv_t);        /* Tensors.pas:648-654 */
    if (tid == 0) {
        double pre = 0.0;
        for (int c = 0; c < nch; ++c) {
            rc[c].beta_l = ss::state_of((float)pre).e;
            /* a prediction only: chunks without a finite estimate add 0 */
            const uint64_t w = ld_dev(reinterpret_cast<const uint64_t*>(&rc[c]) + 1);
            double z = (double)__uint_as_float((uint32_t)w) - (double)m;
            z = z > 50.0 ? 50.0 : (z < -700.0 ? -700.0 : z);
            const double d = (double)__uint_as_float((uint32_t)(w >> 32)) * exp_fast_d(z);
            pre += (d >= 0.0 && d < 1e300) ? d : 0.0;
        }
        FullRow r;
        r.maxkey = km;
        r.amax = am;
        r.m = m;
        r.inv_t = inv_t;
        r.scale = scale;
        /* table window: the 16 binades of |x| below and at the largest one */
        int win = -1;
        if (DT == 1) {
            const int eb = (int)((am >> 23) & 0xFFu); /* am: bits of the largest |x| */
            win = eb - 15 < 0 ? 0 : eb - 15;
        }
        r.win_lo = win;
        r.lsum = 0.0f;
        r.inv = 0.0f;
        r.thr = 0.0f;
        r.argmax = 0;
        r.c_last = -1;
        r.nodraw = 0;
        a.ws.rows[row] = r;
    }
}

/* ------------------------------------------------------------ 2: table */

__global__ __launch_bounds__(kFullBlock) void full_table_kernel(FullArgs a)
{
    const int row = blockIdx.y;
    const int i = blockIdx.x * kFullBlock + threadIdx.x;
    const RowIn ri = row_in(a, row);
    if (!is_full_row(ri.p.top_k, a.vocab) || i >= kFullTab) return;
    const FullRow r = a.ws.rows[row];
    if (r.win_lo < 0) return;
    const float cap = a.softcap;
    const float inv_cap = cap > 0.0f ? div_cr32(1.0f, cap) : 1.0f;
    const uint32_t eb = (uint32_t)r.win_lo + (((uint32_t)i >> 7) & 15u);
    const uint32_t code = (((uint32_t)i >> 11) << 15) | (eb << 7) | ((uint32_t)i & 0x7Fu);
    const float x = __uint_as_float(code << 16);
    a.ws.etab[(int64_t)row * kFullTab + i] =
        exp_diff_cr32(y_exact(x, cap, inv_cap, r.scale, r.inv_t), r.m);
}

/* Load the row's table and context into LDS / registers. */
template <int DT>
__device__ __forceinline__ Ctx load_ctx(const FullArgs& a, int row, const FullRow& r,
                                        FullShared& sh)
{
    Ctx c;
    c.cap = a.softcap;
    c.inv_cap = c.cap > 0.0f ? div_cr32(1.0f, c.cap) : 1.0f;
    c.inv_t = r.inv_t;
    c.m = r.m;
    c.scale = r.scale;
    c.win_lo = r.win_lo;
    if (DT == 1 && r.win_lo >= 0) {
        const float4* src = reinterpret_cast<const float4*>(a.ws.etab + (int64_t)row * kFullTab);
        float4 v[kFullTab / 4 / kFullBlock];
#pragma unroll
        for (int q = 0; q < kFullTab / 4 / kFullBlock; ++q) v[q] = src[threadIdx.x + q * kFullBlock];
#pragma unroll
        for (int q = 0; q < kFullTab / 4 / kFullBlock; ++q)
            reinterpret_cast<float4*>(sh.tab)[threadIdx.x + q * kFullBlock] = v[q];
    }
    __syncthreads();
    return c;
}

/* ------------------------------------------------- 3: lsum chunk maps */

template <int DT>
__global__ __launch_bounds__(kFullBlock) void full_lsum_kernel(FullArgs a)
{
    __shared__ FullShared sh;
    const int tid = threadIdx.x;
    const int row = blockIdx.y, b = blockIdx.x;
    const int V = a.vocab;
    const RowIn ri = row_in(a, row);
    if (!is_full_row(ri.p.top_k, V)) return;
    const char* rowp = reinterpret_cast<const char*>(a.logits) +
                       (int64_t)row * a.row_stride * Elem<DT>::SIZE;
    FullChunk* rc = a.ws.chunks + (int64_t)row * kFullMaxChunks;
    const FullRow r = a.ws.rows[row];
    const Ctx c = load_ctx<DT>(a, row, r, sh);

    uint32_t raw[kFullPer];
    const int64_t e0 = (int64_t)b * kFullChunk + (int64_t)tid * kFullPer;
    const int nvalid = load16<DT>(rowp, e0, V, raw);
    float t[kFullPer];
    double dsum = 0.0;
    uint32_t first1 = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < kFullPer; ++j) {
        t[j] = (j < nvalid) ? e_of<DT>(raw[j], c, sh.tab) : 0.0f;      /* Tensors.pas:660 */
        dsum += (double)t[j];
        if (j < nvalid && t[j] == 1.0f && first1 == 0xFFFFFFFFu) first1 = (uint32_t)(e0 + j);
    }
    const PMap cm = block_chunk_map(thread_map(t, nvalid, rc[b].beta_l), sh);
    dsum = block_sum_d(dsum, sh);
    first1 = block_min_u(first1, sh);
    if (tid == 0) {
        rc[b].lmap = cm;
        rc[b].de = dsum;
        rc[b].first1 = (int32_t)first1;
    }
}

/* ------------------------------------------------------- 4: LSum chain */

/* One workgroup per row: LSum by chaining the chunk maps left to right
 * (Tensors.pas:657-663), re-evaluating the chunks whose map does not apply;
 * then 1/LSum, the argmax, and the predictions for the draw. */
template <int DT>
__global__ __launch_bounds__(kFullBlock) void full_lsum_chain_kernel(FullArgs a)
{
    __shared__ FullShared sh;
    const int tid = threadIdx.x;
    const int row = blockIdx.y;
    const int V = a.vocab;
    const RowIn ri = row_in(a, row);
    if (!is_full_row(ri.p.top_k, V)) return;
    const char* rowp = reinterpret_cast<const char*>(a.logits) +
                       (int64_t)row * a.row_stride * Elem<DT>::SIZE;
    FullChunk* rc = a.ws.chunks + (int64_t)row * kFullMaxChunks;
    const FullRow r = a.ws.rows[row];
    const int nch = a.nch;
    for (int cb = tid; cb < nch; cb += kFullBlock) {
        sh.cmap[cb] = rc[cb].lmap;
        sh.cbeta[cb] = rc[cb].beta_l;
    }
    if (tid == 0) sh.misc[12] = 0;
    const Ctx c = load_ctx<DT>(a, row, r, sh); /* ends with a barrier */

    uint32_t raw[kFullPer];
    float t[kFullPer];
    State st = ss::state_of(0.0f);
    int reev = 0;
    for (int cb = 0; cb < nch; ++cb) {
        if (cb > 0 && st.e == sh.cbeta[cb]) {
            const int32_t m2 = ss::map_apply(sh.cmap[cb], st.m);
            if (m2 < ss::kTop) {
                st.m = m2;
                continue;
            }
        }
        ++reev;
        const int64_t f0 = (int64_t)cb * kFullChunk + (int64_t)tid * kFullPer;
        const int nv = load16<DT>(rowp, f0, V, raw);
#pragma unroll
        for (int j = 0; j < kFullPer; ++j) t[j] = (j < nv) ? e_of<DT>(raw[j], c, sh.tab) : 0.0f;
        int pos = 0;
        if (cb == 0) {
            head_walk(t, __builtin_inff(), sh);
            __syncthreads();
            st.e = sh.misc[9];
            st.m = sh.misc[10];
            __syncthreads();
            pos = kHead / kFullPer;
        }
        int h;
        st = resolve_chunk(t, nv, st, __builtin_inff(), pos, &h, sh);
    }
    const float lsum = ss::value_of(st);
    const float inv = div_cr32(1.0f, lsum);                            /* Tensors.pas:668 */
    /* argmax of p: p = fl32(e * inv) <= inv with equality exactly at e == 1
     * (the next float below 1 gives a p below inv), so the first e == 1 */
    uint32_t f1 = 0xFFFFFFFFu;
    for (int cb = tid; cb < nch; cb += kFullBlock) f1 = g4s_min_u(f1, (uint32_t)rc[cb].first1);
    f1 = block_min_u(f1, sh);
    const int32_t argmax = (int32_t)f1;                                 /* Model.pas:2712-2721 */
    const float T = ri.p.temperature;
    const bool all = a.out.probs && a.out.capacity >= V; /* every p is an output */
    const bool nodraw = !(T > 0.0f);
    if (nodraw && !all) {
        /* no draw: the greedy choice (Model.pas:2723) */
        if (tid < 64) write_row_outputs(a, row, argmax, argmax, lsum, G4S_FLAG_FULL_PATH);
        return;
    }
    const float thr = nodraw ? __builtin_inff() : mul_u_p_cr32(ri.u, ri.p.top_p); /* :2726 */
    if (tid == 0) {
        /* predicted binade of the running sum entering each chunk, and the
         * chunk where it is predicted to reach thr (with margin) */
        double pre = 0.0;
        int last = nch - 1;
        bool found = false;
        for (int cb = 0; cb < nch; ++cb) {
            rc[cb].beta_c = ss::state_of((float)(pre * (double)inv)).e;
            pre += rc[cb].de;
            if (!found && pre * (double)inv >= (double)thr * (1.0 + 0x1p-10)) {
                last = cb;
                found = true;
            }
        }
        FullRow w = r;
        w.lsum = lsum;
        w.inv = inv;
        w.thr = thr;
        w.argmax = argmax;
        w.c_last = all ? nch - 1 : last;
        w.nodraw = nodraw ? 1 : 0;
        w.l_reev = reev;
        w.l_rounds = sh.misc[12];
        w.c_reev = 0;
        w.c_rounds = 0;
        a.ws.rows[row] = w;
    }
}

/* -------------------------------------------------- 5: draw chunk maps */

template <int DT>
__global__ __launch_bounds__(kFullBlock) void full_cdf_kernel(FullArgs a)
{
    __shared__ FullShared sh;
    const int tid = threadIdx.x;
    const int row = blockIdx.y, b = blockIdx.x;
    const int V = a.vocab;
    const RowIn ri = row_in(a, row);
    if (!is_full_row(ri.p.top_k, V)) return;
    const FullRow r = a.ws.rows[row];
    if (r.c_last < 0 || b > r.c_last) return;
    const char* rowp = reinterpret_cast<const char*>(a.logits) +
                       (int64_t)row * a.row_stride * Elem<DT>::SIZE;
    FullChunk* rc = a.ws.chunks + (int64_t)row * kFullMaxChunks;
    const Ctx c = load_ctx<DT>(a, row, r, sh);
    const float inv = r.inv;

    uint32_t raw[kFullPer];
    const int64_t e0 = (int64_t)b * kFullChunk + (int64_t)tid * kFullPer;
    const int nvalid = load16<DT>(rowp, e0, V, raw);
    float t[kFullPer];
#pragma unroll
    for (int j = 0; j < kFullPer; ++j)
        t[j] = (j < nvalid) ? e_of<DT>(raw[j], c, sh.tab) * inv : 0.0f; /* Tensors.pas:671 */
    if (a.out.probs && a.out.capacity >= V) {
        float* po = a.out.probs + (int64_t)row * a.out.capacity;
        int32_t* io = a.out.indices ? a.out.indices + (int64_t)row * a.out.capacity : nullptr;
        for (int j = 0; j < nvalid; ++j) {
            po[e0 + j] = t[j];
            if (io) io[e0 + j] = (int32_t)(e0 + j);
        }
    }
    if (r.nodraw) return;
    const PMap cm = block_chunk_map(thread_map(t, nvalid, rc[b].beta_c), sh);
    if (tid == 0) rc[b].cmap = cm;
}

/* -------------------------------------------------------- 6: the draw */

/* One workgroup per row: the first index whose left-to-right binary32
 * running sum of p reaches thr (Model.pas:2727-2735), else the argmax. */
template <int DT>
__global__ __launch_bounds__(kFullBlock) void full_cdf_chain_kernel(FullArgs a)
{
    __shared__ FullShared sh;
    const int tid = threadIdx.x;
    const int row = blockIdx.y;
    const int V = a.vocab;
    const RowIn ri = row_in(a, row);
    if (!is_full_row(ri.p.top_k, V)) return;
    const FullRow r = a.ws.rows[row];
    if (r.c_last < 0) return;
    if (r.nodraw) {
        if (tid < 64) write_row_outputs(a, row, r.argmax, r.argmax, r.lsum, G4S_FLAG_FULL_PATH);
        return;
    }
    const char* rowp = reinterpret_cast<const char*>(a.logits) +
                       (int64_t)row * a.row_stride * Elem<DT>::SIZE;
    FullChunk* rc = a.ws.chunks + (int64_t)row * kFullMaxChunks;
    const int nch = a.nch;
    for (int cb = tid; cb < nch; cb += kFullBlock) {
        sh.cmap[cb] = cb <= r.c_last ? rc[cb].cmap : ss::map_identity();
        sh.cbeta[cb] = cb <= r.c_last ? rc[cb].beta_c : -1;
    }
    if (tid == 0) sh.misc[12] = 0;
    const Ctx c = load_ctx<DT>(a, row, r, sh); /* ends with a barrier */
    const float inv = r.inv;
    const float thr = r.thr;

    uint32_t raw[kFullPer];
    float t[kFullPer];
    State st = ss::state_of(0.0f);
    int64_t hit = -1;
    int reev = 0;
    for (int cb = 0; cb < nch; ++cb) {
        if (cb > 0 && st.e == sh.cbeta[cb]) {
            const int32_t m2 = ss::map_apply(sh.cmap[cb], st.m);
            if (m2 < ss::kTop && ss::value_of(State{st.e, m2}) < thr) {
                st.m = m2;
                continue;
            }
        }
        ++reev;
        const int64_t f0 = (int64_t)cb * kFullChunk + (int64_t)tid * kFullPer;
        const int nv = load16<DT>(rowp, f0, V, raw);
#pragma unroll
        for (int j = 0; j < kFullPer; ++j)
            t[j] = (j < nv) ? e_of<DT>(raw[j], c, sh.tab) * inv : 0.0f;
        int pos = 0;
        if (cb == 0) {
            head_walk(t, thr, sh);
            __syncthreads();
            st.e = sh.misc[9];
            st.m = sh.misc[10];
            const int hh = sh.misc[11];
            __syncthreads();
            if (hh >= 0) {
                hit = hh;
                break;
            }
            pos = kHead / kFullPer;
        }
        int h;
        st = resolve_chunk(t, nv, st, thr, pos, &h, sh);
        if (h >= 0) {
            hit = (int64_t)cb * kFullChunk + h;
            break;
        }
    }
    if (tid == 0) {
        a.ws.rows[row].c_reev = reev;
        a.ws.rows[row].c_rounds = sh.misc[12];
    }
    uint32_t flags = G4S_FLAG_FULL_PATH | G4S_FLAG_DREW;
    int32_t id = r.argmax;
    if (hit >= 0) {
        id = (int32_t)hit;
        flags |= G4S_FLAG_REACHED;
    }
    if (tid < 64) write_row_outputs(a, row, id, r.argmax, r.lsum, flags);
}

/* ---------------------------------------------------------------- host */

bool full_supported(int32_t vocab)
{
    return (vocab + kFullChunk - 1) / kFullChunk <= kFullMaxChunks;
}

hipError_t full_alloc(FullWorkspace& ws, int32_t vocab, int32_t max_batch)
{
    (void)vocab;
    const size_t mb = (size_t)max_batch;
    hipError_t e = hipMalloc((void**)&ws.rows, mb * sizeof(FullRow));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.chunks, mb * kFullMaxChunks * sizeof(FullChunk));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.etab, mb * kFullTab * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.tickets, mb * 4 * sizeof(uint32_t));
    return e;
}

void full_free(FullWorkspace& ws)
{
    if (ws.rows) (void)hipFree(ws.rows);
    if (ws.chunks) (void)hipFree(ws.chunks);
    if (ws.etab) (void)hipFree(ws.etab);
    if (ws.tickets) (void)hipFree(ws.tickets);
    ws = FullWorkspace{};
}

hipError_t full_init(FullWorkspace& ws, int32_t max_batch, hipStream_t s)
{
    return hipMemsetAsync(ws.tickets, 0, (size_t)max_batch * 4 * sizeof(uint32_t), s);
}

template <int DT>
static hipError_t launch_dt(const FullArgs& a, hipStream_t s)
{
    const dim3 grid((unsigned)a.nch, (unsigned)a.batch);
    hipLaunchKernelGGL((full_max_kernel<DT>), grid, dim3(kFullBlock), 0, s, a);
    if (DT == 1)
        hipLaunchKernelGGL(full_table_kernel, dim3(kFullTab / kFullBlock, (unsigned)a.batch),
                           dim3(kFullBlock), 0, s, a);
    const dim3 rows(1u, (unsigned)a.batch);
    hipLaunchKernelGGL((full_lsum_kernel<DT>), grid, dim3(kFullBlock), 0, s, a);
    hipLaunchKernelGGL((full_lsum_chain_kernel<DT>), rows, dim3(kFullBlock), 0, s, a);
    hipLaunchKernelGGL((full_cdf_kernel<DT>), grid, dim3(kFullBlock), 0, s, a);
    hipLaunchKernelGGL((full_cdf_chain_kernel<DT>), rows, dim3(kFullBlock), 0, s, a);
    return hipGetLastError();
}

hipError_t full_launch(const FullArgs& a, int dtype, hipStream_t s)
{
    return dtype == G4S_DTYPE_BF16 ? launch_dt<1>(a, s) : launch_dt<0>(a, s);
}

}  // namespace g4s
