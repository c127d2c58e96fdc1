/*
 * g4s_device.h -- device-side building blocks shared by the sampler kernels
 * (gfx950, wave64).
 */
#ifndef G4S_DEVICE_H
#define G4S_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemma4_sampler.h"
#include "g4s_crmath.h"

namespace g4s {

constexpr int kMaxTopK = 1024;     /* largest TopK of the top-k path */
constexpr int kCandRow = 16384;    /* workspace candidate slots per row */
constexpr int kMaxSplits = 256;    /* vocabulary chunks per row */
constexpr int kMergeLds = 2048;    /* merge candidates kept in LDS */
constexpr int kRankMax = 512;      /* rank-by-count select up to this many keys */

/* Order-preserving uint32 image of a binary32 value.  -0 maps to +0 (the
 * reference compares Singles, where -0 = +0).  0 is reserved for "not a
 * candidate": values <= fl32(-1e30) never enter the reference's heap
 * (Model.pas:2636,2643). */
__device__ __forceinline__ uint32_t f2key(float f)
{
    uint32_t b = __float_as_uint(f);
    b = (b == 0x80000000u) ? 0u : b;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k)
{
    uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __uint_as_float(b);
}
__device__ __forceinline__ uint32_t cand_key(float f) { return (f > -1e30f) ? f2key(f) : 0u; }

/* Element access: dtype 0 = binary32, 1 = bf16 (bits << 16, Types.pas:417-424). */
template <int DT>
struct Elem;
template <>
struct Elem<0> {
    static constexpr int VW = 4; /* elements per 16-byte load */
    static constexpr int SIZE = 4;
};
template <>
struct Elem<1> {
    static constexpr int VW = 8;
    static constexpr int SIZE = 2;
};

template <int DT>
__device__ __forceinline__ float load_elem(const char* row, int64_t e)
{
    if constexpr (DT == 0) {
        return reinterpret_cast<const float*>(row)[e];
    } else {
        uint32_t b = reinterpret_cast<const uint16_t*>(row)[e];
        return __uint_as_float(b << 16);
    }
}

/* Load VW consecutive elements starting at e0 (a multiple of VW); elements at
 * or beyond `limit` are returned as -inf and flagged invalid by the caller. */
template <int DT>
__device__ __forceinline__ void load_vec(const char* row, int64_t e0, int64_t limit,
                                         float (&v)[Elem<DT>::VW])
{
    constexpr int VW = Elem<DT>::VW;
    if (e0 + VW <= limit) {
        uint4 q = *reinterpret_cast<const uint4*>(row + e0 * Elem<DT>::SIZE);
        if constexpr (DT == 0) {
            v[0] = __uint_as_float(q.x);
            v[1] = __uint_as_float(q.y);
            v[2] = __uint_as_float(q.z);
            v[3] = __uint_as_float(q.w);
        } else {
            uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = __uint_as_float(w[i] << 16);
                v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < VW; ++i)
            v[i] = (e0 + i < limit) ? load_elem<DT>(row, e0 + i) : -__builtin_inff();
    }
}

/* Load VW consecutive in-bounds elements starting at e0 (a multiple of VW):
 * one unconditional 16-byte load. */
template <int DT>
__device__ __forceinline__ void load_vec_full(const char* row, int64_t e0, float (&v)[Elem<DT>::VW])
{
    const uint4 q = *reinterpret_cast<const uint4*>(row + e0 * Elem<DT>::SIZE);
    if constexpr (DT == 0) {
        v[0] = __uint_as_float(q.x);
        v[1] = __uint_as_float(q.y);
        v[2] = __uint_as_float(q.z);
        v[3] = __uint_as_float(q.w);
    } else {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    }
}

/* Cross-workgroup exchange without cache maintenance.  Everything one
 * workgroup hands to another inside a launch is written with device-scope
 * coherent stores (st_dev: written through to the device's point of
 * coherence) and read with device-scope coherent loads (ld_dev), so no L2
 * writeback or invalidate is ever issued (those act on a whole XCD's L2 and
 * serialize when thousands of workgroups issue them). */
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint64_t* p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p)
{
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev(const uint64_t* p)
{
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Elect the last of `count` workgroups that share *ticket.  Each thread's
 * device-coherent stores have completed (s_waitcnt) before the barrier, so
 * they are visible to whichever workgroup takes the last ticket; that one
 * reads them with ld_dev and resets the ticket for the next launch.  `flag`
 * is an LDS word.  Returns true in the elected workgroup. */
__device__ __forceinline__ bool elect_last(uint32_t* ticket, uint32_t count, int* flag)
{
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev =
            __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = prev == count - 1u;
        if (last) st_dev(ticket, 0u);
        *flag = last;
    }
    __syncthreads();
    return *flag != 0;
}

/* Results a host reads as soon as a row's completion word is published (the
 * id and flags in pinned host memory): system-scope stores, written through
 * every cache. */
__device__ __forceinline__ void st_sys(int32_t* p, int32_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void st_sys(uint32_t* p, uint32_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

/* Publish a row's completion for a host that spins on `done` instead of
 * synchronizing the stream.  The host then reads only the row's id and flags,
 * which the calling wave wrote with st_sys: waiting for those stores to
 * complete (they are written through to the system's point of coherence)
 * orders them before the completion word, with no writeback of the L2 (a
 * system-scope release fence would write back the whole XCD's L2).  The
 * runtime uses `done` only for calls without device-memory outputs.  Called
 * by all lanes of the wave that wrote the row's results (lane 0 stores the
 * word). */
__device__ __forceinline__ void publish_done(uint32_t* done, int row, uint32_t seq)
{
    if (!done) return;
    /* the compiler may not move memory operations across the wait: the
     * signal fences are compiler-only barriers (no cache maintenance), the
     * wait itself is the hardware ordering */
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if ((threadIdx.x & 63) == 0)
        __hip_atomic_store(done + row, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

/* ------------------------------------------------------------ wave helpers */

/* Cross-lane steps on DPP (no LDS crossbar).  A wave64 inclusive scan is
 * row_shr 1,2,4,8 inside each 16-lane row, then row_bcast 15 and 31 across
 * rows; a lane without a source keeps the identity `id`. */
#define G4S_DPP_STEP(x, OP, id, T, ctrl, rmask) \
    x = OP(x, (T)__builtin_amdgcn_update_dpp((int)(id), (int)(x), ctrl, rmask, 0xf, false))
#define G4S_DPP_SCAN(x, OP, id, T)                 \
    do {                                           \
        G4S_DPP_STEP(x, OP, id, T, 0x111, 0xf);    \
        G4S_DPP_STEP(x, OP, id, T, 0x112, 0xf);    \
        G4S_DPP_STEP(x, OP, id, T, 0x114, 0xf);    \
        G4S_DPP_STEP(x, OP, id, T, 0x118, 0xf);    \
        G4S_DPP_STEP(x, OP, id, T, 0x142, 0xa);    \
        G4S_DPP_STEP(x, OP, id, T, 0x143, 0xc);    \
    } while (0)

__device__ __forceinline__ int g4s_add_i(int a, int b) { return a + b; }
__device__ __forceinline__ uint32_t g4s_max_u(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t g4s_min_u(uint32_t a, uint32_t b) { return a < b ? a : b; }

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

/* Inclusive prefix sum over the 64 lanes of a wave (all lanes active). */
__device__ __forceinline__ int wave_inclusive_scan(int v)
{
    G4S_DPP_SCAN(v, g4s_add_i, 0, int);
    return v;
}

/* Wave-uniform reductions (all lanes active): the last lane of the scan. */
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    G4S_DPP_SCAN(v, g4s_max_u, 0u, uint32_t);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v)
{
    G4S_DPP_SCAN(v, g4s_min_u, 0xFFFFFFFFu, uint32_t);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ int wave_sum_i32(int v)
{
    G4S_DPP_SCAN(v, g4s_add_i, 0, int);
    return __builtin_amdgcn_readlane(v, 63);
}

/* Lower bounds of the k1-th and k2-th largest (1 <= k <= 64; 0 for k
 * outside that range) of one uint32 per lane (all 64 lanes active), in one
 * MSB-first ballot search over the `bits` bits below the common prefix of
 * the wave's values.  Each result P is the largest value whose bits below
 * those are zero with #{lanes: v >= P} >= k, so at least k lanes hold a
 * value >= P (0 when no positive value qualifies); with bits >= 32 P is the
 * k-th largest itself.  Uniform. */
__device__ __forceinline__ void wave_kth_largest2(uint32_t v, int k1, int k2, int bits,
                                                  uint32_t& r1, uint32_t& r2)
{
    /* both results lie in [min v, max v]: their bits above the highest bit
     * in which min and max differ are the common prefix */
    const uint32_t hi = wave_max_u32(v), lo = wave_min_u32(v);
    const int top = hi == lo ? -1 : 31 - __builtin_clz(hi ^ lo);
    const uint32_t pre = top < 0 ? hi : (top >= 31 ? 0u : (hi & ~((2u << top) - 1u)));
    uint32_t p1 = pre, p2 = pre;
    const bool on1 = k1 >= 1 && k1 <= 64, on2 = k2 >= 1 && k2 <= 64;
    const int stop = top - bits < -1 ? -1 : top - bits;
    for (int bit = top; bit > stop; --bit) {
        const uint32_t c1 = p1 | (1u << bit), c2 = p2 | (1u << bit);
        const int n1 = __popcll(__ballot(v >= c1));
        const int n2 = __popcll(__ballot(v >= c2));
        if (n1 >= k1) p1 = c1;
        if (n2 >= k2) p2 = c2;
    }
    r1 = on1 ? p1 : 0u;
    r2 = on2 ? p2 : 0u;
}

/* k-th largest key (1 <= k <= the number of non-zero keys <= 64*NG) over NG
 * keys per lane of one wave,
 * zero keys ignored (all 64 lanes active), by an MSB-first ballot search;
 * *gt / *eq = how many keys are above / equal to it.  Uniform results. */
template <int NG>
__device__ __forceinline__ uint32_t wave_select_kth(const uint32_t (&v)[NG], int k, int* gt,
                                                    int* eq)
{
    /* with k <= the number of non-zero keys the result lies between the
     * smallest non-zero key and the largest key: search only the bits below
     * their common prefix */
    uint32_t vmax = 0u, vmin = 0xFFFFFFFFu;
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        vmax = v[q] > vmax ? v[q] : vmax;
        vmin = (v[q] != 0u && v[q] < vmin) ? v[q] : vmin;
    }
    vmax = wave_max_u32(vmax);
    vmin = wave_min_u32(vmin);
    const int top = vmax <= vmin ? -1 : 31 - __builtin_clz(vmax ^ vmin);
    uint32_t p = top < 0 ? vmax : (top >= 31 ? 0u : (vmax & ~((2u << top) - 1u)));
    for (int bit = top; bit >= 0; --bit) {
        const uint32_t c = p | (1u << bit);
        int n = 0;
#pragma unroll
        for (int q = 0; q < NG; ++q) n += __popcll(__ballot(v[q] >= c));
        if (n >= k) p = c;
    }
    int g = 0, e = 0;
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        g += __popcll(__ballot(v[q] > p));
        e += __popcll(__ballot(v[q] == p && v[q] != 0u));
    }
    *gt = g;
    *eq = e;
    return p;
}

/* A lower bound of the k-th largest non-zero key over NG keys per lane of
 * one wave (1 <= k <= the number of non-zero keys): the MSB-first ballot
 * search of wave_select_kth stopped after `bits` bits below the keys' common
 * prefix.  Every prefix of that search keeps #{keys >= p} >= k, so the
 * result is a valid bound, within 2^(top-bits) of the exact value. */
template <int NG>
__device__ __forceinline__ uint32_t wave_kth_bound(const uint32_t (&v)[NG], int k, int bits)
{
    uint32_t vmax = 0u, vmin = 0xFFFFFFFFu;
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        vmax = v[q] > vmax ? v[q] : vmax;
        vmin = (v[q] != 0u && v[q] < vmin) ? v[q] : vmin;
    }
    vmax = wave_max_u32(vmax);
    vmin = wave_min_u32(vmin);
    if (vmax <= vmin) return vmax;
    const int top = 31 - __builtin_clz(vmax ^ vmin);
    uint32_t p = top >= 31 ? 0u : (vmax & ~((2u << top) - 1u));
    const int stop = top - bits < -1 ? -1 : top - bits;
    for (int bit = top; bit > stop; --bit) {
        const uint32_t c = p | (1u << bit);
        int n = 0;
#pragma unroll
        for (int q = 0; q < NG; ++q) n += __popcll(__ballot(v[q] >= c));
        if (n >= k) p = c;
    }
    return p;
}

/* Block-wide exclusive prefix sum in thread order; `total` receives the sum.
 * s_wave holds BLOCK/64 ints.  Contains two barriers. */
template <int BLOCK>
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_wave, int& total)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int x = wave_inclusive_scan(v);
    if (lane == 63) s_wave[wid] = x;
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < BLOCK / 64; ++w) {
        const int t = s_wave[w];
        off += (w < wid) ? t : 0;
        tot += t;
    }
    total = tot;
    __syncthreads();
    return off + x - v;
}

template <int BLOCK>
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* s_wave)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wave_max_u32(v);
    if (lane == 0) s_wave[wid] = v;
    __syncthreads();
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < BLOCK / 64; ++w) r = s_wave[w] > r ? s_wave[w] : r;
    __syncthreads();
    return r;
}
template <int BLOCK>
__device__ __forceinline__ uint32_t block_min_u32(uint32_t v, uint32_t* s_wave)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wave_min_u32(v);
    if (lane == 0) s_wave[wid] = v;
    __syncthreads();
    uint32_t r = 0xFFFFFFFFu;
#pragma unroll
    for (int w = 0; w < BLOCK / 64; ++w) r = s_wave[w] < r ? s_wave[w] : r;
    __syncthreads();
    return r;
}
template <int BLOCK>
__device__ __forceinline__ int block_sum_i32(int v, int* s_wave)
{
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wave_sum_i32(v);
    if (lane == 0) s_wave[wid] = v;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int w = 0; w < BLOCK / 64; ++w) r += s_wave[w];
    __syncthreads();
    return r;
}

/* ------------------------------------------------------------- selection */

/* One MSD radix step: from the 256-bin histogram of the current digit, find
 * the digit d with count(> d) < k <= count(>= d).  Writes d, count(> d) and
 * count(== d) to s_misc[0..2].  Called by the whole block; the first wave
 * does the work. */
__device__ __forceinline__ void radix_digit_step(int k, const uint32_t* s_hist, int* s_misc)
{
    const int tid = threadIdx.x;
    if (tid < 64) {
        const int lane = tid;
        int c[4];
        int lsum = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            c[q] = (int)s_hist[255 - (lane * 4 + q)];
            lsum += c[q];
        }
        const int incl = wave_inclusive_scan(lsum);
        int run = incl - lsum;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            int d = 255 - (lane * 4 + q);
            if (run < k && k <= run + c[q]) {
                s_misc[0] = d;
                s_misc[1] = run;
                s_misc[2] = c[q];
            }
            run += c[q];
        }
    }
}

/* k-th largest (1 <= k <= number of selected entries) of key(i) over the
 * entries i in [0, n) with sel(i), by 8-bit MSD radix select with an LDS
 * histogram.  Returns the value; *gt = how many selected entries are larger,
 * *eq = how many equal it.  s_hist: 256 uint32; s_misc: >= 3 ints. */
template <int BLOCK, typename KeyF, typename SelF>
__device__ uint32_t block_radix_kth(int n, int k, KeyF key, SelF sel, uint32_t* s_hist, int* s_misc,
                                   int* gt, int* eq)
{
    const int tid = threadIdx.x;
    uint32_t prefix = 0, mask = 0;
    int above = 0, equal = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int b = tid; b < 256; b += BLOCK) s_hist[b] = 0;
        __syncthreads();
        for (int i = tid; i < n; i += BLOCK) {
            if (!sel(i)) continue;
            uint32_t v = key(i);
            if ((v & mask) == prefix) atomicAdd(&s_hist[(v >> shift) & 255u], 1u);
        }
        __syncthreads();
        radix_digit_step(k, s_hist, s_misc);
        __syncthreads();
        above += s_misc[1];
        equal = s_misc[2];
        k -= s_misc[1];
        prefix |= (uint32_t)s_misc[0] << shift;
        mask |= 255u << shift;
        __syncthreads();
    }
    *gt = above;
    *eq = equal;
    return prefix;
}

/* The same select over keys held in registers (ITEMS per thread, 0 = not
 * selected).  Register arrays are only indexed with constants. */
template <int BLOCK, int ITEMS>
__device__ uint32_t regs_radix_kth(const uint32_t (&keys)[ITEMS], int k, uint32_t* s_hist,
                                   int* s_misc, int* gt, int* eq)
{
    const int tid = threadIdx.x;
    uint32_t prefix = 0, mask = 0;
    int above = 0, equal = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int b = tid; b < 256; b += BLOCK) s_hist[b] = 0;
        __syncthreads();
#pragma unroll
        for (int q = 0; q < ITEMS; ++q) {
            uint32_t v = keys[q];
            if (v != 0u && (v & mask) == prefix) atomicAdd(&s_hist[(v >> shift) & 255u], 1u);
        }
        __syncthreads();
        radix_digit_step(k, s_hist, s_misc);
        __syncthreads();
        above += s_misc[1];
        equal = s_misc[2];
        k -= s_misc[1];
        prefix |= (uint32_t)s_misc[0] << shift;
        mask |= 255u << shift;
        __syncthreads();
    }
    *gt = above;
    *eq = equal;
    return prefix;
}

}  // namespace g4s

#endif
