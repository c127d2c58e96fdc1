/*
 * g4s_decode.hip -- the top-k path for decode-sized batches on gfx950
 * (rows with 0 < TopK <= 256, up to 8 rows per launch).
 *
 * Replaces DoSelectTopKIndices + the top-k branch of DoSample
 * (src/Gemma4.Model.pas:2615-2689, 2765-2826) where one token per sequence
 * is sampled per step and the launch's latency is the cost.  Grid = one
 * 256-thread workgroup per 16 bytes x 256 of a row's logits (256 workgroups
 * per binary32 row of 262144, 128 per bf16 row), x rows:
 *
 *  every workgroup
 *    - one 16-byte load per thread, keys sorted within the thread by
 *      (key descending, index ascending);
 *    - each wave's four largest elements in that order (four rounds of a
 *      wave maximum over the threads' heads; the lowest lane holding it has
 *      the lowest index, since a wave's lanes hold consecutive elements),
 *      written as the wave's list: wave w's lists are a prefix of its
 *      elements in the reference's preference order;
 *    - a two-level election: 16 first-level counters each count one group
 *      of workgroups, the last of a group counts on the row's counter, and
 *      the last there merges (one counter for all workgroups serializes
 *      every arrival on one address).
 *  merge (the elected workgroup of each row)
 *    - the row's lists in one round trip (32 KiB for 262144 binary32 logits);
 *    - L0 = a lower bound of the K-th largest list head (a histogram of the
 *      heads' first 8 bits below their common prefix): the heads are
 *      distinct elements, so the row's K-th largest key is >= L0;
 *    - candidates = list entries >= L0; tau' = their K-th largest key.  When
 *      no wave's fourth entry reaches tau', every element >= tau' of the row
 *      is a candidate, so tau' is the row's K-th largest key and the
 *      candidates decide every tie exactly as the whole row would: all
 *      copies of tau survive, or the lowest-index rule, or (when the heap's
 *      layout decides) a replay of the reference's heap over the row.  A
 *      wave whose fourth entry reaches tau' may hold more such elements:
 *      the merge re-reads up to 64 such waves (one wave each) and adds their
 *      other elements >= tau'; the K-th largest key can only rise, so the
 *      candidates are then complete (more such waves, or more candidates
 *      than LDS holds: the heap is replayed -- exact for every row, slow,
 *      reached only by rows with heavy ties);
 *    - survivors in index order, then one wave runs the reference's tail
 *      (up to four survivors per lane): softcap, 1/T, max, exp, sequential
 *      binary32 LSum, division, argmax, sequential running sum against
 *      fl32(u*TopP).
 * TopK = 1 needs no completeness: a wave's list starts with its lowest-index
 * copy of its maximum, so the row's first maximum is the first list head
 * with the largest key.
 */
#include "g4s_select.h"
#include "g4s_topk.h"

namespace g4s {

using namespace g4s::cr;

namespace {

constexpr int kDB = kDecBlock;
constexpr int kDW = kDB / 64;      /* waves per workgroup */
constexpr int kDL = kDecListLen;   /* entries per wave list */
constexpr int kDMcap = 1024;       /* merge candidates held in LDS; heap-replay tile */
constexpr int kDTile = kDB * 4;    /* heap-replay tile: four elements per thread */
constexpr int kDFast = 128;        /* fast-path candidates: one per thread of two waves */
constexpr int kDInc = 64;          /* waves whose elements the merge can re-read */
static_assert(kDMcap >= kDTile, "replay tiles fit the candidate area");

template <int KMAX>
struct DecShared {
    static_assert(KMAX % 32 == 0, "the tail reads eight float4 of values at a time");
    uint32_t hist[256];
    int misc[8]; /* [0..2] radix step, [3] candidate counter, [4..6] selects, [7] scratch */
    int scan[kDW];
    uint32_t red[4 * kDW];
    int flag;
    alignas(16) uint64_t mc[kDMcap + 64]; /* candidates (the last 64 absorb dropped lane
                                             writes); heap-replay tiles */
    alignas(16) uint32_t mk[kDMcap];      /* the candidates' keys */
    alignas(16) uint32_t mi[kDMcap];      /* the candidates' indices */
    alignas(16) uint32_t ix[kDMcap];      /* survivor indices for the index ranking (else ~0) */
    float vv[kDFast];         /* fast path: each candidate's v */
    float sv[KMAX];           /* the survivors' v in index order */
    uint64_t surv[KMAX];      /* heap storage during a replay */
    uint64_t sorted[KMAX];
    alignas(16) float val[KMAX];
    alignas(16) float prob[KMAX];
    int ninc;                 /* waves to re-read */
    uint32_t incw[kDInc];     /* their numbers */
    uint64_t inc4[kDInc];     /* their lists' last entries */
};

__device__ __forceinline__ uint32_t ent_key(uint64_t e) { return (uint32_t)(e >> 32); }
__device__ __forceinline__ uint32_t ent_idx(uint64_t e) { return (uint32_t)e; }

/* Four consecutive elements from e0 (a multiple of 4); elements at or beyond
 * `limit` are -inf (never screened into the heap: -inf <= -1e30). */
template <int DT>
__device__ __forceinline__ void load4(const char* row, int64_t e0, int64_t limit, float (&v)[4])
{
    if (e0 + 4 <= limit) {
        if constexpr (DT == 0) {
            const float4 q = *reinterpret_cast<const float4*>(row + e0 * 4);
            v[0] = q.x;
            v[1] = q.y;
            v[2] = q.z;
            v[3] = q.w;
        } else {
            const uint2 q = *reinterpret_cast<const uint2*>(row + e0 * 2);
            v[0] = __uint_as_float(q.x << 16);
            v[1] = __uint_as_float(q.x & 0xFFFF0000u);
            v[2] = __uint_as_float(q.y << 16);
            v[3] = __uint_as_float(q.y & 0xFFFF0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            v[i] = (e0 + i < limit) ? load_elem<DT>(row, e0 + i) : -__builtin_inff();
    }
}

/* The reference's min-heap pass (Model.pas:2632-2664) over the whole row:
 * tiles of 1024 elements screened against the current root (an element at
 * or below it would be rejected by every later root too), the screened ones
 * inserted in index order by one lane with the reference's comparisons; the
 * next tile is loaded while one is screened.  On return hv[0..K) / hi[0..K)
 * hold the heap (hi = -1 where the row had fewer than K logits above -1e30). */
template <int DT, typename SH>
__device__ void replay_heap(const char* row, int V, int K, SH& sh, float* hv, int32_t* hi)
{
    float* qv = reinterpret_cast<float*>(sh.mc);
    int32_t* qi = reinterpret_cast<int32_t*>(sh.mc) + kDTile;
    const int tid = threadIdx.x;
    for (int i = tid; i < K; i += kDB) {
        hv[i] = -1e30f; /* :2634-2638 */
        hi[i] = -1;
    }
    __syncthreads();
    float cur[4];
    load4<DT>(row, (int64_t)tid * 4, V, cur);
    for (int base = 0; base < V; base += kDTile) {
        float nxt[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (base + kDTile < V) load4<DT>(row, (int64_t)base + kDTile + (int64_t)tid * 4, V, nxt);
        const float root = hv[0];
        int take = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) take += !(cur[q] <= root) ? 1 : 0; /* :2643-2644 */
        if (__syncthreads_or(take)) {
            int total;
            int pos = block_exclusive_scan<kDB>(take, sh.scan, total);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (!(cur[q] <= root)) {
                    qv[pos] = cur[q];
                    qi[pos] = base + tid * 4 + q;
                    ++pos;
                }
            __syncthreads();
            if (tid == 0) {
                for (int q = 0; q < total; ++q) {
                    const float v = qv[q];
                    if (v <= hv[0]) continue; /* :2643-2644 */
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
                    hi[p] = qi[q];
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) cur[q] = nxt[q];
    }
}

/* Lanes 0..n-1 of wave 0: the index rank of entry i among the n entries of
 * ix[] (entries that are not survivors hold ~0 and rank last). */
__device__ __forceinline__ uint32_t rank_below(const uint32_t* ix, int n, uint32_t mine)
{
    uint32_t r = 0u;
    int j = 0;
    for (; j + 4 <= n; j += 4) {
        const uint4 w = *reinterpret_cast<const uint4*>(ix + j);
        r += (w.x < mine ? 1u : 0u) + (w.y < mine ? 1u : 0u) + (w.z < mine ? 1u : 0u) +
             (w.w < mine ? 1u : 0u);
    }
    for (; j < n; ++j) r += ix[j] < mine ? 1u : 0u;
    return r;
}

/* The K-th largest of the M candidate keys (K <= M; every key in [lo, hi]),
 * with the counts of keys above and equal to it.  Up to 512 keys: one wave
 * holds them in registers and searches the bits below the prefix that lo
 * and hi share, one ballot count per bit (the count of keys >= the trial
 * value decides each bit).  More keys: the block's radix select. */
template <typename SH>
__device__ uint32_t dec_kth(int M, int K, uint32_t lo, uint32_t hi, SH& sh, int* gt, int* eq)
{
    if (M > 512) return select_kth<kDB>(M, K, [&](int i) { return sh.mk[i]; }, sh, gt, eq);
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid < 64) {
        uint32_t k[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int i = q * 64 + lane;
            k[q] = i < M ? sh.mk[i] : 0u; /* 0: no key (every candidate key is >= 1) */
        }
        const uint32_t d = lo ^ hi;
        const int top = d ? 31 - __builtin_clz(d) : -1;
        uint32_t tau = top < 0 ? hi : (top >= 31 ? 0u : (hi & ~((2u << top) - 1u)));
        for (int b = top; b >= 0; --b) {
            const uint32_t t = tau | (1u << b);
            int c = 0;
#pragma unroll
            for (int q = 0; q < 8; ++q) c += __popcll(__ballot(k[q] >= t));
            if (c >= K) tau = t;
        }
        int g = 0, e = 0;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            g += __popcll(__ballot(k[q] > tau));
            e += __popcll(__ballot(k[q] == tau));
        }
        if (lane == 0) {
            sh.misc[4] = (int)tau;
            sh.misc[5] = g;
            sh.misc[6] = e;
        }
    }
    __syncthreads();
    const uint32_t r = (uint32_t)sh.misc[4];
    *gt = sh.misc[5];
    *eq = sh.misc[6];
    __syncthreads();
    return r;
}

}  // namespace

template <int DT, int KMAX>
__global__ __launch_bounds__(kDB) void topk_decode_kernel(TopkArgs a)
{
    constexpr int VW = Elem<DT>::VW;
    constexpr int CH = kDB * VW;
    constexpr int Q = KMAX / 64; /* survivors per lane of the tail */
    __shared__ DecShared<KMAX> sh;

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int row = blockIdx.y;
    const int chunk = blockIdx.x;
    const int S = gridDim.x;
    const int V = a.vocab;

    const g4s_params rp = a.params ? a.params[row] : a.p0;
    const double u = a.u ? a.u[row] : a.u0;
    const int K = rp.top_k;
    if (!(K >= 1 && K < V)) {
        /* full-vocabulary row (Model.pas:2756): the softmax launches take it,
         * or it is rejected here when none follows */
        if (!a.full_on && chunk == 0 && wid == 0) {
            if (lane == 0) {
                st_sys(&a.ids[row], -1);
                if (a.out.flags) st_sys(&a.out.flags[row], G4S_FLAG_ERROR | G4S_FLAG_FULL_PATH);
            }
            publish_done(a.done, row, a.seq);
        }
        return;
    }
    if (K > a.kbound) {
        if (a.wide_on && K > kMaxTopK) return; /* a wide row (g4s_full.hip) */
        if (chunk == 0 && wid == 0) {
            if (lane == 0) {
                st_sys(&a.ids[row], -1);
                if (a.out.flags) st_sys(&a.out.flags[row], G4S_FLAG_ERROR | G4S_FLAG_TOPK_PATH);
            }
            publish_done(a.done, row, a.seq);
        }
        return;
    }

    const char* rowp = reinterpret_cast<const char*>(a.logits) +
                       (int64_t)row * a.row_stride * Elem<DT>::SIZE;
    uint64_t* lists = a.cand + (int64_t)row * kCandRow;

    /* ------------------------------------------------------- phase 1 */
    {
        const int64_t e0 = (int64_t)chunk * CH + (int64_t)tid * VW;
        float v[VW];
        load_vec<DT>(rowp, e0, V, v);
        /* entries (key << 32 | ~index): larger = larger key, or the same key
         * at a lower index; 0 = no element (out of range or <= -1e30) */
        uint64_t o[VW];
#pragma unroll
        for (int q = 0; q < VW; ++q) {
            const uint32_t k = (e0 + q < V) ? cand_key(v[q]) : 0u;
            o[q] = k ? (((uint64_t)k << 32) | (uint32_t)~(uint32_t)(e0 + q)) : 0ull;
        }
        /* descending sorting network (0-1 principle checked for both sizes) */
#define G4S_CS(i, j)                                     \
    {                                                    \
        const uint64_t hi_ = o[i] > o[j] ? o[i] : o[j];  \
        const uint64_t lo_ = o[i] > o[j] ? o[j] : o[i];  \
        o[i] = hi_;                                      \
        o[j] = lo_;                                      \
    }
        if constexpr (VW == 4) {
            G4S_CS(0, 1) G4S_CS(2, 3) G4S_CS(0, 2) G4S_CS(1, 3) G4S_CS(1, 2)
        } else {
            G4S_CS(0, 2) G4S_CS(1, 3) G4S_CS(4, 6) G4S_CS(5, 7)
            G4S_CS(0, 4) G4S_CS(1, 5) G4S_CS(2, 6) G4S_CS(3, 7)
            G4S_CS(0, 1) G4S_CS(2, 3) G4S_CS(4, 5) G4S_CS(6, 7)
            G4S_CS(2, 4) G4S_CS(3, 5) G4S_CS(1, 4) G4S_CS(3, 6)
            G4S_CS(1, 2) G4S_CS(3, 4) G4S_CS(5, 6)
        }
#undef G4S_CS
        /* the wave's kDL largest: the largest head key, taken from the
         * lowest lane holding it (lanes hold consecutive elements, so that is
         * the lowest index with that key) */
        uint64_t mine = 0ull;
#pragma unroll
        for (int r = 0; r < kDL; ++r) {
            const uint32_t hk = (uint32_t)(o[0] >> 32);
            const uint32_t m = wave_max_u32(hk);
            if (m == 0u) break; /* wave-uniform */
            const int l = (int)__builtin_ctzll(__ballot(hk == m));
            const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)o[0], l);
            if (lane == r) mine = ((uint64_t)m << 32) | (uint32_t)~lo;
            if (lane == l) {
#pragma unroll
                for (int q = 0; q + 1 < VW; ++q) o[q] = o[q + 1];
                o[VW - 1] = 0ull;
            }
        }
        if (lane < kDL) st_dev(&lists[(int64_t)(chunk * kDW + wid) * kDL + lane], mine);
    }

    /* ------------------------------------------ two-level election */
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0); /* the lists are written through before the count */
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0) {
        const int gs = (S + kDecGroups - 1) / kDecGroups;
        const int g = chunk / gs, ng = (S + gs - 1) / gs;
        const int gn = (S - g * gs) < gs ? (S - g * gs) : gs;
        uint32_t* tk = a.dec_tickets + (int64_t)row * kDecTicketWords;
        uint32_t* c1 = tk + kDecCounterStride * (1 + g);
        int last = 0;
        if (__hip_atomic_fetch_add(c1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            (uint32_t)gn - 1u) {
            st_dev(c1, 0u);
            if (__hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                (uint32_t)ng - 1u) {
                st_dev(tk, 0u);
                last = 1;
            }
        }
        sh.flag = last;
    }
    __syncthreads();
    if (!sh.flag) return;

    /* ------------------------------------------------------------ merge */
    uint32_t flags = G4S_FLAG_TOPK_PATH;
    /* thread t: the lists of workgroup t (its four waves), one round trip of
     * device-coherent 16-byte loads */
    constexpr int kE = kDW * kDL;
    uint64_t e[kE];
    {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            lists, (short)0, S * kE * (int)sizeof(uint64_t), 0x00020000);
        typedef unsigned v4u __attribute__((ext_vector_type(4)));
        v4u q[kE / 2];
#pragma unroll
        for (int i = 0; i < kE / 2; ++i)
            q[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (tid * kE + 2 * i) * 8, 0,
                                                         16 /* sc1: device coherent */);
#pragma unroll
        for (int i = 0; i < kE / 2; ++i) {
            e[2 * i] = tid < S ? (((uint64_t)q[i].y << 32) | q[i].x) : 0ull;
            e[2 * i + 1] = tid < S ? (((uint64_t)q[i].w << 32) | q[i].z) : 0ull;
        }
    }
    /* heads (each wave's largest), the largest fourth entry, non-empty heads */
    uint32_t hmax = 0u, hmin = 0xFFFFFFFFu, w4 = 0u;
    int nz = 0;
#pragma unroll
    for (int w = 0; w < kDW; ++w) {
        const uint32_t hk = ent_key(e[w * kDL]);
        hmax = hk > hmax ? hk : hmax;
        hmin = (hk != 0u && hk < hmin) ? hk : hmin;
        nz += hk != 0u ? 1 : 0;
        const uint32_t k4 = ent_key(e[w * kDL + kDL - 1]);
        w4 = k4 > w4 ? k4 : w4;
    }
    hmax = wave_max_u32(hmax);
    hmin = wave_min_u32(hmin);
    w4 = wave_max_u32(w4);
    nz = wave_sum_i32(nz);
    if (lane == 0) {
        sh.red[wid] = hmax;
        sh.red[kDW + wid] = hmin;
        sh.red[2 * kDW + wid] = w4;
        sh.red[3 * kDW + wid] = (uint32_t)nz;
    }
    sh.hist[tid] = 0u; /* kDB == 256 bins */
    if (tid == 0) sh.misc[3] = 0;
    __syncthreads();
    hmax = 0u;
    hmin = 0xFFFFFFFFu;
    w4 = 0u;
    nz = 0;
#pragma unroll
    for (int w = 0; w < kDW; ++w) {
        hmax = g4s_max_u(hmax, sh.red[w]);
        hmin = g4s_min_u(hmin, sh.red[kDW + w]);
        w4 = g4s_max_u(w4, sh.red[2 * kDW + w]);
        nz += (int)sh.red[3 * kDW + w];
    }

    /* L0 <= the K-th largest head (K = 1: the largest): the 8 bits of the
     * heads below their common prefix */
    uint32_t L0 = 1u;
    int shift = 0, above = 0;
    uint32_t pre = 0u, dig = 0u;
    const bool radix = nz >= K && !(K == 1 || hmax == hmin);
    if (nz >= K) {
        if (!radix) {
            L0 = K == 1 ? hmax : hmin;
        } else {
            const int top = 31 - __builtin_clz(hmax ^ hmin);
            shift = top >= 7 ? top - 7 : 0;
            pre = top >= 31 ? 0u : (hmax & ~((2u << top) - 1u));
#pragma unroll
            for (int w = 0; w < kDW; ++w) {
                const uint32_t hk = ent_key(e[w * kDL]);
                if (hk != 0u) atomicAdd(&sh.hist[(hk >> shift) & 255u], 1u);
            }
            __syncthreads();
            radix_digit_step(K, sh.hist, sh.misc);
            __syncthreads();
            dig = (uint32_t)sh.misc[0];
            above = sh.misc[1];
            L0 = pre | (dig << shift);
        }
    }
    L0 = L0 < 1u ? 1u : L0;

    /* candidates: list entries >= L0 (each wave list's candidates are a
     * prefix of it; only candidates are written).  When they overflow LDS
     * and the bound kept low bits below the digit, a second digit of the
     * heads inside the first one raises it, and they are compacted again. */
    if (tid == 0) {
        sh.misc[4] = 0; /* tau of the fast path */
        sh.misc[5] = 0; /* copies of tau to split */
    }
    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1) {
            if (!(sh.misc[3] > kDMcap && radix && shift > 0)) break; /* uniform */
            const int shift2 = shift >= 8 ? shift - 8 : 0;
            const uint32_t hi_mask = ~((1u << shift) - 1u); /* the prefix and the first digit */
            const uint32_t lo_mask = (1u << (shift - shift2)) - 1u;
            __syncthreads();
            sh.hist[tid] = 0u;
            __syncthreads();
#pragma unroll
            for (int w = 0; w < kDW; ++w) {
                const uint32_t hk = ent_key(e[w * kDL]);
                if (hk != 0u && (hk & hi_mask) == (pre | (dig << shift)))
                    atomicAdd(&sh.hist[(hk >> shift2) & lo_mask], 1u);
            }
            __syncthreads();
            radix_digit_step(K - above, sh.hist, sh.misc);
            __syncthreads();
            L0 = pre | (dig << shift) | ((uint32_t)sh.misc[0] << shift2);
            if (tid == 0) sh.misc[3] = 0;
            __syncthreads();
        }
        /* in index order: thread t holds workgroup t's lists, wave by wave,
         * and a wave's elements precede the next wave's; inside one list an
         * entry's place is its index rank among the list's candidates */
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < kE; ++i) cnt += ent_key(e[i]) >= L0 ? 1 : 0;
        int total;
        int pos = block_exclusive_scan<kDB>(cnt, sh.scan, total);
#pragma unroll
        for (int w = 0; w < kDW; ++w) {
            int cw = 0;
#pragma unroll
            for (int l = 0; l < kDL; ++l) {
                const uint64_t x = e[w * kDL + l];
                if (ent_key(x) >= L0) {
                    int r = 0;
#pragma unroll
                    for (int l2 = 0; l2 < kDL; ++l2) {
                        const uint64_t y = e[w * kDL + l2];
                        r += (l2 != l && ent_key(y) >= L0 && ent_idx(y) < ent_idx(x)) ? 1 : 0;
                    }
                    if (pos + r < kDMcap) {
                        sh.mc[pos + r] = x;
                        sh.mk[pos + r] = ent_key(x);
                        sh.mi[pos + r] = ent_idx(x);
                    }
                    ++cw;
                }
            }
            pos += cw;
        }
        if (tid == 0) sh.misc[3] = total;
        __syncthreads();
    }
    int M = sh.misc[3];
    const float cap_v = a.softcap;
    const float T = rp.temperature;
    const bool scale = (T > 0.0f) && (T != 1.0f);
    const float inv_t = scale ? div_cr32(1.0f, T) : 1.0f;               /* :2782 */
    /* the survivors' softcapped, scaled values (v of the reference's tail),
     * computed here only on the fast path */
    auto scaled = [&](uint32_t key) {
        const float x = key2f(key);                                     /* :2774 */
        float v = (cap_v > 0.0f) ? softcap_topk_cr32(x, cap_v) : x;     /* :2775-2776 */
        if (scale) v = v * inv_t;                                       /* :2783-2784 */
        return v;
    };

    int nsurv = 0;
    bool have_v = false;
    if (K >= 2 && M >= K && M <= kDFast) {
        /* fast path: wave 0 finds the K-th largest key tau of the candidates
         * (a ballot search, two keys per lane) while waves 2-3 compute every
         * candidate's v.  With no copies of tau to split and no wave list
         * reaching tau, the K candidates >= tau are the survivors, already in
         * index order, and their v are ready. */
        if (wid == 0) {
            const uint32_t k0 = lane < M ? sh.mk[lane] : 0u;
            const uint32_t k1 = lane + 64 < M ? sh.mk[lane + 64] : 0u;
            /* every candidate key lies in [L0, hmax] */
            const uint32_t d = L0 ^ hmax;
            const int top = d ? 31 - __builtin_clz(d) : -1;
            uint32_t tau = top < 0 ? hmax : (top >= 31 ? 0u : (hmax & ~((2u << top) - 1u)));
            for (int b = top; b >= 0; --b) {
                const uint32_t t = tau | (1u << b);
                if (__popcll(__ballot(k0 >= t)) + __popcll(__ballot(k1 >= t)) >= K) tau = t;
            }
            const int G = __popcll(__ballot(k0 > tau)) + __popcll(__ballot(k1 > tau));
            const int E = __popcll(__ballot(k0 == tau)) + __popcll(__ballot(k1 == tau));
            if (lane == 0) {
                sh.misc[4] = (int)tau;
                sh.misc[5] = (E == K - G && w4 < tau) ? 0 : 1;
            }
        } else if (wid >= 2) {
            const int c = tid - 2 * 64;
            if (c < M) sh.vv[c] = scaled(sh.mk[c]);
        }
        __syncthreads();
        if (sh.misc[5] == 0) {
            if (wid != 0) return;
            const uint32_t tau = (uint32_t)sh.misc[4];
            const int q0 = lane, q1 = lane + 64;
            const bool s0 = q0 < M && sh.mk[q0] >= tau;
            const bool s1 = q1 < M && sh.mk[q1] >= tau;
            const uint64_t m0 = __ballot(s0), m1 = __ballot(s1);
            const uint64_t lt = (1ull << lane) - 1ull;
            if (s0) {
                const int at = __popcll(m0 & lt);
                sh.sorted[at] = cand_pack(sh.mk[q0], sh.mi[q0]);
                sh.sv[at] = sh.vv[q0];
            }
            if (s1) {
                const int at = __popcll(m0) + __popcll(m1 & lt);
                sh.sorted[at] = cand_pack(sh.mk[q1], sh.mi[q1]);
                sh.sv[at] = sh.vv[q1];
            }
            __builtin_amdgcn_wave_barrier();
            nsurv = K;
            have_v = true;
        }
    }

    if (!have_v) {
        /* general path: exact survivors by mode 0 (all candidates >= tau),
         * 1 (lowest-index ties) or 2 (heap replay) */
        int mode = 0;
        uint32_t tau = 1u;
        int32_t idx_thr = 0x7FFFFFFF;
        bool ordered = false;
        if (nz == 0) {
            nsurv = 0; /* no logit above -1e30 */
            ordered = true;
        } else if (K == 1) {
            /* the first (lowest-index) copy of the largest key (Model.pas:
             * 2643-2644 rejects later equal keys): a wave's list starts with
             * its lowest-index copy of its maximum, so it is the lowest-index
             * head with the largest key; a second copy anywhere is listed */
            uint32_t imin = 0xFFFFFFFFu;
            int copies = 0;
#pragma unroll
            for (int i = 0; i < kE; ++i) {
                const bool c = ent_key(e[i]) == hmax;
                if (c && (i % kDL) == 0) imin = g4s_min_u(imin, ent_idx(e[i]));
                copies += c ? 1 : 0;
            }
            imin = block_min_u32<kDB>(imin, sh.red);
            copies = block_sum_i32<kDB>(copies, sh.scan);
            if (copies > 1) flags |= G4S_FLAG_TIE_LOWEST;
            if (tid == 0) sh.sorted[0] = cand_pack(hmax, imin);
            nsurv = 1;
            ordered = true;
        } else if (M > kDMcap) {
            mode = 2; /* heavy ties beyond the candidate area */
        } else {
            int G = 0, E = 0;
            if (M >= K) tau = dec_kth(M, K, L0, hmax, sh, &G, &E);
            /* a wave whose list ends at or above tau (fewer than K candidates:
             * above -1e30) may hold more such elements: the merge re-reads
             * those waves and adds the rest of their elements >= tau, after
             * which every element >= the new tau (>= tau) is a candidate */
            const uint32_t thr = M >= K ? tau : 1u;
            if (w4 >= thr) { /* block-uniform */
                if (tid == 0) sh.ninc = 0;
                __syncthreads();
#pragma unroll
                for (int w = 0; w < kDW; ++w) {
                    const uint64_t e4 = e[w * kDL + kDL - 1];
                    if (ent_key(e4) >= thr) {
                        const int jn = atomicAdd(&sh.ninc, 1);
                        if (jn < kDInc) {
                            sh.incw[jn] = (uint32_t)(tid * kDW + w);
                            sh.inc4[jn] = e4;
                        }
                    }
                }
                __syncthreads();
                const int ninc = sh.ninc;
                if (ninc > kDInc) {
                    mode = 2;
                } else {
                    for (int i = wid; i < ninc; i += kDW) { /* one wave per listed wave */
                        const int gw = (int)sh.incw[i];
                        /* the list's last entry in the sorting order of phase 1
                         * (key, then ~index: larger = preferred) */
                        const uint64_t e4 = (sh.inc4[i] & 0xFFFFFFFF00000000ull) |
                                            (uint32_t)~(uint32_t)sh.inc4[i];
                        const int64_t b0 = (int64_t)(gw / kDW) * CH + (int64_t)((gw % kDW) * 64 + lane) * VW;
                        float v[VW];
                        load_vec<DT>(rowp, b0, V, v);
                        uint64_t o[VW];
                        int cnt = 0;
#pragma unroll
                        for (int q = 0; q < VW; ++q) {
                            const uint32_t k = (b0 + q < V) ? cand_key(v[q]) : 0u;
                            o[q] = k ? (((uint64_t)k << 32) | (uint32_t)~(uint32_t)(b0 + q)) : 0ull;
                            /* entries below the list's last are not in the list */
                            o[q] = (k >= thr && o[q] < e4) ? o[q] : 0ull;
                            cnt += o[q] ? 1 : 0;
                        }
                        const int incl = wave_inclusive_scan(cnt);
                        int base = 0;
                        if (lane == 63) base = atomicAdd(&sh.misc[3], incl);
                        base = __builtin_amdgcn_readlane(base, 63);
                        int pos = base + incl - cnt;
#pragma unroll
                        for (int q = 0; q < VW; ++q) {
                            if (o[q]) {
                                if (pos < kDMcap) {
                                    sh.mc[pos] = o[q] ^ 0xFFFFFFFFull; /* index back */
                                    sh.mk[pos] = ent_key(o[q]);
                                    sh.mi[pos] = ~(uint32_t)o[q];
                                }
                                ++pos;
                            }
                        }
                    }
                    __syncthreads();
                    M = sh.misc[3];
                    if (M > kDMcap)
                        mode = 2;
                    else if (M >= K)
                        tau = dec_kth(M, K, L0, hmax, sh, &G, &E);
                }
            }
            if (mode == 2) {
                /* the heap replay below */
            } else if (M < K) {
                nsurv = M; /* every logit above -1e30 survives */
            } else {
                const int need = K - G;
                nsurv = K;
                if (E != need) {
                    /* t* = index of the K-th element >= tau in index order */
                    int g2, e2;
                    const uint32_t tstar_inv = block_radix_kth<kDB>(
                        M, K, [&](int i) { return ~sh.mi[i]; },
                        [&](int i) { return sh.mk[i] >= tau; }, sh.hist, sh.misc + 4, &g2, &e2);
                    const int32_t tstar = (int32_t)~tstar_inv;
                    uint32_t mg = 0u;
                    for (int i = tid; i < M; i += kDB)
                        if (sh.mk[i] > tau) mg = g4s_max_u(mg, sh.mi[i] + 1u);
                    mg = block_max_u32<kDB>(mg, sh.red);
                    const int32_t max_gt = (int32_t)mg - 1; /* -1 when nothing is above tau */
                    if (max_gt < tstar) {
                        /* every key above tau precedes the K-th key >= tau: the
                         * heap keeps them and the first `need` copies of tau */
                        mode = 1;
                        const uint32_t thr_inv = block_radix_kth<kDB>(
                            M, need, [&](int i) { return ~sh.mi[i]; },
                            [&](int i) { return sh.mk[i] == tau; }, sh.hist, sh.misc + 4, &g2,
                            &e2);
                        idx_thr = (int32_t)~thr_inv;
                        flags |= G4S_FLAG_TIE_LOWEST;
                    } else {
                        mode = 2;
                    }
                }
            }
        }

        if (mode == 2) {
            flags |= G4S_FLAG_HEAP_REPLAY;
            float* hv = reinterpret_cast<float*>(sh.surv);
            int32_t* hi = reinterpret_cast<int32_t*>(sh.surv) + KMAX;
            replay_heap<DT>(rowp, V, K, sh, hv, hi);
            /* keep the entries holding an index (Model.pas:2668-2676), then
             * rank them by index (:2678-2688) */
            if (tid < K) sh.ix[tid] = hi[tid] >= 0 ? (uint32_t)hi[tid] : 0xFFFFFFFFu;
            __syncthreads();
            int valid = 0;
            if (tid < K && hi[tid] >= 0) {
                const uint32_t r = rank_below(sh.ix, K, (uint32_t)hi[tid]);
                sh.sorted[r] = cand_pack(f2key(hv[tid]), (uint32_t)hi[tid]);
                valid = 1;
            }
            nsurv = block_sum_i32<kDB>(valid, sh.scan);
            ordered = true;
        }
        if (!ordered) {
            /* survivors in index order: compacted (in any order), then each
             * ranks itself by index among them */
            auto surv_ok = [&](int i) {
                const uint32_t k = sh.mk[i];
                return mode == 0 ? (k >= tau)
                                 : (k > tau || (k == tau && (int32_t)sh.mi[i] <= idx_thr));
            };
            if (tid == 0) sh.misc[7] = 0;
            __syncthreads();
            for (int i0 = 0; i0 < M; i0 += kDB) { /* uniform */
                const int i = i0 + tid;
                const bool ok = i < M && surv_ok(i);
                const uint64_t m = __ballot(ok);
                int base = 0;
                if (lane == 0 && m) base = atomicAdd(&sh.misc[7], __popcll(m));
                base = __builtin_amdgcn_readfirstlane(base);
                if (ok) {
                    const int at = base + __popcll(m & ((1ull << lane) - 1ull));
                    sh.ix[at] = sh.mi[i];
                    sh.surv[at] = sh.mc[i];
                }
            }
            __syncthreads();
            const int ns = sh.misc[7]; /* == nsurv <= K */
            if (tid < 4) sh.ix[ns + tid] = 0xFFFFFFFFu; /* rank padding */
            __syncthreads();
            if (tid < ns) {
                const uint32_t mine = sh.ix[tid];
                uint32_t r0 = 0u, r1 = 0u;
                int j = 0;
                for (; j + 8 <= ns + 3; j += 8) {
                    const uint4 w0 = *reinterpret_cast<const uint4*>(sh.ix + j);
                    const uint4 w1 = *reinterpret_cast<const uint4*>(sh.ix + j + 4);
                    r0 += (w0.x < mine ? 1u : 0u) + (w0.y < mine ? 1u : 0u) +
                          (w0.z < mine ? 1u : 0u) + (w0.w < mine ? 1u : 0u);
                    r1 += (w1.x < mine ? 1u : 0u) + (w1.y < mine ? 1u : 0u) +
                          (w1.z < mine ? 1u : 0u) + (w1.w < mine ? 1u : 0u);
                }
                for (; j < ns; j += 4) {
                    const uint4 w0 = *reinterpret_cast<const uint4*>(sh.ix + j);
                    r0 += (w0.x < mine ? 1u : 0u) + (w0.y < mine ? 1u : 0u) +
                          (w0.z < mine ? 1u : 0u) + (w0.w < mine ? 1u : 0u);
                }
                sh.sorted[r0 + r1] = sh.surv[tid];
            }
        }
        __syncthreads();
        if (wid != 0) return;
    }

    /* ------------------------------------------------ tail (wave 0 only) */
    if (nsurv == 0) {
        if (lane == 0) {
            st_sys(&a.ids[row], -1);
            if (a.out.flags) st_sys(&a.out.flags[row], flags | G4S_FLAG_EMPTY);
            if (a.out.count) a.out.count[row] = 0;
        }
        publish_done(a.done, row, a.seq);
        return;
    }
    /* survivor j = q * 64 + lane of lane `lane` */
    bool act[Q];
    uint64_t my[Q];
    float vv[Q], ev[Q], p[Q];
    uint32_t vk = 0u;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int j = q * 64 + lane;
        act[q] = j < nsurv;
        my[q] = act[q] ? sh.sorted[j] : 0ull;
        /* one survivor: e = Exp(v - v) = 1 whatever v is */
        vv[q] = 0.0f;
        if (act[q] && nsurv > 1) vv[q] = have_v ? sh.sv[j] : scaled(ent_key(my[q]));
        vk = act[q] ? g4s_max_u(vk, f2key(vv[q])) : vk;
    }
    const float vmax = key2f(wave_max_u32(vk));                         /* :2789-2792 */
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        ev[q] = !act[q] ? 0.0f : (nsurv == 1 ? 1.0f : exp_diff_cr32(vv[q], vmax)); /* :2797 */
        sh.val[q * 64 + lane] = ev[q]; /* +0 beyond the survivors */
    }
    __builtin_amdgcn_wave_barrier();
    /* LSum := LSum + LVals[LI], left to right in binary32 (:2798), every lane
     * on the same broadcast LDS reads; +0 padding leaves the sum unchanged */
    const int n4 = (nsurv + 3) >> 2; /* uniform */
    float lsum = 0.0f;
    {
        /* eight float4 reads in flight, then their 32 additions in order */
        const float4* src = reinterpret_cast<const float4*>(sh.val);
        for (int b4 = 0; b4 < n4; b4 += 8) {
            float4 x[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) x[t] = src[b4 + t]; /* KMAX / 4 is a multiple of 8 */
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                lsum = lsum + x[t].x;
                lsum = lsum + x[t].y;
                lsum = lsum + x[t].z;
                lsum = lsum + x[t].w;
            }
        }
    }
    uint32_t pk = 0u;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        p[q] = act[q] ? div_cr32(ev[q], lsum) : 0.0f;                   /* :2800-2801 */
        sh.prob[q * 64 + lane] = p[q];
        pk = act[q] ? g4s_max_u(pk, __float_as_uint(p[q])) : pk;
    }
    /* greedy choice: the first position of the largest p (p >= 0, so its bits
     * order like the values) */
    const uint32_t pmax = wave_max_u32(pk);                              /* :2804-2807 */
    int jarg = 0;
#pragma unroll
    for (int q = Q - 1; q >= 0; --q) {
        const uint64_t m = __ballot(act[q] && __float_as_uint(p[q]) == pmax);
        if (m) jarg = q * 64 + (int)__builtin_ctzll(m);
    }
    __builtin_amdgcn_wave_barrier();
    int chosen = jarg;
    if (T > 0.0f) {                                                     /* :2811-2824 */
        flags |= G4S_FLAG_DREW;
        const float thr = mul_u_p_cr32(u, rp.top_p);
        /* LCum := LCum + LVals[LI] left to right; every running sum goes back
         * to LDS, then ballots find the first that reaches thr */
        float cum = 0.0f;
        const float4* src = reinterpret_cast<const float4*>(sh.prob);
        float4* dst = reinterpret_cast<float4*>(sh.val);
        for (int b4 = 0; b4 < n4; b4 += 8) {
            float4 x[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) x[t] = src[b4 + t];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                float4 c;
                cum = cum + x[t].x;
                c.x = cum;
                cum = cum + x[t].y;
                c.y = cum;
                cum = cum + x[t].z;
                c.z = cum;
                cum = cum + x[t].w;
                c.w = cum;
                dst[b4 + t] = c; /* the same value from every lane */
            }
        }
        __builtin_amdgcn_wave_barrier();
        int first = -1;
#pragma unroll
        for (int q = Q - 1; q >= 0; --q) {
            const uint64_t reach = __ballot(act[q] && sh.val[q * 64 + lane] >= thr);
            if (reach) first = q * 64 + (int)__builtin_ctzll(reach);
        }
        if (first >= 0) {
            chosen = first;
            flags |= G4S_FLAG_REACHED;
        }
    }
    if (lane == 0) {
        st_sys(&a.ids[row], (int32_t)ent_idx(sh.sorted[chosen]));       /* :2826 */
        if (a.out.count) a.out.count[row] = nsurv;
        if (a.out.argmax) a.out.argmax[row] = (int32_t)ent_idx(sh.sorted[jarg]);
        if (a.out.lsum) a.out.lsum[row] = lsum;
        if (a.out.flags) st_sys(&a.out.flags[row], flags);
    }
    if (a.out.indices || a.out.probs) {
        const int capn = a.out.capacity < nsurv ? a.out.capacity : nsurv;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int j = q * 64 + lane;
            if (j < capn) {
                if (a.out.indices)
                    a.out.indices[(int64_t)row * a.out.capacity + j] = (int32_t)ent_idx(my[q]);
                if (a.out.probs) a.out.probs[(int64_t)row * a.out.capacity + j] = p[q];
            }
        }
    }
    publish_done(a.done, row, a.seq);
}

bool decode_eligible(const TopkArgs& a, int dtype)
{
    if (!a.dec_tickets || a.batch < 1 || a.batch > a.dec_rows) return false;
    if (a.kbound < 1 || a.kbound > kDecMaxK) return false;
    const int64_t ch = (int64_t)kDB * (dtype == G4S_DTYPE_F32 ? 4 : 8);
    return (a.vocab + ch - 1) / ch <= kDecMaxChunks;
}

hipError_t decode_launch(const TopkArgs& a, int dtype, hipStream_t s)
{
    const int64_t ch = (int64_t)kDB * (dtype == G4S_DTYPE_F32 ? 4 : 8);
    const dim3 grid((unsigned)((a.vocab + ch - 1) / ch), (unsigned)a.batch);
    /* LDS (and so the resident workgroups of the row pass) sized by the K bound */
    const bool small = a.kbound <= kDecSmallK;
    if (dtype == G4S_DTYPE_F32) {
        if (small)
            hipLaunchKernelGGL((topk_decode_kernel<0, kDecSmallK>), grid, dim3(kDB), 0, s, a);
        else
            hipLaunchKernelGGL((topk_decode_kernel<0, kDecMaxK>), grid, dim3(kDB), 0, s, a);
    } else {
        if (small)
            hipLaunchKernelGGL((topk_decode_kernel<1, kDecSmallK>), grid, dim3(kDB), 0, s, a);
        else
            hipLaunchKernelGGL((topk_decode_kernel<1, kDecMaxK>), grid, dim3(kDB), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace g4s
