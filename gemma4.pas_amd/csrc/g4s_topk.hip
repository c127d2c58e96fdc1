/*
 * g4s_topk.hip -- the top-k sampling path on gfx950 (rows with 0 < TopK < V).
 *
 * Replaces DoSelectTopKIndices + the top-k branch of DoSample
 * (src/Gemma4.Model.pas:2615-2689, 2765-2826).  One kernel launch per batch,
 * grid = splits x rows, one workgroup per vocabulary chunk:
 *
 *  phase 1 (every workgroup)
 *    - 16-byte loads of the chunk into registers as order-preserving keys;
 *    - a provable lower bound theta of the chunk's K-th largest key: each
 *      wave bounds the ceil(K/waves)-th largest of its 64 thread maxima
 *      from below (ballot binary search over 14 bits below their common
 *      prefix; distinct threads, so the wave holds at least that many keys
 *      >= its value) and the block keeps the minimum;
 *    - every key >= theta is a candidate (a superset of the chunk's top-K):
 *      wave-level compaction into LDS with one store per item and no
 *      branch, then coalesced stores to the chunk's HBM slots; if more than
 *      the chunk's slot count qualify (heavy ties), an exact per-chunk radix
 *      select emits the keys above the chunk's K-th value plus its first K
 *      copies in index order;
 *    - per wave, the r-th largest of its 64 thread maxima, r =
 *      ceil(2K / waves in the row): the wave holds at least r distinct keys
 *      >= it, so the ceil(K/r)-th largest of these over the row's waves is a
 *      second lower bound of the row's K-th largest (a tight one: the top
 *      keys of a row rarely share a thread);
 *    - an atomic ticket elects the last workgroup of the row; a batch
 *      whose chunk workgroups do not all fit the device at once skips the
 *      ticket and runs the merges as a second launch (one workgroup per
 *      row, TopkArgs::mode), so no merge holds a compute unit that a chunk
 *      of the second round is waiting for.
 *  merge + tail (last workgroup of each row, or the merge launch)
 *    - loads every chunk record, wave bound and candidate slot of the row
 *      with independent loads (one memory round trip), keeps candidates
 *      >= the larger bound (branch-free LDS compaction), selects the exact
 *      K-th value tau, resolves ties at tau like the reference's min-heap
 *      (lowest index when the heap layout cannot matter, a full heap replay
 *      otherwise), and orders the survivors by vocab index (for at most 128
 *      candidates the other waves rank them by index while wave 0 selects);
 *    - wave 0 runs the reference's tail in index order: softcap, 1/T, max,
 *      exp, sequential binary32 LSum, division, argmax, sequential running
 *      sum against fl32(u*TopP).  The sequential sums are exact left-to-right
 *      binary32 chains over broadcast LDS reads.
 */
#include "g4s_select.h"
#include "g4s_topk.h"
#include "g4s_lmhead.h"

#include <type_traits>

namespace g4s {

using namespace g4s::cr;

namespace {

/* candidate slots one merge thread loads per round */
template <int BLOCK, int KCAP>
constexpr int batch_loads()
{
    return (BLOCK == 1024 && KCAP <= 256) ? 8 : 16;
}

/* LDS of the kernel, sized by the launch's K bound (KCAP >= every K of the
 * launch) so that the many phase-1 workgroups of a batch stay resident
 * together: MCAP merge candidates are kept on chip. */
template <int KCAP, int MCAP>
struct TopkShared {
    static constexpr int kKcap = KCAP;
    static constexpr int kMcap = MCAP;
    uint32_t wtheta[16];
    int scan[16];
    uint32_t red[48];
    int misc[8]; /* [0..3] counters and flags (see the kernel), [4..6] select results,
                    [7] the wave-bound lower bound of the merge */
    int flag_last;
    uint32_t hist[256];
    ChunkRec rec[kMaxSplits];
    uint32_t wb[kWaveBounds];
    uint64_t mc[MCAP + 64]; /* phase-1 candidate staging, then merge candidates, then
                               replay tiles; the last 64 absorb dropped lane writes */
    uint64_t surv[KCAP];   /* survivors (unsorted); min-heap storage during a replay */
    uint64_t sorted[KCAP]; /* survivors ascending by vocab index */
    uint64_t byidx[128];          /* small merges: the candidates in index order */
    alignas(16) float val[KCAP];  /* tail: v, then e; +0 up to a multiple of 64 */
    alignas(16) float prob[KCAP]; /* tail: p; +0 up to a multiple of 64 */
};

/* ------------------------------------------------------------ heap replay */

/* Exact replay of the reference's min-heap pass (Model.pas:2632-2664) over a
 * whole row, for rows whose K-th value is tied in a way the heap layout
 * decides.  Elements are screened in tiles against the current root; the
 * screened ones (in index order) are inserted by one lane.  On return
 * hv[0..K) / hi[0..K) hold the heap. */
template <int BLOCK, int DT, typename SH>
__device__ void heap_replay(const char* row, int vocab, int K, SH& sh, float* hv, int32_t* hi)
{
    static_assert(SH::kMcap >= BLOCK, "replay tiles fit the merge area");
    float* qv = reinterpret_cast<float*>(sh.mc);
    int32_t* qi = reinterpret_cast<int32_t*>(sh.mc) + SH::kMcap;
    const int tid = threadIdx.x;
    for (int i = tid; i < K; i += BLOCK) {
        hv[i] = -1e30f; /* :2634-2638 */
        hi[i] = -1;
    }
    __syncthreads();
    for (int base = 0; base < vocab; base += BLOCK) {
        const int e = base + tid;
        const float x = (e < vocab) ? load_elem<DT>(row, e) : 0.0f;
        const float root = hv[0];
        const int take = (e < vocab) && !(x <= root);
        int total;
        const int pos = block_exclusive_scan<BLOCK>(take, sh.scan, total);
        if (take) {
            qv[pos] = x;
            qi[pos] = e;
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
}

/* One wave: the K-th largest key tau of the M <= 64*NG candidates (K < M).
 * When exactly K candidates are >= tau they are the survivors: written to
 * surv (any order) and true is returned; otherwise false (copies of tau must
 * be split by the tie rules). */
template <int NG>
__device__ __forceinline__ bool wave_fast_select(const uint64_t* mc, int M, int K, uint64_t* surv,
                                                 uint32_t* tau_out = nullptr)
{
    const int lane = threadIdx.x & 63;
    uint32_t kk[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        const int i = lane + 64 * q;
        kk[q] = i < M ? cand_key_of(mc[i]) : 0u;
    }
    int G, E;
    const uint32_t tau = wave_select_kth<NG>(kk, K, &G, &E);
    if (tau_out) *tau_out = tau;
    const bool fast = E == K - G;
    if (fast) {
        int off = 0;
#pragma unroll
        for (int q = 0; q < NG; ++q) {
            const bool t = kk[q] >= tau; /* tau >= 1: padding keys are 0 */
            const uint64_t mask = __ballot(t);
            if (t) surv[off + __popcll(mask & ((1ull << lane) - 1ull))] = mc[lane + 64 * q];
            off += __popcll(mask);
        }
    }
    return fast;
}


/* The K-th largest key tau of the M <= BLOCK candidates in LDS (K < M),
 * over the whole workgroup: 8-bit MSD radix passes over the bits below the
 * keys' common prefix only (every candidate key is >= 1), one candidate
 * per thread.  When exactly K candidates are >= tau they are the survivors:
 * written to surv (any order) and true is returned; otherwise false. */
template <int BLOCK, typename SH>
__device__ __forceinline__ bool block_fast_select(SH& sh, int M, int K, uint64_t* surv)
{
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    constexpr int NW = BLOCK / 64;
    const uint64_t c = tid < M ? sh.mc[tid] : 0ull;
    const uint32_t k = cand_key_of(c);
    const uint32_t hw = wave_max_u32(k), lw = wave_min_u32(tid < M ? k : 0xFFFFFFFFu);
    if (lane == 0) {
        sh.red[wid] = hw;
        sh.red[NW + wid] = lw;
    }
    __syncthreads();
    uint32_t hi = 0u, lo = 0xFFFFFFFFu;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        hi = g4s_max_u(hi, sh.red[w]);
        lo = g4s_min_u(lo, sh.red[NW + w]);
    }
    uint32_t tau;
    int G = 0, E;
    if (hi == lo) {
        tau = hi;
        E = M;
    } else {
        int top = 31 - __builtin_clz(hi ^ lo);
        uint32_t prefix = top >= 31 ? 0u : (hi & ~((2u << top) - 1u));
        uint32_t mask = top >= 31 ? 0u : ~((2u << top) - 1u);
        int kk = K;
        E = 0;
        for (;;) {
            const int shift = top >= 7 ? top - 7 : 0;
            for (int b = tid; b < 256; b += BLOCK) sh.hist[b] = 0u;
            __syncthreads();
            if (tid < M && (k & mask) == prefix) atomicAdd(&sh.hist[(k >> shift) & 255u], 1u);
            __syncthreads();
            radix_digit_step(kk, sh.hist, sh.misc + 4);
            __syncthreads();
            G += sh.misc[5];
            E = sh.misc[6];
            kk -= sh.misc[5];
            prefix |= (uint32_t)sh.misc[4] << shift;
            mask |= ((top - shift == 31) ? 0xFFFFFFFFu : ((2u << (top - shift)) - 1u)) << shift;
            if (shift == 0) break;
            top = shift - 1;
            __syncthreads(); /* the digit step's words are read before the next pass */
        }
        tau = prefix;
    }
    if (E != K - G) return false; /* uniform */
    int tot;
    const bool keep = tid < M && k >= tau;
    const int pos = block_exclusive_scan<BLOCK>(keep ? 1 : 0, sh.scan, tot);
    if (keep) surv[pos] = c;
    return true;
}

}  // namespace

template <int BLOCK, int ITEMS, int DT, int KCAP>
__global__ __launch_bounds__(BLOCK) void topk_kernel(TopkArgs a)
{
    constexpr int VW = Elem<DT>::VW;
    constexpr int NV = ITEMS / VW;
    constexpr int NW = BLOCK / 64;
    constexpr int CHUNK = BLOCK * ITEMS;
    constexpr int MCAP = KCAP <= 64 ? (BLOCK > 512 ? BLOCK : 512) : kMergeLds; /* >= BLOCK */
    constexpr int kBatchLoads = batch_loads<BLOCK, KCAP>();
    static_assert(BLOCK >= kMaxSplits, "one merge thread per chunk record");
    static_assert(KCAP <= BLOCK, "one survivor per thread");
    __shared__ TopkShared<KCAP, MCAP> sh;

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int row = blockIdx.y;
    const int chunk = blockIdx.x;
    const int S = a.splits;
    const int V = a.vocab;

    const g4s_params rp = a.params ? a.params[row] : a.p0;
    const double u = a.u ? a.u[row] : a.u0;
    const int K = rp.top_k;
    if (!(K >= 1 && K < V)) {
        /* full-vocabulary row (Model.pas:2756): the softmax launches take it,
         * or, when none follows this launch, it is rejected here so that no
         * stale id of an earlier call survives */
        if (!a.full_on && chunk == 0 && wid == 0 && a.mode != 1) {
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
        if (chunk == 0 && wid == 0 && a.mode != 1) {
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
    const int64_t cbase = (int64_t)chunk * CHUNK;
    const int cap = 1 << a.cap_log2;
    uint64_t* gcand = a.cand + (int64_t)row * kCandRow + ((int64_t)chunk << a.cap_log2);
    if (tid == 0) {
        sh.misc[0] = 0; /* emission counter */
        sh.misc[1] = 0; /* merge counter */
        sh.misc[2] = 0; /* survivor counter */
        sh.misc[3] = 0; /* K-th key tie flag */
    }

    const int nwave = S * NW;
    /* rank of each wave's recorded bound among its 64 thread maxima */
    int r1 = (2 * K + nwave - 1) / nwave;
    r1 = r1 < 1 ? 1 : (r1 > 64 ? 64 : r1);
    if (a.mode != 2) {
    /* ------------------------------------------------------- phase 1 */
    uint32_t keys[ITEMS];
    if (cbase + CHUNK <= V) {
        /* whole chunk in bounds: independent unconditional 16-byte loads */
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            float v[VW];
            load_vec_full<DT>(rowp, cbase + ((int64_t)j * BLOCK + tid) * VW, v);
#pragma unroll
            for (int q = 0; q < VW; ++q) keys[j * VW + q] = cand_key(v[q]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            float v[VW];
            const int64_t e0 = cbase + ((int64_t)j * BLOCK + tid) * VW;
            load_vec<DT>(rowp, e0, V, v);
#pragma unroll
            for (int q = 0; q < VW; ++q) keys[j * VW + q] = (e0 + q < V) ? cand_key(v[q]) : 0u;
        }
    }
    uint32_t tmax = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) tmax = keys[i] > tmax ? keys[i] : tmax;
    /* per wave: lower bounds of the ceil(K/waves)-th and the r1-th largest of
     * the 64 thread maxima (distinct elements, so the wave holds at least
     * that many keys >= each value) */
    const int kw = (K + NW - 1) / NW;
    uint32_t wth, wr1;
    /* 14 bits below the common prefix of the thread maxima: a bound a hair
     * under the exact value costs a candidate or two and saves half of the
     * search */
    wave_kth_largest2(tmax, kw, r1, 14, wth, wr1);
    if (lane == 0) {
        sh.wtheta[wid] = wth;
        if (nwave <= kWaveBounds && nwave <= BLOCK)
            st_dev(&a.wbounds[(int64_t)row * kWaveBounds + chunk * NW + wid], wr1);
    }
    __syncthreads();
    /* theta: every wave has >= kw keys >= theta, so the chunk has >= K */
    uint32_t theta = 0xFFFFFFFFu;
#pragma unroll
    for (int w = 0; w < NW; ++w) theta = sh.wtheta[w] < theta ? sh.wtheta[w] : theta;
    theta = theta < 1u ? 1u : theta;

    /* every key >= theta is a candidate: wave-level compaction (one LDS
     * atomic per wave for the wave's base) into the LDS staging area with a
     * store per item and no branch (an item that is not a candidate, or
     * beyond the slots, goes to its lane's spare entry), then coalesced
     * stores to the chunk's HBM slots when they all fit */
    static_assert(MCAP >= 4 * KCAP || MCAP >= kMergeLds, "staging holds a chunk's slots");
    int mine = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) mine += keys[i] >= theta;
    {
        const int incl = wave_inclusive_scan(mine);
        int base = 0;
        if (lane == 63) base = atomicAdd(&sh.misc[0], incl);
        base = __builtin_amdgcn_readlane(base, 63);
        int pos = base + incl - mine;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int q = 0; q < VW; ++q) {
                const uint32_t k = keys[j * VW + q];
                const bool c = k >= theta;
                sh.mc[(c && pos < cap) ? pos : MCAP + lane] =
                    cand_pack(k, (uint32_t)(cbase + ((int64_t)j * BLOCK + tid) * VW + q));
                pos += c ? 1 : 0;
            }
    }
    __syncthreads();
    const int total = sh.misc[0];
    if (total <= cap)
        for (int i = tid; i < total; i += BLOCK) st_dev(&gcand[i], sh.mc[i]);

    uint32_t rec_bound = theta, rec_mode_e = 0;
    int emitted = total;
    if (total > cap) {
        /* heavy ties or a weak theta: exact K-th largest of the chunk (the
         * chunk holds more than cap >= 2K keys >= theta >= 1, so at least K);
         * nothing was written to the slots */
        int gt_c, eq_c;
        const uint32_t tau_c =
            regs_radix_kth<BLOCK, ITEMS>(keys, K, sh.hist, sh.misc + 4, &gt_c, &eq_c);
        /* keys strictly above tau_c, any order (fewer than K of them) */
        int gmine = 0;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) gmine += keys[i] > tau_c;
        int gtot;
        int goff = block_exclusive_scan<BLOCK>(gmine, sh.scan, gtot);
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int q = 0; q < VW; ++q) {
                const uint32_t k = keys[j * VW + q];
                if (k > tau_c) {
                    st_dev(&gcand[goff],
                           cand_pack(k, (uint32_t)(cbase + ((int64_t)j * BLOCK + tid) * VW + q)));
                    ++goff;
                }
            }
        /* the first min(eq, K) copies of tau_c in index order: load slot j,
         * then thread, then position within the vector */
        const int want = eq_c < K ? eq_c : K;
        const int base = gtot;
        int taken = 0;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            int c = 0;
#pragma unroll
            for (int q = 0; q < VW; ++q) c += keys[j * VW + q] == tau_c;
            int tot_j;
            int r = block_exclusive_scan<BLOCK>(c, sh.scan, tot_j);
#pragma unroll
            for (int q = 0; q < VW; ++q) {
                if (keys[j * VW + q] == tau_c) {
                    if (taken + r < want)
                        st_dev(&gcand[base + taken + r],
                               cand_pack(tau_c,
                                         (uint32_t)(cbase + ((int64_t)j * BLOCK + tid) * VW + q)));
                    ++r;
                }
            }
            taken += tot_j;
        }
        emitted = gtot + want;
        rec_bound = tau_c;
        rec_mode_e = 0x80000000u | (uint32_t)eq_c;
    }
    if (tid == 0) {
        uint64_t* rp64 = reinterpret_cast<uint64_t*>(a.recs + (int64_t)row * kMaxSplits + chunk);
        st_dev(rp64, ((uint64_t)rec_bound << 32) | (uint32_t)emitted);
        st_dev(rp64 + 1, (uint64_t)rec_mode_e << 32);
    }

    if (a.mode == 1) return; /* the merge launch follows */

    /* ----------------------------------------------- last workgroup elects */
    if (!elect_last(&a.tickets[row], (uint32_t)S, &sh.flag_last)) return;
    } /* phase 1 */

    /* ------------------------------------------------------------ merge */
    uint32_t flags = G4S_FLAG_TOPK_PATH;
    const uint64_t* rcand = a.cand + (int64_t)row * kCandRow;
    uint64_t* gmerge = a.merge + (int64_t)row * kCandRow;
    const int span = S << a.cap_log2;

    /* one round trip: the chunk records, the wave bounds and the first
     * batch of slots (the index is clamped instead of branched on, so every
     * load is issued) */
    const bool use_wb = nwave <= kWaveBounds && nwave <= BLOCK; /* one per merge thread */
    uint32_t wbv = 0u;
    if (use_wb && tid < nwave) wbv = ld_dev(&a.wbounds[(int64_t)row * kWaveBounds + tid]);
    if (tid < S) {
        const uint64_t* rp64 =
            reinterpret_cast<const uint64_t*>(a.recs + (int64_t)row * kMaxSplits + tid);
        const uint64_t w0 = ld_dev(rp64), w1 = ld_dev(rp64 + 1);
        ChunkRec r;
        r.count = (uint32_t)w0;
        r.bound = (uint32_t)(w0 >> 32);
        r.rsv = (uint32_t)w1;
        r.mode_e = (uint32_t)(w1 >> 32);
        sh.rec[tid] = r;
    }
    uint64_t v[kBatchLoads];
#pragma unroll
    for (int i = 0; i < kBatchLoads; ++i) {
        const int f = tid + i * BLOCK;
        v[i] = ld_dev(&rcand[f < span ? f : span - 1]);
    }
    if (use_wb && tid < nwave) sh.wb[tid] = wbv;
    __syncthreads();
    /* a row the candidates cannot decide without its logits (none written) */
    bool need_row = sh.rec[0].rsv == kRecNeedRow;
    if (need_row) {
        if (wid == 0) {
            if (lane == 0) {
                st_sys(&a.ids[row], -1);
                if (a.out.flags) st_sys(&a.out.flags[row], flags | G4S_FLAG_ROW_RECOMPUTED);
                if (a.out.count) a.out.count[row] = 0;
            }
            publish_done(a.done, row, a.seq);
        }
        return;
    }
    uint32_t lb, l1 = 0u;
    bool any_exact;
    {
        uint32_t mb = 1u, ex = 0u;
        if (tid < S) {
            const ChunkRec r = sh.rec[tid];
            mb = r.bound > 1u ? r.bound : 1u;
            ex = r.mode_e >> 31;
        }
        mb = wave_max_u32(mb);
        ex = wave_max_u32(ex);
        if (lane == 0) {
            sh.red[wid] = mb;
            sh.red[32 + wid] = ex;
        }
        /* a lower bound of the ceil(K/r1)-th largest wave bound, by every
         * wave (no barrier); 10 bits below the common prefix are enough to
         * cut the candidates to about K */
        if (use_wb && wid == 0) {
            const int j = (K + r1 - 1) / r1;
            const auto bound = [&](auto ng) {
                constexpr int NG = decltype(ng)::value;
                uint32_t kk[NG];
                int nz = 0;
#pragma unroll
                for (int q = 0; q < NG; ++q) {
                    const int i = lane + 64 * q;
                    kk[q] = i < nwave ? sh.wb[i] : 0u;
                    nz += __popcll(__ballot(kk[q] != 0u));
                }
                return nz >= j ? wave_kth_bound<NG>(kk, j, 10) : 0u;
            };
            const uint32_t b = nwave <= 128   ? bound(std::integral_constant<int, 2>{})
                               : nwave <= 256 ? bound(std::integral_constant<int, 4>{})
                                              : bound(std::integral_constant<int, kWaveBounds / 64>{});
            if (lane == 0) sh.misc[7] = (int)b;
        }
        __syncthreads();
        if (use_wb) l1 = (uint32_t)sh.misc[7];
        lb = 1u;
        ex = 0u;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            lb = sh.red[w] > lb ? sh.red[w] : lb;
            ex |= sh.red[32 + w];
        }
        any_exact = ex != 0u;
    }
    if (any_exact) flags |= G4S_FLAG_CHUNK_EXACT;
    const uint32_t L = lb > l1 ? lb : l1;
    /* counters of the small select below (the wave bounds are consumed; the
     * compaction's barrier orders these stores before their use) */
    constexpr int kSmallM = 128;
    static_assert(kWaveBounds >= kSmallM, "small-select counters");
    for (int i = tid; i < kSmallM; i += BLOCK) sh.wb[i] = 0u;

    /* keep the candidates >= L (wave-level compaction); LDS holds the first
     * MCAP of them, the rest go to the row's HBM merge area */

    for (int b0 = 0; b0 < span; b0 += kBatchLoads * BLOCK) {
        if (b0 > 0) {
#pragma unroll
            for (int i = 0; i < kBatchLoads; ++i) {
                const int f = b0 + tid + i * BLOCK;
                v[i] = ld_dev(&rcand[f < span ? f : span - 1]);
            }
        }
        /* bit i: slot i is kept (inside the row's span, below its chunk's
         * count, key >= L); the counts are read unconditionally (clamped
         * index) so that the LDS reads overlap */
        uint32_t cnt_of[kBatchLoads];
#pragma unroll
        for (int i = 0; i < kBatchLoads; ++i) {
            const int f = b0 + tid + i * BLOCK;
            cnt_of[i] = sh.rec[(f < span ? f : span - 1) >> a.cap_log2].count;
        }
        uint32_t km = 0u;
#pragma unroll
        for (int i = 0; i < kBatchLoads; ++i) {
            const int f = b0 + tid + i * BLOCK;
            const bool k = (f < span) & ((uint32_t)(f & (cap - 1)) < cnt_of[i]) &
                           (cand_key_of(v[i]) >= L);
            km |= (uint32_t)k << i;
        }
        const int cnt = __popc(km);
        const int incl = wave_inclusive_scan(cnt);
        int base = 0;
        if (lane == 63) base = atomicAdd(&sh.misc[1], incl);
        base = __builtin_amdgcn_readlane(base, 63);
        int pos = base + incl - cnt;
        if (__builtin_amdgcn_readlane(base + incl, 63) <= MCAP) {
            /* the wave's candidates all fit in LDS: a store per slot, no
             * branch (a slot not kept goes to its lane's spare entry) */
#pragma unroll
            for (int i = 0; i < kBatchLoads; ++i) {
                const bool k = (km >> i) & 1u;
                sh.mc[k ? pos : MCAP + lane] = v[i];
                pos += k ? 1 : 0;
            }
        } else {
#pragma unroll
            for (int i = 0; i < kBatchLoads; ++i) {
                if ((km >> i) & 1u) {
                    if (pos < MCAP)
                        sh.mc[pos] = v[i];
                    else
                        gmerge[pos] = v[i];
                    ++pos;
                }
            }
        }
    }
    __syncthreads();
    const int M = sh.misc[1];
    if (M > MCAP) flags |= G4S_FLAG_WIDE_MERGE;
    auto ent = [&](int i) -> uint64_t { return i < MCAP ? sh.mc[i] : gmerge[i]; };
    auto ekey = [&](int i) { return cand_key_of(ent(i)); };
    auto eidx = [&](int i) { return cand_idx_of(ent(i)); };

    /* exact top K of the M candidates */
    int nsurv = 0;
    bool general = any_exact || M > MCAP;
    bool ordered = false; /* survivors already in sh.sorted by index */
    if (!general && K == 1 && M > 1) {
        /* K = 1: the reference's one-entry heap keeps the first (lowest-index)
         * copy of the largest key, as a later equal key is rejected (v <=
         * root, Model.pas:2643-2644); every copy of it is a candidate */
        if (wid == 0) {
            uint32_t kmax = 0u;
            for (int i = lane; i < M; i += 64) kmax = g4s_max_u(kmax, cand_key_of(sh.mc[i]));
            kmax = wave_max_u32(kmax);
            uint32_t imin = 0xFFFFFFFFu;
            int copies = 0;
            for (int i = lane; i < M; i += 64) {
                const uint64_t c = sh.mc[i];
                if (cand_key_of(c) == kmax) {
                    imin = g4s_min_u(imin, cand_idx_of(c));
                    ++copies;
                }
            }
            imin = wave_min_u32(imin);
            if (wave_sum_i32(copies) > 1) flags |= G4S_FLAG_TIE_LOWEST;
            if (lane == 0) sh.sorted[0] = cand_pack(kmax, imin);
        }
        nsurv = 1;
        ordered = true;
    } else if (!general && M > K && M <= kSmallM && NW >= 4) {
        /* wave 0 selects tau by its ballot search while the other waves rank
         * the M candidates by vocabulary index (distinct indices; thread
         * (i, s) counts the smaller indices in slice s into an LDS counter) */
        uint32_t tau = 0u;
        if (wid == 0) {
            const bool fast = wave_fast_select<2>(sh.mc, M, K, sh.surv, &tau);
            if (lane == 0) sh.misc[5] = fast ? 0 : 1;
        } else {
            constexpr int SL = (NW - 1) * 64 / kSmallM; /* slices over waves 1.. */
            const int t = tid - 64;
            const int ci = t % kSmallM, sl = t / kSmallM;
            const int per = ((M + SL - 1) / SL + 7) & ~7; /* whole steps of 8 */
            const int j0 = sl * per, j1 = j0 + per < M ? j0 + per : M;
            if (sl < SL && ci < M) {
                const uint32_t mi = cand_idx_of(sh.mc[ci]);
                uint32_t r = 0u;
                for (int j = j0; j < j1; j += 8) {
                    /* 16-byte reads issued together; entries past the slice
                     * (within the merge area) are read and masked */
                    uint32_t ij[8];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint4 w = reinterpret_cast<const uint4*>(sh.mc + j)[q];
                        ij[2 * q] = w.x;
                        ij[2 * q + 1] = w.z;
                    }
#pragma unroll
                    for (int q = 0; q < 8; ++q) r += (j + q < j1 && ij[q] < mi) ? 1u : 0u;
                }
                atomicAdd(&sh.wb[ci], r);
            }
        }
        __syncthreads();
        general = sh.misc[5] != 0;
        if (!general) {
            /* exactly K keys >= tau: wave 0 places every candidate at its
             * index rank, then compacts the ones >= tau in that order */
            nsurv = K;
            ordered = true;
            if (wid == 0) {
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int i = lane + 64 * q;
                    if (i < M) sh.byidx[sh.wb[i]] = sh.mc[i];
                }
                __builtin_amdgcn_wave_barrier();
                int off = 0;
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int i = lane + 64 * q;
                    const uint64_t c = i < M ? sh.byidx[i] : 0ull;
                    const bool keep = i < M && cand_key_of(c) >= tau;
                    const uint64_t m = __ballot(keep);
                    if (keep) sh.sorted[off + __popcll(m & ((1ull << lane) - 1ull))] = c;
                    off += __popcll(m);
                }
            }
        }
    } else if (!general) {
        /* one wave finds the K-th largest key tau of the M candidates (ballot
         * search over registers); when the candidates hold exactly K keys
         * >= tau there is no choice to make and they are the survivors.
         * Otherwise (copies of tau must be split) the general path decides. */
        if (M <= K) {
            for (int i = tid; i < M; i += BLOCK) sh.surv[i] = sh.mc[i];
            nsurv = M;
        } else if (M <= 128 && M <= MCAP) {
            if (wid == 0) {
                const bool fast = wave_fast_select<2>(sh.mc, M, K, sh.surv);
                if (lane == 0) sh.misc[5] = fast ? 0 : 1;
            }
            __syncthreads();
            general = sh.misc[5] != 0;
            if (!general) nsurv = K;
        } else if (M <= 512 && M <= MCAP && M <= BLOCK) {
            /* the whole workgroup's radix select (one wave's ballot search
             * over 4-8 keys per lane takes longer) */
            general = !block_fast_select<BLOCK>(sh, M, K, sh.surv);
            if (!general) nsurv = K;
        } else {
            general = true;
        }
    }
    if (general) {
        if (M <= K) {
            /* M < K: fewer than K logits above -1e30 in the whole row; M == K:
             * the candidates are exactly the top K.  Either way all survive. */
            for (int i = tid; i < M; i += BLOCK) sh.surv[i] = ent(i);
            nsurv = M;
        } else {
            int G, E;
            const uint32_t tau = select_kth<BLOCK>(M, K, ekey, sh, &G, &E);
            const int need = K - G;
            /* a chunk whose exact select truncated copies of tau */
            int trunc = 0;
            if (tid < S) {
                const ChunkRec r = sh.rec[tid];
                trunc = (r.mode_e >> 31) && r.bound == tau && (int)(r.mode_e & 0x7FFFFFFFu) > K;
            }
            trunc = block_sum_i32<BLOCK>(trunc, sh.scan);
            int mode = 0; /* 0: all >= tau survive, 1: lowest-index ties, 2: heap replay */
            int32_t idx_thr = 0x7FFFFFFF;
            if (E != need || trunc) {
                /* t* = index of the K-th element >= tau in index order */
                int g2, e2;
                const uint32_t tstar_inv = block_radix_kth<BLOCK>(
                    M, K, [&](int i) { return ~eidx(i); }, [&](int i) { return ekey(i) >= tau; },
                    sh.hist, sh.misc + 4, &g2, &e2);
                const int32_t tstar = (int32_t)~tstar_inv;
                uint32_t mg = 0;
                for (int i = tid; i < M; i += BLOCK)
                    if (ekey(i) > tau) mg = (eidx(i) + 1u) > mg ? (eidx(i) + 1u) : mg;
                mg = block_max_u32<BLOCK>(mg, sh.red);
                const int32_t max_gt = (int32_t)mg - 1; /* -1 when nothing is above tau */
                if (max_gt < tstar) {
                    /* every key above tau precedes the K-th key >= tau: the heap
                     * keeps them and the first `need` copies of tau */
                    mode = 1;
                    const uint32_t thr_inv = block_radix_kth<BLOCK>(
                        M, need, [&](int i) { return ~eidx(i); },
                        [&](int i) { return ekey(i) == tau; }, sh.hist, sh.misc + 4, &g2, &e2);
                    idx_thr = (int32_t)~thr_inv;
                    flags |= G4S_FLAG_TIE_LOWEST;
                } else {
                    mode = 2;
                    flags |= G4S_FLAG_HEAP_REPLAY;
                }
            }
            if (mode < 2) {
                auto surv_ok = [&](int i) {
                    const uint32_t k = ekey(i);
                    return (k > tau) || (k == tau && (mode == 0 || (int32_t)eidx(i) <= idx_thr));
                };
                int take_n = 0;
                for (int i = tid; i < M; i += BLOCK) take_n += surv_ok(i);
                int sv;
                int soff = block_exclusive_scan<BLOCK>(take_n, sh.scan, sv);
                for (int i = tid; i < M; i += BLOCK)
                    if (surv_ok(i)) sh.surv[soff++] = ent(i);
                nsurv = sv;
            } else if (!a.logits) {
                need_row = true; /* the replay needs every logit */
            } else {
                float* hv = reinterpret_cast<float*>(sh.surv);
                int32_t* hi = reinterpret_cast<int32_t*>(sh.surv) + KCAP;
                heap_replay<BLOCK, DT>(rowp, V, K, sh, hv, hi);
                /* the heap holds K entries, all with index >= 0 here (M > K);
                 * K <= kbound <= BLOCK, so one entry per thread */
                uint64_t mine_e = 0;
                if (tid < K) mine_e = cand_pack(f2key(hv[tid]), (uint32_t)hi[tid]);
                __syncthreads();
                if (tid < K) sh.surv[tid] = mine_e;
                nsurv = K;
            }
        }
    }
    __syncthreads();

    if (nsurv == 0) {
        if (wid == 0) {
            if (lane == 0) {
                st_sys(&a.ids[row], -1);
                if (a.out.flags)
                    st_sys(&a.out.flags[row],
                           flags | (need_row ? G4S_FLAG_ROW_RECOMPUTED : G4S_FLAG_EMPTY));
                if (a.out.count) a.out.count[row] = 0;
            }
            publish_done(a.done, row, a.seq);
        }
        return;
    }

    /* one survivor per thread (nsurv <= K <= BLOCK): its slot in vocab-index
     * order (given by the small select, else rank by count; indices are
     * distinct), then the reference's per-survivor steps */
    const float cap_v = a.softcap;
    const float T = rp.temperature;
    const bool scale = (T > 0.0f) && (T != 1.0f);
    const float inv_t = scale ? div_cr32(1.0f, T) : 1.0f;               /* :2782 */
    uint32_t kv = 0u;
    float vv = 0.0f;
    int pos = 0;
    /* p's storage holds the rank counters until the tail writes p */
    uint32_t* rk = reinterpret_cast<uint32_t*>(sh.prob);
    if (!ordered) {
        /* rank by count over the whole workgroup: thread (i, s) counts the
         * survivors of slice s with an index below survivor i's into i's
         * counter */
        for (int i = tid; i < nsurv; i += BLOCK) rk[i] = 0u;
        __syncthreads();
        const int npad = (nsurv + 63) & ~63; /* <= KCAP <= BLOCK */
        const int SL = BLOCK / npad;
        const int i = tid % npad, sl = tid / npad;
        if (sl < SL && i < nsurv) {
            const int per = (nsurv + SL - 1) / SL;
            const int j0 = sl * per, j1 = j0 + per < nsurv ? j0 + per : nsurv;
            const uint32_t mi = cand_idx_of(sh.surv[i]);
            uint32_t c = 0u;
            int j = j0;
            for (; j + 8 <= j1; j += 8) {
                uint32_t xx[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) xx[t] = cand_idx_of(sh.surv[j + t]);
#pragma unroll
                for (int t = 0; t < 8; ++t) c += xx[t] < mi ? 1u : 0u;
            }
            for (; j < j1; ++j) c += cand_idx_of(sh.surv[j]) < mi ? 1u : 0u;
            if (c != 0u) atomicAdd(&rk[i], c);
        }
        __syncthreads();
    }
    if (tid < nsurv) {
        uint64_t my;
        if (ordered) {
            pos = tid;
            my = sh.sorted[tid];
        } else {
            my = sh.surv[tid];
            pos = (int)rk[tid];
            sh.sorted[pos] = my;
        }
        const float x = key2f(cand_key_of(my));                         /* :2774 */
        vv = (cap_v > 0.0f) ? softcap_topk_cr32(x, cap_v) : x;          /* :2775-2776 */
        if (scale) vv = vv * inv_t;                                     /* :2783-2784 */
        kv = f2key(vv);
    }
    kv = wave_max_u32(kv);
    if (lane == 0) sh.red[wid] = kv;
    __syncthreads();
    uint32_t kmax = 0u;
#pragma unroll
    for (int w = 0; w < NW; ++w) kmax = g4s_max_u(kmax, sh.red[w]);
    const float vmax = key2f(kmax);                                     /* :2789-2792 */
    if (tid < nsurv) sh.val[pos] = exp_diff_cr32(vv, vmax);             /* :2797 */
    const int npad = (nsurv + 63) & ~63; /* <= KCAP, a multiple of 64 */
    if (tid >= nsurv && tid < npad) {
        sh.val[tid] = 0.0f;
        sh.prob[tid] = 0.0f;
    }
    __syncthreads();

    /* ------------------------------------------------ tail (wave 0 only) */
    if (wid != 0) return;
    /* LSum := LSum + LVals[LI], left to right in binary32 (:2798), every
     * lane on the same broadcast LDS reads; the padding adds +0, which
     * leaves a non-negative sum unchanged */
    float lsum = 0.0f;
    for (int base = 0; base < npad; base += 64) {
        const float4* src = reinterpret_cast<const float4*>(sh.val + base);
#pragma unroll
        for (int l4 = 0; l4 < 16; ++l4) {
            const float4 x = src[l4];
            lsum = lsum + x.x;
            lsum = lsum + x.y;
            lsum = lsum + x.z;
            lsum = lsum + x.w;
        }
    }
    /* greedy choice: first position of the largest p (p >= 0, so its bits
     * order like the values) */
    uint32_t pbest = 0u;
    int jbest = 0x7FFFFFFF;
    for (int j = lane; j < nsurv; j += 64) {
        const float p = div_cr32(sh.val[j], lsum);                      /* :2800-2801 */
        sh.prob[j] = p;
        if (__float_as_uint(p) > pbest || jbest == 0x7FFFFFFF) {
            pbest = __float_as_uint(p);
            jbest = j;
        }
    }
    const uint32_t pmax = wave_max_u32(jbest == 0x7FFFFFFF ? 0u : pbest); /* :2804-2807 */
    const int jarg =
        (int)wave_min_u32((jbest != 0x7FFFFFFF && pbest == pmax) ? (uint32_t)jbest : 0xFFFFFFFFu);
    __builtin_amdgcn_wave_barrier();
    int chosen = jarg;
    if (T > 0.0f) {                                                     /* :2811-2824 */
        flags |= G4S_FLAG_DREW;
        const float thr = mul_u_p_cr32(u, rp.top_p);
        /* LCum := LCum + LVals[LI] left to right (broadcast LDS reads as
         * for LSum); every running sum goes back to LDS (the e values are no
         * longer needed), then lane l reads the one after term base + l and
         * one ballot finds the first that reaches thr (a +0 padding term
         * leaves the sum unchanged, so it never reaches thr first) */
        float cum = 0.0f;
        int hit = -1;
        __builtin_amdgcn_wave_barrier();
        for (int base = 0; base < npad; base += 64) {
            const float4* src = reinterpret_cast<const float4*>(sh.prob + base);
            float4* dst = reinterpret_cast<float4*>(sh.val + base);
#pragma unroll
            for (int l4 = 0; l4 < 16; ++l4) {
                const float4 x = src[l4];
                float4 c;
                cum = cum + x.x;
                c.x = cum;
                cum = cum + x.y;
                c.y = cum;
                cum = cum + x.z;
                c.z = cum;
                cum = cum + x.w;
                c.w = cum;
                dst[l4] = c; /* the same value from every lane */
            }
            __builtin_amdgcn_wave_barrier();
            const uint64_t reach = __ballot(sh.val[base + lane] >= thr);
            if (reach) {
                hit = base + (int)__builtin_ctzll(reach);
                break;
            }
        }
        if (hit >= 0) {
            chosen = hit;
            flags |= G4S_FLAG_REACHED;
        }
    }
    if (lane == 0) {
        st_sys(&a.ids[row], (int32_t)cand_idx_of(sh.sorted[chosen]));   /* :2826 */
        if (a.out.count) a.out.count[row] = nsurv;
        if (a.out.argmax) a.out.argmax[row] = (int32_t)cand_idx_of(sh.sorted[jarg]);
        if (a.out.lsum) a.out.lsum[row] = lsum;
        if (a.out.flags) st_sys(&a.out.flags[row], flags);
    }
    if (a.out.indices || a.out.probs) {
        const int capn = a.out.capacity < nsurv ? a.out.capacity : nsurv;
        for (int j = lane; j < capn; j += 64) {
            if (a.out.indices)
                a.out.indices[(int64_t)row * a.out.capacity + j] = (int32_t)cand_idx_of(sh.sorted[j]);
            if (a.out.probs) a.out.probs[(int64_t)row * a.out.capacity + j] = sh.prob[j];
        }
    }
    publish_done(a.done, row, a.seq);
}

/* ------------------------------------- candidates from 64-row group maxima */

/* regs_radix_kth over the top DIGITS bytes only, with a wave-aggregated
 * update of the wave's first digit.  The result is the k-th largest key with
 * its lower bytes cleared: a lower bound of it that at least k keys reach.
 * The group maxima of a row mostly share their leading digit, and LDS
 * atomics to one address serialize, so the lanes holding the first active
 * lane's digit add their count with one atomic; the other lanes (spread over
 * many digits in the later pass) add theirs directly. */
template <int BLOCK, int ITEMS, int DIGITS>
__device__ uint32_t regs_radix_kth_agg(const uint32_t (&keys)[ITEMS], int k, uint32_t* s_hist,
                                       int* s_misc)
{
    const int tid = threadIdx.x, lane = tid & 63;
    uint32_t prefix = 0, mask = 0;
    for (int shift = 24; shift >= 32 - 8 * DIGITS; shift -= 8) {
        for (int b = tid; b < 256; b += BLOCK) s_hist[b] = 0;
        __syncthreads();
#pragma unroll
        for (int q = 0; q < ITEMS; ++q) {
            const uint32_t v = keys[q];
            const bool act = v != 0u && (v & mask) == prefix;
            const uint32_t d = (v >> shift) & 255u;
            const uint64_t left = __ballot(act);
            if (left) {
                const int leader = __builtin_ctzll(left);
                const uint32_t ld = (uint32_t)__builtin_amdgcn_readlane((int)d, leader);
                const bool same = act && d == ld;
                const uint64_t m = __ballot(same);
                if (lane == leader) atomicAdd(&s_hist[ld], (uint32_t)__popcll(m));
                if (act && !same) atomicAdd(&s_hist[d], 1u);
            }
        }
        __syncthreads();
        radix_digit_step(k, s_hist, s_misc);
        __syncthreads();
        k -= s_misc[1];
        prefix |= (uint32_t)s_misc[0] << shift;
        mask |= 255u << shift;
        __syncthreads();
    }
    return prefix;
}

/* The top-k candidates of rows whose logits come from the tiled LM head,
 * which also leaves each 64-logit group's summary (gsum_pack: its largest
 * candidate key, that key's row, a bound of the others).  tau0 is the K-th
 * largest group maximum with its low 16 bits cleared (1 when at most K
 * groups hold a key): K groups hold a key >= tau0, so tau0 is at most the
 * row's K-th largest key, and every key >= tau0 lies in a group whose
 * maximum is >= tau0.  Those groups (about K of them) give the merge's
 * candidates, laid out as the chunk launch would leave them: slot i of the
 * row belongs to chunk i >> cap_log2, every chunk's record carries tau0 as
 * its bound, and the per-wave bounds are 0 (no information).
 *  - with the logits written, a candidate group's keys >= tau0 are read back;
 *    when they outnumber the row's slots (heavy ties), the row is written
 *    as one exact chunk record instead: the keys above the row's K-th largest
 *    key tau and the first min(copies, K) copies of tau in index order, as
 *    the chunk launch's exact select does;
 *  - without them, a candidate group whose other keys are all below tau0
 *    (by the summary's bound) gives its maximum; any other candidate group
 *    becomes a recompute job: its 64 logits are recomputed for this row
 *    (group_logits_kernel) into 64 slots after the maxima.  Too many jobs,
 *    or candidates beyond the slots, mark the row kRecNeedRow.
 * The merge launch (mode 2) then runs unchanged. */
constexpr int kGcBlock = 1024;
constexpr int kGcItems = 8; /* group maxima per thread: up to 8192 groups */
constexpr int kGcLoads = 8; /* candidate groups per wave whose logits are loaded together */

__global__ __launch_bounds__(kGcBlock) void group_cand_kernel(TopkArgs a, const uint64_t* gsum,
                                                              int32_t ngroups, int32_t nwave)
{
    __shared__ uint32_t s_hist[256];
    __shared__ int s_misc[8];
    __shared__ int s_scan[kGcBlock / 64];
    __shared__ int s_list[kGcBlock * kGcItems];
    __shared__ int s_cnt, s_njob;
    __shared__ int s_jobs[kGcMaxJobs];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    constexpr int NW = kGcBlock / 64;
    const int row = blockIdx.x;
    const g4s_params rp = a.params ? a.params[row] : a.p0;
    const int K = rp.top_k;
    int32_t* jobs = a.gc_jobs ? a.gc_jobs + (int64_t)row * kGcJobStride : nullptr;
    if (!(K >= 1 && K < a.vocab) || K > a.kbound) {
        if (tid == 0 && jobs) jobs[0] = 0;
        return; /* the merge launch flags the row */
    }
    const float* lg = a.logits ? reinterpret_cast<const float*>(a.logits) + (int64_t)row * a.row_stride
                               : nullptr;
    const uint64_t* gs = gsum + (int64_t)row * ngroups;
    const int S = a.splits;
    const int cap = 1 << a.cap_log2;
    const int slots = S << a.cap_log2;
    uint64_t* rc = a.cand + (int64_t)row * kCandRow;
    ChunkRec* recs = a.recs + (int64_t)row * kMaxSplits;
    if (tid == 0) {
        s_cnt = 0;
        s_njob = 0;
    }

    /* thread t holds groups kGcItems*t .. +kGcItems-1 */
    uint32_t keys[kGcItems];
    int nz = 0;
#pragma unroll
    for (int q = 0; q < kGcItems; ++q) {
        const int g = tid * kGcItems + q;
        keys[q] = g < ngroups ? gsum_key(gs[g]) : 0u;
        nz += keys[q] != 0u;
    }
    nz = block_sum_i32<kGcBlock>(nz, s_scan);
    uint32_t tau0 = 1u;
    if (nz > K) {
        /* two bytes: the K-th largest group maximum to 7 mantissa bits; the
         * few groups between it and the cleared bound are read back too */
        tau0 = regs_radix_kth_agg<kGcBlock, kGcItems, 2>(keys, K, s_hist, s_misc);
        tau0 = tau0 > 1u ? tau0 : 1u;
    }
    /* the candidate groups, ascending */
    int ng;
    {
        int f = 0;
#pragma unroll
        for (int q = 0; q < kGcItems; ++q) f += keys[q] >= tau0 ? 1 : 0;
        int pos = block_exclusive_scan<kGcBlock>(f, s_scan, ng);
#pragma unroll
        for (int q = 0; q < kGcItems; ++q)
            if (keys[q] >= tau0) s_list[pos++] = tid * kGcItems + q;
    }
    __syncthreads();
    if (!lg) {
        /* no logits: a candidate group's maximum, or a recompute job */
        for (int t = tid; t < ng; t += kGcBlock) {
            const int g = s_list[t];
            const uint64_t sm = gs[g];
            if (gsum_bound2(sm) >= tau0) {
                const int j = atomicAdd(&s_njob, 1);
                if (j < kGcMaxJobs) s_jobs[j] = g;
            } else {
                const int pos = atomicAdd(&s_cnt, 1);
                if (pos < slots)
                    rc[pos] = cand_pack(gsum_key(sm), (uint32_t)(g * 64) + gsum_row(sm));
            }
        }
        __syncthreads();
        const int nmax = s_cnt, njob = s_njob;
        const int M0 = nmax + 64 * njob;
        const bool need_row = njob > kGcMaxJobs || M0 > slots;
        if (tid == 0) {
            jobs[0] = need_row ? 0 : njob;
            jobs[1] = nmax;
        }
        if (!need_row)
            for (int j = tid; j < njob; j += kGcBlock) jobs[2 + j] = s_jobs[j];
        for (int i = tid; i < nwave && i < kWaveBounds; i += kGcBlock)
            a.wbounds[(int64_t)row * kWaveBounds + i] = 0u;
        for (int c = tid; c < S; c += kGcBlock) {
            const int n = M0 - c * cap;
            const int cnt = need_row ? 0 : (n < 0 ? 0 : (n > cap ? cap : n));
            recs[c] = ChunkRec{(uint32_t)cnt, cnt > 0 ? tau0 : 1u,
                               (need_row && c == 0) ? kRecNeedRow : 0u, 0u};
        }
        return;
    }
    /* their keys >= tau0, one group per wave at a time (lane = logit) */
    const auto gkey = [&](int g) -> uint32_t {
        const int64_t i = (int64_t)g * 64 + lane;
        return i < a.vocab ? cand_key(lg[i]) : 0u;
    };
    /* kGcLoads groups per wave per round: their loads are issued together */
    for (int t0 = 0; t0 < ng; t0 += NW * kGcLoads) {
        uint32_t k[kGcLoads];
        int g[kGcLoads];
#pragma unroll
        for (int j = 0; j < kGcLoads; ++j) {
            const int t = t0 + wid + NW * j;
            g[j] = t < ng ? s_list[t] : -1;
            k[j] = g[j] >= 0 ? gkey(g[j]) : 0u;
        }
#pragma unroll
        for (int j = 0; j < kGcLoads; ++j) {
            const bool c = g[j] >= 0 && k[j] >= tau0;
            const uint64_t m = __ballot(c);
            if (m == 0ull) continue; /* wave-uniform */
            int base = 0;
            if (lane == 0) base = atomicAdd(&s_cnt, __popcll(m));
            base = __builtin_amdgcn_readfirstlane(base);
            const int pos = base + __popcll(m & ((1ull << lane) - 1ull));
            if (c && pos < slots) rc[pos] = cand_pack(k[j], (uint32_t)(g[j] * 64 + lane));
        }
    }
    __syncthreads();
    const int M0 = s_cnt;
    for (int i = tid; i < nwave && i < kWaveBounds; i += kGcBlock)
        a.wbounds[(int64_t)row * kWaveBounds + i] = 0u;
    if (M0 <= slots) {
        for (int c = tid; c < S; c += kGcBlock) {
            const int n = M0 - c * cap;
            const int cnt = n < 0 ? 0 : (n > cap ? cap : n);
            recs[c] = ChunkRec{(uint32_t)cnt, cnt > 0 ? tau0 : 1u, 0u, 0u};
        }
        return;
    }
    /* heavy ties: the row's K-th largest key over the candidate groups (M0 >
     * slots >= 2K keys >= tau0 hold it) */
    int gt, eq;
    const uint32_t tau = block_radix_kth<kGcBlock>(
        ng * 64, K,
        [&](int i) -> uint32_t {
            const int64_t e = (int64_t)s_list[i >> 6] * 64 + (i & 63);
            return e < a.vocab ? cand_key(lg[e]) : 0u;
        },
        [&](int) { return true; }, s_hist, s_misc, &gt, &eq);
    /* keys above tau (fewer than K), any order */
    if (tid == 0) s_cnt = 0;
    __syncthreads();
    for (int t = wid; t < ng; t += NW) {
        const int g = s_list[t];
        const uint32_t k = gkey(g);
        const bool c = k > tau;
        const uint64_t m = __ballot(c);
        int base = 0;
        if (lane == 0 && m) base = atomicAdd(&s_cnt, __popcll(m));
        base = __builtin_amdgcn_readfirstlane(base);
        if (c) rc[base + __popcll(m & ((1ull << lane) - 1ull))] = cand_pack(k, (uint32_t)(g * 64 + lane));
    }
    /* the first min(eq, K) copies of tau in index order: NW groups per step,
     * in list order */
    const int want = eq < K ? eq : K;
    int taken = 0;
    for (int t0 = 0; t0 < ng && taken < want; t0 += NW) {
        const int t = t0 + wid;
        const int g = t < ng ? s_list[t] : 0;
        const bool c = t < ng && gkey(g) == tau;
        const uint64_t m = __ballot(c);
        if (lane == 0) s_scan[wid] = __popcll(m);
        __syncthreads();
        int off = 0, tot = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            off += w < wid ? s_scan[w] : 0;
            tot += s_scan[w];
        }
        const int r = taken + off + __popcll(m & ((1ull << lane) - 1ull));
        if (c && r < want) rc[gt + r] = cand_pack(tau, (uint32_t)(g * 64 + lane));
        taken += tot;
        __syncthreads();
    }
    for (int c = tid; c < S; c += kGcBlock)
        recs[c] = c == 0 ? ChunkRec{(uint32_t)(gt + want), tau, 0u, 0x80000000u | (uint32_t)eq}
                         : ChunkRec{0u, 1u, 0u, 0u};
}

/* The recompute jobs of group_cand_kernel (fused LM head without logits):
 * one workgroup per job computes the group's 64 logits for the row's hidden
 * vector in the LM head's term order (one fma per term, block after block,
 * column order; bit-exact with the logits it did not write) and leaves them
 * as candidates in the job's 64 slots; a row past the vocabulary gets key 0,
 * which the merge drops with every key below tau0.  Each logit is one chain
 * of dependent fmas and a single wave issues about one instruction per
 * 2 ns, so one wave (lane = the group's row) runs the chains while three
 * others, one per SIMD, dequantize the next blocks into LDS: per term the
 * chain wave issues one fma and half an LDS read (the next block's reads
 * issued before the current block's fmas), instead of the dequantization's
 * three instructions per weight. */
constexpr int kGlBlocks = 3;                       /* weight blocks per stage */
constexpr int kGlStride = 36;                      /* floats per row of a staged block */
constexpr int kGlBlockF = 64 * kGlStride + 32;     /* a staged block: weights, then x */
constexpr int kGlAhead = 8;                        /* stages of tile loads in flight */
constexpr int kGlProd = 192;                       /* producer threads (three waves) */
constexpr int kGlThreads = 64 + kGlProd;
constexpr int kGlItems = kGlBlocks * 128 / kGlProd; /* (block, row, half) items per producer */
static_assert(kGlItems * kGlProd == kGlBlocks * 128, "whole items per producer thread");
static_assert(8 * kGlBlocks <= kGlProd, "x staging threads");

template <int NST>
__global__ __launch_bounds__(kGlThreads) void group_logits_kernel(TopkArgs a)
{
    __shared__ __align__(16) float s_w[2][kGlBlocks][kGlBlockF];
    __shared__ float4 s_xsink[64];
    const int row = blockIdx.y, j = blockIdx.x;
    const int32_t* jobs = a.gc_jobs + (int64_t)row * kGcJobStride;
    const int njob = jobs[0];
    if (j >= njob) return;
    const int g = jobs[2 + j];
    const int base = jobs[1] + 64 * j;
    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    const int32_t nblk = a.lm_cols / 32;
    const int32_t nst = NST > 0 ? NST : (nblk + kGlBlocks - 1) / kGlBlocks;
    const uint8_t* gt = a.lm_tiles + (int64_t)g * nblk * kQ4TileBytes;
    const float* hx = a.lm_hidden + (int64_t)row * a.lm_cols;
    /* producer thread p, item q: item i = p + q * kGlProd of the stage is
     * block i >> 7, row (i >> 1) & 63, bytes 8 (i & 1) .. +7 of its nibbles
     * (columns 16 (i & 1) .. +15); p < 8 * kGlBlocks also stages the x
     * values of block p >> 3, columns 4 (p & 7) .. +3 (the others load them
     * too, unused, so that the loads stay unconditional) */
    const int p = tid - 64;
    const int px = p < 8 * kGlBlocks ? p : 0;
    float rsc[kGlAhead][kGlItems];
    uint32_t rq0[kGlAhead][kGlItems], rq1[kGlAhead][kGlItems];
    float rx[kGlAhead][4];
    /* the ring slot is a template argument, so that the ring stays in
     * registers */
    const auto load_stage = [&]<int SLOT>(std::integral_constant<int, SLOT>, int32_t st) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < kGlItems; ++q) {
            const int it = p + q * kGlProd;
            int32_t k = st * kGlBlocks + (it >> 7);
            k = k < nblk ? k : nblk - 1;
            const uint8_t* tile = gt + (int64_t)k * kQ4TileBytes;
            rsc[SLOT][q] = reinterpret_cast<const float*>(tile)[(it >> 1) & 63];
            const uint2 w = *reinterpret_cast<const uint2*>(tile + kQ4TileRows * 4 +
                                                           ((it >> 1) & 63) * 16 + (it & 1) * 8);
            rq0[SLOT][q] = w.x;
            rq1[SLOT][q] = w.y;
        }
        int32_t kx = st * kGlBlocks + (px >> 3);
        kx = kx < nblk ? kx : nblk - 1;
        const float4 xv = reinterpret_cast<const float4*>(hx + 32 * kx)[px & 7];
        rx[SLOT][0] = xv.x;
        rx[SLOT][1] = xv.y;
        rx[SLOT][2] = xv.z;
        rx[SLOT][3] = xv.w;
    };
    const auto produce = [&]<int SLOT>(std::integral_constant<int, SLOT>, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < kGlItems; ++q) {
            const int it = p + q * kGlProd;
            const float sc = rsc[SLOT][q];
            const float m8 = -8.0f * sc;
            const uint32_t ws[2] = {rq0[SLOT][q], rq1[SLOT][q]};
            float w[16];
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                const uint32_t lo = ws[d] & 0x0F0F0F0Fu, hi = (ws[d] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    w[8 * d + 2 * i] = __builtin_fmaf((float)((lo >> (8 * i)) & 0xFFu), sc, m8);
                    w[8 * d + 2 * i + 1] = __builtin_fmaf((float)((hi >> (8 * i)) & 0xFFu), sc, m8);
                }
            }
            float4* dst = reinterpret_cast<float4*>(
                &s_w[buf][it >> 7][((it >> 1) & 63) * kGlStride + (it & 1) * 16]);
#pragma unroll
            for (int c = 0; c < 4; ++c)
                dst[c] = make_float4(w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]);
        }
        /* every producer stores its x values: those past the stage's blocks
         * into slots nobody reads (no branch around the ring register) */
        float4* xd = p < 8 * kGlBlocks
                         ? reinterpret_cast<float4*>(&s_w[buf][p >> 3][64 * kGlStride]) + (p & 7)
                         : &s_xsink[p & 63];
        *xd = make_float4(rx[SLOT][0], rx[SLOT][1], rx[SLOT][2], rx[SLOT][3]);
    };
    float S = 0.0f;
    /* the chain over one stage; block b + 1's operands are read from LDS
     * before block b's fmas */
    const auto consume = [&](int32_t st, int buf) __attribute__((always_inline)) {
        float4 w0[8], w1[8], x0[8], x1[8];
        const auto ld = [&](int b, float4 (&wv)[8], float4 (&xv)[8]) __attribute__((always_inline)) {
            const float4* wr = reinterpret_cast<const float4*>(&s_w[buf][b][lane * kGlStride]);
            const float4* xr = reinterpret_cast<const float4*>(&s_w[buf][b][64 * kGlStride]);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                wv[c] = wr[c];
                xv[c] = xr[c];
            }
        };
        const auto chain = [&](const float4 (&wv)[8], const float4 (&xv)[8]) __attribute__((always_inline)) {
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                S = __builtin_fmaf(xv[c].x, wv[c].x, S);
                S = __builtin_fmaf(xv[c].y, wv[c].y, S);
                S = __builtin_fmaf(xv[c].z, wv[c].z, S);
                S = __builtin_fmaf(xv[c].w, wv[c].w, S);
            }
        };
        ld(0, w0, x0);
#pragma unroll
        for (int b = 0; b < kGlBlocks; ++b) {
            if (st * kGlBlocks + b < nblk) { /* uniform */
                if (b % 2 == 0) {
                    if (b + 1 < kGlBlocks) ld(b + 1, w1, x1);
                    chain(w0, x0);
                } else {
                    if (b + 1 < kGlBlocks) ld(b + 1, w0, x0);
                    chain(w1, x1);
                }
            }
        }
    };
    const auto clamp_st = [&](int32_t st) __attribute__((always_inline)) { return st < nst ? st : nst - 1; };
    /* prologue: stages 0 .. kGlAhead-1 in flight, stage 0 staged */
    if (wid > 0) {
        [&]<int... I>(std::integer_sequence<int, I...>) {
            (load_stage(std::integral_constant<int, I>{}, clamp_st(I)), ...);
        }(std::make_integer_sequence<int, kGlAhead>{});
        produce(std::integral_constant<int, 0>{}, 0);
        load_stage(std::integral_constant<int, 0>{}, clamp_st(kGlAhead));
    }
    __syncthreads();
    /* stage st = s0 + I: the chain wave takes buffer st & 1 (= I & 1, s0
     * being a multiple of kGlAhead); the producers stage st + 1 from ring
     * slot (st + 1) mod kGlAhead into the other buffer and refill that
     * slot with stage st + 1 + kGlAhead */
    const auto step = [&]<int I>(std::integral_constant<int, I>, int32_t s0) __attribute__((always_inline)) {
        const int32_t st = s0 + I;
        if (st >= nst) return; /* uniform */
        if (wid == 0) {
            consume(st, I & 1);
        } else if (st + 1 < nst) {
            constexpr int kSlot = (I + 1) % kGlAhead;
            produce(std::integral_constant<int, kSlot>{}, (I + 1) & 1);
            load_stage(std::integral_constant<int, kSlot>{}, clamp_st(st + 1 + kGlAhead));
        }
        __syncthreads();
    };
    if constexpr (NST > 0) {
        /* every stage in straight-line code: the compiler then knows which
         * loads are still in flight at each use and waits for those only
         * (across a loop's back edge it waits for nearly all of them) */
        [&]<int... J>(std::integer_sequence<int, J...>) {
            (step(std::integral_constant<int, J % kGlAhead>{}, J - J % kGlAhead), ...);
        }(std::make_integer_sequence<int, NST>{});
    } else {
        for (int32_t s0 = 0; s0 < nst; s0 += kGlAhead) {
            [&]<int... I>(std::integer_sequence<int, I...>) {
                (step(std::integral_constant<int, I>{}, s0), ...);
            }(std::make_integer_sequence<int, kGlAhead>{});
        }
    }
    if (wid == 0) {
        const int64_t idx = (int64_t)g * 64 + lane;
        const uint32_t key = idx < a.vocab ? cand_key(S) : 0u;
        a.cand[(int64_t)row * kCandRow + base + lane] = cand_pack(key, (uint32_t)idx);
    }
}
static_assert(kGlAhead % 2 == 0, "buffers alternate with the unrolled stage index");

/* ---------------------------------------------------------------- launch */

template <int BLOCK, int ITEMS, int DT>
static hipError_t launch_one(const TopkArgs& a, int kcap, hipStream_t s)
{
    dim3 grid(a.mode == 2 ? 1u : (unsigned)a.splits, (unsigned)a.batch);
    if constexpr (BLOCK < 1024) {
        (void)kcap;
        hipLaunchKernelGGL((topk_kernel<BLOCK, ITEMS, DT, 64>), grid, dim3(BLOCK), 0, s, a);
    } else {
        if (kcap <= 64)
            hipLaunchKernelGGL((topk_kernel<BLOCK, ITEMS, DT, 64>), grid, dim3(BLOCK), 0, s, a);
        else if (kcap <= 256)
            hipLaunchKernelGGL((topk_kernel<BLOCK, ITEMS, DT, 256>), grid, dim3(BLOCK), 0, s, a);
        else
            hipLaunchKernelGGL((topk_kernel<BLOCK, ITEMS, DT, 1024>), grid, dim3(BLOCK), 0, s, a);
    }
    return hipGetLastError();
}

template <int BLOCK, int ITEMS, int DT>
static hipError_t launch_cfg(const TopkArgs& a, int kcap, hipStream_t s, int32_t ncu)
{
    if (ncu <= 0 || (int64_t)a.batch * a.splits * BLOCK <= (int64_t)ncu * 1024)
        return launch_one<BLOCK, ITEMS, DT>(a, kcap, s);
    TopkArgs b = a;
    b.mode = 1;
    hipError_t e = launch_one<BLOCK, ITEMS, DT>(b, kcap, s);
    if (e != hipSuccess) return e;
    b.mode = 2;
    return launch_one<BLOCK, ITEMS, DT>(b, kcap, s);
}

/* Launch shape: 512 x 16 for K bounds up to 64 (eight waves per 8192-term
 * chunk), 1024 x 32 above; twice the items per thread when the vocabulary
 * needs more than kMaxSplits chunks.  Slots per chunk: 4 x kbound (at least
 * 128) when the workspace holds them, else 2 x kbound (>= 2 x kbound keeps a
 * chunk's candidates >= theta within its slots except under heavy ties; 4 x
 * also covers the spread of theta when K is near kbound, and the floor the
 * several waves' candidates when K is small). */
TopkConfig topk_plan(int32_t vocab, int32_t kbound)
{
    struct Shape {
        int block, items;
    };
    static constexpr Shape kSmallK[3] = {{512, 16}, {1024, 32}, {1024, 64}};
    static constexpr Shape kLargeK[2] = {{1024, 32}, {1024, 64}};
    const Shape* shapes = kbound <= 64 ? kSmallK : kLargeK;
    const int nshape = kbound <= 64 ? 3 : 2;
    TopkConfig c{};
    c.ok = false;
    for (int mult = 4; mult >= 2 && !c.ok; mult -= 2) {
        /* at least 128 slots: with a small K the chunk bound is the least of
         * the waves' own bounds, so every wave contributes candidates */
        c.cap_log2 = 7;
        while ((1 << c.cap_log2) < mult * kbound) ++c.cap_log2;
        for (int i = 0; i < nshape && !c.ok; ++i) {
            c.block = shapes[i].block;
            c.items = shapes[i].items;
            c.chunk = c.block * c.items;
            c.splits = (vocab + c.chunk - 1) / c.chunk;
            c.ok = ((c.splits << c.cap_log2) <= kCandRow) && (c.splits <= kMaxSplits) &&
                   (1 << c.cap_log2) <= kMergeLds;
        }
    }
    return c;
}

hipError_t topk_groups_launch(const TopkConfig& c, const TopkArgs& a, const uint64_t* gsum,
                              int32_t ngroups, hipStream_t s)
{
    if (ngroups > kGcBlock * kGcItems) return hipErrorNotSupported;
    /* two chunks' slots (>= 8 x kbound) hold the candidates of all but
     * heavily tied rows, which take the exact record; the merge then loads
     * only those slots.  Without logits, four chunks' slots: the groups'
     * maxima and 64 slots per recompute job. */
    TopkArgs b = a;
    const int smax = a.logits ? 2 : 4;
    b.splits = c.splits < smax ? c.splits : smax;
    hipLaunchKernelGGL(group_cand_kernel, dim3((unsigned)a.batch), dim3(kGcBlock), 0, s, b, gsum,
                       ngroups, (int32_t)(b.splits * (c.block / 64)));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (!a.logits) {
        /* straight-line instantiations for hidden sizes 1536, 2048, 2560, 3072
         * and 4096; a loop otherwise */
        const dim3 grid((unsigned)kGcMaxJobs, (unsigned)a.batch);
        constexpr int kS = 32 * kGlBlocks; /* columns per stage */
        switch ((a.lm_cols + kS - 1) / kS) {
        case (1536 + kS - 1) / kS: hipLaunchKernelGGL(group_logits_kernel<(1536 + kS - 1) / kS>, grid, dim3(kGlThreads), 0, s, b); break;
        case (2048 + kS - 1) / kS: hipLaunchKernelGGL(group_logits_kernel<(2048 + kS - 1) / kS>, grid, dim3(kGlThreads), 0, s, b); break;
        case (2560 + kS - 1) / kS: hipLaunchKernelGGL(group_logits_kernel<(2560 + kS - 1) / kS>, grid, dim3(kGlThreads), 0, s, b); break;
        case (3072 + kS - 1) / kS: hipLaunchKernelGGL(group_logits_kernel<(3072 + kS - 1) / kS>, grid, dim3(kGlThreads), 0, s, b); break;
        case (4096 + kS - 1) / kS: hipLaunchKernelGGL(group_logits_kernel<(4096 + kS - 1) / kS>, grid, dim3(kGlThreads), 0, s, b); break;
        default: hipLaunchKernelGGL(group_logits_kernel<0>, grid, dim3(kGlThreads), 0, s, b); break;
        }
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    b.mode = 2;
    if (c.block == 512 && c.items == 16) return launch_one<512, 16, 0>(b, a.kbound, s);
    if (c.block == 1024 && c.items == 32) return launch_one<1024, 32, 0>(b, a.kbound, s);
    return launch_one<1024, 64, 0>(b, a.kbound, s);
}

hipError_t topk_launch(const TopkConfig& c, const TopkArgs& a, int dtype, hipStream_t s,
                       int32_t ncu)
{
    if (decode_eligible(a, dtype)) return decode_launch(a, dtype, s);
    const int kc = a.kbound;
    if (dtype == G4S_DTYPE_F32) {
        if (c.block == 512 && c.items == 16) return launch_cfg<512, 16, 0>(a, kc, s, ncu);
        if (c.block == 1024 && c.items == 32) return launch_cfg<1024, 32, 0>(a, kc, s, ncu);
        return launch_cfg<1024, 64, 0>(a, kc, s, ncu);
    }
    if (c.block == 512 && c.items == 16) return launch_cfg<512, 16, 1>(a, kc, s, ncu);
    if (c.block == 1024 && c.items == 32) return launch_cfg<1024, 32, 1>(a, kc, s, ncu);
    return launch_cfg<1024, 64, 1>(a, kc, s, ncu);
}

}  // namespace g4s
