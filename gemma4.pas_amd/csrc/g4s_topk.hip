/*
 * g4s_topk.hip -- the top-k sampling path on gfx950 (rows with 0 < TopK < V).
 *
 * Replaces DoSelectTopKIndices + the top-k branch of DoSample
 * (src/Gemma4.Model.pas:2615-2689, 2765-2826).  One kernel launch per batch:
 *
 *  phase 1 (grid = splits x rows, one workgroup per vocabulary chunk)
 *    - 16-byte loads of the chunk into registers as order-preserving keys;
 *    - a provable lower bound theta of the chunk's K-th largest key: each
 *      wave takes the ceil(K/waves)-th largest of its per-thread maxima
 *      (ballot binary search) and the block keeps the minimum;
 *    - every key >= theta is a candidate (a superset of the chunk's top-K);
 *      if more than 2K qualify (heavy ties), an exact per-chunk radix select
 *      emits the keys above the chunk's K-th value plus its first K copies
 *      in index order;
 *    - rc = the ceil(K/splits)-th largest key of the chunk: min over chunks
 *      of rc is a second lower bound of the row's K-th largest;
 *    - candidates and the chunk record go to the HBM workspace, then an
 *      atomic ticket elects the last workgroup of the row.
 *  merge + tail (last workgroup of each row)
 *    - keeps candidates >= max(bounds) (typically ~K..2K of them), selects
 *      the exact K-th value tau, resolves ties at tau like the reference's
 *      min-heap (lowest index when the heap layout cannot matter, a full
 *      heap replay otherwise), sorts the survivors by vocab index;
 *    - wave 0 runs the reference's tail in index order: softcap, 1/T,
 *      max, exp, sequential binary32 LSum, division, argmax, sequential
 *      running sum against fl32(u*TopP).
 */
#include "g4s_topk.h"

namespace g4s {

using namespace g4s::cr;

namespace {

struct TopkShared {
    /* phase 1 */
    uint32_t wtheta[16];
    int scan[16];
    uint32_t red[16];
    int misc[8];
    uint32_t hist[256];
    /* merge */
    ChunkRec rec[kMaxSplits];
    uint32_t mkey[kMergeLds]; /* phase-1 emission buffer, then merge candidates */
    uint32_t midx[kMergeLds];
    uint32_t skey[kMaxTopK]; /* survivors (unsorted), heap values during a replay */
    int32_t sidx[kMaxTopK];
    uint32_t tkey[kMaxTopK]; /* survivors sorted by index */
    int32_t tidx[kMaxTopK];
    float val[kMaxTopK];     /* tail: v, then e, then p */
    float prob[kMaxTopK];
    int flag_last;
};

/* ------------------------------------------------------------ heap replay */

/* Exact replay of the reference's min-heap pass (Model.pas:2632-2664) over a
 * whole row, for rows whose K-th value is tied in a way the heap layout
 * decides.  Elements are screened in tiles against the current root; the
 * screened ones (in index order) are inserted by one lane.  Returns the heap
 * size in use (entries with index >= 0 are the survivors). */
template <int BLOCK, int DT>
__device__ int heap_replay(const char* row, int vocab, int K, TopkShared& sh)
{
    float* hv = reinterpret_cast<float*>(sh.skey);
    int32_t* hi = sh.sidx;
    float* qv = reinterpret_cast<float*>(sh.mkey);
    int32_t* qi = reinterpret_cast<int32_t*>(sh.midx);
    const int tid = threadIdx.x;
    for (int i = tid; i < K; i += BLOCK) {
        hv[i] = -1e30f;
        hi[i] = -1;
    }
    __syncthreads();
    for (int base = 0; base < vocab; base += BLOCK) {
        int e = base + tid;
        float x = (e < vocab) ? load_elem<DT>(row, e) : 0.0f;
        float root = hv[0];
        int take = (e < vocab) && !(x <= root);
        int total;
        int pos = block_exclusive_scan<BLOCK>(take, sh.scan, total);
        if (take) {
            qv[pos] = x;
            qi[pos] = e;
        }
        __syncthreads();
        if (tid == 0) {
            for (int q = 0; q < total; ++q) {
                float v = qv[q];
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
    return K;
}

/* Rank-by-count k-th largest over an LDS/global array (n <= kRankMax). */
template <int BLOCK, typename KeyF>
__device__ uint32_t rank_kth(int n, int k, KeyF key, int* s_misc, int* gt, int* eq)
{
    const int tid = threadIdx.x;
    for (int i = tid; i < n; i += BLOCK) {
        uint32_t ki = key(i);
        int g = 0, q = 0;
        for (int j = 0; j < n; ++j) {
            uint32_t kj = key(j);
            g += kj > ki;
            q += kj == ki;
        }
        if (g < k && k <= g + q) {
            s_misc[4] = (int)ki; /* all writers agree */
            s_misc[5] = g;
            s_misc[6] = q;
        }
    }
    __syncthreads();
    uint32_t r = (uint32_t)s_misc[4];
    *gt = s_misc[5];
    *eq = s_misc[6];
    __syncthreads();
    return r;
}

}  // namespace

template <int BLOCK, int ITEMS, int DT>
__global__ __launch_bounds__(BLOCK) void topk_kernel(TopkArgs a)
{
    constexpr int VW = Elem<DT>::VW;
    constexpr int NV = ITEMS / VW;
    constexpr int NW = BLOCK / 64;
    constexpr int CHUNK = BLOCK * ITEMS;
    __shared__ TopkShared sh;

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int row = blockIdx.y;
    const int chunk = blockIdx.x;
    const int S = a.splits;
    const int V = a.vocab;

    const g4s_params rp = a.params ? a.params[row] : a.p0;
    const double u = a.u ? a.u[row] : a.u0;
    const int K = rp.top_k;
    if (!(K >= 1 && K < V)) return; /* full-vocabulary row (Model.pas:2756) */
    if (K > a.kbound) {
        if (chunk == 0 && tid == 0) {
            a.ids[row] = -1;
            if (a.out.flags) a.out.flags[row] = G4S_FLAG_ERROR | G4S_FLAG_TOPK_PATH;
        }
        return;
    }

    const char* rowp = reinterpret_cast<const char*>(a.logits) +
                       (int64_t)row * a.row_stride * Elem<DT>::SIZE;
    const int64_t cbase = (int64_t)chunk * CHUNK;
    const int cap_c = a.cap_c;
    uint32_t* gkey = a.cand_key + (int64_t)row * kCandRow + (int64_t)chunk * cap_c;
    uint32_t* gidx = a.cand_idx + (int64_t)row * kCandRow + (int64_t)chunk * cap_c;

    /* ------------------------------------------------------- phase 1 */
    uint32_t keys[ITEMS];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        float v[VW];
        int64_t e0 = cbase + ((int64_t)j * BLOCK + tid) * VW;
        load_vec<DT>(rowp, e0, V, v);
#pragma unroll
        for (int q = 0; q < VW; ++q) keys[j * VW + q] = (e0 + q < V) ? cand_key(v[q]) : 0u;
    }
    uint32_t tmax = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) tmax = keys[i] > tmax ? keys[i] : tmax;
    const int kw = (K + NW - 1) / NW;
    uint32_t wth = (kw <= 64) ? wave_kth_largest(tmax, kw) : 0u;
    if (lane == 0) sh.wtheta[wid] = wth;
    __syncthreads();
    uint32_t theta = 0xFFFFFFFFu;
#pragma unroll
    for (int w = 0; w < NW; ++w) theta = sh.wtheta[w] < theta ? sh.wtheta[w] : theta;
    theta = theta < 1u ? 1u : theta;

    int mine = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) mine += keys[i] >= theta;
    int total;
    int off = block_exclusive_scan<BLOCK>(mine, sh.scan, total);

    uint32_t rec_bound, rec_mode_e;
    int emitted;
    if (total <= cap_c) {
        /* common case: every key >= theta is a candidate */
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int q = 0; q < VW; ++q) {
                uint32_t k = keys[j * VW + q];
                if (k >= theta) {
                    sh.mkey[off] = k;
                    sh.midx[off] = (uint32_t)(cbase + ((int64_t)j * BLOCK + tid) * VW + q);
                    ++off;
                }
            }
        emitted = total;
        rec_bound = theta;
        rec_mode_e = 0;
    } else {
        /* heavy ties or a weak theta: exact K-th largest of the chunk */
        int gt_c, eq_c;
        uint32_t tau_c = regs_radix_kth<BLOCK, ITEMS>(keys, K, sh.hist, sh.misc, &gt_c, &eq_c);
        /* keys strictly above tau_c, any order */
        int gmine = 0;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) gmine += keys[i] > tau_c;
        int gtot;
        int goff = block_exclusive_scan<BLOCK>(gmine, sh.scan, gtot);
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int q = 0; q < VW; ++q) {
                uint32_t k = keys[j * VW + q];
                if (k > tau_c) {
                    sh.mkey[goff] = k;
                    sh.midx[goff] = (uint32_t)(cbase + ((int64_t)j * BLOCK + tid) * VW + q);
                    ++goff;
                }
            }
        /* the first min(eq, K) copies of tau_c in index order: load slot j,
         * then thread, then position within the vector */
        const int want = eq_c < K ? eq_c : K;
        int base = gtot;
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
                    if (taken + r < want) {
                        sh.mkey[base + taken + r] = tau_c;
                        sh.midx[base + taken + r] =
                            (uint32_t)(cbase + ((int64_t)j * BLOCK + tid) * VW + q);
                    }
                    ++r;
                }
            }
            taken += tot_j;
        }
        emitted = gtot + want;
        rec_bound = tau_c;
        rec_mode_e = 0x80000000u | (uint32_t)eq_c;
    }
    __syncthreads();

    /* rc = m-th largest key of the chunk, m = ceil(K / splits) */
    const int m = (K + S - 1) / S;
    uint32_t rc = 0;
    if (emitted >= m) {
        int g, q;
        if (emitted <= kRankMax)
            rc = rank_kth<BLOCK>(emitted, m, [&](int i) { return sh.mkey[i]; }, sh.misc, &g, &q);
        else
            rc = block_radix_kth<BLOCK>(
                emitted, m, [&](int i) { return sh.mkey[i]; }, [&](int) { return true; }, sh.hist,
                sh.misc, &g, &q);
    }
    for (int i = tid; i < emitted; i += BLOCK) {
        gkey[i] = sh.mkey[i];
        gidx[i] = sh.midx[i];
    }
    if (tid == 0) {
        ChunkRec r;
        r.count = (uint32_t)emitted;
        r.bound = rec_bound;
        r.rc = rc;
        r.mode_e = rec_mode_e;
        a.recs[(int64_t)row * kMaxSplits + chunk] = r;
    }

    /* ----------------------------------------------- last workgroup elects */
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        uint32_t prev = atomicAdd(&a.tickets[row], 1u);
        sh.flag_last = (prev == (uint32_t)(S - 1));
    }
    __syncthreads();
    if (!sh.flag_last) return;
    __threadfence();
    if (tid == 0) a.tickets[row] = 0u;

    /* ------------------------------------------------------------ merge */
    uint32_t flags = G4S_FLAG_TOPK_PATH;
    uint32_t lb = 1u, lr = 0xFFFFFFFFu;
    bool any_exact = false;
    for (int c = tid; c < S; c += BLOCK) {
        ChunkRec r = a.recs[(int64_t)row * kMaxSplits + c];
        sh.rec[c] = r;
    }
    __syncthreads();
    {
        uint32_t mb = 1u, mr = 0xFFFFFFFFu;
        int ex = 0;
        for (int c = tid; c < S; c += BLOCK) {
            mb = sh.rec[c].bound > mb ? sh.rec[c].bound : mb;
            mr = sh.rec[c].rc < mr ? sh.rec[c].rc : mr;
            ex |= (sh.rec[c].mode_e >> 31) != 0;
        }
        lb = block_max_u32<BLOCK>(mb, sh.red);
        lr = block_min_u32<BLOCK>(mr, sh.red);
        any_exact = block_sum_i32<BLOCK>(ex, sh.scan) != 0;
    }
    if (any_exact) flags |= G4S_FLAG_CHUNK_EXACT;
    const uint32_t L = lb > lr ? lb : lr;

    /* candidates >= L: count, then gather (LDS when they fit, else HBM) */
    const uint32_t* rkey = a.cand_key + (int64_t)row * kCandRow;
    const uint32_t* ridx = a.cand_idx + (int64_t)row * kCandRow;
    const int span = S * cap_c;
    int cnt = 0;
    for (int f = tid; f < span; f += BLOCK) {
        int c = f / cap_c, p = f - c * cap_c;
        if (p < (int)sh.rec[c].count && rkey[f] >= L) ++cnt;
    }
    int M;
    int moff = block_exclusive_scan<BLOCK>(cnt, sh.scan, M);
    const bool wide = M > kMergeLds;
    uint32_t* mk = wide ? a.merge_key + (int64_t)row * kCandRow : sh.mkey;
    uint32_t* mi = wide ? a.merge_idx + (int64_t)row * kCandRow : sh.midx;
    if (wide) flags |= G4S_FLAG_WIDE_MERGE;
    for (int f = tid; f < span; f += BLOCK) {
        int c = f / cap_c, p = f - c * cap_c;
        if (p < (int)sh.rec[c].count) {
            uint32_t k = rkey[f];
            if (k >= L) {
                mk[moff] = k;
                mi[moff] = ridx[f];
                ++moff;
            }
        }
    }
    __syncthreads();

    /* exact K-th largest among the M candidates */
    int nsurv = 0;
    if (M <= K) {
        /* M < K: fewer than K logits above -1e30 in the whole row; M == K:
         * the candidates are exactly the top K.  Either way all survive. */
        for (int i = tid; i < M; i += BLOCK) {
            sh.skey[i] = mk[i];
            sh.sidx[i] = (int32_t)mi[i];
        }
        nsurv = M;
    } else {
        int G, E;
        uint32_t tau;
        if (M <= kRankMax)
            tau = rank_kth<BLOCK>(M, K, [&](int i) { return mk[i]; }, sh.misc, &G, &E);
        else
            tau = block_radix_kth<BLOCK>(
                M, K, [&](int i) { return mk[i]; }, [&](int) { return true; }, sh.hist, sh.misc,
                &G, &E);
        const int need = K - G;
        /* a chunk whose exact select truncated copies of tau */
        int trunc = 0;
        for (int c = tid; c < S; c += BLOCK) {
            uint32_t me = sh.rec[c].mode_e;
            if ((me >> 31) && sh.rec[c].bound == tau && (int)(me & 0x7FFFFFFFu) > K) trunc = 1;
        }
        trunc = block_sum_i32<BLOCK>(trunc, sh.scan);
        int mode = 0; /* 0: all >= tau survive, 1: lowest-index ties, 2: heap replay */
        int32_t idx_thr = 0x7FFFFFFF;
        if (E != need || trunc) {
            /* t* = index of the K-th element >= tau in index order */
            int g2, e2;
            uint32_t tstar_inv = block_radix_kth<BLOCK>(
                M, K, [&](int i) { return ~mi[i]; }, [&](int i) { return mk[i] >= tau; }, sh.hist,
                sh.misc, &g2, &e2);
            int32_t tstar = (int32_t)~tstar_inv;
            uint32_t mg = 0;
            for (int i = tid; i < M; i += BLOCK)
                if (mk[i] > tau) mg = (mi[i] + 1u) > mg ? (mi[i] + 1u) : mg;
            mg = block_max_u32<BLOCK>(mg, sh.red);
            const int32_t max_gt = (int32_t)mg - 1; /* -1 when nothing is above tau */
            if (max_gt < tstar) {
                mode = 1;
                uint32_t thr_inv = block_radix_kth<BLOCK>(
                    M, need, [&](int i) { return ~mi[i]; }, [&](int i) { return mk[i] == tau; },
                    sh.hist, sh.misc, &g2, &e2);
                idx_thr = (int32_t)~thr_inv;
                flags |= G4S_FLAG_TIE_LOWEST;
            } else {
                mode = 2;
                flags |= G4S_FLAG_HEAP_REPLAY;
            }
        }
        if (mode < 2) {
            int take_n = 0;
            for (int i = tid; i < M; i += BLOCK) {
                uint32_t k = mk[i];
                take_n += (k > tau) || (k == tau && (mode == 0 || (int32_t)mi[i] <= idx_thr));
            }
            int sv;
            int soff = block_exclusive_scan<BLOCK>(take_n, sh.scan, sv);
            for (int i = tid; i < M; i += BLOCK) {
                uint32_t k = mk[i];
                if ((k > tau) || (k == tau && (mode == 0 || (int32_t)mi[i] <= idx_thr))) {
                    sh.skey[soff] = k;
                    sh.sidx[soff] = (int32_t)mi[i];
                    ++soff;
                }
            }
            nsurv = sv;
        } else {
            heap_replay<BLOCK, DT>(rowp, V, K, sh);
            /* the heap holds K entries, all with index >= 0 here (M > K) */
            for (int i = tid; i < K; i += BLOCK) {
                float hv = reinterpret_cast<float*>(sh.skey)[i];
                sh.skey[i] = f2key(hv);
            }
            nsurv = K;
        }
    }
    __syncthreads();

    if (nsurv == 0) {
        if (tid == 0) {
            a.ids[row] = -1;
            if (a.out.flags) a.out.flags[row] = flags | G4S_FLAG_EMPTY;
            if (a.out.count) a.out.count[row] = 0;
        }
        return;
    }

    /* survivors ascending by vocab index (rank by count; indices distinct) */
    for (int i = tid; i < nsurv; i += BLOCK) {
        int32_t my = sh.sidx[i];
        int r = 0;
        for (int j = 0; j < nsurv; ++j) r += sh.sidx[j] < my;
        sh.tidx[r] = my;
        sh.tkey[r] = sh.skey[i];
    }
    __syncthreads();

    /* ------------------------------------------------ tail (wave 0 only) */
    if (wid != 0) return;
    const float cap = a.softcap;
    const float T = rp.temperature;
    const bool scale = (T > 0.0f) && (T != 1.0f);
    const float inv_t = scale ? div_cr32(1.0f, T) : 1.0f;               /* :2782 */
    float vmax = -__builtin_inff();
    for (int j = lane; j < nsurv; j += 64) {
        float x = key2f(sh.tkey[j]);                                    /* :2774 */
        float v = (cap > 0.0f) ? softcap_topk_cr32(x, cap) : x;         /* :2775-2776 */
        if (scale) v = v * inv_t;                                       /* :2783-2784 */
        sh.val[j] = v;
        vmax = v > vmax ? v : vmax;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float w = __shfl_xor(vmax, o, 64);
        vmax = w > vmax ? w : vmax;                                     /* :2789-2792 */
    }
    for (int j = lane; j < nsurv; j += 64) sh.val[j] = exp_diff_cr32(sh.val[j], vmax); /* :2797 */
    __builtin_amdgcn_wave_barrier();
    float lsum = 0.0f;
    if (lane == 0) {
        for (int j = 0; j < nsurv; ++j) lsum = lsum + sh.val[j];        /* :2798 */
    }
    lsum = __shfl(lsum, 0, 64);
    float pbest = -1.0f;
    int jbest = 0x7FFFFFFF;
    for (int j = lane; j < nsurv; j += 64) {
        float p = div_cr32(sh.val[j], lsum);                            /* :2800-2801 */
        sh.prob[j] = p;
        if (p > pbest) {
            pbest = p;
            jbest = j;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {                                  /* :2804-2807 */
        float pw = __shfl_xor(pbest, o, 64);
        int jw = __shfl_xor(jbest, o, 64);
        if (pw > pbest || (pw == pbest && jw < jbest)) {
            pbest = pw;
            jbest = jw;
        }
    }
    __builtin_amdgcn_wave_barrier();
    const int jarg = jbest;
    int chosen = jarg;
    if (T > 0.0f) {                                                     /* :2811-2824 */
        flags |= G4S_FLAG_DREW;
        const float thr = mul_u_p_cr32(u, rp.top_p);
        int hit = -1;
        if (lane == 0) {
            float cum = 0.0f;
            for (int j = 0; j < nsurv; ++j) {
                cum = cum + sh.prob[j];
                if (cum >= thr) {
                    hit = j;
                    break;
                }
            }
        }
        hit = __shfl(hit, 0, 64);
        if (hit >= 0) {
            chosen = hit;
            flags |= G4S_FLAG_REACHED;
        }
    }
    if (lane == 0) {
        a.ids[row] = sh.tidx[chosen];                                   /* :2826 */
        if (a.out.count) a.out.count[row] = nsurv;
        if (a.out.argmax) a.out.argmax[row] = sh.tidx[jarg];
        if (a.out.lsum) a.out.lsum[row] = lsum;
        if (a.out.flags) a.out.flags[row] = flags;
    }
    if (a.out.indices || a.out.probs) {
        const int capn = a.out.capacity < nsurv ? a.out.capacity : nsurv;
        for (int j = lane; j < capn; j += 64) {
            if (a.out.indices) a.out.indices[(int64_t)row * a.out.capacity + j] = sh.tidx[j];
            if (a.out.probs) a.out.probs[(int64_t)row * a.out.capacity + j] = sh.prob[j];
        }
    }
}

/* ---------------------------------------------------------------- launch */

template <int BLOCK, int ITEMS, int DT>
static hipError_t launch_cfg(const TopkArgs& a, hipStream_t s)
{
    dim3 grid((unsigned)a.splits, (unsigned)a.batch);
    hipLaunchKernelGGL((topk_kernel<BLOCK, ITEMS, DT>), grid, dim3(BLOCK), 0, s, a);
    return hipGetLastError();
}

TopkConfig topk_plan(int32_t vocab, int32_t kbound)
{
    TopkConfig c{};
    c.block = kbound <= 64 ? 256 : 1024;
    c.items = 32;
    c.chunk = c.block * c.items;
    c.splits = (vocab + c.chunk - 1) / c.chunk;
    c.cap_c = 2 * kbound;
    if (c.splits * c.cap_c > kCandRow || c.splits > kMaxSplits) {
        c.items = 64;
        c.chunk = c.block * c.items;
        c.splits = (vocab + c.chunk - 1) / c.chunk;
    }
    c.ok = (c.splits * c.cap_c <= kCandRow) && (c.splits <= kMaxSplits);
    return c;
}

hipError_t topk_launch(const TopkConfig& c, const TopkArgs& a, int dtype, hipStream_t s)
{
    if (dtype == G4S_DTYPE_F32) {
        if (c.block == 256 && c.items == 32) return launch_cfg<256, 32, 0>(a, s);
        if (c.block == 256 && c.items == 64) return launch_cfg<256, 64, 0>(a, s);
        if (c.block == 1024 && c.items == 32) return launch_cfg<1024, 32, 0>(a, s);
        return launch_cfg<1024, 64, 0>(a, s);
    }
    if (c.block == 256 && c.items == 32) return launch_cfg<256, 32, 1>(a, s);
    if (c.block == 256 && c.items == 64) return launch_cfg<256, 64, 1>(a, s);
    if (c.block == 1024 && c.items == 32) return launch_cfg<1024, 32, 1>(a, s);
    return launch_cfg<1024, 64, 1>(a, s);
}

}  // namespace g4s
