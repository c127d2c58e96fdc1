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

#include "g4s_fullcore.h"

namespace g4s {

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
                st_sys(&a.ids[row], -1);
                if (a.out.count) a.out.count[row] = 0;
                if (a.out.flags)
                    st_sys(&a.out.flags[row], G4S_FLAG_TOPK_PATH | G4S_FLAG_WIDE_K | G4S_FLAG_EMPTY);
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
    if (e == hipSuccess) e = hipMalloc((void**)&ws.ytab, (size_t)65536 * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.fbrow, mb * sizeof(FbRow));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.etab8, mb * kBfTab * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.ptab8, mb * kBfTab * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.stage, mb * kBfStage * sizeof(BfStage));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.cpost, nc * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&ws.head, mb * kFullChunk * sizeof(float));
    return e;
}

void full_free(FullWorkspace& ws)
{
    void* ptrs[] = {ws.rows, ws.chunks, ws.lmap, ws.cmap, ws.beta_l, ws.beta_c, ws.etab, ws.ptab, ws.tmask,
                    ws.sel, ws.hist, ws.ties, ws.bits, ws.heap_v, ws.heap_i, ws.ytab, ws.fbrow,
                    ws.etab8, ws.ptab8, ws.stage, ws.cpost, ws.head};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
    ws = FullWorkspace{};
}

hipError_t full_init(FullWorkspace& ws, int32_t max_batch, float softcap, hipStream_t s)
{
    hipError_t e = hipMemsetAsync(ws.hist, 0, (size_t)max_batch * kWideBins * sizeof(uint32_t), s);
    if (e == hipSuccess) e = fb_init(ws, max_batch, softcap, s);
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
    if (dtype == G4S_DTYPE_BF16 && !a.wide_on && fb_supported(a.vocab)) return fb_launch(a, s);
    return dtype == G4S_DTYPE_BF16 ? launch_dt<1>(a, s) : launch_dt<0>(a, s);
}

}  // namespace g4s
