/*
 * g4s_select.h -- block-wide k-th largest selection shared by the top-k
 * kernels (g4s_topk.hip, g4s_decode.hip).
 */
#ifndef G4S_SELECT_H
#define G4S_SELECT_H

#include "g4s_device.h"

namespace g4s {

/* Rank-by-count k-th largest of key(i), i in [0, n) (n <= kRankMax).  The
 * inner scan reads eight keys per step so the LDS loads overlap. */
template <int BLOCK, typename KeyF>
__device__ uint32_t rank_kth(int n, int k, KeyF key, int* s_misc, int* gt, int* eq)
{
    const int tid = threadIdx.x;
    for (int i = tid; i < n; i += BLOCK) {
        const uint32_t ki = key(i);
        int g = 0, q = 0;
        int j = 0;
        for (; j + 8 <= n; j += 8) {
            uint32_t kk[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) kk[t] = key(j + t);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                g += kk[t] > ki;
                q += kk[t] == ki;
            }
        }
        for (; j < n; ++j) {
            const uint32_t kj = key(j);
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
    const uint32_t r = (uint32_t)s_misc[4];
    *gt = s_misc[5];
    *eq = s_misc[6];
    __syncthreads();
    return r;
}

template <int BLOCK, typename KeyF, typename SH>
__device__ uint32_t select_kth(int n, int k, KeyF key, SH& sh, int* gt, int* eq)
{
    if (n <= kRankMax) return rank_kth<BLOCK>(n, k, key, sh.misc, gt, eq);
    return block_radix_kth<BLOCK>(n, k, key, [](int) { return true; }, sh.hist, sh.misc + 4, gt,
                                  eq);
}

}  // namespace g4s

#endif
