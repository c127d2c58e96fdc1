/*
 * g4s_lmhead.h -- Q4_0 LM head (g4s_lmhead.hip).
 */
#ifndef G4S_LMHEAD_H
#define G4S_LMHEAD_H

#include "g4s_device.h"

namespace g4s {

hipError_t lmhead_q4_0_launch(const uint8_t* w, int32_t rows, int32_t cols, const float* h,
                              int32_t batch, float* logits, int64_t stride, hipStream_t s);

/* The TILED64 layout: per 64 rows x 32 columns, 64 binary32 scales then the
 * 64 rows' 16 nibble bytes. */
constexpr int kQ4TileRows = 64;
constexpr int kQ4TileBytes = kQ4TileRows * 4 + kQ4TileRows * 16;

/* Weight j of a block: term (Single(q) * LScale) of CpuMatVecQ4
 * (src/Gemma4.Tensors.pas:586,590) with q = nibble - 8; fma(nibble, s, -8s)
 * is exact and equal to it (both are (nibble - 8) * s, at most 15
 * significant bits).  w: the row's 16 nibble bytes, low nibble of byte j is
 * weight 2j, high nibble weight 2j + 1. */
__device__ __forceinline__ void q4_dequant32(const uint4 w, float sc, float (&q)[32])
{
    const float m8 = -8.0f * sc;
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        /* the nibble masks stay opaque so that each nibble converts with one
         * v_cvt_f32_ubyteN (instead of a field extract and a convert) */
        uint32_t lo, hi;
        asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(lo) : "v"(ws[d]));
        asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(hi) : "v"(ws[d] >> 4));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q[8 * d + 2 * i] = __builtin_fmaf((float)((lo >> (8 * i)) & 0xFFu), sc, m8);
            q[8 * d + 2 * i + 1] = __builtin_fmaf((float)((hi >> (8 * i)) & 0xFFu), sc, m8);
        }
    }
}

/* A 64-row group's summary for one hidden vector: bits 63-32 the group's
 * largest candidate key (cand_key; 0 when no row is valid), bits 31-26 the
 * lowest row of the group holding it, bits 25-0 the largest key of the
 * group's other rows shifted right by 6. */
__host__ __device__ __forceinline__ uint64_t gsum_pack(uint32_t kmax, uint32_t row6, uint32_t k2)
{
    return ((uint64_t)kmax << 32) | ((row6 & 63u) << 26) | (k2 >> 6);
}
__host__ __device__ __forceinline__ uint32_t gsum_key(uint64_t s) { return (uint32_t)(s >> 32); }
__host__ __device__ __forceinline__ uint32_t gsum_row(uint64_t s) { return ((uint32_t)s >> 26) & 63u; }
/* an upper bound of the key of every row but gsum_row's */
__host__ __device__ __forceinline__ uint32_t gsum_bound2(uint64_t s) { return ((uint32_t)s << 6) | 63u; }

/* ROWS -> TILED64 for `rows` rows starting at a 64-row boundary of the
 * destination (dst points at the first row's tile). */
hipError_t q4_tile_launch(const uint8_t* src_rows, int32_t rows, int32_t nblk, uint8_t* dst,
                          hipStream_t s);

/* The LM head on TILED64 weights.  logits may be NULL (nothing written);
 * `gsum` (optional, [batch][ceil(rows/64)]) receives each 64-row group's
 * summary (gsum_pack). */
hipError_t lmhead_tiled_launch(const uint8_t* tiles, int32_t rows, int32_t cols, const float* h,
                               int32_t batch, float* logits, int64_t stride, uint64_t* gsum,
                               hipStream_t s);

/* DoEmbeddingLookup of a ROWS-layout Q4_0 table: hidden[b] = dequantised
 * row tokens[b] (device) times `scale`. */
hipError_t embed_q4_0_launch(const uint8_t* w, int32_t rows, int32_t cols, const int32_t* tokens,
                             int32_t batch, float scale, float* hidden, hipStream_t s);

}  // namespace g4s

#endif
