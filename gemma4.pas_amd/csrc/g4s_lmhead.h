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

/* ROWS -> TILED64 for `rows` rows starting at a 64-row boundary of the
 * destination (dst points at the first row's tile). */
hipError_t q4_tile_launch(const uint8_t* src_rows, int32_t rows, int32_t nblk, uint8_t* dst,
                          hipStream_t s);

/* The LM head on TILED64 weights; `gmax` (optional, [batch][ceil(rows/64)])
 * receives each 64-row group's largest logit as a candidate key (cand_key). */
hipError_t lmhead_tiled_launch(const uint8_t* tiles, int32_t rows, int32_t cols, const float* h,
                               int32_t batch, float* logits, int64_t stride, uint32_t* gmax,
                               hipStream_t s);

/* DoEmbeddingLookup of a ROWS-layout Q4_0 table: hidden[b] = dequantised
 * row tokens[b] (device) times `scale`. */
hipError_t embed_q4_0_launch(const uint8_t* w, int32_t rows, int32_t cols, const int32_t* tokens,
                             int32_t batch, float scale, float* hidden, hipStream_t s);

}  // namespace g4s

#endif
