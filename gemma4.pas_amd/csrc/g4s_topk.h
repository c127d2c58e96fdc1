/*
 * g4s_topk.h -- launch interface of the top-k path kernel (g4s_topk.hip).
 */
#ifndef G4S_TOPK_H
#define G4S_TOPK_H

#include "g4s_device.h"

namespace g4s {

/* Per-chunk record written by phase 1 (16 bytes). */
struct ChunkRec {
    uint32_t count;  /* candidates emitted */
    uint32_t bound;  /* lower bound of the chunk's K-th largest key (exact when mode bit set) */
    uint32_t rc;     /* ceil(K/splits)-th largest key of the chunk, 0 if fewer keys */
    uint32_t mode_e; /* bit 31: exact select; bits 0-30: copies of the K-th key in the chunk */
};

struct TopkArgs {
    const void* logits;
    int64_t row_stride; /* elements */
    int32_t vocab;
    int32_t batch;
    const g4s_params* params; /* device [batch], or NULL: use p0/u0 (batch == 1) */
    const double* u;
    g4s_params p0;
    double u0;
    int32_t splits;
    int32_t cap_c;  /* candidate slots per chunk (2 * kbound) */
    int32_t kbound; /* every top-k row has TopK <= kbound */
    float softcap;
    uint32_t* cand_key; /* [batch][kCandRow] */
    uint32_t* cand_idx;
    uint32_t* merge_key; /* [batch][kCandRow] merge scratch when candidates exceed LDS */
    uint32_t* merge_idx;
    ChunkRec* recs;     /* [batch][kMaxSplits] */
    uint32_t* tickets;  /* [batch], zero between launches */
    int32_t* ids;       /* device [batch] */
    g4s_outputs out;
};

struct TopkConfig {
    int block, items, chunk, splits, cap_c;
    bool ok;
};

TopkConfig topk_plan(int32_t vocab, int32_t kbound);
hipError_t topk_launch(const TopkConfig& c, const TopkArgs& a, int dtype, hipStream_t s);

}  // namespace g4s

#endif
