/*
 * g4s_topk.h -- launch interface of the top-k path kernel (g4s_topk.hip).
 */
#ifndef G4S_TOPK_H
#define G4S_TOPK_H

#include "g4s_device.h"

namespace g4s {

constexpr int kWaveBounds = 512; /* per-wave bounds kept per row (splits * waves) */

/* The decode-sized launch (g4s_decode.hip): batches of up to kDecMaxBatch
 * rows (as many as the handle's election counters hold) whose TopK bound is
 * at most kDecMaxK, on vocabularies of at most kDecMaxChunks
 * 16-byte-per-thread workgroup chunks (262144 binary32 logits, 524288 bf16).
 * K bounds up to kDecSmallK take an instantiation with less LDS.  (Larger
 * batches take the chunked launch: screening a row into 1024 wave lists
 * costs more instructions per logit than the chunk workgroups' bounds: with
 * this launch a B=64 batch of mixed K took 76.1 us against 37.2 us.) */
constexpr int kDecMaxBatch = 8;
constexpr int kDecMaxK = 256;
constexpr int kDecSmallK = 64;
constexpr int kDecBlock = 256;                 /* threads per workgroup */
constexpr int kDecMaxChunks = 256;             /* workgroups per row */
constexpr int kDecListLen = 4;                 /* entries per wave list */
constexpr int kDecCounterStride = 32;          /* words between election counters (128 B) */
constexpr int kDecGroups = 16;                 /* first-level election counters per row */
constexpr int kDecTicketWords = kDecCounterStride * (kDecGroups + 1);
constexpr int kDecSlotsPerRow = kDecMaxChunks * (kDecBlock / 64) * kDecListLen;
static_assert(kDecSlotsPerRow <= 16384, "the wave lists fit a row's candidate slots");

/* Per-chunk record written by phase 1 (16 bytes). */
struct ChunkRec {
    uint32_t count;  /* candidates emitted */
    uint32_t bound;  /* lower bound of the chunk's K-th largest key (exact when mode bit set) */
    uint32_t rsv;    /* 0, or kRecNeedRow in the row's first record */
    uint32_t mode_e; /* bit 31: exact select; bits 0-30: copies of the K-th key in the chunk */
};

/* rsv of a row's first record: the candidates cannot decide the row without
 * logits that were never written (the fused LM head without d_logits); the
 * merge gives the row id -1 and G4S_FLAG_ROW_RECOMPUTED, and the host
 * samples it again from recomputed logits. */
constexpr uint32_t kRecNeedRow = 1u;

/* Fused LM head without logits: per row, the 64-row groups whose logits the
 * recompute launch produces: [0] count, [1] first candidate slot of the
 * recomputed logits (64 slots per group), [2 ..] the groups. */
constexpr int kGcMaxJobs = 32;
constexpr int kGcJobStride = kGcMaxJobs + 2;

/* A candidate: order-preserving key in the high word, vocab index in the low word. */
__host__ __device__ inline uint64_t cand_pack(uint32_t key, uint32_t idx)
{
    return ((uint64_t)key << 32) | idx;
}
__host__ __device__ inline uint32_t cand_key_of(uint64_t c) { return (uint32_t)(c >> 32); }
__host__ __device__ inline uint32_t cand_idx_of(uint64_t c) { return (uint32_t)c; }

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
    int32_t cap_log2; /* candidate slots per chunk = 1 << cap_log2 (>= 2 * kbound) */
    int32_t kbound;   /* every top-k row has TopK <= kbound */
    int32_t wide_on;  /* rows with TopK > kMaxTopK are left to the wide launches */
    int32_t full_on;  /* the softmax launches follow for full rows; when 0 a full row
                         gets id -1 and G4S_FLAG_ERROR | G4S_FLAG_FULL_PATH here */
    int32_t mode;     /* 0: chunks + last-workgroup merge in one launch; 1: chunks
                         only; 2: merges only (one workgroup per row) */
    float softcap;
    uint64_t* cand;   /* [batch][kCandRow] chunk candidates */
    uint64_t* merge;  /* [batch][kCandRow] merge candidates beyond what LDS holds */
    ChunkRec* recs;   /* [batch][kMaxSplits] */
    uint32_t* wbounds; /* [batch][kWaveBounds]: per wave, the r-th largest thread maximum */
    uint32_t* tickets; /* [batch], zero between launches */
    int32_t* ids;      /* [batch] (device or host-pinned) */
    uint32_t* done;    /* [batch] host-pinned completion words, or NULL */
    uint32_t seq;      /* value written to done[row] once the row's outputs are visible */
    g4s_outputs out;
    uint32_t* dec_tickets; /* [dec_rows][kDecTicketWords] election counters of the decode
                              launch, zero between launches; NULL: no decode launch */
    int32_t dec_rows;      /* rows dec_tickets holds (the decode launch's batch bound) */
    /* the fused LM head without logits (logits == NULL): its TILED64
     * weights, hidden vectors [batch][lm_cols] and the recompute jobs
     * [batch][kGcJobStride] */
    const uint8_t* lm_tiles;
    const float* lm_hidden;
    int32_t lm_cols;
    int32_t* gc_jobs;
};

struct TopkConfig {
    int block, items, chunk, splits, cap_log2;
    bool ok;
};

TopkConfig topk_plan(int32_t vocab, int32_t kbound);
/* One launch (mode 0) while the batch's chunk workgroups fit the device at
 * once (`ncu` compute units, 1024 resident threads each), else a chunk
 * launch followed by a merge launch, so that no merge holds a compute unit
 * that a later chunk is waiting for. */
hipError_t topk_launch(const TopkConfig& c, const TopkArgs& a, int dtype, hipStream_t s,
                       int32_t ncu = 0);

/* Whether topk_launch takes the decode-sized launch for these rows. */
bool decode_eligible(const TopkArgs& a, int dtype);
/* The decode-sized launch (g4s_decode.hip): per-wave candidate lists written
 * by every workgroup, a two-level election, and the merge + tail in the last
 * workgroup of each row.  The lists use the rows' candidate slots (a.cand). */
hipError_t decode_launch(const TopkArgs& a, int dtype, hipStream_t s);

/* Rows whose f32 logits come from the tiled LM head with its 64-logit group
 * summaries (gsum [batch][ngroups], gsum_pack): candidates from the groups
 * whose maximum reaches the K-th largest group maximum, then the merge launch
 * (mode 2).  With a.logits == NULL a candidate group gives its maximum, or,
 * when its second largest key may reach the bound, its 64 logits recomputed
 * by a launch in between.  hipErrorNotSupported above 8192 groups. */
hipError_t topk_groups_launch(const TopkConfig& c, const TopkArgs& a, const uint64_t* gsum,
                              int32_t ngroups, hipStream_t s);

}  // namespace g4s

#endif
