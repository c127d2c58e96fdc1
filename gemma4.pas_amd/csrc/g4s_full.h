/*
 * g4s_full.h -- launch interface of the full-vocabulary path (g4s_full.hip).
 */
#ifndef G4S_FULL_H
#define G4S_FULL_H

#include "g4s_device.h"
#include "g4s_seqsum.h"

namespace g4s {

constexpr int kFullBlock = 256;                     /* threads per chunk workgroup */
constexpr int kFullPer = 16;                        /* consecutive terms per thread */
constexpr int kFullChunk = kFullBlock * kFullPer;   /* terms per chunk */
constexpr int kFullMaxChunks = 1024;                /* chunks per row: vocab <= 2^22 */
constexpr int kFullTab = 4096;                      /* bf16 codes with a tabulated e */

/* Per-row state shared by the four kernels (device workspace). */
struct FullRow {
    uint32_t maxkey;  /* order-preserving key of the largest raw logit */
    uint32_t amax;    /* largest |logit| as a key of |x| */
    float m;          /* max over the row of y = softcap(x) [* 1/T] */
    float inv_t;      /* fl32(1/T) when scaling, else 1 */
    int32_t scale;    /* T > 0 and T <> 1 */
    int32_t win_lo;   /* bf16 exponent field of the table's lowest binade, -1: no table */
    float lsum;       /* LSum (exact) */
    float inv;        /* fl32(1/LSum) */
    float thr;        /* fl32(u * TopP) */
    int32_t argmax;   /* first index of the largest p */
    int32_t c_last;   /* last chunk the draw kernel visits, -1: none */
    int32_t nodraw;   /* T <= 0: the greedy choice, no draw (probabilities still written) */
    /* diagnostics: chunks re-evaluated and re-evaluation rounds, LSum chain
     * then draw chain */
    int32_t l_reev, l_rounds, c_reev, c_rounds;
};

/* Per-chunk records.  Fields exchanged between workgroups of one launch are
 * aligned 64-bit words written and read with device-coherent accesses. */
struct FullChunk {
    uint32_t maxkey;  /* max kernel: chunk's largest key          } word 0 */
    uint32_t amax;    /* max kernel: largest |x| as a key          }        */
    float ymax;       /* approximate y at the chunk's largest logit } word 1 */
    float sapx;       /* approximate sum of exp(y - ymax)           }        */
    ss::PMap lmap;    /* lsum kernel: the chunk's terms in beta_l     word 2 */
    ss::PMap cmap;    /* draw kernel: the chunk's p in beta_c         word 3 */
    double de;        /* lsum kernel: sum of the chunk's e in binary64  word 4 */
    int32_t first1;   /* lsum kernel: first index with e == 1, or INT_MAX */
    int32_t beta_l;   /* predicted binade of LSum entering the chunk */
    int32_t beta_c;   /* predicted binade of the running sum entering the chunk */
    int32_t pad[3];
};

static_assert(sizeof(FullChunk) == 64, "FullChunk layout");
static_assert(__builtin_offsetof(FullChunk, ymax) == 8 && __builtin_offsetof(FullChunk, lmap) == 16 &&
                  __builtin_offsetof(FullChunk, cmap) == 24 && __builtin_offsetof(FullChunk, de) == 32,
              "FullChunk words");

struct FullWorkspace {
    FullRow* rows = nullptr;     /* [max_batch] */
    FullChunk* chunks = nullptr; /* [max_batch][kFullMaxChunks] */
    float* etab = nullptr;       /* [max_batch][kFullTab] */
    uint32_t* tickets = nullptr; /* [max_batch][4], zero between launches */
};

struct FullArgs {
    const void* logits;
    int64_t row_stride;
    int32_t vocab;
    int32_t batch;
    const g4s_params* params;
    const double* u;
    g4s_params p0;
    double u0;
    float softcap;
    int32_t nch;
    FullWorkspace ws;
    int32_t* ids;
    uint32_t* done;
    uint32_t seq;
    g4s_outputs out;
};

hipError_t full_alloc(FullWorkspace& ws, int32_t vocab, int32_t max_batch);
void full_free(FullWorkspace& ws);
hipError_t full_init(FullWorkspace& ws, int32_t max_batch, hipStream_t s);
bool full_supported(int32_t vocab);
hipError_t full_launch(const FullArgs& a, int dtype, hipStream_t s);

}  // namespace g4s

#endif
