/*
 * g4s_full.h -- launch interface of the softmax-path kernels (g4s_full.hip):
 * full-vocabulary rows (TopK <= 0 or TopK >= V) and wide top-k rows
 * (g4s_max_top_k() < TopK < V).
 */
#ifndef G4S_FULL_H
#define G4S_FULL_H

#include "g4s_device.h"
#include "g4s_seqsum.h"

namespace g4s {

constexpr int kFullBlock = 256;                     /* threads of the streaming workgroups */
constexpr int kFullPer = 16;                        /* consecutive terms per lane */
constexpr int kFullChunk = 64 * kFullPer;           /* terms per chunk: one wave's 1024 */
constexpr int kFullMaxChunks = 4096;                /* chunks per row: vocab <= 2^22 */
constexpr int kFullTab = 4096;                      /* bf16 codes with a tabulated e */
constexpr int kNear = 8;  /* e = 1 - j*2^-24 (j < kNear): the values whose p can tie the
                             largest p under the top-k tail's division */
constexpr int kWideBins = 2048;                     /* radix-select histogram bins */
constexpr int kSelChunk = kFullBlock * kFullPer;    /* terms per wide-select workgroup */
constexpr int kSelMaxChunks = 1024;                 /* select chunks per row */

/* Row classes (DoSample's dispatch, src/Gemma4.Model.pas:2756). */
enum : int32_t { kRowTopk = 0, kRowFull = 1, kRowWide = 2 };

/* Per-row state shared by the kernels (device workspace). */
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
    int32_t count;    /* terms that take part: V, or the wide row's survivors */
    int32_t first;    /* index of the first term that takes part */
    int32_t beta_end; /* predicted binade of LSum after the last chunk */
    int32_t near[kNear]; /* first index with e == 1 - j*2^-24 (atomic min), INT_MAX: none */
    /* diagnostics: chunks re-evaluated and re-evaluation rounds, LSum chain
     * then draw chain */
    int32_t l_reev, l_rounds, c_reev, c_rounds;
};

/* Per-chunk record of the max kernel (and the survivor offsets of the row
 * kernel). */
struct FullChunk {
    uint32_t maxkey;  /* chunk's largest key */
    uint32_t amax;    /* largest |x| as a key */
    float ymax;       /* approximate y at the chunk's largest logit */
    float sapx;       /* approximate sum of exp(y - ymax) over the terms taking part */
    int32_t nsurv;    /* terms of the chunk taking part */
    int32_t fsurv;    /* first index taking part, INT_MAX: none */
    int32_t soff;     /* row kernel: terms taking part before the chunk */
    int32_t pad;
};
static_assert(sizeof(FullChunk) == 32, "FullChunk layout");

/* Radix select of a wide row's K-th largest key and its tie resolution. */
struct WideSel {
    uint32_t prefix;  /* key digits fixed so far */
    int32_t krem;     /* rank still to find among keys with that prefix */
    int32_t state;    /* kSel* */
    uint32_t tau;     /* the K-th largest key */
    int32_t need;     /* copies of tau that survive */
    int32_t eq;       /* copies of tau in the row */
    int32_t idx_thr;  /* lowest-index rule: copies with index <= idx_thr survive */
    int32_t count;    /* survivors */
};
enum : int32_t {
    kSelSearch = 0,   /* digits being fixed */
    kSelAll = 1,      /* every key >= tau survives */
    kSelTies = 2,     /* tau tied beyond the remaining slots: resolution pending */
    kSelLowest = 3,   /* the first `need` copies of tau in index order survive */
    kSelReplay = 4,   /* the min-heap decides: replay pending */
    kSelBits = 5,     /* the surviving copies of tau are marked in the row's bitmask */
    kSelEmpty = 6     /* no logit above -1e30 */
};

struct TieRec {
    int32_t cge;      /* keys >= tau in the chunk */
    int32_t ceq;      /* keys == tau in the chunk */
    int32_t maxgt;    /* last index with key > tau, -1: none */
    int32_t pad;
};

struct FullWorkspace {
    FullRow* rows = nullptr;     /* [max_batch] */
    FullChunk* chunks = nullptr; /* [max_batch][cstride] */
    ss::PMap* lmap = nullptr;    /* [max_batch][cstride] chunk's terms in beta_l */
    ss::PMap* cmap = nullptr;    /* [max_batch][cstride] chunk's p in beta_c */
    int32_t* beta_l = nullptr;   /* [max_batch][cstride] predicted binade of LSum entering */
    int32_t* beta_c = nullptr;   /* [max_batch][cstride] same for the draw's running sum */
    float* etab = nullptr;       /* [max_batch][kFullTab] e of the tabulated bf16 codes */
    float* ptab = nullptr;       /* [max_batch][kFullTab] p of the same codes */
    uint64_t* tmask = nullptr;   /* [max_batch][2] binades where a table e ([0]) or p
                                    ([1]) is a half-unit tie (64-binade windows) */
    /* wide rows */
    WideSel* sel = nullptr;      /* [max_batch] */
    uint32_t* hist = nullptr;    /* [max_batch][kWideBins], zero between launches */
    TieRec* ties = nullptr;      /* [max_batch][kSelMaxChunks] */
    uint32_t* bits = nullptr;    /* [max_batch][ceil(vocab/32)] surviving tied copies */
    float* heap_v = nullptr;     /* [vocab] replay heap (one row at a time) */
    int32_t* heap_i = nullptr;   /* [vocab] */
    int32_t bits_stride = 0;     /* words per row of `bits` */
    int32_t cstride = 0;         /* chunk records per row (= chunks of the vocabulary) */
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
    int32_t nch;      /* chunks of kFullChunk terms per row */
    int32_t nsel;     /* chunks of kSelChunk terms per row (wide select) */
    int32_t nstage;   /* chunks each chain precomputes (set by full_launch) */
    int32_t cpw;      /* chunks per wave of the streaming passes (set by full_launch) */
    int32_t wide_on;  /* wide rows are handled by this launch */
    int32_t topk_on;  /* a top-k launch takes the top-k rows; when 0 such a row gets
                         id -1 and G4S_FLAG_ERROR | G4S_FLAG_TOPK_PATH here */
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
