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

/* Streaming pipeline of full bf16 rows (g4s_fullbf.hip). */
constexpr int kBfTab = 8192;       /* e / p table: 32 binades of |x| x 128 mantissas x 2 signs */
constexpr int kBfWin = 32;         /* binades of |x| in the table */
constexpr int kBfStage = 16;       /* chunks per row staged for a chain */
constexpr int kBfBlock = 512;      /* threads of the table-lookup passes */
constexpr int kBfMaxChunks = 1024; /* chunks per row: vocab <= 2^20 */

/* Per-row words of the streaming pipeline that several workgroups update. */
struct FbRow {
    uint32_t kmax;  /* largest key of the row (atomic max, max pass) */
    uint32_t amax;  /* largest |x| of the row as binary32 bits (atomic max, max pass) */
    uint32_t key1;  /* smallest order key of a code whose e is 1 (atomic min) */
    int32_t amx;    /* first index whose key >= key1: the argmax of p (atomic min) */
    float s0;       /* LSum after chunk 0, exact */
    float c0;       /* the draw's running sum after chunk 0, exact (when hit0 < 0) */
    int32_t hit0;   /* first index of chunk 0 whose running sum reaches thr, -1: none */
    int32_t nsl;    /* chunks staged for the LSum chain */
    int32_t nsc;    /* chunks staged for the draw chain */
    /* the terms of codes outside the table: -inf, +inf, and every code below
     * the table's binades when they share one value (NaN: they do not) --
     * e (row kernel), then p (LSum chain) */
    float e_ninf, e_pinf, e_tiny;
    float p_ninf, p_pinf, p_tiny;
    int32_t pad;
};
static_assert(sizeof(FbRow) == 64, "FbRow layout");

/* A chunk staged for a chain (a predicted binade crossing): its lane maps
 * in binade b and b + 1 and its 1024 terms (lane l's 16 at l*16). */
struct BfStage {
    ss::PMap lo[64];
    ss::PMap hi[64];
    int32_t b;
    int32_t chunk;
    int32_t pad[2];
    /* inclusive lane scans of the lo maps from an even [0..63] and an odd
     * [64..127] entering significand, and of the hi maps [128..255] */
    int32_t xs[256];
    float t[kFullChunk];
};
static_assert(sizeof(BfStage) % 16 == 0, "BfStage copies in 16-byte units");

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
                                    ([1]) is a half-unit tie (64-binade windows); the
                                    bf16 rows' draw pass keeps its p mask in LDS */
    /* wide rows */
    WideSel* sel = nullptr;      /* [max_batch] */
    uint32_t* hist = nullptr;    /* [max_batch][kWideBins], zero between launches */
    TieRec* ties = nullptr;      /* [max_batch][kSelMaxChunks] */
    uint32_t* bits = nullptr;    /* [max_batch][ceil(vocab/32)] surviving tied copies */
    float* heap_v = nullptr;     /* [vocab] replay heap (one row at a time) */
    int32_t* heap_i = nullptr;   /* [vocab] */
    /* streaming pipeline of full bf16 rows */
    float* ytab = nullptr;       /* [65536] y = softcap(x) of every bf16 code (full-row form) */
    FbRow* fbrow = nullptr;      /* [max_batch] */
    float* etab8 = nullptr;      /* [max_batch][kBfTab] e of the tabulated codes */
    float* ptab8 = nullptr;      /* [max_batch][kBfTab] p of the same codes */
    BfStage* stage = nullptr;    /* [max_batch][kBfStage] staged chunks (LSum, then the draw) */
    float* cpost = nullptr;      /* [max_batch][cstride] exact LSum after every chunk */
    float* head = nullptr;       /* [max_batch][kFullChunk] e of every row's chunk 0 */
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
hipError_t full_init(FullWorkspace& ws, int32_t max_batch, float softcap, hipStream_t s);
bool full_supported(int32_t vocab);

/* The streaming pipeline (g4s_fullbf.hip): full bf16 rows of a batch
 * without wide rows, vocab a multiple of kFullChunk up to kBfMaxChunks
 * chunks. */
bool fb_supported(int32_t vocab);
hipError_t fb_init(FullWorkspace& ws, int32_t max_batch, float softcap, hipStream_t s);
hipError_t fb_launch(const FullArgs& a, hipStream_t s);
hipError_t full_launch(const FullArgs& a, int dtype, hipStream_t s);

}  // namespace g4s

#endif
