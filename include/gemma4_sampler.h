/*
 * gemma4_sampler.h -- C ABI of libgemma4_sampler.so, the MI355X (gfx950)
 * token sampler for the Gemma4.pas engine.
 *
 * The library replaces the engine's CPU sampler, TModel.DoSample and its
 * helpers (src/Gemma4.Model.pas:2615-2827, src/Gemma4.Tensors.pas:638-673,
 * src/Gemma4.Layers.pas:300-316), on logits that stay in device memory.  It
 * keeps the reference's sampling surface (TSamplingParams:
 * Temperature / TopK / TopP) and its order of operations:
 *   top-k path (0 < TopK < V): top-K on raw logits (min-heap tie semantics)
 *     -> survivors ascending by vocab index -> softcap cap*tanh(x/cap)
 *     -> * fl32(1/T) when T > 0 and T <> 1 -> softmax (sequential binary32
 *     sum, division) -> greedy argmax -> if T > 0: first survivor, in index
 *     order, whose running binary32 sum is >= fl32(u*TopP), else the argmax;
 *   full path (TopK <= 0 or TopK >= V): softcap tanh(x*fl32(1/cap))*cap on
 *     every logit -> temperature -> softmax over V (sequential binary32 sum,
 *     reciprocal multiply) -> argmax -> the same index-order draw over V.
 * Transcendental steps are correctly rounded to binary32.  System.Random is
 * replaced by a caller-supplied uniform u in [0,1) per row, so a caller that
 * passes the values its RNG would have produced reproduces the reference
 * exactly.
 *
 * Conventions: functions return 0 (G4S_OK) or a negative g4s_status; the
 * message of the last failure is kept per handle (g4s_last_error).  One
 * handle = one HIP stream; a handle is not thread-safe; several handles may
 * coexist.  Device pointers are HIP device memory of the handle's device.
 */
#ifndef GEMMA4_SAMPLER_H
#define GEMMA4_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G4S_ABI_VERSION 1

typedef struct g4s_sampler g4s_sampler;

typedef enum g4s_dtype {
    G4S_DTYPE_F32 = 0,  /* binary32 logits (the engine's FLogits) */
    G4S_DTYPE_BF16 = 1  /* bf16 logits, widened exactly as TBFloat16.ToSingle (Types.pas:417-424) */
} g4s_dtype;

typedef enum g4s_status {
    G4S_OK = 0,
    G4S_ERR_INVALID_ARGUMENT = -1, /* null pointer, bad size, misaligned logits, ... */
    G4S_ERR_UNSUPPORTED = -2,      /* e.g. a vocabulary above 2^22 on the softmax path */
    G4S_ERR_NO_DEVICE = -3,        /* no HIP device / wrong architecture */
    G4S_ERR_OUT_OF_MEMORY = -4,    /* workspace allocation failed at create */
    G4S_ERR_HIP = -5,              /* a HIP runtime call failed */
    G4S_ERR_EMPTY_ROW = -6,        /* a top-k row had no logit above -1e30 (id set to -1) */
    G4S_ERR_IO = -7,               /* weight store: the archive could not be opened or mapped */
    G4S_ERR_FORMAT = -8,           /* weight store: not a VPK / manifest the engine would accept */
    G4S_ERR_NOT_FOUND = -9,        /* weight store: no such archive entry or tensor */
    G4S_ERR_ABORTED = -10          /* decode loop: the forward callback reported a failure */
} g4s_status;

/* TSamplingParams, src/Gemma4.Model.pas:70-76 (same fields, same meaning).
 * repetition_penalty is carried for layout parity and, as in the reference,
 * never read. */
typedef struct g4s_params {
    float temperature;
    int32_t top_k;
    float top_p;
    float repetition_penalty;
} g4s_params;

/* Per-row flags (g4s_outputs.flags) */
#define G4S_FLAG_TOPK_PATH 0x1u     /* row took the top-k path */
#define G4S_FLAG_FULL_PATH 0x2u     /* row took the full-vocabulary path */
#define G4S_FLAG_DREW 0x4u          /* T > 0: a draw against u*TopP happened */
#define G4S_FLAG_REACHED 0x8u       /* the running sum reached u*TopP */
#define G4S_FLAG_TIE_LOWEST 0x10u   /* K-th value tied; resolved by the lowest-index rule */
#define G4S_FLAG_HEAP_REPLAY 0x20u  /* K-th value tied; resolved by replaying the min-heap */
#define G4S_FLAG_CHUNK_EXACT 0x40u  /* a vocabulary chunk needed the exact per-chunk select */
#define G4S_FLAG_WIDE_MERGE 0x80u   /* the merge candidate set exceeded on-chip memory */
#define G4S_FLAG_WIDE_K 0x100u      /* TopK above g4s_max_top_k(): radix select over the whole row */
#define G4S_FLAG_ROW_RECOMPUTED 0x200u /* g4s_lmhead_sample_q4_0 without d_logits: the row's ties
                                          needed every logit, so the call recomputed the row and
                                          sampled it again (same result, slower) */
#define G4S_FLAG_EMPTY 0x40000000u  /* no logit above -1e30 on the top-k path */
#define G4S_FLAG_ERROR 0x80000000u  /* row rejected (e.g. TopK above the launch bound) */

/* Optional per-row outputs; every pointer is device memory and may be NULL.
 *   count   [batch]           candidates: K' survivors (top-k path) or V (full path)
 *   indices [batch*capacity]  top-k path: survivor vocab indices, ascending
 *   probs   [batch*capacity]  top-k path: normalised survivor probabilities
 *                             (LVals after the division, Model.pas:2800-2801);
 *                             full path: p_i over the vocabulary when capacity >= V
 *   argmax  [batch]           token id of the greedy choice (first maximum of p)
 *   lsum    [batch]           softmax denominator (LSum)
 *   flags   [batch]           G4S_FLAG_* */
typedef struct g4s_outputs {
    int32_t* count;
    int32_t* indices;
    float* probs;
    int32_t capacity;
    int32_t* argmax;
    float* lsum;
    uint32_t* flags;
} g4s_outputs;

/* Library version string, e.g. "gemma4_sampler 0.1.0 (gfx950)". */
const char* g4s_version(void);

/* TSamplingParams.SetDefaults, src/Gemma4.Model.pas:346-352:
 * T = 1.0, TopK = 64, TopP = 0.95, RepetitionPenalty = 1.0. */
void g4s_params_set_defaults(g4s_params* params);

/* Largest TopK of the single-launch top-k kernel.  Rows with a larger TopK
 * (below V) take the wide top-k path: a radix select over the whole row with
 * the same semantics (G4S_FLAG_WIDE_K).  TopK <= 0 or >= V selects the full
 * path. */
int32_t g4s_max_top_k(void);

/* Create a sampler for `vocab` logits per row and up to `max_batch` rows per
 * call.  `softcap` is the model's final_logit_softcapping
 * (Gemma4.Config.pas:74,209; 30.0 for Gemma 4; <= 0 disables it).
 * `hip_stream` (hipStream_t, may be NULL = default stream) orders all work.
 * Allocates the whole workspace; no later call allocates device memory.
 * Replaces: the sampler state of TModel (FLogits/FConfig, Model.pas:131,161). */
int g4s_create(g4s_sampler** out, int32_t vocab, int32_t max_batch, float softcap,
               void* hip_stream);

/* Release the handle and its workspace.  NULL is accepted. */
int g4s_destroy(g4s_sampler* sampler);

/* Message of the most recent failure on this handle ("" if none).  With a
 * NULL handle, the message of the most recent failed g4s_create or
 * g4s_sample_topk_noalloc on the calling thread. */
const char* g4s_last_error(const g4s_sampler* sampler);

/* Sample `batch` rows synchronously.  Replaces TModel.DoSample
 * (src/Gemma4.Model.pas:2739-2827) and the per-token logits readback
 * (Model.pas:1382-1385): the logits stay on the device, only ids return.
 *   d_logits   device, `batch` rows of `vocab` logits, row i at
 *              d_logits + i*row_stride elements; 16-byte aligned base and
 *              row_stride*sizeof(dtype) a multiple of 16
 *   params     host, `batch` entries (one TSamplingParams per row)
 *   u          host, `batch` uniforms in [0,1) standing in for System.Random
 *   ids        host, `batch` token ids written on return */
int g4s_sample(g4s_sampler* sampler, const void* d_logits, int32_t dtype, int64_t row_stride,
               int32_t batch, const g4s_params* params, const double* u, int32_t* ids);

/* g4s_sample plus the optional device-side outputs described above. */
int g4s_sample_ex(g4s_sampler* sampler, const void* d_logits, int32_t dtype, int64_t row_stride,
                  int32_t batch, const g4s_params* params, const double* u, int32_t* ids,
                  const g4s_outputs* outputs);

/* Stream-ordered variant for callers that keep parameters on the device
 * (graph capture, serving loops).  d_params, d_u and d_ids are device
 * arrays of `batch` entries.  `k_bound` >= every TopK of a top-k-path row
 * (0 < TopK < V; k_bound 0 when no row takes the top-k path) sizes the
 * launch: above g4s_max_top_k() the wide top-k launches are added;
 * `full_rows` != 0 when some row may take the full-vocabulary path.  Rows
 * that violate k_bound get id -1 and G4S_FLAG_ERROR, and so does a row whose
 * path is not enqueued: a full-vocabulary row when full_rows == 0
 * (G4S_FLAG_ERROR | G4S_FLAG_FULL_PATH) or a top-k row when k_bound == 0
 * (G4S_FLAG_ERROR | G4S_FLAG_TOPK_PATH); no row keeps an earlier call's id.
 * Returns after enqueueing; results are valid once the stream reaches this
 * point. */
int g4s_sample_async(g4s_sampler* sampler, const void* d_logits, int32_t dtype,
                     int64_t row_stride, int32_t batch, const g4s_params* d_params,
                     const double* d_u, int32_t k_bound, int32_t full_rows, int32_t* d_ids,
                     const g4s_outputs* outputs);

/* g4s_sample_async launched from a hipGraph the handle owns: the first call
 * with a given set of arguments (the pointers, dtype, row_stride, batch,
 * k_bound, full_rows and the outputs' pointers) captures the launches on the
 * handle's stream and instantiates them; later calls with the same arguments
 * replay that graph (up to 8 argument sets are kept, the least recently used
 * replaced first).  The graph reads the logits, parameters and uniforms when
 * it runs, so a decode loop rewrites the same buffers and calls again.  Under
 * a capture of the caller's own on the handle's stream the launches are
 * recorded into that capture instead.  Same arguments, results and errors
 * as g4s_sample_async; the handle needs a stream other than the null stream.
 * Replaces the engine's per-token record + submit of its sampling work
 * (src/Gemma4.Model.pas:1331-1375; src/Gemma4.Vulkan.pas:1449-1461) for
 * the sampling step. */
int g4s_sample_graph(g4s_sampler* sampler, const void* d_logits, int32_t dtype,
                     int64_t row_stride, int32_t batch, const g4s_params* d_params,
                     const double* d_u, int32_t k_bound, int32_t full_rows, int32_t* d_ids,
                     const g4s_outputs* outputs);

/* Rows and bytes of the device scratch array behind g4s_sample_topk_noalloc
 * (held by every GPU the library runs on until the process ends). */
#define G4S_NOALLOC_MAX_ROWS 32
#define G4S_NOALLOC_SCRATCH_BYTES 8602880

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the top-k path of g4s_sample_async without a handle,
 * with its workspace in a fixed device array of G4S_NOALLOC_SCRATCH_BYTES
 * per GPU instead of memory allocated by g4s_create.  Calls no hipMalloc,
 * hipFree or allocating library routine.
 *   d_logits, dtype, row_stride  as for g4s_sample_async (`vocab` logits per row)
 *   batch      1 .. G4S_NOALLOC_MAX_ROWS; larger batches are rejected
 *   d_params, d_u, d_ids  device arrays of `batch` entries
 *   k_bound    1 .. min(g4s_max_top_k(), vocab - 1), >= every row's TopK
 *   softcap    final_logit_softcapping (<= 0 disables it)
 *   outputs    optional device outputs, as for g4s_sample_ex
 *   hip_stream the stream the work is enqueued on (NULL = default stream)
 * Rows whose TopK is <= 0, >= vocab or above k_bound get id -1 and
 * G4S_FLAG_ERROR.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU race, so run one at a time per device.  Returns after
 * enqueueing; failures are reported by g4s_last_error(NULL). */
int g4s_sample_topk_noalloc(const void* d_logits, int32_t dtype, int32_t vocab,
                            int64_t row_stride, int32_t batch, const g4s_params* d_params,
                            const double* d_u, int32_t k_bound, float softcap, int32_t* d_ids,
                            const g4s_outputs* outputs, void* hip_stream);

/* LM head for the sampler's config-5 workload: logits = W * h for `batch`
 * hidden vectors, with W in the engine's Q4_0 layout (TQ4Block rows,
 * src/Gemma4.Types.pas:139-142: fp16 scale + 16 interleaved nibble bytes per
 * 32 weights).  Bit-exact with CpuMatVecQ4 (src/Gemma4.Tensors.pas:546-598):
 * each logit is the left-to-right single-rounding sum over the row.
 *   d_weights  device, rows*(cols/32)*18 bytes; d_hidden device [batch*cols] fp32;
 *   d_logits   device [batch*logits_stride] fp32 output.  cols % 32 == 0.
 * Stream-ordered on the handle's stream. */
int g4s_lmhead_q4_0(g4s_sampler* sampler, const void* d_weights, int32_t rows, int32_t cols,
                    const float* d_hidden, int32_t batch, float* d_logits,
                    int64_t logits_stride);

/* The LM head of g4s_lmhead_q4_0 (same arguments, same bit-exact logits) on
 * weights in the TILED64 layout (g4s_store_upload_q4_0 / g4s_q4_0_repack):
 * one wave per 64 weight rows with coalesced weight loads.  d_tiles and
 * d_hidden 16-byte aligned, batch*cols*4 < 2 GiB.  Stream-ordered.
 * Replaces the engine's LM-head projection before the sampler
 * (src/Gemma4.Model.pas:1285-1300; CPU form CpuMatVecQ4,
 * src/Gemma4.Tensors.pas:546-598). */
int g4s_lmhead_q4_0_tiled(g4s_sampler* sampler, const void* d_tiles, int32_t rows, int32_t cols,
                          const float* d_hidden, int32_t batch, float* d_logits,
                          int64_t logits_stride);

/* The LM head fused with the sampler: logits of `batch` hidden vectors over
 * the handle's `vocab` rows of TILED64 weights, then g4s_sample_ex on them
 * (same params / u / ids / outputs, same results).  The LM head keeps, per
 * hidden vector and 64-row group, the group's largest logit (as a candidate
 * key), its row and a bound of the group's second largest; top-k rows then
 * take only the groups that can hold their top K (the K-th largest group
 * maximum bounds the K-th largest logit from below).
 *   d_logits != NULL: the logits are also written (f32, logits_stride >=
 *     vocab, a multiple of 4); candidate groups are read back from them and
 *     rows with TopK <= 0, >= V or above g4s_max_top_k() take the usual
 *     paths on them.
 *   d_logits == NULL: no logits are written (logits_stride is ignored).  A
 *     candidate group contributes its largest logit, unless its second
 *     largest may also be a candidate: then its 64 logits for that vector
 *     are recomputed in the LM head's term order (bit-exact).  A row whose
 *     ties at the K-th value need every logit is recomputed whole and
 *     sampled again (G4S_FLAG_ROW_RECOMPUTED); the call allocates that row's
 *     buffer (vocab floats) once per handle.  Every row must be a top-k row
 *     with 0 < TopK <= g4s_max_top_k() (G4S_ERR_INVALID_ARGUMENT otherwise)
 *     and vocab <= 524288 (G4S_ERR_UNSUPPORTED otherwise).
 * Synchronous.  Replaces: Forward's LM head + readback + DoSample
 * (src/Gemma4.Model.pas:1285-1300,1379-1387,2739-2827). */
int g4s_lmhead_sample_q4_0(g4s_sampler* sampler, const void* d_tiles, int32_t cols,
                           const float* d_hidden, int32_t batch, float* d_logits,
                           int64_t logits_stride, const g4s_params* params, const double* u,
                           int32_t* ids, const g4s_outputs* outputs);

/* ------------------------------------------------------------------------
 * Batched decode loop: TModel.Generate (src/Gemma4.Model.pas:2829-2938) for
 * `batch` sequences at once, around a forward pass the caller supplies.
 * ---------------------------------------------------------------------- */

/* IsEosToken, src/Gemma4.Types.pas:65-67,554-559 */
#define G4S_EOS_TOKEN_1 1
#define G4S_EOS_TOKEN_2 106
#define G4S_EOS_TOKEN_3 50

/* The caller's model step (Generate's Forward(LTokenId)): tokens[b] is the
 * token sequence b feeds next, or -1 when sequence b takes no further step.
 * On return the raw logits of every sequence with tokens[b] >= 0 must be in
 * row b of the loop's logits buffer, written by work on the sampler's stream
 * or already complete.  Return 0 to go on; anything else ends the loop with
 * G4S_ERR_ABORTED. */
typedef int (*g4s_forward_fn)(void* user, const int32_t* tokens, int32_t batch);

/* System.Random for sequence `seq`: the uniform in [0,1) its next draw uses.
 * Called only for rows with T > 0, once per sampled token, sequences in
 * index order within a step (each sequence sees its own draws in the order
 * Generate would make them). */
typedef double (*g4s_random_fn)(void* user, int32_t seq);

/* Generate's ACallback (TGenerateCallback, Model.pas:78-84), per sequence:
 * return 0 to stop that sequence after `token`. */
typedef int (*g4s_token_fn)(void* user, int32_t seq, int32_t token);

/* DoEmbeddingLookup (src/Gemma4.Model.pas:2047-2080) for a Q4_0 table in the
 * ROWS layout: d_hidden[b*cols ..] = dequantised row d_tokens[b] times
 * `scale` (the engine passes fl32(sqrt(hidden_size))); a token outside
 * [0, rows) gives zeros.  d_tokens device int32 [batch].  Stream-ordered. */
int g4s_embed_q4_0(g4s_sampler* sampler, const void* d_weights, int32_t rows, int32_t cols,
                   const int32_t* d_tokens, int32_t batch, float scale, float* d_hidden);

/* Generate for `batch` sequences (params[b] each), every sequence following
 * Model.pas:2887-2928: d_logits (dtype, row_stride as for g4s_sample) holds
 * each sequence's logits after its prompt; the first token is sampled from
 * them; then, while fewer than max_tokens tokens are out, the token is
 * appended, an EOS token or a 0 from on_token (may be NULL) ends the
 * sequence, and otherwise `forward` is called and the next token sampled.
 * As in the reference, the sequence that appends its max_tokens-th token
 * still takes that last forward and sample (their token is not returned),
 * so a caller's random stream advances exactly as Generate's would.
 * Sequences that end stop taking steps; the rest go on together.  Outputs:
 * tokens[b*max_tokens + i] (host) and lengths[b] (host).  Synchronous. */
int g4s_generate(g4s_sampler* sampler, int32_t batch, const g4s_params* params,
                 int32_t max_tokens, const void* d_logits, int32_t dtype, int64_t row_stride,
                 g4s_forward_fn forward, g4s_random_fn random, g4s_token_fn on_token, void* user,
                 int32_t* tokens, int32_t* lengths);

/* ------------------------------------------------------------------------
 * Weight store: the engine's VPK archive and the Q4_0 LM head weight.
 *
 * TWeightStore (src/Gemma4.Tensors.pas:321-506) over TVFS
 * (src/vendor/StdApp/StdApp.VFS.pas:243-363): a memory-mapped VPK0 archive
 * holding a JSON manifest and one weights file.  The tied embedding of
 * Gemma 4 ("model.language_model.embed_tokens.weight", Q4_0 [262144, 2560],
 * src/Gemma4.Model.pas:1297-1298) is the LM head of the sampler's config-5
 * workload; g4s_store_upload_q4_0 puts it in device memory.
 * ---------------------------------------------------------------------- */

typedef struct g4s_store g4s_store;

/* TDtypeKind, src/Gemma4.Types.pas:94-100 (same order). */
typedef enum g4s_wdtype {
    G4S_WDTYPE_UNKNOWN = 0,
    G4S_WDTYPE_BF16 = 1,
    G4S_WDTYPE_F16 = 2,
    G4S_WDTYPE_F32 = 3,
    G4S_WDTYPE_Q4_0 = 4
} g4s_wdtype;

#define G4S_MAX_DIMS 8

/* TTensorInfo, src/Gemma4.Types.pas:119-129 (the name is returned apart). */
typedef struct g4s_tensor_info {
    int32_t source_dtype; /* g4s_wdtype */
    int32_t output_dtype; /* g4s_wdtype */
    uint64_t offset;      /* bytes from the start of the weights file */
    uint64_t size;        /* bytes */
    int32_t ndim;
    int32_t shape[G4S_MAX_DIMS];
} g4s_tensor_info;

/* Device layouts of a Q4_0 matrix [rows, cols] (cols % 32 == 0).
 *   ROWS     the engine's TQ4Block rows as stored (src/Gemma4.Types.pas:
 *            139-142): per 32 weights an fp16 scale and 16 bytes whose low
 *            nibble is weight 2j and high nibble weight 2j+1;
 *            rows*(cols/32)*18 bytes.  The layout of g4s_lmhead_q4_0.
 *   TILED64  tiles of 64 rows x 32 columns, tile (g, k) at byte
 *            (g*(cols/32) + k)*1280: 64 binary32 scales (each fp16 scale
 *            widened as TFloat16.ToSingle, src/Gemma4.Types.pas:438-481),
 *            then the 64 rows' 16 nibble bytes as stored; rows past the end
 *            of the matrix have scale 0.  ceil(rows/64)*(cols/32)*1280 bytes.
 *            The layout of g4s_lmhead_q4_0_tiled. */
#define G4S_Q4_LAYOUT_ROWS 0
#define G4S_Q4_LAYOUT_TILED64 1

/* TWeightStore.Open (src/Gemma4.Tensors.pas:321-380): map the archive
 * (its extension is forced to .vpk as TVFS.Open does), read and parse the
 * manifest, find the weights file.  manifest_path / weights_path NULL mean
 * the engine's "E4B/manifest.json" / "E4B/weights.bin" (Types.pas:79,85);
 * paths are matched case-insensitively with '\' read as '/'.  On failure
 * *out is NULL and g4s_store_last_error(NULL) says why. */
int g4s_store_open(g4s_store** out, const char* vpk_path, const char* manifest_path,
                   const char* weights_path);

/* TWeightStore.Close (Tensors.pas:382-389): unmap and release.  NULL is accepted. */
int g4s_store_close(g4s_store* store);

/* Message of the last failure on `store`; with NULL, of the last failed
 * g4s_store_open, g4s_q4_0_repack or handle-free call on this thread. */
const char* g4s_store_last_error(const g4s_store* store);

/* TWeightStore.TensorCount / GetTensorInfo / FindTensor (Tensors.pas:508-
 * 516, 457-467).  `name` (optional) receives the NUL-terminated tensor name. */
int32_t g4s_store_tensor_count(const g4s_store* store);
int g4s_store_tensor_info(g4s_store* store, int32_t index, g4s_tensor_info* info, char* name,
                          int32_t name_capacity);
int g4s_store_find_tensor(g4s_store* store, const char* name, g4s_tensor_info* info);

/* TWeightStore.GetRawPointer (Tensors.pas:469-475): the tensor's bytes in
 * the mapped archive (host memory, valid until g4s_store_close), or NULL. */
const void* g4s_store_raw_pointer(g4s_store* store, const char* name);

/* CRC-32 of every archive entry against its directory record (the checksum
 * TVFS writes when packing, StdApp.VFS.pas:600-602). */
int g4s_store_verify(g4s_store* store);

/* Bytes a Q4_0 matrix takes in `layout`, or -1 for bad sizes / layouts. */
int64_t g4s_q4_0_device_bytes(int32_t rows, int32_t cols, int32_t layout);

/* LoadTensor of a Q4_0 tensor (Tensors.pas:477-506) plus the engine's
 * staged GPU upload (src/Gemma4.Model.pas:494-640): the [rows, cols] Q4_0
 * tensor `name` is copied into d_dst (device, 16-byte aligned,
 * dst_bytes >= g4s_q4_0_device_bytes) in `layout`.  Returns when the data
 * is in place; work is ordered on hip_stream (NULL = default stream). */
int g4s_store_upload_q4_0(g4s_store* store, const char* name, int32_t layout, void* d_dst,
                          uint64_t dst_bytes, void* hip_stream);

/* Device-side conversion of a ROWS-layout matrix into TILED64 (stream-
 * ordered; d_tiled 16-byte aligned, g4s_q4_0_device_bytes(.., TILED64)
 * bytes).  No counterpart in the reference: the engine repacks on the host
 * (Model.pas:513-530) into its own planar layout. */
int g4s_q4_0_repack(const void* d_rows, int32_t rows, int32_t cols, void* d_tiled,
                    void* hip_stream);

#ifdef __cplusplus
}
#endif
#endif
