/*
 * g4s_oracle.h -- CPU restatement of the Gemma4.pas token sampler.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * MI355X sampler (libgemma4_sampler.so).  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product never does.
 *
 * Every function restates one reference routine statement by statement
 * (file:line given on each declaration, paths relative to the reference
 * repository root).  The reference is Object Pascal (Delphi 12, Win64 only)
 * and cannot be compiled here, so its floating-point semantics are fixed as:
 *   - each assignment to a Single rounds once to binary32;
 *   - compound right-hand sides are evaluated in Extended, modelled as
 *     `long double` (x87 80-bit).  Build with -DORC_EXTENDED_IS_DOUBLE to
 *     model Extended as binary64 instead (Win64 Delphi);
 *   - System.Exp / System.Math.Tanh are evaluated in Extended (expl / tanhl)
 *     and rounded once to Single on assignment;
 *   - System.Random is replaced by a caller-supplied uniform u (double).
 * Compile with -ffp-contract=off so no product/sum pair is fused.
 */
#ifndef G4S_ORACLE_H
#define G4S_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* TSamplingParams, src/Gemma4.Model.pas:70-76 */
typedef struct orc_params {
    float   temperature;
    int32_t top_k;
    float   top_p;
    float   repetition_penalty; /* never read by DoSample (Model.pas:2739-2827) */
} orc_params;

/* Everything DoSample computed on the way to its answer. */
typedef struct orc_detail {
    int32_t path;        /* 0 = top-k path (Model.pas:2765-2826), 1 = full-vocab path (:2756-2763) */
    int32_t count;       /* survivors on the top-k path, V on the full path */
    int32_t argmax_pos;  /* greedy position (LBest / argmax of p) before any draw */
    int32_t chosen_pos;  /* position of the returned token among the candidates */
    int32_t drew;        /* 1 when Temperature > 0 (a draw against u*TopP happened) */
    int32_t reached;     /* 1 when the running sum reached the threshold */
    float   lsum;        /* softmax denominator LSum */
    float   threshold;   /* LRand = fl32(u * TopP) */
    float   cum_prev;    /* running sum just before chosen_pos (0 when chosen_pos == 0) */
    float   cum_at;      /* running sum at chosen_pos */
    float   max_val;     /* LMax after softcap and temperature */
    int32_t token;       /* returned token id */
} orc_detail;

const char* orc_semantics(void);

/* TBFloat16.ToSingle / FromSingle, src/Gemma4.Types.pas:417-434 */
float    orc_bf16_to_f32(uint16_t v);
uint16_t orc_f32_to_bf16(float v);
/* TFloat16.ToSingle / FromSingle, src/Gemma4.Types.pas:438-501 */
float    orc_f16_to_f32(uint16_t v);
uint16_t orc_f16_from_f32(float v);

/* CpuLogitSoftcap, src/Gemma4.Layers.pas:300-316 (in place) */
void  orc_logit_softcap(float* data, int32_t count, float cap);
/* The inline softcap of the top-k path, src/Gemma4.Model.pas:2775-2776 */
float orc_softcap_topk(float x, float cap);
/* CpuSoftmaxF32, src/Gemma4.Tensors.pas:638-673 (in place); returns LSum */
float orc_softmax_f32(float* data, int32_t count);
/* One `Exp(a - b)` assignment to a Single (Tensors.pas:660, Model.pas:2797) */
float orc_exp_diff(float a, float b);

/* DoSelectTopKIndices, src/Gemma4.Model.pas:2615-2689.  Writes the survivor
 * indices ascending and returns their count (<= K). */
int32_t orc_select_topk_indices(const float* logits, int32_t vocab, int32_t k, int32_t* out_idx);

/* DoSampleTopP, src/Gemma4.Model.pas:2691-2737 (modifies logits in place:
 * on return they hold the normalized probabilities). */
int32_t orc_sample_topp(float* logits, int32_t count, float top_p, float temperature,
                        double u, orc_detail* detail);

/* DoSample, src/Gemma4.Model.pas:2739-2827 on one row of fp32 logits.
 * out_idx/out_probs (optional) receive the candidates and their normalized
 * probabilities: K' survivors on the top-k path, all V on the full path
 * (capacity `cap` entries; the full path writes them only when cap >= V). */
int32_t orc_do_sample(const float* logits, int32_t vocab, float softcap, const orc_params* params,
                      double u, int32_t* out_idx, float* out_probs, int32_t cap,
                      orc_detail* detail);

/* DoSample over a batch of rows (dtype 0 = fp32, 1 = bf16 widened by
 * TBFloat16.ToSingle), rows spread over `threads` host threads.  This is the
 * CPU baseline the benchmark times.  Returns 0. */
int32_t orc_sample_batch(const void* logits, int32_t dtype, int32_t vocab, int64_t row_stride,
                         int32_t batch, const orc_params* params, const double* u, float softcap,
                         int32_t* ids, int32_t threads);

/* TQ4Block (src/Gemma4.Types.pas:139-142) helpers */
void     orc_dequant_q4_block(const uint8_t* block18, float* dst32);         /* Quant.pas:209-239 */
uint64_t orc_f32_to_q4_buffer(const float* src, uint8_t* dst, uint64_t count); /* Quant.pas:121-197 */
/* CpuMatVecQ4, src/Gemma4.Tensors.pas:546-598; rows [row0, row0+nrows) only */
void orc_matvec_q4(const uint8_t* matrix, const float* vec, float* dst, int32_t rows, int32_t cols,
                   int32_t row0, int32_t nrows);
/* CpuMatVecQ4 for `batch` hidden vectors, rows split across threads. */
void orc_matvec_q4_batch(const uint8_t* matrix, const float* vecs, float* dst, int32_t rows,
                         int32_t cols, int32_t batch, int32_t threads);

/* Literal left-to-right binary32 running sum; returns the final sum and,
 * when `threshold` is reached, the first index with sum >= threshold in
 * *first_reach (else -1).  (The loops at Tensors.pas:657-663, Model.pas:2727-2735.) */
float orc_seqsum_f32(const float* a, int64_t n, float threshold, int64_t* first_reach);

#ifdef __cplusplus
}
#endif
#endif
