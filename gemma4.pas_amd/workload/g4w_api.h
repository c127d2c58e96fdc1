/*
 * g4w_api.h -- exported functions of libg4s_workload.so (workload/g4w.hip):
 * the synthetic rows of the sampler's benchmark configurations, generated
 * bit-identically on the host and on the device.
 */
#ifndef G4W_API_H
#define G4W_API_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void g4w_host_peaky_rows(uint64_t seed, int64_t row0, int64_t nrows, int32_t vocab, int64_t stride,
                         float* out, int32_t greedy_every, int32_t threads);
void g4w_host_flat_bf16_rows(uint64_t seed, int64_t row0, int64_t nrows, int32_t vocab,
                             int64_t stride, uint16_t* out, int32_t threads);
void g4w_host_row_u(uint64_t seed, int64_t row0, int64_t nrows, double* u);
void g4w_host_mixed_params(uint64_t seed, int64_t row0, int64_t nrows, float* t, int32_t* k,
                           float* p);
void g4w_host_hidden(uint64_t seed, int32_t batch, int32_t cols, float* out);
void g4w_host_q4_weights(uint64_t seed, int64_t block0, int64_t nblocks, uint8_t* out,
                         int32_t threads);

/* device generators: pointers are device memory, work is ordered on `stream` */
int g4w_dev_peaky_rows(uint64_t seed, int64_t row0, int64_t nrows, int32_t vocab, int64_t stride,
                       float* out, int32_t greedy_every, void* stream);
int g4w_dev_flat_bf16_rows(uint64_t seed, int64_t row0, int64_t nrows, int32_t vocab,
                           int64_t stride, uint16_t* out, void* stream);
int g4w_dev_q4_weights(uint64_t seed, int64_t block0, int64_t nblocks, uint8_t* out, void* stream);
int g4w_dev_hidden(uint64_t seed, int32_t batch, int32_t cols, float* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif
