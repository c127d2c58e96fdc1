/*
 * g4w.hip -- host and gfx950 generators for the sampler's synthetic workloads
 * (libg4s_workload.so).  The host functions and the kernels evaluate the same
 * g4w.h expressions, so both sides produce bit-identical rows.  Used by the
 * benchmark and the parity tests; not part of the sampler library.
 */
#include <hip/hip_runtime.h>

#include <thread>
#include <vector>

#include "g4w.h"
#include "g4w_api.h"

#define G4W_API extern "C" __attribute__((visibility("default")))

namespace {

template <typename F>
void parallel_rows(int64_t nrows, int threads, F f)
{
    if (threads < 1) threads = 1;
    if (threads == 1 || nrows < 2) {
        for (int64_t r = 0; r < nrows; ++r) f(r);
        return;
    }
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t)
        pool.emplace_back([=]() {
            for (int64_t r = t; r < nrows; r += threads) f(r);
        });
    for (auto& th : pool) th.join();
}

/* Greedy planting on one host row: copy the row maximum to 2..4 indices. */
void plant_host(uint64_t seed, uint64_t row, int32_t vocab, float* x)
{
    int32_t best = 0;
    for (int32_t i = 1; i < vocab; ++i)
        if (x[i] > x[best]) best = i;
    int32_t idx[4];
    int n = g4w_plant_indices(seed, row, vocab, best, idx);
    for (int j = 0; j < n; ++j) x[idx[j]] = x[best];
}

}  // namespace

/* Peaky rows [row0, row0+nrows): rows with (row % greedy_every == greedy_every-1)
 * get the greedy planting when greedy_every > 0. */
G4W_API void g4w_host_peaky_rows(uint64_t seed, int64_t row0, int64_t nrows, int32_t vocab,
                                 int64_t stride, float* out, int32_t greedy_every, int32_t threads)
{
    parallel_rows(nrows, threads, [=](int64_t r) {
        uint64_t row = (uint64_t)(row0 + r);
        float* x = out + r * stride;
        for (int32_t i = 0; i < vocab; ++i) x[i] = g4w_peaky_base(seed, row, (uint64_t)i);
        int32_t sidx[G4W_NSPIKES];
        float sval[G4W_NSPIKES];
        g4w_peaky_spikes(seed, row, vocab, sidx, sval);
        int ns = G4W_NSPIKES < vocab ? G4W_NSPIKES : vocab;
        for (int j = 0; j < ns; ++j) x[sidx[j]] = sval[j];
        if (greedy_every > 0 && (row % (uint64_t)greedy_every) == (uint64_t)(greedy_every - 1))
            plant_host(seed, row, vocab, x);
    });
}

G4W_API void g4w_host_flat_bf16_rows(uint64_t seed, int64_t row0, int64_t nrows, int32_t vocab,
                                     int64_t stride, uint16_t* out, int32_t threads)
{
    parallel_rows(nrows, threads, [=](int64_t r) {
        uint64_t row = (uint64_t)(row0 + r);
        uint16_t* x = out + r * stride;
        for (int32_t i = 0; i < vocab; ++i) x[i] = g4w_flat_bf16(seed, row, (uint64_t)i);
    });
}

G4W_API void g4w_host_row_u(uint64_t seed, int64_t row0, int64_t nrows, double* u)
{
    for (int64_t r = 0; r < nrows; ++r) u[r] = g4w_row_u(seed, (uint64_t)(row0 + r));
}

G4W_API void g4w_host_mixed_params(uint64_t seed, int64_t row0, int64_t nrows, float* t,
                                   int32_t* k, float* p)
{
    for (int64_t r = 0; r < nrows; ++r)
        g4w_mixed_params(seed, (uint64_t)(row0 + r), &t[r], &k[r], &p[r]);
}

G4W_API void g4w_host_hidden(uint64_t seed, int32_t batch, int32_t cols, float* out)
{
    for (int32_t b = 0; b < batch; ++b)
        for (int32_t c = 0; c < cols; ++c)
            out[(int64_t)b * cols + c] = g4w_hidden(seed, (uint64_t)b, (uint64_t)c);
}

G4W_API void g4w_host_q4_weights(uint64_t seed, int64_t block0, int64_t nblocks, uint8_t* out,
                                 int32_t threads)
{
    int64_t per = 4096;
    int64_t nchunks = (nblocks + per - 1) / per;
    parallel_rows(nchunks, threads, [=](int64_t c) {
        int64_t b0 = c * per, b1 = b0 + per < nblocks ? b0 + per : nblocks;
        for (int64_t b = b0; b < b1; ++b) g4w_q4_block(seed, (uint64_t)(block0 + b), out + b * 18);
    });
}

/* ------------------------------------------------------------------ kernels */

__global__ void k_peaky_base(uint64_t seed, int64_t row0, int32_t vocab, int64_t stride, float* out)
{
    int64_t r = blockIdx.y;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < vocab) out[r * stride + i] = g4w_peaky_base(seed, (uint64_t)(row0 + r), (uint64_t)i);
}

__global__ void k_peaky_spikes(uint64_t seed, int64_t row0, int64_t nrows, int32_t vocab,
                               int64_t stride, float* out)
{
    int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= nrows) return;
    int32_t sidx[G4W_NSPIKES];
    float sval[G4W_NSPIKES];
    g4w_peaky_spikes(seed, (uint64_t)(row0 + r), vocab, sidx, sval);
    int ns = G4W_NSPIKES < vocab ? G4W_NSPIKES : vocab;
    for (int j = 0; j < ns; ++j) out[r * stride + sidx[j]] = sval[j];
}

/* One 256-thread block per row: first index of the maximum, then planting. */
__global__ __launch_bounds__(256) void k_plant(uint64_t seed, int64_t row0, int32_t vocab,
                                               int64_t stride, float* out, int32_t greedy_every)
{
    int64_t r = blockIdx.x;
    uint64_t row = (uint64_t)(row0 + r);
    if ((row % (uint64_t)greedy_every) != (uint64_t)(greedy_every - 1)) return;
    float* x = out + r * stride;
    __shared__ float sv[256];
    __shared__ int32_t si[256];
    float bv = -__builtin_inff();
    int32_t bi = vocab;
    for (int32_t i = threadIdx.x; i < vocab; i += 256) {
        float v = x[i];
        if (v > bv) {
            bv = v;
            bi = i;
        }
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            float ov = sv[threadIdx.x + s];
            int32_t oi = si[threadIdx.x + s];
            if (ov > sv[threadIdx.x] || (ov == sv[threadIdx.x] && oi < si[threadIdx.x])) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        int32_t best = si[0];
        int32_t idx[4];
        int n = g4w_plant_indices(seed, row, vocab, best, idx);
        for (int j = 0; j < n; ++j) x[idx[j]] = x[best];
    }
}

__global__ void k_flat_bf16(uint64_t seed, int64_t row0, int32_t vocab, int64_t stride, uint16_t* out)
{
    int64_t r = blockIdx.y;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < vocab) out[r * stride + i] = g4w_flat_bf16(seed, (uint64_t)(row0 + r), (uint64_t)i);
}

__global__ void k_q4_blocks(uint64_t seed, int64_t block0, int64_t nblocks, uint8_t* out)
{
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    uint8_t tmp[18];
    g4w_q4_block(seed, (uint64_t)(block0 + b), tmp);
    for (int j = 0; j < 18; ++j) out[b * 18 + j] = tmp[j];
}

__global__ void k_hidden(uint64_t seed, int32_t batch, int32_t cols, float* out)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)batch * cols) return;
    out[i] = g4w_hidden(seed, (uint64_t)(i / cols), (uint64_t)(i % cols));
}

/* Device generators: all pointers are device memory, work is stream-ordered.
 * Return 0 on success or the hipError_t of the failing launch. */
G4W_API int g4w_dev_peaky_rows(uint64_t seed, int64_t row0, int64_t nrows, int32_t vocab,
                               int64_t stride, float* out, int32_t greedy_every, void* stream)
{
    hipStream_t s = (hipStream_t)stream;
    for (int64_t r0 = 0; r0 < nrows; r0 += 65535) {
        int64_t nr = nrows - r0 < 65535 ? nrows - r0 : 65535;
        dim3 g((unsigned)((vocab + 255) / 256), (unsigned)nr);
        hipLaunchKernelGGL(k_peaky_base, g, dim3(256), 0, s, seed, row0 + r0, vocab, stride,
                           out + r0 * stride);
        hipLaunchKernelGGL(k_peaky_spikes, dim3((unsigned)((nr + 63) / 64)), dim3(64), 0, s, seed,
                           row0 + r0, nr, vocab, stride, out + r0 * stride);
        if (greedy_every > 0)
            hipLaunchKernelGGL(k_plant, dim3((unsigned)nr), dim3(256), 0, s, seed, row0 + r0, vocab,
                               stride, out + r0 * stride, greedy_every);
    }
    return (int)hipGetLastError();
}

G4W_API int g4w_dev_flat_bf16_rows(uint64_t seed, int64_t row0, int64_t nrows, int32_t vocab,
                                   int64_t stride, uint16_t* out, void* stream)
{
    hipStream_t s = (hipStream_t)stream;
    for (int64_t r0 = 0; r0 < nrows; r0 += 65535) {
        int64_t nr = nrows - r0 < 65535 ? nrows - r0 : 65535;
        dim3 g((unsigned)((vocab + 255) / 256), (unsigned)nr);
        hipLaunchKernelGGL(k_flat_bf16, g, dim3(256), 0, s, seed, row0 + r0, vocab, stride,
                           out + r0 * stride);
    }
    return (int)hipGetLastError();
}

G4W_API int g4w_dev_q4_weights(uint64_t seed, int64_t block0, int64_t nblocks, uint8_t* out,
                               void* stream)
{
    hipLaunchKernelGGL(k_q4_blocks, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, seed, block0, nblocks, out);
    return (int)hipGetLastError();
}

G4W_API int g4w_dev_hidden(uint64_t seed, int32_t batch, int32_t cols, float* out, void* stream)
{
    int64_t n = (int64_t)batch * cols;
    hipLaunchKernelGGL(k_hidden, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, seed, batch, cols, out);
    return (int)hipGetLastError();
}
