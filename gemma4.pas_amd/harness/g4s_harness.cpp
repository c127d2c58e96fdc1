/*
 * g4s_harness.cpp -- native timing loops over the libgemma4_sampler.so C ABI.
 *
 * Benchmark plumbing, not part of the sampler: it drives the same entry
 * points a host engine binds (g4s_sample, g4s_sample_async) and times them
 * without an interpreter between the clock and the call.  Rows are produced
 * on the device by the workload generator (libg4s_workload.so) outside the
 * timed region, into the buffer the sampler then reads, so every sample sees
 * freshly written logits the way the engine's LM head leaves them.
 */
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <vector>

#include "gemma4_sampler.h"
#include "../workload/g4w_api.h"

#define G4H_API extern "C" __attribute__((visibility("default")))

namespace {

inline double now_us()
{
    return std::chrono::duration<double, std::micro>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

__global__ void g4h_null_kernel(uint32_t* flag, uint32_t seq)
{
    if (threadIdx.x == 0 && flag)
        __hip_atomic_store(flag, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace

/*
 * Host-side floor of a synchronous single-kernel call: `n` launches of an
 * empty one-wave kernel, each followed by
 *   mode 0: hipStreamSynchronize
 *   mode 1: a host spin on a pinned flag the kernel stores (system scope),
 *           then hipStreamSynchronize only after the timed region
 * us[i] = wall clock from before the launch to the end of the wait.
 */
G4H_API int g4h_null_roundtrip(void* stream, int32_t n, int32_t mode, double* us)
{
    hipStream_t st = (hipStream_t)stream;
    uint32_t* flag = nullptr;
    if (hipHostMalloc((void**)&flag, 64, hipHostMallocCoherent) != hipSuccess) return -101;
    *flag = 0;
    int rc = 0;
    for (int32_t i = 0; i < n && rc == 0; ++i) {
        const uint32_t seq = (uint32_t)i + 1u;
        double t0 = now_us();
        hipLaunchKernelGGL(g4h_null_kernel, dim3(1), dim3(64), 0, st, mode == 1 ? flag : nullptr,
                           seq);
        if (hipGetLastError() != hipSuccess) {
            rc = -102;
            break;
        }
        if (mode == 1) {
            /* bounded spin: ~2 s, then give up and report */
            uint64_t spins = 0;
            while (__atomic_load_n(flag, __ATOMIC_ACQUIRE) != seq && ++spins < 2000000000ull) {
            }
            if (spins >= 2000000000ull) rc = -103;
        } else if (hipStreamSynchronize(st) != hipSuccess) {
            rc = -104;
        }
        us[i] = now_us() - t0;
        if (mode == 1 && hipStreamSynchronize(st) != hipSuccess) rc = -104;
    }
    (void)hipStreamSynchronize(st);
    (void)hipHostFree(flag);
    return rc;
}

/*
 * The floor of a one-kernel hipGraph launch on this stream, measured as the
 * graph leg of the decode stream measures the sampler (g4h_graph_decode): a
 * graph holding one launch of a null kernel, captured once, launched `n`
 * times from an idle stream, each launch between two events; gpu_us[i] =
 * event time of launch i, call_us[i] = host time spent inside the
 * hipGraphLaunch call itself.
 */
G4H_API int g4h_graph_floor(void* stream, int32_t n, float* gpu_us, double* call_us)
{
    hipStream_t st = (hipStream_t)stream;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipGraph_t g = nullptr;
    hipGraphExec_t gx = nullptr;
    int rc = 0;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) rc = -101;
    if (rc == 0 && hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess)
        rc = -102;
    if (rc == 0) {
        hipLaunchKernelGGL(g4h_null_kernel, dim3(1), dim3(64), 0, st, nullptr, 1u);
        if (hipStreamEndCapture(st, &g) != hipSuccess) rc = -103;
    }
    if (rc == 0 && hipGraphInstantiate(&gx, g, nullptr, nullptr, 0) != hipSuccess) rc = -104;
    for (int32_t i = 0; rc == 0 && i < n; ++i) {
        if (hipStreamSynchronize(st) != hipSuccess) rc = -105;
        (void)hipEventRecord(e0, st);
        const double t0 = now_us();
        if (rc == 0 && hipGraphLaunch(gx, st) != hipSuccess) rc = -106;
        call_us[i] = now_us() - t0;
        (void)hipEventRecord(e1, st);
        if (rc == 0 && hipEventSynchronize(e1) != hipSuccess) rc = -107;
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        gpu_us[i] = ms * 1000.0f;
    }
    (void)hipStreamSynchronize(st);
    if (gx) (void)hipGraphExecDestroy(gx);
    if (g) (void)hipGraphDestroy(g);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    return rc;
}

/*
 * Decode-style latency: `nrows` single-row samples back to back.  Row r of
 * the peaky workload (every `greedy_every`-th row greedy, TopK = 1, with the
 * maximum planted 2-4 more times) is generated into d_row, then sampled with
 * T, K, P and u of that row.
 *   mode 0: g4s_sample (synchronous; host params in, host id out), nothing
 *           else inside the timed region (gpu_us[r] = 0)
 *   mode 1: g4s_sample_async (params and u already on the device) + a
 *           4-byte id readback and a stream sync, between two hipEvents
 *   mode 2: g4s_sample as in mode 0, between two hipEvents
 * host_us[r]: wall clock of the sampler call, entry to id on the host
 *             (modes 1 and 2: including the two event records).
 * gpu_us[r] : hipEvent time of the same work on the sampler's stream.
 * ids[r]    : the sampled token id.
 */
G4H_API int g4h_decode_latency(g4s_sampler* s, void* stream, void* d_row, uint64_t seed,
                               int32_t row0, int32_t nrows, int32_t vocab, int32_t greedy_every,
                               float temperature, int32_t top_k, float top_p, int32_t mode,
                               double* host_us, float* gpu_us, int32_t* ids)
{
    hipStream_t st = (hipStream_t)stream;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -100;
    g4s_params* dpar = nullptr;
    double* du = nullptr;
    int32_t* did = nullptr;
    int32_t* hid = nullptr;
    g4s_params* hpar = nullptr;
    double* hu = nullptr;
    int rc = 0;
    if (hipMalloc((void**)&dpar, sizeof(g4s_params)) != hipSuccess ||
        hipMalloc((void**)&du, sizeof(double)) != hipSuccess ||
        hipMalloc((void**)&did, sizeof(int32_t)) != hipSuccess ||
        hipHostMalloc((void**)&hid, sizeof(int32_t), hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc((void**)&hpar, sizeof(g4s_params), hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc((void**)&hu, sizeof(double), hipHostMallocDefault) != hipSuccess)
        rc = -101;
    for (int32_t i = 0; rc == 0 && i < nrows; ++i) {
        const int32_t r = row0 + i;
        g4s_params p;
        p.temperature = temperature;
        p.top_k = (greedy_every > 0 && (r % greedy_every) == greedy_every - 1) ? 1 : top_k;
        p.top_p = top_p;
        p.repetition_penalty = 1.0f;
        double u = 0.0;
        g4w_host_row_u(seed, r, 1, &u);
        if (g4w_dev_peaky_rows(seed, r, 1, vocab, vocab, (float*)d_row, greedy_every, st) != 0) {
            rc = -102;
            break;
        }
        if (mode == 1) {
            *hpar = p;
            *hu = u;
            if (hipMemcpyAsync(dpar, hpar, sizeof(p), hipMemcpyHostToDevice, st) != hipSuccess ||
                hipMemcpyAsync(du, hu, sizeof(u), hipMemcpyHostToDevice, st) != hipSuccess) {
                rc = -103;
                break;
            }
        }
        if (hipStreamSynchronize(st) != hipSuccess) {
            rc = -104;
            break;
        }
        int32_t id = -1;
        double t0 = now_us();
        if (mode == 0) {
            rc = g4s_sample(s, d_row, G4S_DTYPE_F32, vocab, 1, &p, &u, &id);
            const double t1 = now_us();
            if (rc != 0) break;
            host_us[i] = t1 - t0;
            gpu_us[i] = 0.0f;
            ids[i] = id;
            continue;
        }
        (void)hipEventRecord(e0, st);
        if (mode == 2) {
            rc = g4s_sample(s, d_row, G4S_DTYPE_F32, vocab, 1, &p, &u, &id);
            (void)hipEventRecord(e1, st);
        } else {
            rc = g4s_sample_async(s, d_row, G4S_DTYPE_F32, vocab, 1, dpar, du, top_k, 0, did,
                                  nullptr);
            if (rc == 0 && hipMemcpyAsync(hid, did, 4, hipMemcpyDeviceToHost, st) != hipSuccess)
                rc = -105;
            (void)hipEventRecord(e1, st);
            if (rc == 0 && hipStreamSynchronize(st) != hipSuccess) rc = -106;
            id = *hid;
        }
        double t1 = now_us();
        if (rc != 0) break;
        (void)hipEventSynchronize(e1);
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        host_us[i] = t1 - t0;
        gpu_us[i] = ms * 1000.0f;
        ids[i] = id;
    }
    (void)hipStreamSynchronize(st);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (dpar) (void)hipFree(dpar);
    if (du) (void)hipFree(du);
    if (did) (void)hipFree(did);
    if (hid) (void)hipHostFree(hid);
    if (hpar) (void)hipHostFree(hpar);
    if (hu) (void)hipHostFree(hu);
    return rc;
}

/*
 * A train of `steps` stream-ordered samples of the same resident batch with
 * no event between them: *total_us is the event time from before the first
 * to after the last, so total_us / steps is the average launch duration
 * including only the gap between consecutive kernels.
 */
G4H_API int g4h_launch_train(g4s_sampler* s, void* stream, const void* d_logits, int32_t dtype,
                             int64_t row_stride, int32_t batch, const g4s_params* d_params,
                             const double* d_u, int32_t k_bound, int32_t full_rows,
                             int32_t* d_ids, int32_t warmup, int32_t steps, float* total_us)
{
    hipStream_t st = (hipStream_t)stream;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess) return -100;
    if (hipEventCreate(&e1) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return -100;
    }
    int rc = 0;
    for (int32_t i = 0; rc == 0 && i < warmup; ++i)
        rc = g4s_sample_async(s, d_logits, dtype, row_stride, batch, d_params, d_u, k_bound,
                              full_rows, d_ids, nullptr);
    if (rc == 0 && hipStreamSynchronize(st) != hipSuccess) rc = -104;
    if (rc == 0) (void)hipEventRecord(e0, st);
    for (int32_t i = 0; rc == 0 && i < steps; ++i)
        rc = g4s_sample_async(s, d_logits, dtype, row_stride, batch, d_params, d_u, k_bound,
                              full_rows, d_ids, nullptr);
    if (rc == 0) (void)hipEventRecord(e1, st);
    if (rc == 0 && hipStreamSynchronize(st) != hipSuccess) rc = -104;
    if (rc == 0) {
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        *total_us = ms * 1000.0f;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

/*
 * Batched throughput: `steps` stream-ordered samples of the same resident
 * batch (g4s_sample_async, parameters on the device), each bracketed by a
 * pair of events on the sampler's stream.  step_us[i] = event time of step
 * i.  `warmup` untimed steps run first.  The whole timed loop is also
 * bracketed by one event pair (total_us) and the host clock (wall_us).
 */
G4H_API int g4h_batch_throughput(g4s_sampler* s, void* stream, const void* d_logits, int32_t dtype,
                                 int64_t row_stride, int32_t batch, const g4s_params* d_params,
                                 const double* d_u, int32_t k_bound, int32_t full_rows,
                                 int32_t* d_ids, int32_t warmup, int32_t steps, float* step_us,
                                 float* total_us, double* wall_us)
{
    hipStream_t st = (hipStream_t)stream;
    std::vector<hipEvent_t> ev((size_t)steps + 1);
    for (auto& e : ev)
        if (hipEventCreate(&e) != hipSuccess) return -100;
    int rc = 0;
    for (int32_t i = 0; rc == 0 && i < warmup; ++i)
        rc = g4s_sample_async(s, d_logits, dtype, row_stride, batch, d_params, d_u, k_bound,
                              full_rows, d_ids, nullptr);
    if (rc == 0 && hipStreamSynchronize(st) != hipSuccess) rc = -104;
    double t0 = now_us();
    if (rc == 0) (void)hipEventRecord(ev[0], st);
    for (int32_t i = 0; rc == 0 && i < steps; ++i) {
        rc = g4s_sample_async(s, d_logits, dtype, row_stride, batch, d_params, d_u, k_bound,
                              full_rows, d_ids, nullptr);
        (void)hipEventRecord(ev[(size_t)i + 1], st);
    }
    if (rc == 0 && hipStreamSynchronize(st) != hipSuccess) rc = -104;
    double t1 = now_us();
    if (rc == 0) {
        for (int32_t i = 0; i < steps; ++i) {
            float ms = 0.0f;
            (void)hipEventElapsedTime(&ms, ev[(size_t)i], ev[(size_t)i + 1]);
            step_us[i] = ms * 1000.0f;
        }
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, ev[0], ev[(size_t)steps]);
        *total_us = ms * 1000.0f;
        *wall_us = t1 - t0;
    }
    for (auto& e : ev) (void)hipEventDestroy(e);
    return rc;
}

/*
 * The decode stream launched from the sampler's own hipGraph
 * (g4s_sample_graph), as a device-resident decode loop runs it: one row on
 * fixed device buffers (logits, parameters, uniform, id; the id stays on the
 * device for the next step), so every call after the first replays the graph
 * the handle captured.  For each row i of d_rows (fp32, row i at
 * d_rows + i*vocab, parameters and uniforms in device arrays) the row is
 * copied into those buffers untimed, then g4s_sample_graph is called:
 * gpu_us[i] = event time around the call on the stream, host_us[i] = call
 * until the host sees the closing event complete, call_us[i] = host time
 * inside g4s_sample_graph, ids[i] = the id (read back untimed).
 */
G4H_API int g4h_graph_decode(g4s_sampler* s, void* stream, const float* d_rows, int32_t vocab,
                             int32_t nrows, const g4s_params* d_params, const double* d_u,
                             int32_t k_bound, double* host_us, float* gpu_us, double* call_us,
                             int32_t* ids)
{
    hipStream_t st = (hipStream_t)stream;
    if (nrows < 1) return -100;
    float* row = nullptr;
    g4s_params* par = nullptr;
    double* u = nullptr;
    int32_t* did = nullptr;
    int32_t* hid = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = 0;
    if (hipMalloc((void**)&row, (size_t)vocab * sizeof(float)) != hipSuccess ||
        hipMalloc((void**)&par, sizeof(g4s_params)) != hipSuccess ||
        hipMalloc((void**)&u, sizeof(double)) != hipSuccess ||
        hipMalloc((void**)&did, sizeof(int32_t)) != hipSuccess ||
        hipHostMalloc((void**)&hid, sizeof(int32_t), hipHostMallocDefault) != hipSuccess ||
        hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
        rc = -101;
    /* the first call captures; it is not timed */
    if (rc == 0 && (hipMemcpyAsync(row, d_rows, (size_t)vocab * sizeof(float),
                                   hipMemcpyDeviceToDevice, st) != hipSuccess ||
                    hipMemcpyAsync(par, d_params, sizeof(g4s_params), hipMemcpyDeviceToDevice,
                                   st) != hipSuccess ||
                    hipMemcpyAsync(u, d_u, sizeof(double), hipMemcpyDeviceToDevice, st) !=
                        hipSuccess ||
                    hipStreamSynchronize(st) != hipSuccess))
        rc = -102;
    if (rc == 0) rc = g4s_sample_graph(s, row, G4S_DTYPE_F32, vocab, 1, par, u, k_bound, 0, did,
                                       nullptr);
    if (rc == 0 && hipStreamSynchronize(st) != hipSuccess) rc = -103;
    for (int32_t i = 0; rc == 0 && i < nrows; ++i) {
        if (hipMemcpyAsync(row, d_rows + (int64_t)i * vocab, (size_t)vocab * sizeof(float),
                           hipMemcpyDeviceToDevice, st) != hipSuccess ||
            hipMemcpyAsync(par, d_params + i, sizeof(g4s_params), hipMemcpyDeviceToDevice, st) !=
                hipSuccess ||
            hipMemcpyAsync(u, d_u + i, sizeof(double), hipMemcpyDeviceToDevice, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
            rc = -106;
            break;
        }
        const double t0 = now_us();
        (void)hipEventRecord(e0, st);
        const double c0 = now_us();
        rc = g4s_sample_graph(s, row, G4S_DTYPE_F32, vocab, 1, par, u, k_bound, 0, did, nullptr);
        const double c1 = now_us();
        (void)hipEventRecord(e1, st);
        while (rc == 0 && hipEventQuery(e1) == hipErrorNotReady) {
        }
        const double t1 = now_us();
        if (rc == 0 && (hipMemcpyAsync(hid, did, sizeof(int32_t), hipMemcpyDeviceToHost, st) !=
                            hipSuccess ||
                        hipStreamSynchronize(st) != hipSuccess))
            rc = -108;
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        host_us[i] = t1 - t0;
        gpu_us[i] = ms * 1000.0f;
        call_us[i] = c1 - c0;
        ids[i] = *hid;
    }
    (void)hipStreamSynchronize(st);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (row) (void)hipFree(row);
    if (par) (void)hipFree(par);
    if (u) (void)hipFree(u);
    if (did) (void)hipFree(did);
    if (hid) (void)hipHostFree(hid);
    return rc;
}

/*
 * The decode stream sampled back to back from hipGraphs: rows i = 0 ..
 * nrows-1 resident at d_rows + i*vocab (fp32, parameters and uniforms in
 * device arrays); each run of `chunk` rows is captured once as one graph of
 * `chunk` g4s_sample_async calls (one row each), launched once untimed and
 * once between two events: chunk_us[c] = event time of chunk c's graph
 * (chunk rows back to back); d_ids[i] receives row i's id.
 */
G4H_API int g4h_graph_chunks(g4s_sampler* s, void* stream, const float* d_rows, int32_t vocab,
                             int32_t nrows, const g4s_params* d_params, const double* d_u,
                             int32_t k_bound, int32_t* d_ids, int32_t chunk, float* chunk_us)
{
    hipStream_t st = (hipStream_t)stream;
    if (nrows < 1 || chunk < 1) return -100;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = 0;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) rc = -101;
    for (int32_t c0 = 0, c = 0; rc == 0 && c0 < nrows; c0 += chunk, ++c) {
        const int32_t n = std::min(chunk, nrows - c0);
        hipGraph_t g = nullptr;
        hipGraphExec_t gx = nullptr;
        if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess) {
            rc = -102;
            break;
        }
        for (int32_t i = 0; i < n && rc == 0; ++i) {
            const int32_t r = c0 + i;
            rc = g4s_sample_async(s, d_rows + (int64_t)r * vocab, G4S_DTYPE_F32, vocab, 1,
                                  d_params + r, d_u + r, k_bound, 0, d_ids + r, nullptr);
        }
        const hipError_t ec = hipStreamEndCapture(st, &g);
        if (rc == 0 && ec != hipSuccess) rc = -104;
        if (rc == 0 && hipGraphInstantiate(&gx, g, nullptr, nullptr, 0) != hipSuccess) rc = -105;
        if (rc == 0 && (hipGraphLaunch(gx, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess))
            rc = -106;
        if (rc == 0) {
            (void)hipEventRecord(e0, st);
            if (hipGraphLaunch(gx, st) != hipSuccess) rc = -107;
            (void)hipEventRecord(e1, st);
            if (rc == 0 && hipEventSynchronize(e1) != hipSuccess) rc = -108;
            float ms = 0.0f;
            (void)hipEventElapsedTime(&ms, e0, e1);
            chunk_us[c] = ms * 1000.0f;
        }
        if (gx) (void)hipGraphExecDestroy(gx);
        if (g) (void)hipGraphDestroy(g);
    }
    (void)hipStreamSynchronize(st);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    return rc;
}

namespace {

/* Plain streaming copy, 16 bytes per lane per step: the calibration kernel
 * for HBM traffic counters (its bytes read and written are known exactly). */
__global__ void g4h_copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, int64_t n)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = src[i];
}

}  // namespace

/*
 * `steps` launches of the calibration copy of `bytes` (a multiple of 16)
 * from src to dst on `stream`; us[i] = event time of launch i.
 */
G4H_API int g4h_copy_throughput(void* stream, const void* src, void* dst, int64_t bytes,
                                int32_t steps, float* us)
{
    hipStream_t st = (hipStream_t)stream;
    if (bytes <= 0 || (bytes & 15) || steps <= 0) return -1;
    const int64_t n = bytes / 16;
    std::vector<hipEvent_t> ev((size_t)steps + 1);
    for (auto& e : ev)
        if (hipEventCreate(&e) != hipSuccess) return -100;
    int rc = 0;
    const int grid = (int)std::min<int64_t>((n + 255) / 256, 4096);
    (void)hipEventRecord(ev[0], st);
    for (int32_t i = 0; i < steps && rc == 0; ++i) {
        hipLaunchKernelGGL(g4h_copy_kernel, dim3(grid), dim3(256), 0, st, (const uint4*)src,
                           (uint4*)dst, n);
        if (hipGetLastError() != hipSuccess) rc = -102;
        (void)hipEventRecord(ev[(size_t)i + 1], st);
    }
    if (hipStreamSynchronize(st) != hipSuccess && rc == 0) rc = -104;
    if (rc == 0)
        for (int32_t i = 0; i < steps; ++i) {
            float ms = 0.0f;
            (void)hipEventElapsedTime(&ms, ev[(size_t)i], ev[(size_t)i + 1]);
            us[i] = ms * 1000.0f;
        }
    for (auto& e : ev) (void)hipEventDestroy(e);
    return rc;
}

/*
 * LM head + sampler, stream-ordered: per step g4s_lmhead_q4_0 into d_logits
 * then g4s_sample_async on them.  lm_us[i] / total_us[i] = event times of the
 * LM head alone and of the whole step i.  `warmup` untimed steps first.
 */
G4H_API int g4h_lmhead_sampler(g4s_sampler* s, void* stream, const void* d_weights, int32_t rows,
                               int32_t cols, const float* d_hidden, int32_t batch, float* d_logits,
                               const g4s_params* d_params, const double* d_u, int32_t k_bound,
                               int32_t* d_ids, int32_t warmup, int32_t steps, float* lm_us,
                               float* total_us)
{
    hipStream_t st = (hipStream_t)stream;
    std::vector<hipEvent_t> ev((size_t)steps * 3);
    for (auto& e : ev)
        if (hipEventCreate(&e) != hipSuccess) return -100;
    int rc = 0;
    for (int32_t i = 0; rc == 0 && i < warmup; ++i) {
        rc = g4s_lmhead_q4_0(s, d_weights, rows, cols, d_hidden, batch, d_logits, rows);
        if (rc == 0)
            rc = g4s_sample_async(s, d_logits, G4S_DTYPE_F32, rows, batch, d_params, d_u, k_bound,
                                  0, d_ids, nullptr);
    }
    if (rc == 0 && hipStreamSynchronize(st) != hipSuccess) rc = -104;
    for (int32_t i = 0; rc == 0 && i < steps; ++i) {
        (void)hipEventRecord(ev[(size_t)i * 3], st);
        rc = g4s_lmhead_q4_0(s, d_weights, rows, cols, d_hidden, batch, d_logits, rows);
        (void)hipEventRecord(ev[(size_t)i * 3 + 1], st);
        if (rc == 0)
            rc = g4s_sample_async(s, d_logits, G4S_DTYPE_F32, rows, batch, d_params, d_u, k_bound,
                                  0, d_ids, nullptr);
        (void)hipEventRecord(ev[(size_t)i * 3 + 2], st);
    }
    if (rc == 0 && hipStreamSynchronize(st) != hipSuccess) rc = -104;
    if (rc == 0)
        for (int32_t i = 0; i < steps; ++i) {
            float a = 0.0f, b = 0.0f;
            (void)hipEventElapsedTime(&a, ev[(size_t)i * 3], ev[(size_t)i * 3 + 1]);
            (void)hipEventElapsedTime(&b, ev[(size_t)i * 3], ev[(size_t)i * 3 + 2]);
            lm_us[i] = a * 1000.0f;
            total_us[i] = b * 1000.0f;
        }
    for (auto& e : ev) (void)hipEventDestroy(e);
    return rc;
}

/*
 * The LM head on TILED64 weights alone: `steps` launches of
 * g4s_lmhead_q4_0_tiled, each bracketed by events (us[i]).
 */
G4H_API int g4h_lmhead_tiled(g4s_sampler* s, void* stream, const void* d_tiles, int32_t rows,
                             int32_t cols, const float* d_hidden, int32_t batch, float* d_logits,
                             int32_t warmup, int32_t steps, float* us)
{
    hipStream_t st = (hipStream_t)stream;
    std::vector<hipEvent_t> ev((size_t)steps * 2);
    for (auto& e : ev)
        if (hipEventCreate(&e) != hipSuccess) return -100;
    int rc = 0;
    for (int32_t i = 0; rc == 0 && i < warmup; ++i)
        rc = g4s_lmhead_q4_0_tiled(s, d_tiles, rows, cols, d_hidden, batch, d_logits, rows);
    if (rc == 0 && hipStreamSynchronize(st) != hipSuccess) rc = -104;
    for (int32_t i = 0; rc == 0 && i < steps; ++i) {
        (void)hipEventRecord(ev[(size_t)i * 2], st);
        rc = g4s_lmhead_q4_0_tiled(s, d_tiles, rows, cols, d_hidden, batch, d_logits, rows);
        (void)hipEventRecord(ev[(size_t)i * 2 + 1], st);
    }
    if (rc == 0 && hipStreamSynchronize(st) != hipSuccess) rc = -104;
    if (rc == 0)
        for (int32_t i = 0; i < steps; ++i) {
            float a = 0.0f;
            (void)hipEventElapsedTime(&a, ev[(size_t)i * 2], ev[(size_t)i * 2 + 1]);
            us[i] = a * 1000.0f;
        }
    for (auto& e : ev) (void)hipEventDestroy(e);
    return rc;
}

/*
 * The fused LM head + sample (g4s_lmhead_sample_q4_0, synchronous): host
 * wall time of each call in us[i]; the last call's ids in ids.
 */
G4H_API int g4h_lmhead_sample_fused(g4s_sampler* s, const void* d_tiles, int32_t rows,
                                    int32_t cols, const float* d_hidden, int32_t batch,
                                    float* d_logits, const g4s_params* params, const double* u,
                                    int32_t* ids, int32_t warmup, int32_t steps, float* us)
{
    int rc = 0;
    for (int32_t i = 0; rc == 0 && i < warmup; ++i)
        rc = g4s_lmhead_sample_q4_0(s, d_tiles, cols, d_hidden, batch, d_logits, rows, params, u,
                                    ids, nullptr);
    for (int32_t i = 0; rc == 0 && i < steps; ++i) {
        const auto t0 = std::chrono::steady_clock::now();
        rc = g4s_lmhead_sample_q4_0(s, d_tiles, cols, d_hidden, batch, d_logits, rows, params, u,
                                    ids, nullptr);
        const auto t1 = std::chrono::steady_clock::now();
        us[i] = (float)std::chrono::duration<double, std::micro>(t1 - t0).count();
    }
    return rc;
}
