/*
 * g4s_noalloc.hip -- g4s_sample_topk_noalloc: the top-k path of
 * g4s_sample_async for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 *
 * It needs no handle.  The per-row workspace of the top-k kernel (candidate
 * slots, merge overflow, chunk records, wave bounds, election tickets) lives
 * in one file-scope device array, `scratch`, of G4S_NOALLOC_SCRATCH_BYTES:
 * every GPU the library runs on holds its own copy until the process ends.
 * Its device address is taken once per device with hipGetSymbolAddress (the
 * array's name is not a device address in host code) and only that address
 * is handed to kernels.  Nothing here calls hipMalloc, hipFree or an
 * allocating library routine.
 *
 * What must start at zero: the election tickets (the one-word tickets of
 * the chunked launch and the counters of the decode-sized launch).  The
 * kernels return each to zero in the workgroup it elects, so they are zero
 * between launches; they are also cleared once, with a fill kernel on the caller's
 * stream, at the first call on each device.  Calls that overlap on one GPU
 * share the array and race: a caller runs one call at a time per device
 * (e.g. one stream).
 */
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>

#include "g4s_runtime.h"
#include "g4s_topk.h"

#define G4S_API extern "C" __attribute__((visibility("default")))

namespace {

using namespace g4s;

constexpr int kRows = G4S_NOALLOC_MAX_ROWS;
constexpr size_t kTicketsOff = 0;
constexpr size_t kCandOff = 256;
constexpr size_t kMergeOff = kCandOff + (size_t)kRows * kCandRow * sizeof(uint64_t);
constexpr size_t kRecsOff = kMergeOff + (size_t)kRows * kCandRow * sizeof(uint64_t);
constexpr size_t kWbOff = kRecsOff + (size_t)kRows * kMaxSplits * sizeof(ChunkRec);
constexpr size_t kDecTicketsOff = kWbOff + (size_t)kRows * kWaveBounds * sizeof(uint32_t);
constexpr int kDecRows = kRows < kDecMaxBatch ? kRows : kDecMaxBatch;
constexpr int kDecWords = kDecRows * kDecTicketWords;
constexpr size_t kBytes = kDecTicketsOff + (size_t)kDecWords * sizeof(uint32_t);
static_assert(kRows * sizeof(uint32_t) <= kCandOff, "tickets before the candidates");
static_assert(kDecTicketsOff % 256 == 0, "aligned sections");
static_assert(kBytes == G4S_NOALLOC_SCRATCH_BYTES, "header states the scratch size");
static_assert(kRecsOff % 256 == 0 && kWbOff % 256 == 0, "aligned sections");

static __device__ __align__(256) uint8_t scratch[kBytes];

__global__ void noalloc_clear_tickets(uint32_t* tickets, uint32_t* dec_tickets)
{
    if (threadIdx.x < (unsigned)kRows) tickets[threadIdx.x] = 0u;
    for (int i = threadIdx.x; i < kDecWords; i += blockDim.x) dec_tickets[i] = 0u;
}

constexpr int kMaxDevices = 64;

struct DevScratch {
    bool ready = false;
    uint8_t* ptr = nullptr; /* device address of `scratch` on this device */
    int32_t ncu = 0;
};

std::mutex g_mu;
DevScratch g_dev[kMaxDevices];

/* Set-up, once per device with that device current: the architecture, the
 * compute units and the device address of `scratch`.  `first` is true on the
 * call that completed the set-up. */
int device_scratch(int dev, DevScratch& out, bool& first)
{
    std::lock_guard<std::mutex> lock(g_mu);
    DevScratch& d = g_dev[dev];
    first = false;
    if (!d.ready) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess)
            return set_null_handle_error(G4S_ERR_NO_DEVICE, "hipGetDeviceProperties failed");
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            return set_null_handle_error(G4S_ERR_NO_DEVICE,
                                         "device %d is %s; this library targets gfx950", dev,
                                         prop.gcnArchName);
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return set_null_handle_error(G4S_ERR_HIP, "hipGetSymbolAddress(scratch): %s",
                                         hipGetErrorString(e));
        d.ptr = static_cast<uint8_t*>(p);
        d.ncu = prop.multiProcessorCount;
        d.ready = true;
        first = true;
    }
    out = d;
    return G4S_OK;
}

}  // namespace

G4S_API int g4s_sample_topk_noalloc(const void* d_logits, int32_t dtype, int32_t vocab,
                                    int64_t row_stride, int32_t batch, const g4s_params* d_params,
                                    const double* d_u, int32_t k_bound, float softcap,
                                    int32_t* d_ids, const g4s_outputs* outputs, void* hip_stream)
{
    clear_null_handle_error();
    if (!d_logits || !d_params || !d_u || !d_ids)
        return set_null_handle_error(G4S_ERR_INVALID_ARGUMENT,
                                     "d_logits, d_params, d_u and d_ids must be non-NULL");
    if (dtype != G4S_DTYPE_F32 && dtype != G4S_DTYPE_BF16)
        return set_null_handle_error(G4S_ERR_INVALID_ARGUMENT, "dtype %d is neither F32 nor BF16",
                                     dtype);
    if (vocab < 2 || vocab > (1 << 30))
        return set_null_handle_error(G4S_ERR_INVALID_ARGUMENT, "vocab %d outside [2, 2^30]",
                                     vocab);
    if (batch < 1 || batch > kRows)
        return set_null_handle_error(G4S_ERR_INVALID_ARGUMENT,
                                     "batch %d outside [1, %d] (G4S_NOALLOC_MAX_ROWS)", batch,
                                     kRows);
    const int64_t esize = dtype == G4S_DTYPE_F32 ? 4 : 2;
    if (((uintptr_t)d_logits & 15u) != 0)
        return set_null_handle_error(G4S_ERR_INVALID_ARGUMENT, "d_logits must be 16-byte aligned");
    if (batch > 1 && (row_stride < vocab || ((row_stride * esize) & 15) != 0))
        return set_null_handle_error(G4S_ERR_INVALID_ARGUMENT,
                                     "row_stride %lld: below vocab %d or not a multiple of 16 "
                                     "bytes",
                                     (long long)row_stride, vocab);
    if (k_bound < 1 || k_bound > kMaxTopK || k_bound >= vocab)
        return set_null_handle_error(G4S_ERR_INVALID_ARGUMENT,
                                     "k_bound %d outside [1, min(%d, vocab - 1)]", k_bound,
                                     kMaxTopK);
    if (!(softcap == softcap)) return set_null_handle_error(G4S_ERR_INVALID_ARGUMENT, "softcap is NaN");
    g4s_outputs out{};
    if (outputs) out = *outputs;
    if ((out.indices || out.probs) && out.capacity < 1)
        return set_null_handle_error(G4S_ERR_INVALID_ARGUMENT, "outputs.capacity must be >= 1");
    const TopkConfig cfg = topk_plan(vocab, k_bound);
    if (!cfg.ok)
        return set_null_handle_error(G4S_ERR_UNSUPPORTED, "no top-k launch plan for K=%d",
                                     k_bound);

    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return set_null_handle_error(G4S_ERR_NO_DEVICE, "no usable current HIP device");
    DevScratch ds;
    bool first = false;
    int rc = device_scratch(dev, ds, first);
    if (rc) return rc;
    hipStream_t stream = (hipStream_t)hip_stream;
    uint8_t* base = ds.ptr;
    if (first) {
        /* a kernel, not hipMemsetAsync: the call may be under graph capture */
        hipLaunchKernelGGL(noalloc_clear_tickets, dim3(1), dim3(256), 0, stream,
                           reinterpret_cast<uint32_t*>(base + kTicketsOff),
                           reinterpret_cast<uint32_t*>(base + kDecTicketsOff));
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess)
            return set_null_handle_error(G4S_ERR_HIP, "scratch set-up: %s", hipGetErrorString(e));
    }

    TopkArgs a{};
    a.logits = d_logits;
    a.row_stride = batch > 1 ? row_stride : vocab;
    a.vocab = vocab;
    a.batch = batch;
    a.params = d_params;
    a.u = d_u;
    a.splits = cfg.splits;
    a.cap_log2 = cfg.cap_log2;
    a.kbound = k_bound;
    a.wide_on = 0;
    a.full_on = 0; /* full-vocabulary rows get id -1 and G4S_FLAG_ERROR */
    a.softcap = softcap;
    a.cand = reinterpret_cast<uint64_t*>(base + kCandOff);
    a.merge = reinterpret_cast<uint64_t*>(base + kMergeOff);
    a.recs = reinterpret_cast<ChunkRec*>(base + kRecsOff);
    a.wbounds = reinterpret_cast<uint32_t*>(base + kWbOff);
    a.tickets = reinterpret_cast<uint32_t*>(base + kTicketsOff);
    a.dec_tickets = reinterpret_cast<uint32_t*>(base + kDecTicketsOff);
    a.dec_rows = kDecRows;
    a.ids = d_ids;
    a.done = nullptr;
    a.seq = 0;
    a.out = out;
    const hipError_t e = topk_launch(cfg, a, dtype, stream, ds.ncu);
    if (e != hipSuccess)
        return set_null_handle_error(G4S_ERR_HIP, "top-k kernel launch: %s", hipGetErrorString(e));
    return G4S_OK;
}
