/*
 * g4s_runtime.hip -- host runtime and C ABI of libgemma4_sampler.so.
 *
 * Owns the per-handle HBM workspace (allocated once in g4s_create, reused by
 * every call), validates arguments the way the engine would have to, and
 * dispatches each row to the top-k path or the full-vocabulary path exactly
 * as DoSample's branch does (src/Gemma4.Model.pas:2756).  Errors follow the
 * engine's convention of a failing result plus a message (StdApp.Base.pas
 * TErrors), here a negative g4s_status and g4s_last_error().
 */
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "g4s_full.h"
#include "g4s_lmhead.h"
#include "g4s_runtime.h"
#include "g4s_topk.h"

#define G4S_API extern "C" __attribute__((visibility("default")))

namespace {

thread_local std::string g_create_error;

/* The fused LM head's weights and hidden vectors, for the rows whose
 * logits were not written (recomputed groups). */
struct LmSource {
    const uint8_t* tiles;
    const float* hidden;
    int32_t cols;
};

}  // namespace

namespace g4s {

int set_null_handle_error(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_create_error = buf;
    return code;
}

void clear_null_handle_error() { g_create_error.clear(); }

}  // namespace g4s

struct g4s_sampler {
    int device = 0;
    int32_t ncu = 0; /* compute units of the device (top-k launch split) */
    int32_t vocab = 0;
    int32_t max_batch = 0;
    float softcap = 0.0f;
    hipStream_t stream = nullptr;
    std::string err;

    /* top-k path workspace */
    uint64_t* cand = nullptr;
    uint64_t* merge = nullptr;
    g4s::ChunkRec* recs = nullptr;
    uint32_t* wbounds = nullptr;
    uint32_t* tickets = nullptr;
    uint32_t* dec_tickets = nullptr; /* [dec_rows][kDecTicketWords] */
    int32_t dec_rows = 0;            /* min(max_batch, kDecMaxBatch) */
    uint64_t* gsum = nullptr;     /* [max_batch][ceil(vocab/64)] LM-head group summaries */
    int32_t* gc_jobs = nullptr;   /* [max_batch][kGcJobStride] group recompute jobs */
    float* row_logits = nullptr;  /* one row of logits for a recomputed row (allocated by
                                     the first fused call without d_logits that needs it) */
    /* full path workspace */
    g4s::FullWorkspace full{};
    /* per-call staging */
    g4s_params* d_params = nullptr;
    double* d_u = nullptr;
    g4s_params* h_params = nullptr; /* pinned */
    double* h_u = nullptr;          /* pinned */
    int32_t* h_ids = nullptr;       /* pinned */
    uint32_t* h_flags = nullptr;    /* pinned */
    uint32_t* h_done = nullptr;     /* pinned, coherent: per-row completion words */
    uint32_t seq = 0;               /* last completion value handed to a launch */

    /* g4s_sample_graph: captured stream-ordered samples, one per argument set */
    struct GraphEntry {
        bool used = false;
        uint64_t last = 0; /* least recently launched entry is replaced first */
        const void* logits = nullptr;
        int32_t dtype = 0;
        int64_t row_stride = 0;
        int32_t batch = 0;
        const g4s_params* params = nullptr;
        const double* u = nullptr;
        int32_t k_bound = 0;
        int32_t full_rows = 0;
        int32_t* ids = nullptr;
        g4s_outputs out{};
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
    };
    static constexpr int kGraphs = 8;
    GraphEntry graphs[kGraphs];
    uint64_t graph_clock = 0;
};

namespace {

int fail(g4s_sampler* s, int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (s)
        s->err = buf;
    else
        g_create_error = buf;
    return code;
}

int hip_fail(g4s_sampler* s, hipError_t e, const char* what)
{
    return fail(s, G4S_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

void release(g4s_sampler* s)
{
    auto f = [](void* p) {
        if (p) (void)hipFree(p);
    };
    auto fh = [](void* p) {
        if (p) (void)hipHostFree(p);
    };
    f(s->cand);
    f(s->merge);
    f(s->recs);
    f(s->wbounds);
    f(s->tickets);
    f(s->dec_tickets);
    f(s->gsum);
    f(s->gc_jobs);
    f(s->row_logits);
    g4s::full_free(s->full);
    f(s->d_params);
    f(s->d_u);
    fh(s->h_params);
    fh(s->h_u);
    fh(s->h_ids);
    fh(s->h_flags);
    fh(s->h_done);
    for (auto& g : s->graphs) {
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
        if (g.graph) (void)hipGraphDestroy(g.graph);
        g = g4s_sampler::GraphEntry{};
    }
}

bool is_topk_row(const g4s_params& p, int32_t vocab) { return p.top_k >= 1 && p.top_k < vocab; }

int check_logits(g4s_sampler* s, const void* d_logits, int32_t dtype, int64_t row_stride,
                 int32_t batch)
{
    if (!d_logits) return fail(s, G4S_ERR_INVALID_ARGUMENT, "d_logits is NULL");
    if (dtype != G4S_DTYPE_F32 && dtype != G4S_DTYPE_BF16)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "dtype %d is neither F32 nor BF16", dtype);
    if (batch < 1 || batch > s->max_batch)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "batch %d outside [1, %d]", batch, s->max_batch);
    if (batch > 1 && row_stride < s->vocab)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "row_stride %lld < vocab %d",
                    (long long)row_stride, s->vocab);
    const int64_t esize = dtype == G4S_DTYPE_F32 ? 4 : 2;
    if (((uintptr_t)d_logits & 15u) != 0)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "d_logits must be 16-byte aligned");
    if (batch > 1 && ((row_stride * esize) & 15) != 0)
        return fail(s, G4S_ERR_INVALID_ARGUMENT,
                    "row_stride * sizeof(dtype) must be a multiple of 16 bytes");
    return G4S_OK;
}

/* Enqueue both paths for `batch` rows whose parameters are at d_params/d_u
 * (or inline p0/u0 when d_params is NULL). */
int enqueue(g4s_sampler* s, const void* d_logits, int32_t dtype, int64_t row_stride, int32_t batch,
            const g4s_params* d_params, const double* d_u, const g4s_params* p0, double u0,
            int32_t kbound, bool full_rows, bool wide, int32_t* d_ids,
            const g4s_outputs* outputs, uint32_t* done = nullptr, uint32_t seq = 0,
            const uint64_t* gsum = nullptr, const LmSource* lm = nullptr)
{
    g4s_outputs out{};
    if (outputs) out = *outputs;
    if ((out.indices || out.probs) && out.capacity < 1)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "outputs.capacity must be >= 1");
    if (kbound > 0) {
        g4s::TopkConfig cfg = g4s::topk_plan(s->vocab, kbound);
        if (!cfg.ok) return fail(s, G4S_ERR_UNSUPPORTED, "no top-k launch plan for K=%d", kbound);
        g4s::TopkArgs a{};
        a.logits = d_logits;
        a.row_stride = row_stride;
        a.vocab = s->vocab;
        a.batch = batch;
        a.params = d_params;
        a.u = d_u;
        if (p0) a.p0 = *p0;
        a.u0 = u0;
        a.splits = cfg.splits;
        a.cap_log2 = cfg.cap_log2;
        a.kbound = kbound;
        a.wide_on = wide ? 1 : 0;
        a.full_on = (full_rows || wide) ? 1 : 0;
        a.softcap = s->softcap;
        a.cand = s->cand;
        a.merge = s->merge;
        a.recs = s->recs;
        a.wbounds = s->wbounds;
        a.tickets = s->tickets;
        a.dec_tickets = s->dec_tickets;
        a.dec_rows = s->dec_rows;
        if (lm) {
            a.lm_tiles = lm->tiles;
            a.lm_hidden = lm->hidden;
            a.lm_cols = lm->cols;
            a.gc_jobs = s->gc_jobs;
        }
        a.ids = d_ids;
        a.done = done;
        a.seq = seq;
        a.out = out;
        hipError_t e = hipErrorNotSupported;
        if (gsum && dtype == G4S_DTYPE_F32)
            e = g4s::topk_groups_launch(cfg, a, gsum, (s->vocab + 63) / 64, s->stream);
        if (e == hipErrorNotSupported) {
            (void)hipGetLastError();
            if (!d_logits) return fail(s, G4S_ERR_UNSUPPORTED, "top-k rows without logits");
            e = g4s::topk_launch(cfg, a, dtype, s->stream, s->ncu);
        }
        if (e != hipSuccess) return hip_fail(s, e, "top-k kernel launch");
    }
    if (full_rows || wide) {
        if (!g4s::full_supported(s->vocab))
            return fail(s, G4S_ERR_UNSUPPORTED,
                        "the softmax path (TopK <= 0, TopK >= V, or TopK > %d) supports vocab "
                        "<= %d",
                        g4s::kMaxTopK, g4s::kFullChunk * g4s::kFullMaxChunks);
        g4s::FullArgs f{};
        f.logits = d_logits;
        f.row_stride = row_stride;
        f.vocab = s->vocab;
        f.batch = batch;
        f.params = d_params;
        f.u = d_u;
        if (p0) f.p0 = *p0;
        f.u0 = u0;
        f.softcap = s->softcap;
        f.nch = (s->vocab + g4s::kFullChunk - 1) / g4s::kFullChunk;
        f.nsel = (s->vocab + g4s::kSelChunk - 1) / g4s::kSelChunk;
        f.wide_on = wide ? 1 : 0;
        f.topk_on = kbound > 0 ? 1 : 0;
        f.ws = s->full;
        f.ids = d_ids;
        f.done = done;
        f.seq = seq;
        f.out = out;
        hipError_t e = g4s::full_launch(f, dtype, s->stream);
        if (e != hipSuccess) return hip_fail(s, e, "full-vocabulary kernel launch");
    }
    return G4S_OK;
}

}  // namespace

G4S_API const char* g4s_version(void) { return "gemma4_sampler 0.1.0 (gfx950)"; }

G4S_API void g4s_params_set_defaults(g4s_params* p)
{
    /* TSamplingParams.SetDefaults, Model.pas:346-352 */
    if (!p) return;
    p->temperature = 1.0f;
    p->top_k = 64;
    p->top_p = 0.95f;
    p->repetition_penalty = 1.0f;
}

G4S_API int32_t g4s_max_top_k(void) { return g4s::kMaxTopK; }

G4S_API const char* g4s_last_error(const g4s_sampler* s)
{
    return s ? s->err.c_str() : g_create_error.c_str();
}

G4S_API int g4s_create(g4s_sampler** out, int32_t vocab, int32_t max_batch, float softcap,
                       void* hip_stream)
{
    g_create_error.clear();
    if (!out) return fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "out is NULL");
    *out = nullptr;
    if (vocab < 2 || vocab > (1 << 30))
        return fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "vocab %d outside [2, 2^30]", vocab);
    if (max_batch < 1 || max_batch > 65535)
        return fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "max_batch %d outside [1, 65535]",
                    max_batch);
    if (!(softcap == softcap))
        return fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "softcap is NaN");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1)
        return fail(nullptr, G4S_ERR_NO_DEVICE, "no HIP device visible");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return fail(nullptr, G4S_ERR_NO_DEVICE, "hipGetDevice failed");
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess)
        return fail(nullptr, G4S_ERR_NO_DEVICE, "hipGetDeviceProperties failed");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(nullptr, G4S_ERR_NO_DEVICE, "device %d is %s; this library targets gfx950",
                    dev, prop.gcnArchName);

    g4s_sampler* s = new g4s_sampler();
    s->device = dev;
    s->ncu = prop.multiProcessorCount;
    s->vocab = vocab;
    s->max_batch = max_batch;
    s->softcap = softcap;
    s->stream = (hipStream_t)hip_stream;

    const size_t mb = (size_t)max_batch;
    bool ok = true;
    auto dm = [&](void** p, size_t bytes) {
        if (ok && hipMalloc(p, bytes) != hipSuccess) ok = false;
    };
    auto hm = [&](void** p, size_t bytes) {
        if (ok && hipHostMalloc(p, bytes, hipHostMallocDefault) != hipSuccess) ok = false;
    };
    dm((void**)&s->cand, mb * g4s::kCandRow * sizeof(uint64_t));
    dm((void**)&s->merge, mb * g4s::kCandRow * sizeof(uint64_t));
    dm((void**)&s->recs, mb * g4s::kMaxSplits * sizeof(g4s::ChunkRec));
    dm((void**)&s->wbounds, mb * g4s::kWaveBounds * sizeof(uint32_t));
    dm((void**)&s->tickets, mb * sizeof(uint32_t));
    const size_t dec_rows = mb < (size_t)g4s::kDecMaxBatch ? mb : (size_t)g4s::kDecMaxBatch;
    s->dec_rows = (int32_t)dec_rows;
    dm((void**)&s->dec_tickets, dec_rows * g4s::kDecTicketWords * sizeof(uint32_t));
    dm((void**)&s->gsum, mb * (size_t)((vocab + 63) / 64) * sizeof(uint64_t));
    dm((void**)&s->gc_jobs, mb * g4s::kGcJobStride * sizeof(int32_t));
    dm((void**)&s->d_params, mb * sizeof(g4s_params));
    dm((void**)&s->d_u, mb * sizeof(double));
    hm((void**)&s->h_params, mb * sizeof(g4s_params));
    hm((void**)&s->h_u, mb * sizeof(double));
    hm((void**)&s->h_ids, mb * sizeof(int32_t));
    hm((void**)&s->h_flags, mb * sizeof(uint32_t));
    if (ok && hipHostMalloc((void**)&s->h_done, mb * sizeof(uint32_t), hipHostMallocCoherent) !=
                  hipSuccess)
        ok = false;
    if (ok && g4s::full_alloc(s->full, vocab, max_batch) != hipSuccess) ok = false;
    if (!ok) {
        release(s);
        delete s;
        return fail(nullptr, G4S_ERR_OUT_OF_MEMORY,
                    "workspace allocation failed (vocab %d, max_batch %d)", vocab, max_batch);
    }
    /* pinned allocations can be recycled memory: the completion words must
     * start below the first sequence value */
    std::memset(s->h_done, 0, mb * sizeof(uint32_t));
    hipError_t e = hipMemsetAsync(s->tickets, 0, mb * sizeof(uint32_t), s->stream);
    if (e == hipSuccess)
        e = hipMemsetAsync(s->dec_tickets, 0, dec_rows * g4s::kDecTicketWords * sizeof(uint32_t),
                           s->stream);
    if (e == hipSuccess) e = g4s::full_init(s->full, max_batch, softcap, s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) {
        release(s);
        delete s;
        return fail(nullptr, G4S_ERR_HIP, "workspace initialisation: %s", hipGetErrorString(e));
    }
    *out = s;
    return G4S_OK;
}

G4S_API int g4s_destroy(g4s_sampler* s)
{
    if (!s) return G4S_OK;
    (void)hipStreamSynchronize(s->stream);
    release(s);
    delete s;
    return G4S_OK;
}

namespace {

int check_params(g4s_sampler* s, int32_t batch, const g4s_params* params, const double* u,
                 int32_t* ids)
{
    if (!params || !u || !ids)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "params, u and ids must be non-NULL");
    /* u must be a probability-like number; the reference's Random is in [0,1) */
    for (int32_t r = 0; r < batch; ++r)
        if (!(u[r] >= 0.0 && u[r] < 1.0))
            return fail(s, G4S_ERR_INVALID_ARGUMENT, "row %d: u = %g outside [0, 1)", r, u[r]);
    return G4S_OK;
}

/* The synchronous sample of g4s_sample_ex (arguments checked), optionally on
 * logits from the tiled LM head with their group maxima. */
int sample_sync(g4s_sampler* s, const void* d_logits, int32_t dtype, int64_t row_stride,
                int32_t batch, const g4s_params* params, const double* u, int32_t* ids,
                const g4s_outputs* outputs, const uint64_t* gsum = nullptr,
                const LmSource* lm = nullptr)
{
    int rc;
    int32_t kbound = 0;
    bool full_rows = false, wide = false;
    for (int32_t r = 0; r < batch; ++r) {
        if (is_topk_row(params[r], s->vocab)) {
            if (params[r].top_k > g4s::kMaxTopK)
                wide = true;
            else
                kbound = params[r].top_k > kbound ? params[r].top_k : kbound;
        } else {
            full_rows = true;
        }
    }
    g4s_outputs out{};
    if (outputs) out = *outputs;
    /* ids (and flags, unless the caller wants them on the device) are written
     * by the kernel straight into this handle's pinned host buffers, and each
     * row then publishes a completion word: the synchronous call spins on
     * those words instead of synchronizing the stream, and needs no copy
     * after the kernel. */
    uint32_t* user_flags = out.flags;
    if (++s->seq == 0) s->seq = 1;
    const uint32_t seq = s->seq;
    for (int32_t r = 0; r < batch; ++r) {
        s->h_ids[r] = -1;
        s->h_flags[r] = 0u;
    }
    /* the completion words carry only the ids and flags: a call that also
     * asks for device-memory outputs waits for the stream instead */
    const bool dev_out = user_flags || out.count || out.indices || out.probs || out.argmax ||
                         out.lsum;
    if (!user_flags) out.flags = s->h_flags;
    uint32_t* done = !dev_out ? s->h_done : nullptr;

    if (batch == 1) {
        rc = enqueue(s, d_logits, dtype, row_stride, 1, nullptr, nullptr, &params[0], u[0], kbound,
                     full_rows, wide, s->h_ids, &out, done, seq, gsum, lm);
    } else {
        std::memcpy(s->h_params, params, sizeof(g4s_params) * batch);
        std::memcpy(s->h_u, u, sizeof(double) * batch);
        hipError_t e = hipMemcpyAsync(s->d_params, s->h_params, sizeof(g4s_params) * batch,
                                      hipMemcpyHostToDevice, s->stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(s->d_u, s->h_u, sizeof(double) * batch, hipMemcpyHostToDevice,
                               s->stream);
        if (e != hipSuccess) return hip_fail(s, e, "parameter upload");
        rc = enqueue(s, d_logits, dtype, row_stride, batch, s->d_params, s->d_u, nullptr, 0.0,
                     kbound, full_rows, wide, s->h_ids, &out, done, seq, gsum, lm);
    }
    if (rc) return rc;
    hipError_t e = hipSuccess;
    bool published = false;
    if (done) {
        /* bounded spin (about a second), then the stream decides */
        const auto t0 = std::chrono::steady_clock::now();
        for (uint64_t spin = 0;; ++spin) {
            int32_t r = 0;
            while (r < batch && __atomic_load_n(&s->h_done[r], __ATOMIC_ACQUIRE) == seq) ++r;
            if (r == batch) {
                published = true;
                break;
            }
            if ((spin & 1023u) == 1023u &&
                std::chrono::steady_clock::now() - t0 > std::chrono::seconds(1))
                break;
        }
    }
    if (!published) {
        if (user_flags)
            e = hipMemcpyAsync(s->h_flags, user_flags, sizeof(uint32_t) * batch,
                               hipMemcpyDeviceToHost, s->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
        if (e != hipSuccess) return hip_fail(s, e, "sampling");
    }
    std::memcpy(ids, s->h_ids, sizeof(int32_t) * batch);
    for (int32_t r = 0; r < batch; ++r)
        if (s->h_flags[r] & G4S_FLAG_EMPTY)
            return fail(s, G4S_ERR_EMPTY_ROW, "row %d: no logit above -1e30 on the top-k path", r);
    return G4S_OK;
}

}  // namespace

G4S_API int g4s_sample_ex(g4s_sampler* s, const void* d_logits, int32_t dtype, int64_t row_stride,
                          int32_t batch, const g4s_params* params, const double* u, int32_t* ids,
                          const g4s_outputs* outputs)
{
    if (!s) return fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "sampler is NULL");
    s->err.clear();
    int rc = check_logits(s, d_logits, dtype, row_stride, batch);
    if (rc) return rc;
    rc = check_params(s, batch, params, u, ids);
    if (rc) return rc;
    return sample_sync(s, d_logits, dtype, row_stride, batch, params, u, ids, outputs, nullptr);
}

G4S_API int g4s_sample(g4s_sampler* s, const void* d_logits, int32_t dtype, int64_t row_stride,
                       int32_t batch, const g4s_params* params, const double* u, int32_t* ids)
{
    return g4s_sample_ex(s, d_logits, dtype, row_stride, batch, params, u, ids, nullptr);
}

namespace {

int check_async(g4s_sampler* s, const void* d_logits, int32_t dtype, int64_t row_stride,
                int32_t batch, const g4s_params* d_params, const double* d_u, int32_t k_bound,
                int32_t full_rows, int32_t* d_ids)
{
    int rc = check_logits(s, d_logits, dtype, row_stride, batch);
    if (rc) return rc;
    if (!d_params || !d_u || !d_ids)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "d_params, d_u and d_ids must be non-NULL");
    if (k_bound < 0 || k_bound >= s->vocab)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "k_bound %d outside [0, %d)", k_bound, s->vocab);
    if (k_bound == 0 && !full_rows)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "k_bound == 0 and full_rows == 0: nothing to do");
    return G4S_OK;
}

int enqueue_async(g4s_sampler* s, const void* d_logits, int32_t dtype, int64_t row_stride,
                  int32_t batch, const g4s_params* d_params, const double* d_u, int32_t k_bound,
                  int32_t full_rows, int32_t* d_ids, const g4s_outputs* outputs)
{
    const bool wide = k_bound > g4s::kMaxTopK;
    return enqueue(s, d_logits, dtype, row_stride, batch, d_params, d_u, nullptr, 0.0,
                   wide ? g4s::kMaxTopK : k_bound, full_rows != 0, wide, d_ids, outputs);
}

bool same_outputs(const g4s_outputs& a, const g4s_outputs& b)
{
    return a.count == b.count && a.indices == b.indices && a.probs == b.probs &&
           a.capacity == b.capacity && a.argmax == b.argmax && a.lsum == b.lsum &&
           a.flags == b.flags;
}

}  // namespace

G4S_API int g4s_sample_async(g4s_sampler* s, const void* d_logits, int32_t dtype,
                             int64_t row_stride, int32_t batch, const g4s_params* d_params,
                             const double* d_u, int32_t k_bound, int32_t full_rows, int32_t* d_ids,
                             const g4s_outputs* outputs)
{
    if (!s) return fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "sampler is NULL");
    s->err.clear();
    const int rc = check_async(s, d_logits, dtype, row_stride, batch, d_params, d_u, k_bound,
                               full_rows, d_ids);
    if (rc) return rc;
    return enqueue_async(s, d_logits, dtype, row_stride, batch, d_params, d_u, k_bound, full_rows,
                         d_ids, outputs);
}

G4S_API int g4s_sample_graph(g4s_sampler* s, const void* d_logits, int32_t dtype,
                             int64_t row_stride, int32_t batch, const g4s_params* d_params,
                             const double* d_u, int32_t k_bound, int32_t full_rows, int32_t* d_ids,
                             const g4s_outputs* outputs)
{
    if (!s) return fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "sampler is NULL");
    s->err.clear();
    int rc = check_async(s, d_logits, dtype, row_stride, batch, d_params, d_u, k_bound,
                         full_rows, d_ids);
    if (rc) return rc;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s->stream, &cs);
    if (e != hipSuccess) return hip_fail(s, e, "hipStreamIsCapturing");
    if (cs == hipStreamCaptureStatusActive) /* the caller's own capture records the launches */
        return enqueue_async(s, d_logits, dtype, row_stride, batch, d_params, d_u, k_bound,
                             full_rows, d_ids, outputs);
    if (!s->stream)
        return fail(s, G4S_ERR_UNSUPPORTED,
                    "g4s_sample_graph needs a handle created on a stream (not the null stream)");
    g4s_outputs out{};
    if (outputs) out = *outputs;
    g4s_sampler::GraphEntry* hit = nullptr;
    g4s_sampler::GraphEntry* victim = &s->graphs[0];
    for (auto& g : s->graphs) {
        if (g.used && g.logits == d_logits && g.dtype == dtype && g.row_stride == row_stride &&
            g.batch == batch && g.params == d_params && g.u == d_u && g.k_bound == k_bound &&
            g.full_rows == full_rows && g.ids == d_ids && same_outputs(g.out, out)) {
            hit = &g;
            break;
        }
        if (!g.used || (victim->used && g.last < victim->last)) victim = &g;
    }
    if (!hit) {
        if (victim->exec) (void)hipGraphExecDestroy(victim->exec);
        if (victim->graph) (void)hipGraphDestroy(victim->graph);
        *victim = g4s_sampler::GraphEntry{};
        e = hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return hip_fail(s, e, "hipStreamBeginCapture");
        rc = enqueue_async(s, d_logits, dtype, row_stride, batch, d_params, d_u, k_bound,
                           full_rows, d_ids, outputs);
        hipGraph_t g = nullptr;
        e = hipStreamEndCapture(s->stream, &g);
        if (rc || e != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            return rc ? rc : hip_fail(s, e, "hipStreamEndCapture");
        }
        hipGraphExec_t x = nullptr;
        e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            (void)hipGraphDestroy(g);
            return hip_fail(s, e, "hipGraphInstantiate");
        }
        victim->used = true;
        victim->logits = d_logits;
        victim->dtype = dtype;
        victim->row_stride = row_stride;
        victim->batch = batch;
        victim->params = d_params;
        victim->u = d_u;
        victim->k_bound = k_bound;
        victim->full_rows = full_rows;
        victim->ids = d_ids;
        victim->out = out;
        victim->graph = g;
        victim->exec = x;
        hit = victim;
    }
    hit->last = ++s->graph_clock;
    e = hipGraphLaunch(hit->exec, s->stream);
    if (e != hipSuccess) return hip_fail(s, e, "hipGraphLaunch");
    return G4S_OK;
}

G4S_API int g4s_lmhead_q4_0(g4s_sampler* s, const void* d_weights, int32_t rows, int32_t cols,
                            const float* d_hidden, int32_t batch, float* d_logits,
                            int64_t logits_stride)
{
    if (!s) return fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "sampler is NULL");
    s->err.clear();
    if (!d_weights || !d_hidden || !d_logits)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (rows < 1 || cols < 32 || (cols % 32) != 0)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "rows %d / cols %d (cols must be a multiple of 32)",
                    rows, cols);
    if (batch < 1 || logits_stride < rows)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "batch %d / logits_stride %lld", batch,
                    (long long)logits_stride);
    hipError_t e = g4s::lmhead_q4_0_launch((const uint8_t*)d_weights, rows, cols, d_hidden, batch,
                                           d_logits, logits_stride, s->stream);
    if (e == hipErrorNotSupported)
        return fail(s, G4S_ERR_UNSUPPORTED, "LM-head shape not supported (batch %d)", batch);
    if (e != hipSuccess) return hip_fail(s, e, "LM-head kernel launch");
    return G4S_OK;
}

namespace {

int check_tiled(g4s_sampler* s, const void* d_tiles, int32_t rows, int32_t cols,
                const float* d_hidden, int32_t batch, float* d_logits, int64_t logits_stride,
                bool logits_optional = false)
{
    if (!d_tiles || !d_hidden || (!d_logits && !logits_optional))
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (rows < 1 || cols < 32 || (cols % 32) != 0)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "rows %d / cols %d (cols must be a multiple of 32)",
                    rows, cols);
    if (!d_logits) logits_stride = rows;
    if (batch < 1 || logits_stride < rows)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "batch %d / logits_stride %lld", batch,
                    (long long)logits_stride);
    if (((uintptr_t)d_tiles & 15u) != 0 || ((uintptr_t)d_hidden & 15u) != 0)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "d_tiles and d_hidden must be 16-byte aligned");
    if ((int64_t)batch * cols * 4 > INT32_MAX)
        return fail(s, G4S_ERR_UNSUPPORTED, "hidden matrix of %d x %d floats above 2 GiB", batch,
                    cols);
    return G4S_OK;
}

}  // namespace

G4S_API int g4s_lmhead_q4_0_tiled(g4s_sampler* s, const void* d_tiles, int32_t rows, int32_t cols,
                                  const float* d_hidden, int32_t batch, float* d_logits,
                                  int64_t logits_stride)
{
    if (!s) return fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "sampler is NULL");
    s->err.clear();
    int rc = check_tiled(s, d_tiles, rows, cols, d_hidden, batch, d_logits, logits_stride);
    if (rc) return rc;
    hipError_t e = g4s::lmhead_tiled_launch((const uint8_t*)d_tiles, rows, cols, d_hidden, batch,
                                            d_logits, logits_stride, nullptr, s->stream);
    if (e != hipSuccess) return hip_fail(s, e, "LM-head kernel launch");
    return G4S_OK;
}

G4S_API int g4s_embed_q4_0(g4s_sampler* s, const void* d_weights, int32_t rows, int32_t cols,
                           const int32_t* d_tokens, int32_t batch, float scale, float* d_hidden)
{
    if (!s) return fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "sampler is NULL");
    s->err.clear();
    if (!d_weights || !d_tokens || !d_hidden)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (rows < 1 || cols < 32 || (cols % 32) != 0 || batch < 1)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "rows %d / cols %d / batch %d", rows, cols, batch);
    if (((uintptr_t)d_weights & 1u) != 0)
        return fail(s, G4S_ERR_INVALID_ARGUMENT, "d_weights must be 2-byte aligned");
    hipError_t e = g4s::embed_q4_0_launch((const uint8_t*)d_weights, rows, cols, d_tokens, batch,
                                          scale, d_hidden, s->stream);
    if (e != hipSuccess) return hip_fail(s, e, "embedding kernel launch");
    return G4S_OK;
}

namespace {

bool is_eos(int32_t t)
{
    return t == G4S_EOS_TOKEN_1 || t == G4S_EOS_TOKEN_2 || t == G4S_EOS_TOKEN_3;
}

/* DoSample for the rows b with want[b], as runs of consecutive rows (one
 * synchronous sample per run); u comes from `random` for rows with T > 0. */
int sample_rows(g4s_sampler* s, const void* d_logits, int32_t dtype, int64_t row_stride,
                int32_t batch, const g4s_params* params, g4s_random_fn random, void* user,
                const std::vector<uint8_t>& want, std::vector<int32_t>& ids)
{
    const int64_t esize = dtype == G4S_DTYPE_F32 ? 4 : 2;
    std::vector<double> u((size_t)batch, 0.0);
    for (int32_t b = 0; b < batch; ++b) {
        if (!want[(size_t)b] || !(params[b].temperature > 0.0f)) continue;
        u[(size_t)b] = random(user, b);
        if (!(u[(size_t)b] >= 0.0 && u[(size_t)b] < 1.0))
            return fail(s, G4S_ERR_INVALID_ARGUMENT, "sequence %d: random() = %g outside [0, 1)", b,
                        u[(size_t)b]);
    }
    for (int32_t b0 = 0; b0 < batch;) {
        if (!want[(size_t)b0]) {
            ++b0;
            continue;
        }
        int32_t b1 = b0;
        while (b1 < batch && want[(size_t)b1]) ++b1;
        const char* p = static_cast<const char*>(d_logits) + (int64_t)b0 * row_stride * esize;
        const int rc = sample_sync(s, p, dtype, row_stride, b1 - b0, params + b0, u.data() + b0,
                                   ids.data() + b0, nullptr, nullptr);
        if (rc) return rc;
        b0 = b1;
    }
    return G4S_OK;
}

}  // namespace

G4S_API int g4s_generate(g4s_sampler* s, int32_t batch, const g4s_params* params,
                         int32_t max_tokens, const void* d_logits, int32_t dtype,
                         int64_t row_stride, g4s_forward_fn forward, g4s_random_fn random,
                         g4s_token_fn on_token, void* user, int32_t* tokens, int32_t* lengths)
{
    if (!s) return fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "sampler is NULL");
    s->err.clear();
    int rc = check_logits(s, d_logits, dtype, row_stride, batch);
    if (rc) return rc;
    if (!params || !forward || !random || !lengths || (max_tokens > 0 && !tokens))
        return fail(s, G4S_ERR_INVALID_ARGUMENT,
                    "params, forward, random, lengths (and tokens) must be non-NULL");
    const size_t B = (size_t)batch;
    std::vector<uint8_t> live(B, 1), want(B, 1);
    std::vector<int32_t> cur(B, -1), len(B, 0), fwd(B, -1);
    for (size_t b = 0; b < B; ++b) lengths[b] = 0;
    /* the first token of every sequence, from its prompt's logits (:2889) */
    rc = sample_rows(s, d_logits, dtype, row_stride, batch, params, random, user, want, cur);
    if (rc) return rc;
    for (;;) {
        bool any = false;
        for (size_t b = 0; b < B; ++b) {
            want[b] = 0;
            fwd[b] = -1;
            if (!live[b]) continue;
            if (len[b] >= max_tokens) { /* while LI < AMaxTokens (:2904) */
                live[b] = 0;
                continue;
            }
            tokens[b * (size_t)max_tokens + (size_t)len[b]] = cur[b]; /* :2906 */
            lengths[b] = ++len[b];
            if (is_eos(cur[b]) || (on_token && on_token(user, (int32_t)b, cur[b]) == 0)) {
                live[b] = 0; /* :2908-2916 */
                continue;
            }
            fwd[b] = cur[b];
            want[b] = 1;
            any = true;
        }
        if (!any) break;
        if (forward(user, fwd.data(), batch) != 0) /* :2919 */
            return fail(s, G4S_ERR_ABORTED, "the forward callback failed");
        rc = sample_rows(s, d_logits, dtype, row_stride, batch, params, random, user, want, cur);
        if (rc) return rc; /* :2923 */
    }
    return G4S_OK;
}

namespace {

/* The fused call without logits accepts top-k rows only (0 < TopK <=
 * kMaxTopK, TopK < vocab) and at most 8192 64-row groups. */
int check_no_logits(g4s_sampler* s, int32_t batch, const g4s_params* params)
{
    if ((s->vocab + 63) / 64 > 8192)
        return fail(s, G4S_ERR_UNSUPPORTED, "vocab %d above 524288 without d_logits", s->vocab);
    for (int32_t r = 0; r < batch; ++r)
        if (!is_topk_row(params[r], s->vocab) || params[r].top_k > g4s::kMaxTopK)
            return fail(s, G4S_ERR_INVALID_ARGUMENT,
                        "row %d: TopK %d needs d_logits (only 0 < TopK <= %d without them)", r,
                        params[r].top_k, g4s::kMaxTopK);
    return G4S_OK;
}

/* Row r of a fused call without logits whose ties needed every logit: its
 * logits recomputed into the handle's row buffer, then sampled as
 * g4s_sample_ex would, into row r of the caller's outputs. */
int resample_row(g4s_sampler* s, const void* d_tiles, int32_t cols, const float* d_hidden,
                 int32_t r, const g4s_params* params, const double* u, int32_t* ids,
                 const g4s_outputs* outputs)
{
    const int64_t stride = ((int64_t)s->vocab + 3) & ~(int64_t)3;
    if (!s->row_logits) {
        if (hipMalloc((void**)&s->row_logits, (size_t)stride * sizeof(float)) != hipSuccess) {
            s->row_logits = nullptr;
            return fail(s, G4S_ERR_OUT_OF_MEMORY, "row buffer of %lld floats",
                        (long long)stride);
        }
    }
    hipError_t e = g4s::lmhead_tiled_launch((const uint8_t*)d_tiles, s->vocab, cols,
                                            d_hidden + (int64_t)r * cols, 1, s->row_logits,
                                            stride, nullptr, s->stream);
    if (e != hipSuccess) return hip_fail(s, e, "LM-head kernel launch");
    g4s_outputs o{};
    if (outputs) {
        o = *outputs;
        const int64_t cap = o.capacity > 0 ? o.capacity : 0;
        if (o.count) o.count += r;
        if (o.indices) o.indices += (int64_t)r * cap;
        if (o.probs) o.probs += (int64_t)r * cap;
        if (o.argmax) o.argmax += r;
        if (o.lsum) o.lsum += r;
        if (o.flags) o.flags += r;
    }
    int32_t id = -1;
    const int rc = sample_sync(s, s->row_logits, G4S_DTYPE_F32, stride, 1, &params[r], &u[r], &id,
                               outputs ? &o : nullptr);
    ids[r] = id;
    if (rc) return rc;
    if (o.flags) {
        uint32_t f = 0u;
        e = hipMemcpy(&f, o.flags, sizeof(f), hipMemcpyDeviceToHost);
        f |= G4S_FLAG_ROW_RECOMPUTED;
        if (e == hipSuccess) e = hipMemcpy(o.flags, &f, sizeof(f), hipMemcpyHostToDevice);
        if (e != hipSuccess) return hip_fail(s, e, "flags of a recomputed row");
    }
    return G4S_OK;
}

}  // namespace

G4S_API int g4s_lmhead_sample_q4_0(g4s_sampler* s, const void* d_tiles, int32_t cols,
                                   const float* d_hidden, int32_t batch, float* d_logits,
                                   int64_t logits_stride, const g4s_params* params,
                                   const double* u, int32_t* ids, const g4s_outputs* outputs)
{
    if (!s) return fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "sampler is NULL");
    s->err.clear();
    int rc = check_tiled(s, d_tiles, s->vocab, cols, d_hidden, batch, d_logits, logits_stride,
                         true);
    if (rc) return rc;
    if (d_logits) {
        rc = check_logits(s, d_logits, G4S_DTYPE_F32, logits_stride, batch);
        if (rc) return rc;
    }
    rc = check_params(s, batch, params, u, ids);
    if (rc) return rc;
    if (!d_logits) {
        rc = check_no_logits(s, batch, params);
        if (rc) return rc;
    }
    hipError_t e = g4s::lmhead_tiled_launch((const uint8_t*)d_tiles, s->vocab, cols, d_hidden,
                                            batch, d_logits, logits_stride, s->gsum, s->stream);
    if (e != hipSuccess) return hip_fail(s, e, "LM-head kernel launch");
    if (d_logits)
        return sample_sync(s, d_logits, G4S_DTYPE_F32, logits_stride, batch, params, u, ids,
                           outputs, s->gsum);
    const LmSource lm{(const uint8_t*)d_tiles, d_hidden, cols};
    rc = sample_sync(s, nullptr, G4S_DTYPE_F32, s->vocab, batch, params, u, ids, outputs, s->gsum,
                     &lm);
    if (rc && rc != G4S_ERR_EMPTY_ROW) return rc;
    const int rc_rows = rc;
    std::vector<uint32_t> fl(s->h_flags, s->h_flags + batch);
    for (int32_t r = 0; r < batch; ++r) {
        if (!(fl[r] & G4S_FLAG_ROW_RECOMPUTED)) continue;
        rc = resample_row(s, d_tiles, cols, d_hidden, r, params, u, ids, outputs);
        if (rc) return rc;
    }
    return rc_rows;
}
