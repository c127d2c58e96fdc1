/*
 * g4s_oracle.cpp -- CPU restatement of the Gemma4.pas sampler (test oracle).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for libgemma4_sampler.so, never part
 * of the product path.  Each function follows the cited reference routine
 * statement by statement; the floating-point model is described in
 * g4s_oracle.h.  Build: make -C oracle (g++ -O2 -ffp-contract=off).
 */
#include "g4s_oracle.h"

#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#ifdef ORC_EXTENDED_IS_DOUBLE
typedef double ext_t;
static inline ext_t ext_exp(ext_t x) { return std::exp(x); }
static inline ext_t ext_tanh(ext_t x) { return std::tanh(x); }
static inline ext_t ext_round(ext_t x) { return std::nearbyint(x); }
#define ORC_SEMANTICS "Extended=binary64"
#else
typedef long double ext_t;
static inline ext_t ext_exp(ext_t x) { return expl(x); }
static inline ext_t ext_tanh(ext_t x) { return tanhl(x); }
static inline ext_t ext_round(ext_t x) { return nearbyintl(x); }
#define ORC_SEMANTICS "Extended=x87-80bit"
#endif

/* `LSingle := <ext expression>`: one rounding to binary32. */
static inline float to_single(ext_t v) { return (float)v; }

/* Pascal literal -1e30 assigned to a Single (Model.pas:2636) */
static const float kHeapEmpty = -1e30f;

extern "C" const char* orc_semantics(void) { return ORC_SEMANTICS; }

/* ---------------------------------------------------------------- Types.pas */

extern "C" float orc_bf16_to_f32(uint16_t v)
{
    /* TBFloat16.ToSingle, Types.pas:417-424: bits shl 16 */
    uint32_t bits = (uint32_t)v << 16;
    float r;
    std::memcpy(&r, &bits, 4);
    return r;
}

extern "C" uint16_t orc_f32_to_bf16(float v)
{
    /* TBFloat16.FromSingle, Types.pas:426-434: truncation */
    uint32_t bits;
    std::memcpy(&bits, &v, 4);
    return (uint16_t)(bits >> 16);
}

extern "C" float orc_f16_to_f32(uint16_t v)
{
    /* TFloat16.ToSingle, Types.pas:438-481 */
    uint32_t sign = (v >> 15) & 1u;
    uint32_t expo = (v >> 10) & 0x1Fu;
    uint32_t mant = v & 0x3FFu;
    uint32_t bits;
    if (expo == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            while ((mant & 0x400u) == 0) {
                mant <<= 1;
                expo += 1; /* Types.pas:462: Inc(LExponent) -- the exponent is raised,
                              not lowered, while normalising; restated as written */
            }
            expo += 1;
            mant &= 0x3FFu;
            bits = (sign << 31) | ((expo + (127 - 15)) << 23) | (mant << 13);
        }
    } else if (expo == 0x1F) {
        bits = (sign << 31) | (0xFFu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((expo + (127 - 15)) << 23) | (mant << 13);
    }
    float r;
    std::memcpy(&r, &bits, 4);
    return r;
}

extern "C" uint16_t orc_f16_from_f32(float v)
{
    /* TFloat16.FromSingle, Types.pas:483-501: truncation, flush to zero */
    uint32_t bits;
    std::memcpy(&bits, &v, 4);
    uint32_t sign = (bits >> 31) & 1u;
    int32_t expo = (int32_t)((bits >> 23) & 0xFFu) - 127 + 15;
    uint32_t mant = bits & 0x7FFFFFu;
    if (expo <= 0) return (uint16_t)(sign << 15);
    if (expo >= 0x1F) return (uint16_t)((sign << 15) | (0x1Fu << 10));
    return (uint16_t)((sign << 15) | ((uint32_t)expo << 10) | (mant >> 13));
}

/* --------------------------------------------------------- Layers/Tensors */

extern "C" void orc_logit_softcap(float* data, int32_t count, float cap)
{
    /* CpuLogitSoftcap, Layers.pas:300-316 */
    float inv_cap = to_single((ext_t)1.0 / (ext_t)cap);            /* :309 */
    for (int32_t i = 0; i < count; ++i) {
        float v = data[i];                                          /* :312 */
        data[i] = to_single(ext_tanh((ext_t)v * (ext_t)inv_cap) * (ext_t)cap); /* :313-314 */
    }
}

extern "C" float orc_softcap_topk(float x, float cap)
{
    /* LVals[LI] := LCap * Tanh(LVals[LI] / LCap), Model.pas:2776 */
    return to_single((ext_t)cap * ext_tanh((ext_t)x / (ext_t)cap));
}

extern "C" float orc_exp_diff(float a, float b)
{
    return to_single(ext_exp((ext_t)a - (ext_t)b));
}

extern "C" float orc_softmax_f32(float* data, int32_t count)
{
    /* CpuSoftmaxF32, Tensors.pas:638-673 */
    float lmax = data[0];                                           /* :648 */
    for (int32_t i = 1; i < count; ++i) {                           /* :649-654 */
        float v = data[i];
        if (v > lmax) lmax = v;
    }
    float lsum = 0.0f;                                              /* :657 */
    for (int32_t i = 0; i < count; ++i) {                           /* :658-663 */
        float v = to_single(ext_exp((ext_t)data[i] - (ext_t)lmax));
        data[i] = v;
        lsum = to_single((ext_t)lsum + (ext_t)v);
    }
    if (lsum > 0.0f) {                                              /* :666-672 */
        float inv = to_single((ext_t)1.0 / (ext_t)lsum);
        for (int32_t i = 0; i < count; ++i)
            data[i] = to_single((ext_t)data[i] * (ext_t)inv);
    }
    return lsum;
}

/* ---------------------------------------------------------------- Model.pas */

extern "C" int32_t orc_select_topk_indices(const float* logits, int32_t vocab, int32_t k,
                                           int32_t* out_idx)
{
    /* DoSelectTopKIndices, Model.pas:2615-2689 */
    std::vector<float> hv((size_t)k);
    std::vector<int32_t> hi((size_t)k);
    for (int32_t i = 0; i < k; ++i) {                               /* :2634-2638 */
        hv[i] = kHeapEmpty;
        hi[i] = -1;
    }
    for (int32_t i = 0; i < vocab; ++i) {                           /* :2640-2664 */
        float v = logits[i];
        if (v <= hv[0]) continue;
        int32_t pos = 0;
        for (;;) {
            int32_t child = pos * 2 + 1;
            if (child >= k) break;
            if (child + 1 < k && hv[child + 1] < hv[child]) child += 1;
            if (hv[child] >= v) break;
            hv[pos] = hv[child];
            hi[pos] = hi[child];
            pos = child;
        }
        hv[pos] = v;
        hi[pos] = i;
    }
    int32_t len = 0;                                                /* :2668-2676 */
    for (int32_t i = 0; i < k; ++i)
        if (hi[i] >= 0) out_idx[len++] = hi[i];
    for (int32_t i = 1; i < len; ++i) {                             /* :2678-2688 */
        int32_t tmp = out_idx[i];
        int32_t j = i - 1;
        while (j >= 0 && out_idx[j] > tmp) {
            out_idx[j + 1] = out_idx[j];
            --j;
        }
        out_idx[j + 1] = tmp;
    }
    return len;
}

extern "C" int32_t orc_sample_topp(float* logits, int32_t count, float top_p, float temperature,
                                   double u, orc_detail* detail)
{
    /* DoSampleTopP, Model.pas:2691-2737 */
    if (temperature > 0.0f && temperature != 1.0f) {               /* :2703-2708 */
        float inv = to_single((ext_t)1.0 / (ext_t)temperature);
        for (int32_t i = 0; i < count; ++i)
            logits[i] = to_single((ext_t)logits[i] * (ext_t)inv);
    }
    float vmax = logits[0];
    for (int32_t i = 1; i < count; ++i)
        if (logits[i] > vmax) vmax = logits[i];
    float lsum = orc_softmax_f32(logits, count);                    /* :2710 */

    int32_t result = 0;                                             /* :2712-2721 */
    float lmax = logits[0];
    for (int32_t i = 1; i < count; ++i) {
        if (logits[i] > lmax) {
            lmax = logits[i];
            result = i;
        }
    }
    int32_t argmax = result;
    int32_t reached = 0;
    float cum = 0.0f, cum_prev = 0.0f, rnd = 0.0f;
    if (temperature > 0.0f) {                                       /* :2723-2736 */
        rnd = to_single((ext_t)u * (ext_t)top_p);
        for (int32_t i = 0; i < count; ++i) {
            cum_prev = cum;
            cum = to_single((ext_t)cum + (ext_t)logits[i]);
            if (cum >= rnd) {
                result = i;
                reached = 1;
                break;
            }
        }
    }
    if (detail) {
        detail->path = 1;
        detail->count = count;
        detail->argmax_pos = argmax;
        detail->chosen_pos = result;
        detail->drew = temperature > 0.0f;
        detail->reached = reached;
        detail->lsum = lsum;
        detail->threshold = rnd;
        detail->cum_prev = reached ? cum_prev : 0.0f;
        detail->cum_at = reached ? cum : 0.0f;
        detail->max_val = vmax;
        detail->token = result;
    }
    return result;
}

extern "C" int32_t orc_do_sample(const float* logits, int32_t vocab, float softcap,
                                 const orc_params* params, double u, int32_t* out_idx,
                                 float* out_probs, int32_t cap, orc_detail* detail)
{
    /* DoSample, Model.pas:2739-2827 */
    if (params->top_k <= 0 || params->top_k >= vocab) {             /* :2756-2763 */
        std::vector<float> work(logits, logits + vocab);
        if (softcap > 0.0f) orc_logit_softcap(work.data(), vocab, softcap);
        int32_t r = orc_sample_topp(work.data(), vocab, params->top_p, params->temperature, u,
                                    detail);
        if (out_probs && cap >= vocab) std::memcpy(out_probs, work.data(), sizeof(float) * vocab);
        if (out_idx && cap >= vocab)
            for (int32_t i = 0; i < vocab; ++i) out_idx[i] = i;
        return r;
    }

    std::vector<int32_t> idx((size_t)params->top_k);
    int32_t n = orc_select_topk_indices(logits, vocab, params->top_k, idx.data()); /* :2767 */
    if (n == 0) {
        /* LVals[0] on an empty array: outside the reference's domain */
        if (detail) {
            std::memset(detail, 0, sizeof(*detail));
            detail->token = -1;
        }
        return -1;
    }
    std::vector<float> vals((size_t)n);
    for (int32_t i = 0; i < n; ++i) {                               /* :2772-2777 */
        vals[i] = logits[idx[i]];
        if (softcap > 0.0f) vals[i] = to_single((ext_t)softcap * ext_tanh((ext_t)vals[i] / (ext_t)softcap));
    }
    float temperature = params->temperature;
    if (temperature > 0.0f && temperature != 1.0f) {               /* :2780-2785 */
        float inv = to_single((ext_t)1.0 / (ext_t)temperature);
        for (int32_t i = 0; i < n; ++i) vals[i] = to_single((ext_t)vals[i] * (ext_t)inv);
    }
    float lmax = vals[0];                                           /* :2789-2792 */
    for (int32_t i = 1; i < n; ++i)
        if (vals[i] > lmax) lmax = vals[i];
    float lsum = 0.0f;                                              /* :2794-2799 */
    for (int32_t i = 0; i < n; ++i) {
        vals[i] = to_single(ext_exp((ext_t)vals[i] - (ext_t)lmax));
        lsum = to_single((ext_t)lsum + (ext_t)vals[i]);
    }
    for (int32_t i = 0; i < n; ++i)                                 /* :2800-2801 */
        vals[i] = to_single((ext_t)vals[i] / (ext_t)lsum);
    int32_t best = 0;                                               /* :2804-2807 */
    for (int32_t i = 1; i < n; ++i)
        if (vals[i] > vals[best]) best = i;
    int32_t argmax = best;
    int32_t reached = 0;
    float cum = 0.0f, cum_prev = 0.0f, rnd = 0.0f;
    if (temperature > 0.0f) {                                       /* :2811-2824 */
        rnd = to_single((ext_t)u * (ext_t)params->top_p);
        for (int32_t i = 0; i < n; ++i) {
            cum_prev = cum;
            cum = to_single((ext_t)cum + (ext_t)vals[i]);
            if (cum >= rnd) {
                best = i;
                reached = 1;
                break;
            }
        }
    }
    if (out_idx)
        for (int32_t i = 0; i < n && i < cap; ++i) out_idx[i] = idx[i];
    if (out_probs)
        for (int32_t i = 0; i < n && i < cap; ++i) out_probs[i] = vals[i];
    if (detail) {
        detail->path = 0;
        detail->count = n;
        detail->argmax_pos = argmax;
        detail->chosen_pos = best;
        detail->drew = temperature > 0.0f;
        detail->reached = reached;
        detail->lsum = lsum;
        detail->threshold = rnd;
        detail->cum_prev = reached ? cum_prev : 0.0f;
        detail->cum_at = reached ? cum : 0.0f;
        detail->max_val = lmax;
        detail->token = idx[best];
    }
    return idx[best];                                               /* :2826 */
}

extern "C" int32_t orc_sample_batch(const void* logits, int32_t dtype, int32_t vocab,
                                    int64_t row_stride, int32_t batch, const orc_params* params,
                                    const double* u, float softcap, int32_t* ids, int32_t threads)
{
    if (threads < 1) threads = 1;
    auto work = [&](int32_t t) {
        std::vector<float> row;
        if (dtype == 1) row.resize((size_t)vocab);
        for (int32_t r = t; r < batch; r += threads) {
            const float* src;
            if (dtype == 1) {
                const uint16_t* b = (const uint16_t*)logits + (int64_t)r * row_stride;
                for (int32_t i = 0; i < vocab; ++i) row[i] = orc_bf16_to_f32(b[i]);
                src = row.data();
            } else {
                src = (const float*)logits + (int64_t)r * row_stride;
            }
            ids[r] = orc_do_sample(src, vocab, softcap, &params[r], u[r], nullptr, nullptr, 0,
                                   nullptr);
        }
    };
    if (threads == 1) {
        work(0);
    } else {
        std::vector<std::thread> pool;
        for (int32_t t = 0; t < threads; ++t) pool.emplace_back(work, t);
        for (auto& th : pool) th.join();
    }
    return 0;
}

/* ---------------------------------------------------------------- Quant.pas */

static inline float q4_scale(const uint8_t* block18)
{
    uint16_t s = (uint16_t)(block18[0] | (block18[1] << 8)); /* TQ4Block.Scale: little-endian UInt16 */
    return orc_f16_to_f32(s);
}

extern "C" void orc_dequant_q4_block(const uint8_t* block18, float* dst32)
{
    /* DequantQ4Block, Quant.pas:209-239 */
    float scale = q4_scale(block18);
    for (int i = 0; i < 16; ++i) {
        uint8_t b = block18[2 + i];
        int lo = (int)(b & 0x0F) - 8;
        dst32[i * 2] = to_single((ext_t)(float)lo * (ext_t)scale);
        int hi = (int)(b >> 4) - 8;
        dst32[i * 2 + 1] = to_single((ext_t)(float)hi * (ext_t)scale);
    }
}

extern "C" uint64_t orc_f32_to_q4_buffer(const float* src, uint8_t* dst, uint64_t count)
{
    /* F32ToQ4Buffer, Quant.pas:121-197 */
    uint64_t nblocks = count / 32;
    for (uint64_t b = 0; b < nblocks; ++b) {
        const float* f = src + b * 32;
        uint8_t* out = dst + b * 18;
        float lmax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            float v = std::fabs(f[i]);
            if (v > lmax) lmax = v;
        }
        float scale = to_single((ext_t)lmax / (ext_t)7.0);
        uint16_t s16 = orc_f16_from_f32(scale);
        out[0] = (uint8_t)(s16 & 0xFF);
        out[1] = (uint8_t)(s16 >> 8);
        float inv = scale > 0.0f ? to_single((ext_t)1.0 / (ext_t)scale) : 0.0f;
        for (int i = 0; i < 16; ++i) {
            int q = (int)ext_round((ext_t)f[i * 2] * (ext_t)inv); /* Round(): banker's rounding */
            if (q < -8) q = -8;
            if (q > 7) q = 7;
            uint8_t nib = (uint8_t)(q + 8);
            q = (int)ext_round((ext_t)f[i * 2 + 1] * (ext_t)inv);
            if (q < -8) q = -8;
            if (q > 7) q = 7;
            nib = (uint8_t)(nib | ((uint8_t)(q + 8) << 4));
            out[2 + i] = nib;
        }
    }
    return nblocks;
}

extern "C" void orc_matvec_q4(const uint8_t* matrix, const float* vec, float* dst, int32_t rows,
                              int32_t cols, int32_t row0, int32_t nrows)
{
    /* CpuMatVecQ4, Tensors.pas:546-598 */
    (void)rows;
    int32_t bpr = cols / 32;
    for (int32_t r = row0; r < row0 + nrows; ++r) {
        float lsum = 0.0f;
        const uint8_t* rs = matrix + (int64_t)r * bpr * 18;
        for (int32_t bi = 0; bi < bpr; ++bi) {
            const uint8_t* blk = rs + (int64_t)bi * 18;
            float scale = q4_scale(blk);
            int32_t vi = bi * 32;
            for (int j = 0; j < 16; ++j) {
                uint8_t byte = blk[2 + j];
                int lo = (int)(byte & 0x0F) - 8;
                lsum = to_single((ext_t)lsum + ((ext_t)(float)lo * (ext_t)scale) * (ext_t)vec[vi + j * 2]);
                int hi = (int)(byte >> 4) - 8;
                lsum = to_single((ext_t)lsum + ((ext_t)(float)hi * (ext_t)scale) * (ext_t)vec[vi + j * 2 + 1]);
            }
        }
        dst[r] = lsum;
    }
}

extern "C" void orc_matvec_q4_batch(const uint8_t* matrix, const float* vecs, float* dst,
                                    int32_t rows, int32_t cols, int32_t batch, int32_t threads)
{
    if (threads < 1) threads = 1;
    auto work = [&](int32_t t) {
        int32_t per = (rows + threads - 1) / threads;
        int32_t r0 = t * per;
        int32_t r1 = r0 + per > rows ? rows : r0 + per;
        if (r0 >= r1) return;
        for (int32_t b = 0; b < batch; ++b)
            orc_matvec_q4(matrix, vecs + (int64_t)b * cols, dst + (int64_t)b * rows, rows, cols, r0,
                          r1 - r0);
    };
    std::vector<std::thread> pool;
    for (int32_t t = 0; t < threads; ++t) pool.emplace_back(work, t);
    for (auto& th : pool) th.join();
}

extern "C" float orc_seqsum_f32(const float* a, int64_t n, float threshold, int64_t* first_reach)
{
    float s = 0.0f;
    int64_t first = -1;
    for (int64_t i = 0; i < n; ++i) {
        s = to_single((ext_t)s + (ext_t)a[i]);
        if (first < 0 && s >= threshold) first = i;
    }
    if (first_reach) *first_reach = first;
    return s;
}
