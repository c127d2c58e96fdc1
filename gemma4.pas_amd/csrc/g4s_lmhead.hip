/*
 * g4s_lmhead.hip -- the Q4_0 LM head feeding the sampler, bit-exact with
 * CpuMatVecQ4 (src/Gemma4.Tensors.pas:546-598).
 *
 * Every logit is the reference's left-to-right sum over the row's blocks,
 * each term `LSum := LSum + (Single(q) * LScale) * x` in block order, low
 * nibble (x[2j]) before high nibble (x[2j+1]) of byte j (:581-593).  The
 * product q*s is exact in binary32 (a 4-bit integer times the 11-bit fp16
 * scale) and q*s*x has at most 39 significant bits, so under the reference's
 * Extended intermediates the step rounds the exact S + q*s*x to 64 bits and
 * then to binary32.  One binary32 fma(q*s, x, S) rounds it once, and the
 * two agree unless the 64-bit rounding lands on a binary32 midpoint: that
 * needs the exact sum to span more than 64 bits while sitting within 2^-64
 * of a midpoint, which happens only for 0 < |S| <= 2^-64 |q*s*x| with q*s*x
 * itself a binary32 midpoint -- never for this workload (|S| is then at
 * least 2^-60 unless it is 0).  So the kernel is one fma per term, in the
 * reference's order.
 *
 * Layout: one weight row per thread (the TQ4Block row, 18 bytes per 32
 * weights, read in place), batch tiles of 32 hidden vectors whose values are
 * staged in LDS two blocks at a time (double-buffered, the next group's
 * loads in flight during the current one) and read as broadcasts; 32
 * independent running sums per thread.
 * Compute-bound at B=32: 2*B*rows*cols flops against 377 MB of weights.
 */
#include "g4s_lmhead.h"

namespace g4s {

namespace {

constexpr int kLmBlock = 256;
constexpr int kLmTile = 32; /* hidden vectors per pass over the weights */
constexpr int kLmKb = 2;    /* weight blocks (of 32 terms) per staged group of hidden values */

/* TFloat16.ToSingle (src/Gemma4.Types.pas:438-481) as written, including its
 * handling of subnormal halves (the exponent is raised while normalising). */
__device__ __forceinline__ float f16_to_f32_ref(uint32_t v)
{
    const uint32_t sign = (v >> 15) & 1u;
    uint32_t expo = (v >> 10) & 0x1Fu;
    uint32_t mant = v & 0x3FFu;
    uint32_t bits;
    if (expo == 0u) {
        if (mant == 0u) {
            bits = sign << 31;
        } else {
            const uint32_t shift = (uint32_t)__builtin_clz(mant) - 21u; /* until bit 10 is set */
            mant = (mant << shift) & 0x3FFu;
            expo = shift + 1u;
            bits = (sign << 31) | ((expo + (127u - 15u)) << 23) | (mant << 13);
        }
    } else if (expo == 0x1Fu) {
        bits = (sign << 31) | (0xFFu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((expo + (127u - 15u)) << 23) | (mant << 13);
    }
    return __uint_as_float(bits);
}

__global__ __launch_bounds__(kLmBlock) void lmhead_q4_kernel(const uint8_t* __restrict__ w,
                                                             int32_t rows, int32_t nblk,
                                                             const float* __restrict__ h,
                                                             int32_t cols, int32_t batch,
                                                             float* __restrict__ out,
                                                             int64_t stride, int32_t h_vec4)
{
    /* the hidden values of kLmKb weight blocks for the tile's kLmTile
     * vectors, double-buffered: every lane reads the same entry (an LDS
     * broadcast), so the fma operands come from VGPRs */
    __shared__ __align__(16) float xs[2][kLmTile][kLmKb * 32];
    constexpr int kStage = kLmTile * kLmKb * 8 / kLmBlock; /* float4 per thread per stage */
    static_assert(kLmTile * kLmKb * 8 % kLmBlock == 0, "whole float4 stages");
    const int32_t r = blockIdx.x * kLmBlock + threadIdx.x;
    const bool active = r < rows;
    const int32_t rr = active ? r : rows - 1;
    const uint8_t* wrow = w + (int64_t)rr * nblk * 18;
    const int32_t ngroup = (nblk + kLmKb - 1) / kLmKb;
    for (int32_t b0 = 0; b0 < batch; b0 += kLmTile) {
        const int32_t nb = batch - b0 < kLmTile ? batch - b0 : kLmTile;
        /* hidden values of block group g (zeros past the batch or the row) */
        const auto fetch = [&](int32_t g, float4 (&v)[kStage]) {
#pragma unroll
            for (int q = 0; q < kStage; ++q) {
                const int i = threadIdx.x + q * kLmBlock;
                const int b = i / (kLmKb * 8), c4 = i % (kLmKb * 8);
                const int32_t col = g * kLmKb * 32 + c4 * 4;
                float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (b < nb && col < cols) {
                    const float* src = h + (int64_t)(b0 + b) * cols + col;
                    if (h_vec4)
                        x = *reinterpret_cast<const float4*>(src);
                    else
                        x = make_float4(src[0], src[1], src[2], src[3]);
                }
                v[q] = x;
            }
        };
        const auto stash = [&](int buf, const float4 (&v)[kStage]) {
#pragma unroll
            for (int q = 0; q < kStage; ++q) {
                const int i = threadIdx.x + q * kLmBlock;
                reinterpret_cast<float4*>(&xs[buf][i / (kLmKb * 8)][0])[i % (kLmKb * 8)] = v[q];
            }
        };
        float S[kLmTile];
#pragma unroll
        for (int b = 0; b < kLmTile; ++b) S[b] = 0.0f;
        float4 nx[kStage];
        fetch(0, nx);
        stash(0, nx);
        __syncthreads();
        for (int32_t g = 0; g < ngroup; ++g) {
            const int buf = g & 1;
            if (g + 1 < ngroup) fetch(g + 1, nx); /* in flight during this group */
            for (int kk = 0; kk < kLmKb; ++kk) {
                const int32_t k = g * kLmKb + kk;
                if (k >= nblk) break;
                const uint16_t* blk = reinterpret_cast<const uint16_t*>(wrow + (int64_t)k * 18);
                uint32_t half[9];
#pragma unroll
                for (int i = 0; i < 9; ++i) half[i] = blk[i];
                const float sc = f16_to_f32_ref(half[0]);
                float qs[32];
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const uint32_t byte = (half[1 + (j >> 1)] >> ((j & 1) * 8)) & 0xFFu;
                    qs[2 * j] = (float)((int)(byte & 0x0Fu) - 8) * sc;     /* Tensors.pas:586 */
                    qs[2 * j + 1] = (float)((int)(byte >> 4) - 8) * sc;    /* Tensors.pas:590 */
                }
                /* term j of every vector before term j+4: the 32 running sums
                 * are independent chains, each still in the reference's order */
#pragma unroll
                for (int j4 = 0; j4 < 8; ++j4) {
#pragma unroll
                    for (int b = 0; b < kLmTile; ++b) {
                        const float4 x = reinterpret_cast<const float4*>(&xs[buf][b][kk * 32])[j4];
                        S[b] = __builtin_fmaf(qs[4 * j4], x.x, S[b]);
                        S[b] = __builtin_fmaf(qs[4 * j4 + 1], x.y, S[b]);
                        S[b] = __builtin_fmaf(qs[4 * j4 + 2], x.z, S[b]);
                        S[b] = __builtin_fmaf(qs[4 * j4 + 3], x.w, S[b]);
                    }
                }
            }
            if (g + 1 < ngroup) stash(buf ^ 1, nx); /* read last in group g - 1 */
            __syncthreads();
        }
        if (active) {
#pragma unroll
            for (int b = 0; b < kLmTile; ++b)
                if (b < nb) out[(int64_t)(b0 + b) * stride + r] = S[b];
        }
        __syncthreads(); /* the next tile restages both buffers */
    }
}

}  // namespace

hipError_t lmhead_q4_0_launch(const uint8_t* w, int32_t rows, int32_t cols, const float* h,
                              int32_t batch, float* logits, int64_t stride, hipStream_t s)
{
    const int32_t nblk = cols / 32;
    const int32_t h_vec4 = (reinterpret_cast<uintptr_t>(h) & 15u) == 0 ? 1 : 0;
    hipLaunchKernelGGL(lmhead_q4_kernel, dim3((unsigned)((rows + kLmBlock - 1) / kLmBlock)),
                       dim3(kLmBlock), 0, s, w, rows, nblk, h, cols, batch, logits, stride, h_vec4);
    return hipGetLastError();
}

}  // namespace g4s
