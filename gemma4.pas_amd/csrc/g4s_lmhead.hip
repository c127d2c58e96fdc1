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
 * wave-uniform (scalar loads); 32 independent running sums per thread.
 * Compute-bound at B=32: 2*B*rows*cols flops against 377 MB of weights.
 */
#include "g4s_lmhead.h"

namespace g4s {

namespace {

constexpr int kLmBlock = 256;
constexpr int kLmTile = 32; /* hidden vectors per pass over the weights */

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
                                                             int64_t stride)
{
    const int32_t r = blockIdx.x * kLmBlock + threadIdx.x;
    const bool active = r < rows;
    const int32_t rr = active ? r : rows - 1;
    const uint8_t* wrow = w + (int64_t)rr * nblk * 18;
    for (int32_t b0 = 0; b0 < batch; b0 += kLmTile) {
        const int32_t nb = batch - b0 < kLmTile ? batch - b0 : kLmTile;
        float S[kLmTile];
#pragma unroll
        for (int b = 0; b < kLmTile; ++b) S[b] = 0.0f;
        for (int32_t k = 0; k < nblk; ++k) {
            const uint16_t* blk = reinterpret_cast<const uint16_t*>(wrow + (int64_t)k * 18);
            uint32_t half[9];
#pragma unroll
            for (int i = 0; i < 9; ++i) half[i] = blk[i];
            const float s = f16_to_f32_ref(half[0]);
            float qs[32];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t byte = (half[1 + (j >> 1)] >> ((j & 1) * 8)) & 0xFFu;
                qs[2 * j] = (float)((int)(byte & 0x0Fu) - 8) * s;     /* Tensors.pas:586 */
                qs[2 * j + 1] = (float)((int)(byte >> 4) - 8) * s;    /* Tensors.pas:590 */
            }
            const float* hk = h + (int64_t)b0 * cols + (int64_t)k * 32;
#pragma unroll
            for (int b = 0; b < kLmTile; ++b) {
                if (b < nb) {
                    const float* x = hk + (int64_t)b * cols;
#pragma unroll
                    for (int j = 0; j < 32; ++j) S[b] = __builtin_fmaf(qs[j], x[j], S[b]);
                }
            }
        }
        if (active) {
#pragma unroll
            for (int b = 0; b < kLmTile; ++b)
                if (b < nb) out[(int64_t)(b0 + b) * stride + r] = S[b];
        }
    }
}

}  // namespace

hipError_t lmhead_q4_0_launch(const uint8_t* w, int32_t rows, int32_t cols, const float* h,
                              int32_t batch, float* logits, int64_t stride, hipStream_t s)
{
    const int32_t nblk = cols / 32;
    hipLaunchKernelGGL(lmhead_q4_kernel, dim3((unsigned)((rows + kLmBlock - 1) / kLmBlock)),
                       dim3(kLmBlock), 0, s, w, rows, nblk, h, cols, batch, logits, stride);
    return hipGetLastError();
}

}  // namespace g4s
