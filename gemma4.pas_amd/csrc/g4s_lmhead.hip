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

/* ------------------------------------------------------------------
 * TILED64 layout and the LM head over it.
 *
 * One wave per 64 weight rows (lane = row), waves independent (no LDS, no
 * barrier).  Per 32-column block a lane loads its row's binary32 scale and
 * 16 nibble bytes from the tile (256 + 1024 contiguous bytes per wave) one
 * block ahead, and dequantises the 32 weights once for the 32 hidden
 * vectors of the batch tile.  The hidden values reach the fma without LDS:
 * a 16-byte load per lane brings two vectors' 32 values of the block into
 * four VGPRs (lanes 0-7 of every 16-lane row: vector b, columns 4n..4n+3;
 * lanes 8-15: vector b+1), and v_fmac_f32 with the DPP modifier
 * row_newbcast:n hands lane n's value of its 16-lane row to all lanes of
 * that row -- the same value in all four rows, so every lane sees it.  Each
 * logit is still one fma per term in column order (the order argument at
 * the top of this file), the 32 vectors being 32 independent chains.
 * ------------------------------------------------------------------ */

constexpr int kTileB = 32;        /* hidden vectors per pass over the weights */
constexpr int kTileWaves = 4;     /* waves (64-row groups) per workgroup */
constexpr int kXAhead = 4;        /* vector pairs whose values are in flight */

__global__ __launch_bounds__(256) void q4_tile_kernel(const uint8_t* __restrict__ src, int32_t rows,
                                                      int32_t nblk, uint8_t* __restrict__ dst)
{
    const int32_t groups = (rows + kQ4TileRows - 1) / kQ4TileRows;
    const int64_t total = (int64_t)groups * kQ4TileRows * nblk;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        /* t = (g * nblk + k) * 64 + lane: the destination is written in order */
        const int32_t lane = (int32_t)(t % kQ4TileRows);
        const int64_t tile = t / kQ4TileRows;
        const int32_t k = (int32_t)(tile % nblk);
        const int32_t g = (int32_t)(tile / nblk);
        const int32_t r = g * kQ4TileRows + lane;
        uint8_t* tp = dst + tile * kQ4TileBytes;
        float sc = 0.0f;
        uint32_t q[4] = {0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
        if (r < rows) {
            const uint16_t* b = reinterpret_cast<const uint16_t*>(src + ((int64_t)r * nblk + k) * 18);
            sc = f16_to_f32_ref(b[0]);
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = (uint32_t)b[1 + 2 * i] | ((uint32_t)b[2 + 2 * i] << 16);
        }
        reinterpret_cast<float*>(tp)[lane] = sc;
        reinterpret_cast<uint4*>(tp + kQ4TileRows * 4)[lane] = make_uint4(q[0], q[1], q[2], q[3]);
    }
}

/* 16 fmas: S0 (vector b) and S1 (vector b+1) take terms 8p .. 8p+7 of the
 * block, in order, interleaved; x0..x3 hold the pair's values (lane n:
 * columns 4n..4n+3 of b, lane n+8: of b+1) and q0..q7 the weights. */
#define G4S_FMAC_BCAST(N0, N1, N2, N3)                                                          \
    asm("v_fmac_f32_dpp %0, %2, %6 row_newbcast:" N0 " row_mask:0xf bank_mask:0xf\n\t"          \
        "v_fmac_f32_dpp %1, %2, %6 row_newbcast:" N1 " row_mask:0xf bank_mask:0xf\n\t"          \
        "v_fmac_f32_dpp %0, %3, %7 row_newbcast:" N0 " row_mask:0xf bank_mask:0xf\n\t"          \
        "v_fmac_f32_dpp %1, %3, %7 row_newbcast:" N1 " row_mask:0xf bank_mask:0xf\n\t"          \
        "v_fmac_f32_dpp %0, %4, %8 row_newbcast:" N0 " row_mask:0xf bank_mask:0xf\n\t"          \
        "v_fmac_f32_dpp %1, %4, %8 row_newbcast:" N1 " row_mask:0xf bank_mask:0xf\n\t"          \
        "v_fmac_f32_dpp %0, %5, %9 row_newbcast:" N0 " row_mask:0xf bank_mask:0xf\n\t"          \
        "v_fmac_f32_dpp %1, %5, %9 row_newbcast:" N1 " row_mask:0xf bank_mask:0xf\n\t"          \
        "v_fmac_f32_dpp %0, %2, %10 row_newbcast:" N2 " row_mask:0xf bank_mask:0xf\n\t"         \
        "v_fmac_f32_dpp %1, %2, %10 row_newbcast:" N3 " row_mask:0xf bank_mask:0xf\n\t"         \
        "v_fmac_f32_dpp %0, %3, %11 row_newbcast:" N2 " row_mask:0xf bank_mask:0xf\n\t"         \
        "v_fmac_f32_dpp %1, %3, %11 row_newbcast:" N3 " row_mask:0xf bank_mask:0xf\n\t"         \
        "v_fmac_f32_dpp %0, %4, %12 row_newbcast:" N2 " row_mask:0xf bank_mask:0xf\n\t"         \
        "v_fmac_f32_dpp %1, %4, %12 row_newbcast:" N3 " row_mask:0xf bank_mask:0xf\n\t"         \
        "v_fmac_f32_dpp %0, %5, %13 row_newbcast:" N2 " row_mask:0xf bank_mask:0xf\n\t"         \
        "v_fmac_f32_dpp %1, %5, %13 row_newbcast:" N3 " row_mask:0xf bank_mask:0xf"             \
        : "+v"(S0), "+v"(S1)                                                                    \
        : "v"(x0), "v"(x1), "v"(x2), "v"(x3), "v"(q0), "v"(q1), "v"(q2), "v"(q3), "v"(q4),      \
          "v"(q5), "v"(q6), "v"(q7))

/* The 64 terms of one block for vectors b and b+1 (x: the pair's values). */
__device__ __forceinline__ void fma_pair(float& S0, float& S1, const float4 x, const float (&q)[32])
{
    const float x0 = x.x, x1 = x.y, x2 = x.z, x3 = x.w;
    {
        const float q0 = q[0], q1 = q[1], q2 = q[2], q3 = q[3];
        const float q4 = q[4], q5 = q[5], q6 = q[6], q7 = q[7];
        G4S_FMAC_BCAST("0", "8", "1", "9");
    }
    {
        const float q0 = q[8], q1 = q[9], q2 = q[10], q3 = q[11];
        const float q4 = q[12], q5 = q[13], q6 = q[14], q7 = q[15];
        G4S_FMAC_BCAST("2", "10", "3", "11");
    }
    {
        const float q0 = q[16], q1 = q[17], q2 = q[18], q3 = q[19];
        const float q4 = q[20], q5 = q[21], q6 = q[22], q7 = q[23];
        G4S_FMAC_BCAST("4", "12", "5", "13");
    }
    {
        const float q0 = q[24], q1 = q[25], q2 = q[26], q3 = q[27];
        const float q4 = q[28], q5 = q[29], q6 = q[30], q7 = q[31];
        G4S_FMAC_BCAST("6", "14", "7", "15");
    }
}
#undef G4S_FMAC_BCAST

__global__ __launch_bounds__(64 * kTileWaves) void lmhead_tiled_kernel(
    const uint8_t* __restrict__ tiles, int32_t rows, int32_t nblk, const float* __restrict__ h,
    int32_t cols, int32_t batch, float* __restrict__ out, int64_t stride, uint64_t* __restrict__ gsum,
    int32_t ngroups)
{
    const int lane = threadIdx.x & 63;
    const int32_t g = __builtin_amdgcn_readfirstlane(blockIdx.x * kTileWaves + (threadIdx.x >> 6));
    if (g >= ngroups) return; /* whole waves: no barrier below */
    const int32_t r = g * kQ4TileRows + lane;
    const float* tsc = reinterpret_cast<const float*>(tiles + (int64_t)g * nblk * kQ4TileBytes);
    const uint4* tq = reinterpret_cast<const uint4*>(tiles + (int64_t)g * nblk * kQ4TileBytes +
                                                     kQ4TileRows * 4);
    const uint32_t ul = (uint32_t)lane;
    constexpr int kTileF = kQ4TileBytes / 4;  /* floats per tile */
    constexpr int kTileQ = kQ4TileBytes / 16; /* uint4 per tile */
    /* lane's share of a pair load: vector 2p + (n >> 3), columns 4 (n & 7) .. +3 */
    const int n = lane & 15;
    const int32_t xlane = (n >> 3) * cols + 4 * (n & 7);
    for (int32_t b0 = 0; b0 < batch; b0 += kTileB) {
        /* offset of pair p's load: vectors past the batch read vector batch-1
         * (any valid row; their sums are discarded) */
        /* 32-bit byte offsets from the uniform base (the hidden matrix is
         * below 2 GiB: checked by the launcher) */
        const auto xload = [&](int p, int32_t k) -> float4 {
            const int32_t ub = b0 + 2 * p;
            const int32_t o = ub + 1 < batch ? ub * cols + xlane : (batch - 1) * cols + 4 * (n & 7);
            const uint32_t byte = (uint32_t)(o + 32 * k) * 4u;
            return *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(h) + byte);
        };
        float S[kTileB];
#pragma unroll
        for (int b = 0; b < kTileB; ++b) S[b] = 0.0f;
        /* the first block's weights and vector pairs */
        float sc = tsc[ul];
        uint4 w = tq[ul];
        float4 xr[kXAhead];
#pragma unroll
        for (int p = 0; p < kXAhead; ++p) xr[p] = xload(p, 0);
        for (int32_t k = 0; k < nblk; ++k) {
            float q[32];
            q4_dequant32(w, sc, q);
            const int32_t kn = k + 1 < nblk ? k + 1 : k;
            sc = tsc[(uint32_t)(kn * kTileF) + ul];
            w = tq[(uint32_t)(kn * kTileQ) + ul];
            /* the scheduler keeps each load where it is issued: kXAhead pairs
             * before its use, after the block's weight loads */
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int p = 0; p < kTileB / 2; ++p) {
                const float4 x = xr[p % kXAhead];
                /* the pair kXAhead ahead (wrapping into the next block) */
                const int pa = p + kXAhead;
                const int32_t ka = pa < kTileB / 2 ? k : kn;
                xr[p % kXAhead] = xload(pa % (kTileB / 2), ka);
                __builtin_amdgcn_sched_barrier(0);
                fma_pair(S[2 * p], S[2 * p + 1], x, q);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        const bool live = r < rows;
#pragma unroll
        for (int b = 0; b < kTileB; ++b) {
            if (b0 + b < batch) {
                if (out && live) out[(int64_t)(b0 + b) * stride + r] = S[b];
                if (gsum) {
                    /* the group's summary: its largest key, the lowest row
                     * holding it, and the largest key of the other rows */
                    const uint32_t key = live ? cand_key(S[b]) : 0u;
                    const uint32_t kmax = wave_max_u32(key);
                    const uint32_t r6 = (uint32_t)__builtin_ctzll(__ballot(key == kmax));
                    const uint32_t k2 = wave_max_u32(ul == r6 ? 0u : key);
                    if (lane == 0) gsum[(int64_t)(b0 + b) * ngroups + g] = gsum_pack(kmax, r6, k2);
                }
            }
        }
    }
}

/* DoEmbeddingLookup for a Q4_0 table (src/Gemma4.Model.pas:2047-2080):
 * row `token` dequantised as DequantQ4Block does (Single(q) * LScale,
 * src/Gemma4.Quant.pas:209-239; exact) and multiplied by `scale`
 * (CpuScaleF32, src/Gemma4.Tensors.pas:626-636; one rounding).  One thread
 * per weight; tokens outside [0, rows) give a zero vector. */
__global__ __launch_bounds__(256) void embed_q4_kernel(const uint8_t* __restrict__ w, int32_t rows,
                                                       int32_t nblk, const int32_t* __restrict__ tokens,
                                                       int32_t batch, float scale,
                                                       float* __restrict__ out)
{
    const int32_t cols = nblk * 32;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)batch * cols) return;
    const int32_t b = (int32_t)(i / cols), c = (int32_t)(i % cols);
    const int32_t t = tokens[b];
    float v = 0.0f;
    if (t >= 0 && t < rows) {
        const uint8_t* blk = w + ((int64_t)t * nblk + c / 32) * 18;
        const float sc = f16_to_f32_ref((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        const uint32_t byte = blk[2 + (c % 32) / 2];
        const int q = (int)((c & 1) ? (byte >> 4) : (byte & 0x0Fu)) - 8;
        v = ((float)q * sc) * scale;
    }
    out[i] = v;
}

}  // namespace

hipError_t embed_q4_0_launch(const uint8_t* w, int32_t rows, int32_t cols, const int32_t* tokens,
                             int32_t batch, float scale, float* hidden, hipStream_t s)
{
    const int64_t n = (int64_t)batch * cols;
    hipLaunchKernelGGL(embed_q4_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, w, rows,
                       cols / 32, tokens, batch, scale, hidden);
    return hipGetLastError();
}

hipError_t q4_tile_launch(const uint8_t* src, int32_t rows, int32_t nblk, uint8_t* dst, hipStream_t s)
{
    const int64_t total = (int64_t)((rows + kQ4TileRows - 1) / kQ4TileRows) * kQ4TileRows * nblk;
    const int64_t want = (total + 255) / 256;
    const unsigned grid = (unsigned)(want < 65536 ? want : 65536);
    hipLaunchKernelGGL(q4_tile_kernel, dim3(grid), dim3(256), 0, s, src, rows, nblk, dst);
    return hipGetLastError();
}

hipError_t lmhead_tiled_launch(const uint8_t* tiles, int32_t rows, int32_t cols, const float* h,
                               int32_t batch, float* logits, int64_t stride, uint64_t* gsum,
                               hipStream_t s)
{
    const int32_t ngroups = (rows + kQ4TileRows - 1) / kQ4TileRows;
    const unsigned grid = (unsigned)((ngroups + kTileWaves - 1) / kTileWaves);
    hipLaunchKernelGGL(lmhead_tiled_kernel, dim3(grid), dim3(64 * kTileWaves), 0, s, tiles, rows,
                       cols / 32, h, cols, batch, logits, stride, gsum, ngroups);
    return hipGetLastError();
}

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
