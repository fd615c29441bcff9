// Prefill GEMM on the matrix cores: Y[T, n] = X[T, K] . W[n, K]^T (+ bias),
// X fp16, W int4 (groups of 32, fp16 scales) or int8 (fp16 row scales) in the
// fused step's tiled layout, dequantized on the fly, fp32 accumulation.
//
// Reference: GemmXWtKernel (backends/cuda/qwen_cuda_model.cu:878-908), the
// prefill GEMM of ForwardChunk (:2398-2516): C = X.W^T + b over a chunk of
// prompt rows, in FP32 SIMT tiles there; the CPU path is one MatVec per row
// (model/architectures/qwen/qwen_model.cpp:21-31).
//
// A workgroup (4 waves) computes a 64 x 64 tile of Y: wave w the rows
// 16w..16w+15, four 16 x 16 accumulators across the 64 columns. Each step of
// 32 k is one v_mfma_f32_16x16x32_f16 per accumulator:
//   A: lane l holds X[row l % 16][8 (l / 16) .. +7] (one 16-byte load);
//   B: lane l holds W[column l % 16][8 (l / 16) .. +7] as exact small
//      integers q in fp16 (int4: a code's nibble through a magic-number OR;
//      int8: its byte through v_perm), read straight from the tiled layout.
// The scales stay out of the matrix product, so it is exact in its inputs:
// int4 multiplies each group's product by the column's group scale (every
// 32-k step is one group), int8 the finished sum by the row scale.
#include "common.h"

namespace lyk {
namespace {

constexpr int kGemmThreads = 256;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t lane_of(int r, int unit, int tr, int& blk) {
    const int per = 64 / tr;   // units a block holds per row
    blk = unit / per;
    return (uint32_t)((unit % per) * tr + r);
}

template <bool Q8>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(const uint16_t* __restrict__ x, int ldx, int T, int K,
                                                           const uint8_t* __restrict__ qw,
                                                           const uint16_t* __restrict__ qs, int n, int tr, int nbp,
                                                           int nc, const float* __restrict__ bias,
                                                           float* __restrict__ y, int ldy) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int quad = lane >> 4, col = lane & 15;
    const int t0 = blockIdx.y * 64 + wave * 16, n0 = blockIdx.x * 64;
    const int trow = t0 + col;   // this lane's A row
    f32x4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // this lane's B column in each accumulator: tile, row in tile
    int tt[4], rr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = n0 + 16 * j + col;
        tt[j] = c / tr;
        rr[j] = c % tr;
    }
    const int steps = (K + 31) / 32;
    for (int g = 0; g < steps; ++g) {
        // A: X[trow][32g + 8 quad .. +7], zero past T and K
        const int k0 = 32 * g + 8 * quad;
        uint32_t av[4] = {0u, 0u, 0u, 0u};
        if (trow < T) {
            const uint16_t* xr = x + (size_t)trow * ldx;
            if (k0 + 8 <= K) {
                const u32x4 v = ld(reinterpret_cast<const u32x4*>(xr + k0));
                av[0] = v.x;
                av[1] = v.y;
                av[2] = v.z;
                av[3] = v.w;
            } else {
                for (int e = 0; e < 8; ++e)
                    if (k0 + e < K) av[e / 2] |= (uint32_t)ld(xr + k0 + e) << (16 * (e & 1));
            }
        }
        const f16x8 a = __builtin_bit_cast(f16x8, u32x4{av[0], av[1], av[2], av[3]});
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = n0 + 16 * j + col;
            uint32_t bv[4] = {0u, 0u, 0u, 0u};
            float s = 0.0f;
            if (c < n) {
                if constexpr (!Q8) {
                    // unit = group g; the lane's u32 `quad` of it: k 8 quad .. +7
                    int blk;
                    const uint32_t l = lane_of(rr[j], g, tr, blk);
                    const uint32_t u = ld(reinterpret_cast<const uint32_t*>(
                        qw + (((size_t)tt[j] * nbp + blk) * 64 + l) * 16 + 4 * quad));
                    const uint32_t t = u >> 8, magic = 0x64006400u;
                    // nibbles of k 8q+{0,1} | {2,3} (x16) | {4,5} | {6,7} (x16)
                    const half2_t lo_off = {(half_t)-1032.0f, (half_t)-1032.0f};
                    const half2_t hi_off = {(half_t)-1152.0f, (half_t)-1152.0f};
                    const half2_t sixteenth = {(half_t)0.0625f, (half_t)0.0625f};
                    const half2_t p0 = as_half2((u & 0x000F000Fu) | magic) + lo_off;
                    const half2_t p1 = (as_half2((u & 0x00F000F0u) | magic) + hi_off) * sixteenth;
                    const half2_t p2 = as_half2((t & 0x000F000Fu) | magic) + lo_off;
                    const half2_t p3 = (as_half2((t & 0x00F000F0u) | magic) + hi_off) * sixteenth;
                    bv[0] = __builtin_bit_cast(uint32_t, p0);
                    bv[1] = __builtin_bit_cast(uint32_t, p1);
                    bv[2] = __builtin_bit_cast(uint32_t, p2);
                    bv[3] = __builtin_bit_cast(uint32_t, p3);
                    s = h2f(ld(qs + (((size_t)tt[j] * nc + blk / 4) * 64 + l) * 4 + blk % 4));
                } else {
                    // units of 16 codes: k 8 quad .. +7 is half (quad & 1) of unit 2g + quad / 2
                    int blk;
                    const uint32_t l = lane_of(rr[j], 2 * g + quad / 2, tr, blk);
                    const uint8_t* p = qw + (((size_t)tt[j] * nbp + blk) * 64 + l) * 16 + 8 * (quad & 1);
                    const uint32_t w0 = ld(reinterpret_cast<const uint32_t*>(p));
                    const uint32_t w1 = ld(reinterpret_cast<const uint32_t*>(p + 4));
                    const half2_t off = {(half_t)-1152.0f, (half_t)-1152.0f};
                    const uint32_t ws[2] = {w0, w1};
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const half2_t e0 = as_half2(__builtin_amdgcn_perm(0x64646464u, ws[h], 0x04010400u)) + off;
                        const half2_t e1 = as_half2(__builtin_amdgcn_perm(0x64646464u, ws[h], 0x04030402u)) + off;
                        bv[2 * h] = __builtin_bit_cast(uint32_t, e0);
                        bv[2 * h + 1] = __builtin_bit_cast(uint32_t, e1);
                    }
                }
            }
            const f16x8 b = __builtin_bit_cast(f16x8, u32x4{bv[0], bv[1], bv[2], bv[3]});
            const f32x4 part = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            if constexpr (!Q8) {
                // D lane l: rows 4 quad + i, column l % 16 -- this lane's B column
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[j][i] = fmaf(part[i], s, acc[j][i]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[j][i] += part[i];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = n0 + 16 * j + col;
        if (c >= n) continue;
        float s = 1.0f;
        if constexpr (Q8) s = h2f(ld(qs + (size_t)tt[j] * 64 + rr[j]));
        const float bb = bias ? ld(bias + c) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = t0 + 4 * quad + i;
            if (t < T) y[(size_t)t * ldy + c] = acc[j][i] * s + bb;
        }
    }
}

}  // namespace
}  // namespace lyk

using namespace lyk;

extern "C" {

int lyk_hip_gemm_q(const uint16_t* d_x, int64_t ldx, int64_t T, int64_t K, const void* d_qw, const void* d_qs,
                   int64_t n, int tile_rows, int q8, const float* d_bias, float* d_y, int64_t ldy, void* stream) {
    if (!d_x || !d_qw || !d_qs || !d_y || T < 1 || K < 1 || n < 1 || ldx < K || ldy < n) return LYK_ERR_INVALID_ARG;
    if (tile_rows != 16 && tile_rows != 32 && tile_rows != 64) return LYK_ERR_INVALID_ARG;
    if (T > (1 << 24) || n > (1 << 24) || K > (1 << 24) || ldx % 8) return LYK_ERR_SHAPE;
    // the tiled layout's block and chunk counts per tile (lyk_q*_pack_tiled)
    const int64_t unit = q8 ? 16 : 32, per = 64 / tile_rows;
    const int64_t units = (K + unit - 1) / unit;
    const int64_t nb = (units + per - 1) / per, nc = (nb + 3) / 4, nbp = 4 * nc;
    dim3 grid((unsigned)((n + 63) / 64), (unsigned)((T + 63) / 64));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (q8)
        hipLaunchKernelGGL(gemm_kernel<true>, grid, dim3(kGemmThreads), 0, st, d_x, (int)ldx, (int)T, (int)K,
                           static_cast<const uint8_t*>(d_qw), static_cast<const uint16_t*>(d_qs), (int)n,
                           tile_rows, (int)nbp, (int)nc, d_bias, d_y, (int)ldy);
    else
        hipLaunchKernelGGL(gemm_kernel<false>, grid, dim3(kGemmThreads), 0, st, d_x, (int)ldx, (int)T, (int)K,
                           static_cast<const uint8_t*>(d_qw), static_cast<const uint16_t*>(d_qs), (int)n,
                           tile_rows, (int)nbp, (int)nc, d_bias, d_y, (int)ldy);
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

}  // extern "C"
