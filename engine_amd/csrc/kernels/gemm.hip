// Prefill GEMM on the matrix cores: Y[T, n] = X[T, K] . W[n, K]^T, X fp16, W
// int4 (groups of 32, fp16 scales) or int8 (fp16 row scales) in the fused
// step's tiled layout, fp32 accumulation, with the chunk pass's epilogues:
// store (+ bias: the QKV sums), add into Y (the residual after o and down),
// or, for the paired gate/up matrix, fp16 SiLU(gate) * up.
//
// Reference: GemmXWtKernel (backends/cuda/qwen_cuda_model.cu:878-908), the
// prefill GEMM of ForwardChunk (:2398-2516): C = X.W^T + b over a chunk of
// prompt rows, in FP32 SIMT tiles there; the CPU path is one MatVec per row
// (model/architectures/qwen/qwen_model.cpp:21-31).
//
// A workgroup (4 waves) computes a 128 x 128 tile of Y, each wave a 64 x 64
// quarter as 4 x 4 accumulators of 16 x 16. Per step of 32 k the workgroup
// stages in LDS the X tile (fp16) and the W tile's codes as fp16 (exact: the
// integers -8..7 or -128..127; the next step's global words are fetched into
// registers while this step's MFMAs run), then each wave runs 16
// v_mfma_f32_16x16x32_f16 from LDS operands:
//   A: lane l holds X[row l % 16][8 (l / 16) .. +7];
//   B: lane l holds W[column l % 16][8 (l / 16) .. +7].
// A step's 32 k are one int4 group, so its products land in fresh
// accumulators and join the sums through one fma with the group's scale;
// int8's row scale multiplies the finished sum. Every product is exact, as
// in the decode GEMV: the result differs from the dequantized fp32 product
// by the order of the fp32 additions only.
#include "common.h"

namespace lyk {
namespace {

constexpr int kGemmThreads = 256;


constexpr int kTile = 128;      // rows and columns of Y per workgroup
constexpr int kRowHalves = 40;  // LDS row of a 32-k slice (fp16), padded against bank conflicts

__device__ __forceinline__ uint32_t lane_of(int r, int unit, int tr, int& blk) {
    const int per = 64 / tr;   // units a block holds per row
    blk = unit / per;
    return (uint32_t)((unit % per) * tr + r);
}

// Epilogues (the LYK_GEMM_* values of the C ABI).
constexpr int kStore = 0, kAdd = 1, kSiluPairs = 2;

// ncols: columns of the tiled matrix (rows of W; paired: tiles * tr, the
// gate and up halves of each tile); n: valid columns (paired: gate rows).
template <bool Q8, int EP>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(const uint16_t* __restrict__ x, int ldx, int T, int K,
                                                           const uint8_t* __restrict__ qw,
                                                           const uint16_t* __restrict__ qs, int n, int ncols, int tr,
                                                           int nbp, int nc, const float* __restrict__ bias,
                                                           void* __restrict__ yv, int ldy) {
    __shared__ __align__(16) uint16_t xs[kTile * kRowHalves];
    __shared__ __align__(16) uint16_t ws[kTile * kRowHalves];
    __shared__ float gsc[kTile];   // int4: this step's group scale per column
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int quad = lane >> 4, col = lane & 15;
    const int t0 = blockIdx.y * kTile, n0 = blockIdx.x * kTile;
    const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;   // this wave's quarter
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // staging roles: X row tid / 2, 16 k from 16 (tid & 1); W column tid / 2,
    // 8 k slices 2 (tid & 1) and 2 (tid & 1) + 1
    const int xr = tid >> 1, xh = tid & 1;
    const int wcol = tid >> 1, wd = 2 * (tid & 1);
    const int cn = n0 + wcol;
    const int wt = cn / tr, wrr = cn % tr;
    const half2_t lo_off = {(half_t)-1032.0f, (half_t)-1032.0f};
    const half2_t hi_off = {(half_t)-1152.0f, (half_t)-1152.0f};
    const half2_t sixteenth = {(half_t)0.0625f, (half_t)0.0625f};
    const int steps = (K + 31) / 32;
    // step g's global words, fetched one step ahead so the loads fly while
    // the previous step's MFMAs run: X row slice, W words and scale
    u32x4 xv0, xv1;
    uint32_t wv[2][2];
    uint16_t wsc = 0;
    auto fetch = [&](int g) {
        const int t = t0 + xr, k0 = 32 * g + 16 * xh;
        xv0 = u32x4{0u, 0u, 0u, 0u};
        xv1 = u32x4{0u, 0u, 0u, 0u};
        if (t < T) {
            const uint16_t* p = x + (size_t)t * ldx + k0;
            if (k0 + 16 <= K) {
                xv0 = ld(reinterpret_cast<const u32x4*>(p));
                xv1 = ld(reinterpret_cast<const u32x4*>(p + 8));
            } else {
                uint32_t e[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
                for (int q = 0; q < 16; ++q)
                    if (k0 + q < K) e[q / 2] |= (uint32_t)ld(p + q) << (16 * (q & 1));
                xv0 = u32x4{e[0], e[1], e[2], e[3]};
                xv1 = u32x4{e[4], e[5], e[6], e[7]};
            }
        }
        wsc = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int dd = wd + h;   // 8-k slice of the step
            wv[h][0] = wv[h][1] = 0u;
            if (cn >= ncols) continue;
            if constexpr (!Q8) {
                int blk;
                const uint32_t l = lane_of(wrr, g, tr, blk);
                wv[h][0] = ld(reinterpret_cast<const uint32_t*>(qw + (((size_t)wt * nbp + blk) * 64 + l) * 16 + 4 * dd));
                if (h == 0) wsc = ld(qs + (((size_t)wt * nc + blk / 4) * 64 + l) * 4 + blk % 4);
            } else {
                // 16-code units: slice dd is half (dd & 1) of unit 2g + dd / 2
                int blk;
                const uint32_t l = lane_of(wrr, 2 * g + dd / 2, tr, blk);
                const uint8_t* p = qw + (((size_t)wt * nbp + blk) * 64 + l) * 16 + 8 * (dd & 1);
                wv[h][0] = ld(reinterpret_cast<const uint32_t*>(p));
                wv[h][1] = ld(reinterpret_cast<const uint32_t*>(p + 4));
            }
        }
    };
    // the fetched words into LDS: X as is, W codes as fp16 integers
    auto stage = [&]() {
        u32x4* d = reinterpret_cast<u32x4*>(xs + xr * kRowHalves + 16 * xh);
        d[0] = xv0;
        d[1] = xv1;
        if constexpr (!Q8)
            if (wd == 0) gsc[wcol] = h2f(wsc);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int dd = wd + h;
            u32x4 v;
            if constexpr (!Q8) {
                const uint32_t u = wv[h][0], tt = u >> 8, magic = 0x64006400u;
                // nibbles of k 8dd+{0,1} | {2,3} (x16, then /16: exact) | {4,5} | {6,7}
                const half2_t p0 = as_half2((u & 0x000F000Fu) | magic) + lo_off;
                const half2_t p1 = (as_half2((u & 0x00F000F0u) | magic) + hi_off) * sixteenth;
                const half2_t p2 = as_half2((tt & 0x000F000Fu) | magic) + lo_off;
                const half2_t p3 = (as_half2((tt & 0x00F000F0u) | magic) + hi_off) * sixteenth;
                v = u32x4{as_u32(p0), as_u32(p1), as_u32(p2), as_u32(p3)};
            } else {
                uint32_t e[4];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    e[2 * q] = as_u32(as_half2(__builtin_amdgcn_perm(0x64646464u, wv[h][q], 0x04010400u)) + hi_off);
                    e[2 * q + 1] = as_u32(as_half2(__builtin_amdgcn_perm(0x64646464u, wv[h][q], 0x04030402u)) + hi_off);
                }
                v = u32x4{e[0], e[1], e[2], e[3]};
            }
            if (cn >= ncols) v = u32x4{0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x4*>(ws + wcol * kRowHalves + 8 * dd) = v;
        }
    };
    fetch(0);
    for (int g = 0; g < steps; ++g) {
        stage();
        __syncthreads();
        if (g + 1 < steps) fetch(g + 1);
        // ---- 16 MFMAs from LDS
        f16x8 a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            a[i] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(xs + (wr + 16 * i + col) * kRowHalves + 8 * quad));
#pragma unroll
        for (int j = 0; j < 4; ++j)
            b[j] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(ws + (wc + 16 * j + col) * kRowHalves + 8 * quad));
        if constexpr (Q8) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        } else {
            // the group's sums, scaled into the running ones
            float sg[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) sg[j] = gsc[wc + 16 * j + col];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], f32x4{0.0f, 0.0f, 0.0f, 0.0f},
                                                                           0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][e] = fmaf(p[e], sg[j], acc[i][j][e]);
                }
        }
        __syncthreads();   // the tiles are restaged by the next step
    }
    // D lane l: rows 4 quad + e of the subtile, column l % 16
    if constexpr (EP == kSiluPairs) {
        // tile column r < tr/2 is gate row (c / tr) * tr/2 + r, its up row
        // tr/2 columns on: the next subtile(s) for tr >= 32, 8 lanes on for
        // tr = 16
        uint16_t* act = static_cast<uint16_t*>(yv);
        const int half = tr / 2;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = n0 + wc + 16 * j + col;
            const int r = c % tr, row = c / tr * half + r;
            // int8: the gate and up rows' scales (the sums are of codes)
            float sg = 1.0f, su = 1.0f;
            if constexpr (Q8)
                if (r < half && c < ncols) {
                    sg = h2f(ld(qs + (size_t)(c / tr) * 64 + r));
                    su = h2f(ld(qs + (size_t)(c / tr) * 64 + r + half));
                }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float up;
                    if (tr == 16) {
                        up = __shfl_down(acc[i][j][e], 8, 16);
                    } else {
                        up = 0.0f;
#pragma unroll
                        for (int jj = 0; jj < 4; ++jj)
                            if (jj == j + half / 16) up = acc[i][jj][e];
                    }
                    const float gt = acc[i][j][e] * sg;
                    up *= su;
                    const int t = t0 + wr + 16 * i + 4 * quad + e;
                    if (r < half && row < n && t < T) act[(size_t)t * ldy + row] = f2h(gt / (1.0f + expf(-gt)) * up);
                }
        }
    } else {
        float* y = static_cast<float*>(yv);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = n0 + wc + 16 * j + col;
            if (c >= n) continue;
            float s = 1.0f;
            if constexpr (Q8) s = h2f(ld(qs + (size_t)(c / tr) * 64 + c % tr));
            const float bb = EP == kStore && bias ? ld(bias + c) : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = t0 + wr + 16 * i + 4 * quad + e;
                    if (t >= T) continue;
                    const float v = Q8 ? acc[i][j][e] * s : acc[i][j][e];
                    float* dst = y + (size_t)t * ldy + c;
                    if constexpr (EP == kAdd) *dst = *dst + v;
                    else *dst = v + bb;
                }
        }
    }
}

template <bool Q8>
void launch_gemm(int ep, dim3 grid, hipStream_t st, const uint16_t* x, int ldx, int T, int K, const uint8_t* qw,
                 const uint16_t* qs, int n, int ncols, int tr, int nbp, int nc, const float* bias, void* y, int ldy) {
    auto k = ep == kAdd ? gemm_kernel<Q8, kAdd> : ep == kSiluPairs ? gemm_kernel<Q8, kSiluPairs> : gemm_kernel<Q8, kStore>;
    hipLaunchKernelGGL(k, grid, dim3(kGemmThreads), 0, st, x, ldx, T, K, qw, qs, n, ncols, tr, nbp, nc, bias, y, ldy);
}

}  // namespace
}  // namespace lyk

using namespace lyk;

extern "C" {

int lyk_hip_gemm_q(const uint16_t* d_x, int64_t ldx, int64_t T, int64_t K, const void* d_qw, const void* d_qs,
                   int64_t n, int tile_rows, int q8, int epilogue, const float* d_bias, void* d_y, int64_t ldy,
                   void* stream) {
    if (!d_x || !d_qw || !d_qs || !d_y || T < 1 || K < 1 || n < 1 || ldx < K || ldy < n) return LYK_ERR_INVALID_ARG;
    if (tile_rows != 16 && tile_rows != 32 && tile_rows != 64) return LYK_ERR_INVALID_ARG;
    if (epilogue != LYK_GEMM_STORE && epilogue != LYK_GEMM_ADD && epilogue != LYK_GEMM_SILU_PAIRS)
        return LYK_ERR_INVALID_ARG;
    if (T > (1 << 24) || n > (1 << 24) || K > (1 << 24) || ldx % 8) return LYK_ERR_SHAPE;
    // the tiled layout's block and chunk counts per tile (lyk_q*_pack_tiled)
    const bool paired = epilogue == LYK_GEMM_SILU_PAIRS;
    const int64_t unit = q8 ? 16 : 32, per = 64 / tile_rows;
    const int64_t units = (K + unit - 1) / unit;
    const int64_t nb = (units + per - 1) / per, nc = (nb + 3) / 4, nbp = 4 * nc;
    const int64_t tiles = paired ? (n + tile_rows / 2 - 1) / (tile_rows / 2) : (n + tile_rows - 1) / tile_rows;
    const int64_t ncols = paired ? tiles * tile_rows : n;
    dim3 grid((unsigned)((ncols + kTile - 1) / kTile), (unsigned)((T + kTile - 1) / kTile));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (q8)
        launch_gemm<true>(epilogue, grid, st, d_x, (int)ldx, (int)T, (int)K, static_cast<const uint8_t*>(d_qw),
                          static_cast<const uint16_t*>(d_qs), (int)n, (int)ncols, tile_rows, (int)nbp, (int)nc,
                          d_bias, d_y, (int)ldy);
    else
        launch_gemm<false>(epilogue, grid, st, d_x, (int)ldx, (int)T, (int)K, static_cast<const uint8_t*>(d_qw),
                           static_cast<const uint16_t*>(d_qs), (int)n, (int)ncols, tile_rows, (int)nbp, (int)nc,
                           d_bias, d_y, (int)ldy);
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

}  // extern "C"
