// Weight-only dequant-GEMV for the decode path (int4 group-32 and int8
// per-row), gfx950.
//
// Replaces the reference's MatVecEpi1Kernel / FusedQkv1Kernel /
// FusedGateUp1Kernel / MatVecBatchKernel / MatVecEpilogueKernel
// (backends/cuda/qwen_cuda_model.cu:533-578, 615-819, 1268-1378), whose CPU
// counterpart is MatVec (model/architectures/qwen/qwen_model.cpp:21-31).
//
// Design (one row per lane):
//   * A wave owns a tile of 64 weight rows; lane r computes row 64t+r, so the
//     activation vector is the same for every lane and is read with scalar
//     loads into SGPRs; no cross-lane reduction is needed for the dot product.
//   * Each lane streams 16 bytes per load (one int4 group of 32 weights, or
//     16 int8 weights); the packed layout puts the 64 lanes' 16-byte pieces
//     side by side, so every wave-wide load is one contiguous 1 KiB.
//   * int4 codes become fp16 pairs with one AND/OR against the exponent of
//     1024 and one packed subtract; v_dot2_f32_f16 multiplies them with fp16
//     activation pairs exactly and accumulates in fp32. Each group's sum is
//     scaled by its fp16 scale once.
//   * The K range of a tile is split over the waves of a workgroup and, when
//     there are few tiles, over several workgroups. Waves combine through
//     LDS; workgroups write partial sums to the workspace and the last one to
//     finish (per-tile arrival counter) adds them in split order, so results
//     do not depend on timing.
#include "common.h"

namespace lyk {
namespace {

constexpr int kMaxWaves = 4;
constexpr int kMaxM = 4;

struct Plan {
    int tiles, chunks, waves, splits, cps;  // cps: chunks per split
};

Plan make_plan(int64_t n, int64_t k, int paired, int q8, int ksplit) {
    Plan p;
    p.tiles = paired ? ceil_div(n, 32) : ceil_div(n, 64);
    const int64_t units = q8 ? ceil_div(k, 16) : ceil_div(k, 32);
    p.chunks = ceil_div(units, 8);
    // default: aim for ~4096 waves, at most 16 sharing one tile's K range
    int wpt = ksplit > 0 ? ksplit : ceil_div(4096, p.tiles);
    if (ksplit <= 0 && wpt > 16) wpt = 16;
    if (wpt > p.chunks) wpt = p.chunks;
    if (wpt < 1) wpt = 1;
    p.waves = wpt < kMaxWaves ? wpt : kMaxWaves;
    p.splits = ceil_div(wpt, p.waves);
    p.cps = ceil_div(p.chunks, p.splits);
    p.splits = ceil_div(p.chunks, p.cps);
    if (p.waves > p.cps) p.waves = p.cps;
    return p;
}

uint64_t workspace_for(const Plan& p, int m) {
    if (p.splits <= 1) return 0;
    const uint64_t counters = (uint64_t(p.tiles) * 4 + 255) / 256 * 256;
    return counters + uint64_t(p.splits) * m * p.tiles * 64 * 4;
}

// ---------------------------------------------------------------- epilogue

template <int M, int EPI>
__device__ __forceinline__ void epilogue(const float (&v)[M], int tile, int lane,
                                         int n, void* y, int ldy,
                                         const float* bias) {
    if constexpr (EPI == LYK_EPI_SILU_F16) {
        // paired tile: lanes 0-31 hold gate rows, lanes 32-63 the up rows
        const int j = tile * 32 + lane;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float u = __shfl_down(v[m], 32, 64);
            if (lane < 32 && j < n) {
                const float g = v[m];
                const float a = g / (1.0f + expf(-g)) * u;
                static_cast<uint16_t*>(y)[(size_t)m * ldy + j] = f2h(a);
            }
        }
    } else {
        const int r = tile * 64 + lane;
        if (r >= n) return;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float val = v[m];
            if constexpr (EPI == LYK_EPI_ADD) {
                static_cast<float*>(y)[(size_t)m * ldy + r] += val;
            } else {
                if (bias) val += bias[r];
                if constexpr (EPI == LYK_EPI_STORE_F16)
                    static_cast<uint16_t*>(y)[(size_t)m * ldy + r] = f2h(val);
                else
                    static_cast<float*>(y)[(size_t)m * ldy + r] = val;
            }
        }
    }
}

// Combines the per-wave sums of a workgroup and, across split workgroups,
// the per-split partials; then runs the epilogue (wave 0 only).
template <int M, int EPI>
__device__ __forceinline__ void finish(float (&acc)[M], int tile, int split,
                                       int splits, int n, void* y, int ldy,
                                       const float* bias, float* partial,
                                       unsigned* counters, int tiles) {
    __shared__ float red[kMaxWaves][M][64];
    const int lane = threadIdx.x & 63;
    const int wave = uniform(threadIdx.x >> 6);
    const int waves = uniform(blockDim.x >> 6);
#pragma unroll
    for (int m = 0; m < M; ++m) red[wave][m][lane] = acc[m];
    __syncthreads();
    if (wave != 0) return;
    float v[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float s = red[0][m][lane];
        for (int w = 1; w < waves; ++w) s += red[w][m][lane];
        v[m] = s;
    }
    if (splits > 1) {
        // Split-K across workgroups: partials are agent-scope (sc1) atomic
        // stores, coherent across the XCDs' L2s; they are published before
        // the arrival is counted, and the last arrival adds them in split
        // order, then zeroes them and the counter.
        const size_t npad = (size_t)tiles * 64;
#pragma unroll
        for (int m = 0; m < M; ++m)
            store_sc1(&partial[((size_t)split * M + m) * npad + tile * 64 + lane], v[m]);
        if (!arrive_last(&counters[tile], (unsigned)splits)) return;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float s = 0.0f;
            for (int sp = 0; sp < splits; ++sp) {
                float* p = &partial[((size_t)sp * M + m) * npad + tile * 64 + lane];
                s += load_sc1(p);
                *p = 0.0f;  // the workspace is all zero again after every launch
            }
            v[m] = s;
        }
        if (lane == 0) counters[tile] = 0u;
    }
    epilogue<M, EPI>(v, tile, lane, n, y, ldy, bias);
}

// ------------------------------------------------------------- int4 kernel

template <int M, int EPI>
__global__ __launch_bounds__(256) void gemv_q4_kernel(
    const u32x4* __restrict__ qw, const u32x4* __restrict__ qs,
    const uint16_t* __restrict__ x, int ldx, int groups, int chunks, int cps,
    int n, void* __restrict__ y, int ldy, const float* __restrict__ bias,
    float* __restrict__ partial, unsigned* __restrict__ counters, int splits,
    int tiles, uint32_t mask_lo, uint32_t mask_hi, uint32_t magic) {
    const int tile = blockIdx.x;
    const int split = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = uniform(threadIdx.x >> 6);
    const int waves = uniform(blockDim.x >> 6);
    const int c0 = split * cps;
    const int c1 = min(chunks, c0 + cps);
    const u32x4* wt = qw + (size_t)tile * chunks * 8 * 64 + lane;
    const u32x4* st = qs + (size_t)tile * chunks * 64 + lane;
    const half2_t off_a = {(half_t)-1032.0f, (half_t)-1032.0f};
    const half2_t off_b = {(half_t)-1152.0f, (half_t)-1152.0f};

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;

    // magic lives in a VGPR so that mask-and-or is one v_and_or_b32 (a VOP3
    // instruction may read only one SGPR on gfx9).
    uint32_t vmagic;
    asm("v_mov_b32 %0, %1" : "=v"(vmagic) : "s"(magic));

    // Loads are issued in the order their data is used (weights of groups
    // 0..7, then the scales): vmcnt waits retire in issue order.
    auto load = [&](int c, u32x4 (&w)[8], u32x4& s4) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            w[j] = __builtin_nontemporal_load(wt + ((size_t)c * 8 + j) * 64);
            __builtin_amdgcn_sched_barrier(0);
        }
        s4 = st[(size_t)c * 64];
        __builtin_amdgcn_sched_barrier(0);
    };
    auto compute = [&](int c, const u32x4 (&w)[8], const u32x4& s4) {
        // Group sums first, scales last: the scale vector is the chunk's
        // last-needed operand, so waiting for it never stalls a group.
        float gs[M][8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // Groups past the end of K are packed with scale 0 and code 0;
            // they read the last real group's activations (finite) and add 0.
            const int g = min(c * 8 + j, groups - 1);
            const uint32_t u4[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
            half2_t qa[8], qb[8];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t u = u4[d], t = u >> 8;
                qa[2 * d] = as_half2((u & mask_lo) | vmagic) + off_a;
                qb[2 * d] = as_half2((u & mask_hi) | vmagic) + off_b;
                qa[2 * d + 1] = as_half2((t & mask_lo) | vmagic) + off_a;
                qb[2 * d + 1] = as_half2((t & mask_hi) | vmagic) + off_b;
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint32_t* xg = reinterpret_cast<const uint32_t*>(x + (size_t)m * ldx + (size_t)g * 32);
                float a = 0.0f, b = 0.0f;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    a = dot2(qa[2 * d], as_half2(xg[4 * d + 0]), a);
                    b = dot2(qb[2 * d], as_half2(xg[4 * d + 1]), b);
                    a = dot2(qa[2 * d + 1], as_half2(xg[4 * d + 2]), a);
                    b = dot2(qb[2 * d + 1], as_half2(xg[4 * d + 3]), b);
                }
                gs[m][j] = b * 0.0625f + a;
            }
        }
        const uint32_t sw[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float s = h2f(uint16_t(sw[j >> 1] >> (16 * (j & 1))));
#pragma unroll
            for (int m = 0; m < M; ++m) acc[m] = fmaf(gs[m][j], s, acc[m]);
        }
    };

    // Two buffers in flight per wave: chunk c+waves is requested before
    // chunk c is unpacked. The request is unconditional (past the end it
    // re-reads the wave's last chunk) so the number of loads in flight is
    // the same on every path and the waits before each group stay exact.
    u32x4 wa[8], wb[8], sa, sb;
    int c = c0 + wave;
    if (c < c1) {
        const int last = c + (c1 - 1 - c) / waves * waves;
        load(c, wa, sa);
        while (true) {
            load(min(c + waves, last), wb, sb);
            __builtin_amdgcn_sched_barrier(0);  // keep the requests ahead of the math
            compute(c, wa, sa);
            c += waves;
            if (c > last) break;
            load(min(c + waves, last), wa, sa);
            __builtin_amdgcn_sched_barrier(0);
            compute(c, wb, sb);
            c += waves;
            if (c > last) break;
        }
    }
    finish<M, EPI>(acc, tile, split, splits, n, y, ldy, bias, partial, counters, tiles);
}

// ------------------------------------------------------------- int8 kernel

template <int M, int EPI>
__global__ __launch_bounds__(256) void gemv_q8_kernel(
    const u32x4* __restrict__ qw, const uint16_t* __restrict__ qs,
    const uint16_t* __restrict__ x, int ldx, int blocks, int chunks, int cps,
    int n, void* __restrict__ y, int ldy, const float* __restrict__ bias,
    float* __restrict__ partial, unsigned* __restrict__ counters, int splits,
    int tiles, uint32_t hi_bytes) {
    const int tile = blockIdx.x;
    const int split = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = uniform(threadIdx.x >> 6);
    const int waves = uniform(blockDim.x >> 6);
    const int c0 = split * cps;
    const int c1 = min(chunks, c0 + cps);
    const u32x4* wt = qw + (size_t)tile * chunks * 8 * 64 + lane;
    const half2_t off = {(half_t)-1152.0f, (half_t)-1152.0f};

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;

    auto load = [&](int c, u32x4 (&w)[8]) {
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = __builtin_nontemporal_load(wt + ((size_t)c * 8 + j) * 64);
    };
    auto compute = [&](int c, const u32x4 (&w)[8]) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // blocks past the end of K hold code 0: read the last real
            // block's activations (finite) and add 0
            const int b = min(c * 8 + j, blocks - 1);
            const uint32_t u4[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
            half2_t q[8];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                // bytes q+128 -> fp16 1024+byte via v_perm with 0x64 high bytes
                q[2 * d] = as_half2(__builtin_amdgcn_perm(hi_bytes, u4[d], 0x04010400u)) + off;
                q[2 * d + 1] = as_half2(__builtin_amdgcn_perm(hi_bytes, u4[d], 0x04030402u)) + off;
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint32_t* xb = reinterpret_cast<const uint32_t*>(x + (size_t)m * ldx + (size_t)b * 16);
                float a = acc[m];
#pragma unroll
                for (int i = 0; i < 8; ++i) a = dot2(q[i], as_half2(xb[i]), a);
                acc[m] = a;
            }
        }
    };
    u32x4 wa[8], wb[8];
    int c = c0 + wave;
    if (c < c1) {
        const int last = c + (c1 - 1 - c) / waves * waves;
        load(c, wa);
        while (true) {
            load(min(c + waves, last), wb);
            __builtin_amdgcn_sched_barrier(0);
            compute(c, wa);
            c += waves;
            if (c > last) break;
            load(min(c + waves, last), wa);
            __builtin_amdgcn_sched_barrier(0);
            compute(c, wb);
            c += waves;
            if (c > last) break;
        }
    }
    const float s = h2f(qs[(size_t)tile * 64 + lane]);
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] *= s;
    finish<M, EPI>(acc, tile, split, splits, n, y, ldy, bias, partial, counters, tiles);
}

// ----------------------------------------------------- unpack / dequantize

// One thread per (packed row, group): writes codes and/or dequantized values
// in row-major order; paired packings put the B rows after the A rows.
__global__ void q4_unpack_kernel(const uint4* __restrict__ qw,
                                 const uint16_t* __restrict__ qs, int64_t n,
                                 int64_t k, int paired, int chunks,
                                 int8_t* __restrict__ codes,
                                 uint16_t* __restrict__ scales,
                                 float* __restrict__ wout) {
    const int tile = blockIdx.x;
    const int lane = threadIdx.x;
    const int groups = (int)((k + 31) / 32);
    int64_t row = paired ? tile * 32 + (lane & 31) : (int64_t)tile * 64 + lane;
    if (row >= n) return;
    if (paired && lane >= 32) row += n;
    const int pos[8] = {0, 16, 4, 20, 8, 24, 12, 28};
    for (int g = blockIdx.y; g < groups; g += gridDim.y) {
        const uint4 w = qw[((size_t)tile * chunks * 8 + g) * 64 + lane];
        const uint16_t sbits = qs[(((size_t)tile * chunks + g / 8) * 64 + lane) * 8 + (g & 7)];
        if (scales) scales[row * groups + g] = sbits;
        const float s = h2f(sbits);
        const uint32_t u4[4] = {w.x, w.y, w.z, w.w};
        for (int d = 0; d < 4; ++d)
            for (int j = 0; j < 8; ++j) {
                const int64_t kk = (int64_t)g * 32 + d * 8 + j;
                if (kk >= k) continue;
                const int q = (int)((u4[d] >> pos[j]) & 0xFu) - 8;
                if (codes) codes[row * k + kk] = (int8_t)q;
                if (wout) wout[row * k + kk] = (float)q * s;
            }
    }
}

__global__ void q8_unpack_kernel(const uint4* __restrict__ qw,
                                 const uint16_t* __restrict__ qs, int64_t n,
                                 int64_t k, int paired, int chunks,
                                 int8_t* __restrict__ codes,
                                 uint16_t* __restrict__ scales,
                                 float* __restrict__ wout) {
    const int tile = blockIdx.x;
    const int lane = threadIdx.x;
    const int blocks = (int)((k + 15) / 16);
    int64_t row = paired ? tile * 32 + (lane & 31) : (int64_t)tile * 64 + lane;
    if (row >= n) return;
    if (paired && lane >= 32) row += n;
    const uint16_t sbits = qs[(size_t)tile * 64 + lane];
    if (scales && blockIdx.y == 0) scales[row] = sbits;
    const float s = h2f(sbits);
    for (int b = blockIdx.y; b < blocks; b += gridDim.y) {
        const uint4 w = qw[((size_t)tile * chunks * 8 + b) * 64 + lane];
        const uint32_t u4[4] = {w.x, w.y, w.z, w.w};
        for (int j = 0; j < 16; ++j) {
            const int64_t kk = (int64_t)b * 16 + j;
            if (kk >= k) continue;
            const int q = (int)((u4[j >> 2] >> (8 * (j & 3))) & 0xFFu) - 128;
            if (codes) codes[row * k + kk] = (int8_t)q;
            if (wout) wout[row * k + kk] = (float)q * s;
        }
    }
}

// ---------------------------------------------------------------- launchers

template <int M, int EPI>
void launch_q4(const Plan& p, hipStream_t st, const void* qw, const void* qs,
               const uint16_t* x, int ldx, int groups, int n, void* y, int ldy,
               const float* bias, float* partial, unsigned* counters) {
    hipLaunchKernelGGL((gemv_q4_kernel<M, EPI>), dim3(p.tiles, p.splits), dim3(64 * p.waves), 0, st,
                       (const u32x4*)qw, (const u32x4*)qs, x, ldx, groups, p.chunks, p.cps, n, y,
                       ldy, bias, partial, counters, p.splits, p.tiles, 0x000F000Fu, 0x00F000F0u,
                       0x64006400u);
}

template <int M, int EPI>
void launch_q8(const Plan& p, hipStream_t st, const void* qw, const void* qs,
               const uint16_t* x, int ldx, int blocks, int n, void* y, int ldy,
               const float* bias, float* partial, unsigned* counters) {
    hipLaunchKernelGGL((gemv_q8_kernel<M, EPI>), dim3(p.tiles, p.splits), dim3(64 * p.waves), 0, st,
                       (const u32x4*)qw, (const uint16_t*)qs, x, ldx, blocks, p.chunks, p.cps, n, y,
                       ldy, bias, partial, counters, p.splits, p.tiles, 0x64646464u);
}

template <bool Q8, int M>
void dispatch_epi(int epi, const Plan& p, hipStream_t st, const void* qw, const void* qs,
                  const uint16_t* x, int ldx, int units, int n, void* y, int ldy,
                  const float* bias, float* partial, unsigned* counters) {
#define LYK_CASE(E)                                                                          \
    case E:                                                                                  \
        if constexpr (Q8)                                                                    \
            launch_q8<M, E>(p, st, qw, qs, x, ldx, units, n, y, ldy, bias, partial, counters); \
        else                                                                                 \
            launch_q4<M, E>(p, st, qw, qs, x, ldx, units, n, y, ldy, bias, partial, counters); \
        break;
    switch (epi) {
        LYK_CASE(LYK_EPI_STORE)
        LYK_CASE(LYK_EPI_ADD)
        LYK_CASE(LYK_EPI_STORE_F16)
        LYK_CASE(LYK_EPI_SILU_F16)
    }
#undef LYK_CASE
}

template <bool Q8>
int gemv_entry(const void* qw, const void* qs, int64_t n, int64_t k, const uint16_t* x,
               int64_t ldx, int m, int epi, void* y, int64_t ldy, const float* bias,
               int ksplit, void* ws, uint64_t ws_bytes, void* stream) {
    if (!qw || !qs || !x || !y || n <= 0 || k <= 0) return LYK_ERR_INVALID_ARG;
    if (m < 1 || m > kMaxM || epi < LYK_EPI_STORE || epi > LYK_EPI_SILU_F16) return LYK_ERR_INVALID_ARG;
    const int unit = Q8 ? 16 : 32;
    if (ldx < (k + unit - 1) / unit * unit || (ldx & 1)) return LYK_ERR_INVALID_ARG;
    if (ldy < n || n > (int64_t)1 << 30 || k > (int64_t)1 << 24) return LYK_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) & 3) return LYK_ERR_INVALID_ARG;
    const int paired = epi == LYK_EPI_SILU_F16;
    const Plan p = make_plan(n, k, paired, Q8, ksplit);
    const uint64_t need = workspace_for(p, m);
    if (need > ws_bytes || (need && !ws)) return LYK_ERR_WORKSPACE;
    unsigned* counters = static_cast<unsigned*>(ws);
    float* partial = need ? reinterpret_cast<float*>(static_cast<char*>(ws) +
                                                     (uint64_t(p.tiles) * 4 + 255) / 256 * 256)
                          : nullptr;
    const int units = (int)(Q8 ? (k + 15) / 16 : (k + 31) / 32);
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (m) {
        case 1: dispatch_epi<Q8, 1>(epi, p, st, qw, qs, x, (int)ldx, units, (int)n, y, (int)ldy, bias, partial, counters); break;
        case 2: dispatch_epi<Q8, 2>(epi, p, st, qw, qs, x, (int)ldx, units, (int)n, y, (int)ldy, bias, partial, counters); break;
        case 3: dispatch_epi<Q8, 3>(epi, p, st, qw, qs, x, (int)ldx, units, (int)n, y, (int)ldy, bias, partial, counters); break;
        case 4: dispatch_epi<Q8, 4>(epi, p, st, qw, qs, x, (int)ldx, units, (int)n, y, (int)ldy, bias, partial, counters); break;
    }
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

template <bool Q8>
int unpack_entry(const void* qw, const void* qs, int64_t n, int64_t k, int paired,
                 int8_t* codes, uint16_t* scales, float* wout, void* stream) {
    if (!qw || !qs || n <= 0 || k <= 0 || (!codes && !scales && !wout)) return LYK_ERR_INVALID_ARG;
    const Plan p = make_plan(n, k, paired, Q8, 1);
    const int units = (int)(Q8 ? (k + 15) / 16 : (k + 31) / 32);
    dim3 grid(p.tiles, units < 64 ? units : 64);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (Q8)
        hipLaunchKernelGGL(q8_unpack_kernel, grid, dim3(64), 0, st, (const uint4*)qw,
                           (const uint16_t*)qs, n, k, paired, p.chunks, codes, scales, wout);
    else
        hipLaunchKernelGGL(q4_unpack_kernel, grid, dim3(64), 0, st, (const uint4*)qw,
                           (const uint16_t*)qs, n, k, paired, p.chunks, codes, scales, wout);
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

}  // namespace
}  // namespace lyk

using namespace lyk;

extern "C" {

int lyk_hip_gemv_splits(int64_t n, int64_t k, int m, int paired, int q8) {
    (void)m;
    const Plan p = make_plan(n, k, paired, q8, 0);
    return p.splits * p.waves;
}

uint64_t lyk_hip_gemv_workspace_bytes(int64_t n, int64_t k, int m, int splits, int paired,
                                      int q8) {
    if (n <= 0 || k <= 0 || m < 1) return 0;
    return workspace_for(make_plan(n, k, paired, q8, splits), m);
}

int lyk_hip_gemv_q4(const void* d_qw, const void* d_qs, int64_t n, int64_t k,
                    const uint16_t* d_x, int64_t ldx, int m, int epilogue, void* d_y,
                    int64_t ldy, const float* d_bias, int splits, void* d_workspace,
                    uint64_t workspace_bytes, void* stream) {
    return gemv_entry<false>(d_qw, d_qs, n, k, d_x, ldx, m, epilogue, d_y, ldy, d_bias, splits,
                             d_workspace, workspace_bytes, stream);
}

int lyk_hip_gemv_q8(const void* d_qw, const void* d_qs, int64_t n, int64_t k,
                    const uint16_t* d_x, int64_t ldx, int m, int epilogue, void* d_y,
                    int64_t ldy, const float* d_bias, int splits, void* d_workspace,
                    uint64_t workspace_bytes, void* stream) {
    return gemv_entry<true>(d_qw, d_qs, n, k, d_x, ldx, m, epilogue, d_y, ldy, d_bias, splits,
                            d_workspace, workspace_bytes, stream);
}

int lyk_hip_q4_unpack(const void* d_qw, const void* d_qs, int64_t n, int64_t k, int paired,
                      int8_t* d_codes, uint16_t* d_scales, void* stream) {
    return unpack_entry<false>(d_qw, d_qs, n, k, paired, d_codes, d_scales, nullptr, stream);
}
int lyk_hip_q8_unpack(const void* d_qw, const void* d_qs, int64_t n, int64_t k, int paired,
                      int8_t* d_codes, uint16_t* d_scales, void* stream) {
    return unpack_entry<true>(d_qw, d_qs, n, k, paired, d_codes, d_scales, nullptr, stream);
}
int lyk_hip_q4_dequant(const void* d_qw, const void* d_qs, int64_t n, int64_t k, int paired,
                       float* d_w, void* stream) {
    return unpack_entry<false>(d_qw, d_qs, n, k, paired, nullptr, nullptr, d_w, stream);
}
int lyk_hip_q8_dequant(const void* d_qw, const void* d_qs, int64_t n, int64_t k, int paired,
                       float* d_w, void* stream) {
    return unpack_entry<true>(d_qw, d_qs, n, k, paired, nullptr, nullptr, d_w, stream);
}

}  // extern "C"
