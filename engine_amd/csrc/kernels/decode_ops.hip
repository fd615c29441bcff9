// Small per-token kernels of the decode step: embedding gather + RMSNorm,
// RMSNorm to fp16, RoPE + paged KV append, and greedy argmax.
//
// Reference counterparts: GatherEmbedRowsKernel, NormScaleKernel,
// RmsNormRowsKernel, RopeQkKernel, ScatterKv2Kernel, ArgmaxStage1/2Kernel
// (backends/cuda/qwen_cuda_model.cu:182-218, 591-610, 822-870, 910-944,
// 1388-1458); CPU: RmsNorm / ApplyRope / the embedding copy / Sampler's
// greedy rule (model/architectures/qwen/qwen_model.cpp:33-54, 220-221;
// core/generation/sampler.cpp:48-53).
#include "common.h"

namespace lyk {
namespace {

constexpr int kThreads = 256;

// Sum of x[i]^2 over the row, reduced over the workgroup (fixed tree order).
__device__ float block_sum(float v) {
    __shared__ float part[kThreads / 64];
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) part[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) s += part[w];
    __syncthreads();
    return s;
}

// xn = fp16(x * (1/sqrt(mean(x^2) + eps)) * gamma), the reference order of
// operations (qwen_model.cpp:35-38); the sum of squares is a tree.
__device__ void rmsnorm_row(const float* x, const float* gamma, float eps, int n,
                            uint16_t* out) {
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += kThreads) ss += x[i] * x[i];
    ss = block_sum(ss);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += kThreads) out[i] = f2h(x[i] * scale * gamma[i]);
}

__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float* __restrict__ h, int ldh,
                                                           const float* __restrict__ gamma,
                                                           float eps, int n,
                                                           uint16_t* __restrict__ xn, int ldx) {
    const int m = blockIdx.x;
    rmsnorm_row(h + (size_t)m * ldh, gamma, eps, n, xn + (size_t)m * ldx);
}

__global__ __launch_bounds__(kThreads) void embed_rmsnorm_kernel(
    const float* __restrict__ table, int vocab, const int* __restrict__ tokens, int n,
    float* __restrict__ h, int ldh, const float* __restrict__ gamma, float eps,
    uint16_t* __restrict__ xn, int ldx) {
    const int m = blockIdx.x;
    int tok = tokens[m];
    if (tok < 0 || tok >= vocab) tok = 0;  // host validates; never read out of bounds
    const float* src = table + (size_t)tok * n;
    float* dst = h + (size_t)m * ldh;
    for (int i = threadIdx.x; i < n; i += kThreads) dst[i] = src[i];
    __syncthreads();
    rmsnorm_row(dst, gamma, eps, n, xn + (size_t)m * ldx);
}

// One workgroup per (head, batch row); head < nq are query heads, then nkv
// key heads, then nkv value heads. Rotation pairs (i, i + hd/2) use the
// host-built cos/sin tables, so the products equal the CPU's bit for bit.
__global__ void rope_kv_kernel(const float* __restrict__ qkv, int ldq, int nq, int nkv, int hd,
                               const int* __restrict__ pos, const float* __restrict__ rcos,
                               const float* __restrict__ rsin, int max_pos,
                               float* __restrict__ q_out, uint16_t* __restrict__ kc,
                               uint16_t* __restrict__ vc, const int* __restrict__ table,
                               int table_stride, int block_tokens, int num_blocks) {
    const int head = blockIdx.x, m = blockIdx.y;
    const int p = pos[m];
    if (p < 0 || p >= max_pos) return;  // host validates positions
    const int half = hd / 2;
    const float* src = qkv + (size_t)m * ldq + (size_t)head * hd;
    const float* c = rcos + (size_t)p * half;
    const float* s = rsin + (size_t)p * half;
    if (head < nq) {
        float* dst = q_out + ((size_t)m * nq + head) * hd;
        for (int i = threadIdx.x; i < half; i += blockDim.x) {
            const float a = src[i], b = src[i + half];
            dst[i] = rot_lo(a, b, c[i], s[i]);
            dst[i + half] = rot_hi(a, b, c[i], s[i]);
        }
        return;
    }
    const int blk = table[(size_t)m * table_stride + p / block_tokens];
    if (blk < 0 || blk >= num_blocks) return;
    const int slot = p % block_tokens;
    if (head < nq + nkv) {
        const int kh = head - nq;
        uint16_t* dst = kc + (((size_t)blk * nkv + kh) * block_tokens + slot) * hd;
        for (int i = threadIdx.x; i < half; i += blockDim.x) {
            const float a = src[i], b = src[i + half];
            dst[i] = f2h(rot_lo(a, b, c[i], s[i]));
            dst[i + half] = f2h(rot_hi(a, b, c[i], s[i]));
        }
    } else {
        const int vh = head - nq - nkv;
        uint16_t* dst = vc + (((size_t)blk * nkv + vh) * block_tokens + slot) * hd;
        for (int i = threadIdx.x; i < hd; i += blockDim.x) dst[i] = f2h(src[i]);
    }
}

// ------------------------------------------------------------------ argmax
// Greedy rule of Sampler::Sample: the first index of the maximum; NaN never
// wins (treated as -inf). Stage 1: each workgroup reduces a segment; the
// last workgroup of a row (arrival counter) reduces the partials in order.

constexpr int kMaxRows = 32;  // argmax rows per launch (workspace counter slots)

struct Best {
    float v;
    int i;
};

__device__ __forceinline__ Best better(Best a, Best b) {
    if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
    return a;
}

__device__ Best wave_best(Best b) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        Best other{__shfl_xor(b.v, o, 64), __shfl_xor(b.i, o, 64)};
        b = better(b, other);
    }
    return b;
}

// Result of one row: the token feeds the next step; non-finite logits are
// counted (added, so a multi-step run accumulates); the position advances;
// for single-row greedy runs the token is appended to the history at *step.
__device__ void commit(int m, int token, int bad, int* out, int* nonfinite, int* advance,
                       int* history, int* step) {
    out[m] = token;
    if (nonfinite) nonfinite[m] += bad;
    if (advance) advance[m] += 1;
    if (history) {
        const int s = *step;
        history[s] = token;
        *step = s + 1;
    }
}

__global__ __launch_bounds__(kThreads) void argmax_kernel(
    const float* __restrict__ logits, int ldl, int n, int seg, int* __restrict__ out,
    int* __restrict__ nonfinite, float* __restrict__ pv, int* __restrict__ pi,
    unsigned* __restrict__ counters, int* __restrict__ advance, int* __restrict__ history,
    int* __restrict__ step) {
    const int m = blockIdx.y, b = blockIdx.x, nb = gridDim.x;
    const float* row = logits + (size_t)m * ldl;
    const int i0 = b * seg, i1 = min(n, i0 + seg);
    Best best{-INFINITY, 0x7fffffff};
    int bad = 0;
    for (int i = i0 + threadIdx.x; i < i1; i += kThreads) {
        float v = row[i];
        if (!isfinite(v)) {
            ++bad;
            if (isnan(v)) v = -INFINITY;
        }
        best = better(best, Best{v, i});
    }
    best = wave_best(best);
    __shared__ float sv[kThreads / 64];
    __shared__ int si[kThreads / 64], sb[kThreads / 64];
    bad = (int)wave_sum((float)bad);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { sv[wave] = best.v; si[wave] = best.i; sb[wave] = bad; }
    __syncthreads();
    if (threadIdx.x != 0) return;
    best = Best{sv[0], si[0]};
    bad = sb[0];
    for (int w = 1; w < kThreads / 64; ++w) { best = better(best, Best{sv[w], si[w]}); bad += sb[w]; }
    if (nb == 1) {
        commit(m, best.i < n ? best.i : 0, bad, out, nonfinite, advance, history, step);
        return;
    }
    const size_t slot = (size_t)m * nb + b;
    __hip_atomic_store(&pv[slot], best.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&pi[slot], best.i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(&counters[kMaxRows + m], (unsigned)bad, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    publish_sc1_stores();
    const unsigned prev = __hip_atomic_fetch_add(&counters[m], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev != (unsigned)(nb - 1)) return;
    Best r{-INFINITY, 0x7fffffff};
    for (int j = 0; j < nb; ++j) {
        const size_t sj = (size_t)m * nb + j;
        Best c{__hip_atomic_load(&pv[sj], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
               __hip_atomic_load(&pi[sj], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)};
        r = better(r, c);
        pv[sj] = 0.0f;
        pi[sj] = 0;
    }
    const unsigned total_bad = __hip_atomic_exchange(&counters[kMaxRows + m], 0u,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    commit(m, r.i < n ? r.i : 0, (int)total_bad, out, nonfinite, advance, history, step);
    counters[m] = 0u;
}

int argmax_segments(int64_t n) {
    int nb = ceil_div(n, 4096);
    return nb < 1 ? 1 : (nb > 128 ? 128 : nb);
}

}  // namespace
}  // namespace lyk

using namespace lyk;

extern "C" {

int lyk_hip_rmsnorm_f16(const float* d_h, int64_t ldh, const float* d_gamma, float eps, int m,
                        int64_t n, uint16_t* d_xn, int64_t ldx, void* stream) {
    if (!d_h || !d_gamma || !d_xn || m < 1 || n < 1 || ldh < n || ldx < n) return LYK_ERR_INVALID_ARG;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(m), dim3(kThreads), 0, (hipStream_t)stream, d_h,
                       (int)ldh, d_gamma, eps, (int)n, d_xn, (int)ldx);
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

int lyk_hip_embed_rmsnorm(const float* d_table, int64_t vocab, const int32_t* d_tokens, int m,
                          int64_t n, float* d_h, int64_t ldh, const float* d_gamma, float eps,
                          uint16_t* d_xn, int64_t ldx, void* stream) {
    if (!d_table || !d_tokens || !d_h || !d_gamma || !d_xn || m < 1 || n < 1 || vocab < 1 ||
        ldh < n || ldx < n)
        return LYK_ERR_INVALID_ARG;
    hipLaunchKernelGGL(embed_rmsnorm_kernel, dim3(m), dim3(kThreads), 0, (hipStream_t)stream,
                       d_table, (int)vocab, d_tokens, (int)n, d_h, (int)ldh, d_gamma, eps, d_xn,
                       (int)ldx);
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

int lyk_hip_rope_kv_append(const float* d_qkv, int64_t ldq, int m, int nq, int nkv, int hd,
                           const int32_t* d_pos, const float* d_cos, const float* d_sin,
                           int max_pos, float* d_q, uint16_t* d_kcache, uint16_t* d_vcache,
                           const int32_t* d_table, int table_stride, int block_tokens,
                           int num_blocks, void* stream) {
    if (!d_qkv || !d_pos || !d_cos || !d_sin || !d_q || !d_kcache || !d_vcache || !d_table)
        return LYK_ERR_INVALID_ARG;
    if (m < 1 || nq < 1 || nkv < 1 || hd < 2 || (hd & 1) || block_tokens < 1 || num_blocks < 1 ||
        ldq < (int64_t)(nq + 2 * nkv) * hd || table_stride < 1)
        return LYK_ERR_INVALID_ARG;
    const int threads = hd / 2 < 64 ? 64 : (hd / 2 > 256 ? 256 : hd / 2);
    hipLaunchKernelGGL(rope_kv_kernel, dim3(nq + 2 * nkv, m), dim3(threads), 0, (hipStream_t)stream,
                       d_qkv, (int)ldq, nq, nkv, hd, d_pos, d_cos, d_sin, max_pos, d_q, d_kcache,
                       d_vcache, d_table, table_stride, block_tokens, num_blocks);
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

uint64_t lyk_hip_argmax_workspace_bytes(int m, int64_t n) {
    // [32 arrival counters][32 non-finite counts] then per-segment (value, index)
    return 256 + (uint64_t)m * (uint64_t)argmax_segments(n) * 8;
}

int lyk_hip_argmax(const float* d_logits, int64_t ldl, int m, int64_t n, int32_t* d_tokens,
                   int32_t* d_nonfinite, int32_t* d_advance, int32_t* d_history,
                   int32_t* d_step, void* d_workspace, uint64_t workspace_bytes, void* stream) {
    if (!d_logits || !d_tokens || m < 1 || n < 1 || ldl < n || n > 0x7ffffff0) return LYK_ERR_INVALID_ARG;
    if ((d_history != nullptr) != (d_step != nullptr) || (d_history && m != 1)) return LYK_ERR_INVALID_ARG;
    if (m > kMaxRows) return LYK_ERR_SHAPE;
    const int nb = argmax_segments(n);
    unsigned* counters = nullptr;
    float* pv = nullptr;
    int* pi = nullptr;
    if (nb > 1) {
        if (!d_workspace || workspace_bytes < lyk_hip_argmax_workspace_bytes(m, n)) return LYK_ERR_WORKSPACE;
        char* base = static_cast<char*>(d_workspace);
        counters = reinterpret_cast<unsigned*>(base);
        pv = reinterpret_cast<float*>(base + 256);
        pi = reinterpret_cast<int*>(base + 256 + (size_t)m * nb * 4);
    }
    const int seg = (int)((n + nb - 1) / nb);
    hipLaunchKernelGGL(argmax_kernel, dim3(nb, m), dim3(kThreads), 0, (hipStream_t)stream,
                       d_logits, (int)ldl, (int)n, seg, d_tokens, d_nonfinite, pv, pi, counters,
                       d_advance, d_history, d_step);
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

}  // extern "C"
