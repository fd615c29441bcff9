// GQA decode attention over the paged fp16 KV cache (one query token per
// sequence), gfx950.
//
// Reference: the CPU attention loop (model/architectures/qwen/qwen_model.cpp:
// 255-287) and the CUDA split-K pair BatchSplitAttentionKernel /
// BatchCombineAttentionKernel (backends/cuda/qwen_cuda_model.cu:401-527).
//
// Layout: per layer, K and V pools are fp16 [num_blocks][nkv][bt][hd]; token t
// of a sequence lives in block table[t / bt], slot t % bt. One workgroup
// handles one (kv head, split, sequence): all q heads of the GQA group share
// every K/V element it loads. K and V rows of a chunk of tokens are staged in
// LDS with 16-byte loads (one 4 KiB block of 16 tokens x 128 dims is one
// contiguous run), scores for the whole group are computed from LDS, and an
// online softmax carries the running max / sum across chunks. Splits write
// (max, sum, unnormalised output) partials; the last split to finish merges
// them in split order, so the result is independent of timing.
#include "common.h"

namespace lyk {
namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 64;     // tokens staged per iteration
constexpr int kMaxItems = 16;  // (head, dim) outputs per thread: G*hd <= 4096

struct AttnShape {
    int nq, nkv, hd, G, bt, splits, num_blocks, table_stride;
};

template <int VEC>  // halves per staged load: 8 (16 bytes) or 2
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(
    const float* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const int* __restrict__ table, const int* __restrict__ positions, AttnShape sh, float scale,
    uint16_t* __restrict__ out, int ldo, float* __restrict__ pml, float* __restrict__ pacc,
    unsigned* __restrict__ counters) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int g = blockIdx.x, s = blockIdx.y, m = blockIdx.z;
    const int G = sh.G, hd = sh.hd, tid = threadIdx.x;
    const int ldk = hd + 2;  // padded LDS row (halves): consecutive rows hit different banks
    float* q_s = reinterpret_cast<float*>(smem);                   // [G][hd]
    float* p_s = q_s + G * hd;                                     // [G][kChunk]
    float* m_s = p_s + G * kChunk;                                 // [G] running max
    float* l_s = m_s + 16;                                         // [G] running sum
    float* a_s = l_s + 16;                                         // [G] rescale factor
    uint16_t* k_s = reinterpret_cast<uint16_t*>(a_s + 16);         // [kChunk][ldk]
    uint16_t* v_s = k_s + kChunk * ldk;                            // [kChunk][ldk]

    const int ctx = positions[m] + 1;  // the query at position p sees tokens 0..p
    const int per = (ctx + sh.splits - 1) / sh.splits;
    const int t0 = s * per, t1 = min(ctx, t0 + per);

    for (int i = tid; i < G * hd; i += kThreads)
        q_s[i] = q[((size_t)m * sh.nq + (size_t)g * G) * hd + i];
    if (tid < G) { m_s[tid] = -INFINITY; l_s[tid] = 0.0f; }

    const int items = (G * hd + kThreads - 1) / kThreads;
    float acc[kMaxItems];
#pragma unroll
    for (int i = 0; i < kMaxItems; ++i) acc[i] = 0.0f;
    __syncthreads();

    const int* tab = table + (size_t)m * sh.table_stride;
    const int units = hd / VEC;
    for (int c0 = t0; c0 < t1; c0 += kChunk) {
        const int n = min(kChunk, t1 - c0);
        // stage K and V rows of tokens c0..c0+n-1
        for (int e = tid; e < n * units; e += kThreads) {
            const int j = e / units, u = e % units;
            const int t = c0 + j;
            int blk = tab[t / sh.bt];
            if (blk < 0 || blk >= sh.num_blocks) blk = 0;  // host-validated tables
            const size_t off = (((size_t)blk * sh.nkv + g) * sh.bt + t % sh.bt) * hd + u * VEC;
            if constexpr (VEC == 8) {
                const uint4 kv = *reinterpret_cast<const uint4*>(kc + off);
                const uint4 vv = *reinterpret_cast<const uint4*>(vc + off);
                uint32_t* kd = reinterpret_cast<uint32_t*>(k_s + j * ldk + u * VEC);
                uint32_t* vd = reinterpret_cast<uint32_t*>(v_s + j * ldk + u * VEC);
                kd[0] = kv.x; kd[1] = kv.y; kd[2] = kv.z; kd[3] = kv.w;
                vd[0] = vv.x; vd[1] = vv.y; vd[2] = vv.z; vd[3] = vv.w;
            } else {
                *reinterpret_cast<uint32_t*>(k_s + j * ldk + u * VEC) =
                    *reinterpret_cast<const uint32_t*>(kc + off);
                *reinterpret_cast<uint32_t*>(v_s + j * ldk + u * VEC) =
                    *reinterpret_cast<const uint32_t*>(vc + off);
            }
        }
        __syncthreads();
        // scores: dot(q_h, k_t) * scale, the CPU's order of the final multiply
        for (int e = tid; e < G * n; e += kThreads) {
            const int h = e / n, j = e % n;
            const float* qh = q_s + h * hd;
            const uint32_t* kr = reinterpret_cast<const uint32_t*>(k_s + j * ldk);
            float dot = 0.0f;
            for (int d = 0; d < hd / 2; ++d) {
                const half2_t kk = as_half2(kr[d]);
                dot = fmaf(qh[2 * d], (float)kk.x, dot);
                dot = fmaf(qh[2 * d + 1], (float)kk.y, dot);
            }
            p_s[h * kChunk + j] = dot * scale;
        }
        __syncthreads();
        // online softmax: one wave per head, one lane per token of the chunk
        {
            const int lane = tid & 63, wave = tid >> 6;
            for (int h = wave; h < G; h += kThreads / 64) {
                const float sc = lane < n ? p_s[h * kChunk + lane] : -INFINITY;
                const float mx = wave_max(sc);
                const float mold = m_s[h];
                const float mnew = fmaxf(mold, mx);
                const float p = lane < n ? expf(sc - mnew) : 0.0f;
                const float sum = wave_sum(p);
                if (lane < n) p_s[h * kChunk + lane] = p;
                if (lane == 0) {
                    const float alpha = expf(mold - mnew);  // 0 on the first chunk
                    a_s[h] = alpha;
                    l_s[h] = l_s[h] * alpha + sum;
                    m_s[h] = mnew;
                }
            }
        }
        __syncthreads();
        // out[h][d] = alpha_h * out[h][d] + sum_j p[h][j] * v[j][d]
#pragma unroll
        for (int i = 0; i < kMaxItems; ++i) {
            const int idx = tid + i * kThreads;
            if (i < items && idx < G * hd) {
                const int h = idx / hd, d = idx % hd;
                const float* ph = p_s + h * kChunk;
                float a = acc[i] * a_s[h];
                for (int j = 0; j < n; ++j)
                    a = fmaf(ph[j], h2f(v_s[j * ldk + d]), a);
                acc[i] = a;
            }
        }
        __syncthreads();
    }

    // ---- partials and fixed-order merge across splits
    const int S = sh.splits;
    const size_t grp = (size_t)m * sh.nkv + g;
    if (S == 1) {
#pragma unroll
        for (int i = 0; i < kMaxItems; ++i) {
            const int idx = tid + i * kThreads;
            if (i < items && idx < G * hd) {
                const int h = idx / hd;
                out[(size_t)m * ldo + (size_t)g * G * hd + idx] = f2h(acc[i] / l_s[h]);
            }
        }
        return;
    }
    float* ml = pml + (grp * S + s) * G * 2;
    float* pa = pacc + (grp * S + s) * (size_t)G * hd;
    if (tid < G) { store_sc1(&ml[2 * tid], m_s[tid]); store_sc1(&ml[2 * tid + 1], l_s[tid]); }
#pragma unroll
    for (int i = 0; i < kMaxItems; ++i) {
        const int idx = tid + i * kThreads;
        if (i < items && idx < G * hd) store_sc1(&pa[idx], acc[i]);
    }
    publish_sc1_stores();
    __syncthreads();
    __shared__ int last;
    if (tid < 64) {
        const bool l = arrive_last(&counters[grp], (unsigned)S);
        if (tid == 0) last = l;
    }
    __syncthreads();
    if (!last) return;
    // merged max per head, then weights e^(m_s - M)
    if (tid < G) {
        float M = -INFINITY;
        for (int j = 0; j < S; ++j) M = fmaxf(M, load_sc1(&pml[(grp * S + j) * G * 2 + 2 * tid]));
        float L = 0.0f;
        for (int j = 0; j < S; ++j) {
            float* e = &pml[(grp * S + j) * G * 2 + 2 * tid];
            L += load_sc1(e + 1) * expf(load_sc1(e) - M);
        }
        m_s[tid] = M;
        l_s[tid] = L;
    }
    __syncthreads();
    for (int i = 0; i < items; ++i) {
        const int idx = tid + i * kThreads;
        if (idx < G * hd) {
            const int h = idx / hd;
            float o = 0.0f;
            for (int j = 0; j < S; ++j) {
                float* e = &pml[(grp * S + j) * G * 2 + 2 * h];
                float* pj = &pacc[(grp * S + j) * (size_t)G * hd + idx];
                o += load_sc1(pj) * expf(load_sc1(e) - m_s[h]);
                *pj = 0.0f;
            }
            out[(size_t)m * ldo + (size_t)g * G * hd + idx] = f2h(o / l_s[h]);
        }
    }
    __syncthreads();
    if (tid < G)
        for (int j = 0; j < S; ++j) {
            pml[(grp * S + j) * G * 2 + 2 * tid] = 0.0f;
            pml[(grp * S + j) * G * 2 + 2 * tid + 1] = 0.0f;
        }
    if (tid == 0) counters[grp] = 0u;
}

size_t attn_smem(int G, int hd) {
    return (size_t)(G * hd + G * kChunk + 48) * 4 + (size_t)2 * kChunk * (hd + 2) * 2;
}

}  // namespace
}  // namespace lyk

using namespace lyk;

extern "C" {

uint64_t lyk_hip_attn_workspace_bytes(int m, int nq, int nkv, int hd, int splits) {
    if (m < 1 || nq < 1 || nkv < 1 || hd < 1 || splits < 1) return 0;
    const int G = nq / nkv;
    const uint64_t counters = ((uint64_t)m * nkv * 4 + 255) / 256 * 256;
    return counters + (uint64_t)m * nkv * splits * G * (2 + hd) * 4;
}

int lyk_hip_attn_decode(const float* d_q, const uint16_t* d_kcache, const uint16_t* d_vcache,
                        const int32_t* d_table, int table_stride, const int32_t* d_pos, int m,
                        int nq, int nkv, int hd, int block_tokens, int num_blocks, int splits,
                        uint16_t* d_out, int64_t ldo, void* d_workspace, uint64_t workspace_bytes,
                        void* stream) {
    if (!d_q || !d_kcache || !d_vcache || !d_table || !d_pos || !d_out) return LYK_ERR_INVALID_ARG;
    if (m < 1 || nq < 1 || nkv < 1 || nq % nkv || hd < 2 || (hd & 1) || block_tokens < 1 ||
        num_blocks < 1 || splits < 1 || table_stride < 1 || ldo < (int64_t)nq * hd)
        return LYK_ERR_INVALID_ARG;
    const int G = nq / nkv;
    if (G > 16 || G * hd > kThreads * kMaxItems || hd > 512 || splits > 1024) return LYK_ERR_SHAPE;
    const uint64_t need = splits > 1 ? lyk_hip_attn_workspace_bytes(m, nq, nkv, hd, splits) : 0;
    if (need > workspace_bytes || (need && !d_workspace)) return LYK_ERR_WORKSPACE;
    unsigned* counters = static_cast<unsigned*>(d_workspace);
    const uint64_t cbytes = ((uint64_t)m * nkv * 4 + 255) / 256 * 256;
    float* pml = need ? reinterpret_cast<float*>(static_cast<char*>(d_workspace) + cbytes) : nullptr;
    float* pacc = need ? pml + (size_t)m * nkv * splits * G * 2 : nullptr;
    AttnShape sh{nq, nkv, hd, G, block_tokens, splits, num_blocks, table_stride};
    const float scale = 1.0f / sqrtf((float)hd);
    const size_t smem = attn_smem(G, hd);
    if (smem > 64 * 1024) return LYK_ERR_SHAPE;
    hipStream_t st = static_cast<hipStream_t>(stream);
    dim3 grid(nkv, splits, m);
    if (hd % 8 == 0)
        hipLaunchKernelGGL(attn_decode_kernel<8>, grid, dim3(kThreads), smem, st, d_q, d_kcache,
                           d_vcache, d_table, d_pos, sh, scale, d_out, (int)ldo, pml, pacc, counters);
    else
        hipLaunchKernelGGL(attn_decode_kernel<2>, grid, dim3(kThreads), smem, st, d_q, d_kcache,
                           d_vcache, d_table, d_pos, sh, scale, d_out, (int)ldo, pml, pacc, counters);
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

}  // extern "C"
