// Chunk prefill kernels: RoPE + paged KV append for a chunk of prompt rows of
// one sequence, and causal attention of the chunk's queries over the cache.
// With the prefill GEMM (gemm.hip) and RMSNorm (decode_ops.hip) they make up
// one chunk pass of a layer; the fused decode step then reads the cache they
// fill.
//
// Reference: ForwardChunk's RoPE / KV scatter and ChunkAttentionKernel
// (backends/cuda/qwen_cuda_model.cu:822-870, 981-1030, 2398-2516); the CPU
// path runs the same arithmetic one token at a time
// (model/architectures/qwen/qwen_model.cpp:239-287).
//
// Attention runs on the matrix cores, one wave per (16-token query tile,
// query head), 4 waves to a workgroup on consecutive heads of the tile:
//   * q.k: S^T[key][token] = K[key][:] . q[token][:] with
//     v_mfma_f32_16x16x32_f16, A = a 16-key K tile (lane l: key l % 16, 8
//     dims from 8 (l / 16), 16 bytes of a row-major K row), B = the tile's q
//     (lane l: token l % 16), q fp32 split into two fp16 parts (hi + lo, ~22
//     bits) so the product keeps fp32 precision. Lane (quad, c) gets the
//     scores of token c against keys 4 quad + e.
//   * softmax online over 16-key tiles: the token's running max and sum (the
//     quads of a token exchange theirs through two xor shuffles).
//   * p.v: O[token][dim] += P[token][key] V[key][dim] with
//     v_mfma_f32_16x16x16_f16, A = the lane's own four weights (already in
//     A's layout: token c, keys 4 quad..), split hi + lo like q; B = V from
//     the transposed cache (lane l: dim l % 16, 4 consecutive keys, 8 bytes).
// The arithmetic is the fused step's attention (the same splits and fp32
// sums), so a prompt prefilled in chunks and one prefilled token by token
// differ by the order of fp32 additions only.
#include "common.h"

namespace lyk {
namespace {

constexpr int kRopeThreads = 64;
constexpr int kAttnWaves = 4;

// One workgroup per (head, row); heads < nq are query heads, then nkv key
// heads, then nkv value heads. Row t is position pos0 + t.
__global__ __launch_bounds__(kRopeThreads) void chunk_rope_kv_kernel(
    const float* __restrict__ qkv, int ldq, int pos0, int nq, int nkv, int hd, const float* __restrict__ rcos,
    const float* __restrict__ rsin, float* __restrict__ q_out, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
    const int* __restrict__ table, int bt, int num_blocks) {
    const int head = blockIdx.x, t = blockIdx.y;
    const int p = pos0 + t, half = hd / 2;
    const float* src = qkv + (size_t)t * ldq + (size_t)head * hd;
    const float* c = rcos + (size_t)p * half;
    const float* s = rsin + (size_t)p * half;
    if (head < nq) {
        float* dst = q_out + ((size_t)t * nq + head) * hd;
        for (int i = threadIdx.x; i < half; i += kRopeThreads) {
            const float a = src[i], b = src[i + half];
            dst[i] = rot_lo(a, b, c[i], s[i]);
            dst[i + half] = rot_hi(a, b, c[i], s[i]);
        }
        return;
    }
    const int blk = table[p / bt];
    if (blk < 0 || blk >= num_blocks) return;   // the host hands in valid tables
    const int slot = p % bt;
    if (head < nq + nkv) {
        // K row-major: [blk][nkv][bt][hd]
        uint16_t* dst = kc + (((size_t)blk * nkv + (head - nq)) * bt + slot) * hd;
        for (int i = threadIdx.x; i < half; i += kRopeThreads) {
            const float a = src[i], b = src[i + half];
            dst[i] = f2h(rot_lo(a, b, c[i], s[i]));
            dst[i + half] = f2h(rot_hi(a, b, c[i], s[i]));
        }
    } else {
        // V transposed: [blk][nkv][hd][bt]
        uint16_t* dst = vc + ((size_t)blk * nkv + (head - nq - nkv)) * hd * bt + slot;
        for (int i = threadIdx.x; i < hd; i += kRopeThreads) dst[(size_t)i * bt] = f2h(src[i]);
    }
}

template <int HD>
__global__ __launch_bounds__(kAttnWaves * 64) void chunk_attention_kernel(
    const float* __restrict__ q, int T, int pos0, int nq, int nkv, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int* __restrict__ table, int bt, int num_blocks,
    uint16_t* __restrict__ out, int ldo) {
    constexpr int KS = HD / 32;   // 32-dim steps of q.k
    constexpr int DT = HD / 16;   // 16-dim tiles of p.v
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int quad = lane >> 4, c = lane & 15;
    const int h = blockIdx.x * kAttnWaves + wave;
    if (h >= nq) return;   // no workgroup barrier below: an idle wave may leave
    const int g = h / (nq / nkv);
    const int tok0 = blockIdx.y * 16;
    const int last = min(tok0 + 15, T - 1);
    const int ctx = pos0 + T;                 // keys written so far
    const int pos_c = pos0 + min(tok0 + c, T - 1);   // this lane's token's position
    const float scale = 1.0f / sqrtf((float)HD);

    // B operand of q.k: token c's q, dims 8 quad.. of each 32-dim step
    f16x8 qa[KS], qb[KS];
    {
        const int t = tok0 + c;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            uint16_t hi[8], lo[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = t < T ? q[((size_t)t * nq + h) * HD + ks * 32 + quad * 8 + e] : 0.0f;
                split_f16(v, hi[e], lo[e]);
            }
            qa[ks] = __builtin_bit_cast(f16x8, hi);
            qb[ks] = __builtin_bit_cast(f16x8, lo);
        }
    }
    f32x4 acc[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) acc[d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;   // token c's running max and sum
    const size_t head_k = (size_t)bt * HD;   // one kv head of a block
    const int ntiles = (pos0 + last) / 16 + 1;
    for (int kt = 0; kt < ntiles; ++kt) {
        const int k0 = kt * 16;   // a tile never straddles a block (bt % 16 == 0)
        const int blk = table[k0 / bt];
        const bool blk_ok = blk >= 0 && blk < num_blocks;
        const size_t base = (size_t)(blk_ok ? blk : 0) * nkv * head_k + (size_t)g * head_k;
        const int slot0 = k0 % bt;
        // A operand: key k0 + c's row, dims 8 quad.. of each step (zero past
        // the keys written)
        const bool kvalid = blk_ok && k0 + c < ctx;
        u32x4 kr[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            kr[ks] = kvalid ? ld(reinterpret_cast<const u32x4*>(kc + base + (size_t)(slot0 + c) * HD + ks * 32 + quad * 8))
                            : u32x4{0u, 0u, 0u, 0u};
        // B operands of p.v: dim d*16 + c, keys 4 quad .. +3
        uint64_t vr[DT];
        const int nvalid = blk_ok ? ctx - (k0 + quad * 4) : 0;
#pragma unroll
        for (int d = 0; d < DT; ++d) {
            uint64_t w = 0;
            if (nvalid > 0) {
                w = ld(reinterpret_cast<const uint64_t*>(vc + base + (size_t)(d * 16 + c) * bt + slot0 + quad * 4));
                if (nvalid < 4) w &= (1ull << (16 * nvalid)) - 1;
            }
            vr[d] = w;
        }
        f32x4 sv = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const f16x8 kf = __builtin_bit_cast(f16x8, kr[ks]);
            sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qa[ks], sv, 0, 0, 0);
            sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qb[ks], sv, 0, 0, 0);
        }
        // scores of token c, keys k0 + 4 quad + e; causal mask
        float s[4], mx = -INFINITY;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            s[e] = k0 + quad * 4 + e <= pos_c ? sv[e] * scale : -INFINITY;
            mx = fmaxf(mx, s[e]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(m, mx);   // finite: key 0 is in every token's range
        const float alpha = expf(m - mnew);
        float p[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] = expf(s[e] - mnew);
        float sum = (p[0] + p[1]) + (p[2] + p[3]);
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        l = l * alpha + sum;
        m = mnew;
        // A operand of p.v: token c, keys 4 quad..; hi and lo parts
        uint16_t ph[4], pl[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) split_f16(p[e], ph[e], pl[e]);
        const f16x4 pa = __builtin_bit_cast(f16x4, ph), pb = __builtin_bit_cast(f16x4, pl);
        // rows of O in this lane: tokens 4 quad + e, whose alpha lane 4 quad + e holds
        float al[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) al[e] = __shfl(alpha, quad * 4 + e, 64);
#pragma unroll
        for (int d = 0; d < DT; ++d) {
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[d][e] *= al[e];
            const f16x4 vf = __builtin_bit_cast(f16x4, vr[d]);
            acc[d] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, vf, acc[d], 0, 0, 0);
            acc[d] = __builtin_amdgcn_mfma_f32_16x16x16f16(pb, vf, acc[d], 0, 0, 0);
        }
    }
    // O[token 4 quad + e][dim d*16 + c] / that token's sum, fp16
    float lr[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) lr[e] = __shfl(l, quad * 4 + e, 64);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int t = tok0 + quad * 4 + e;
        if (t >= T) continue;
        uint16_t* o = out + (size_t)t * ldo + (size_t)h * HD + c;
#pragma unroll
        for (int d = 0; d < DT; ++d) o[d * 16] = f2h(acc[d][e] / lr[e]);
    }
}

}  // namespace
}  // namespace lyk

using namespace lyk;

extern "C" {

int lyk_hip_chunk_rope_kv(const float* d_qkv, int64_t ldq, int T, int pos0, int nq, int nkv, int hd,
                          const float* d_cos, const float* d_sin, int max_pos, float* d_q, uint16_t* d_kcache,
                          uint16_t* d_vcache, const int32_t* d_table, int table_len, int block_tokens,
                          int num_blocks, void* stream) {
    if (!d_qkv || !d_cos || !d_sin || !d_q || !d_kcache || !d_vcache || !d_table) return LYK_ERR_INVALID_ARG;
    if (T < 1 || pos0 < 0 || nq < 1 || nkv < 1 || nq % nkv || hd < 2 || hd % 2 || block_tokens < 1 ||
        num_blocks < 1 || table_len < 1)
        return LYK_ERR_INVALID_ARG;
    if (ldq < (int64_t)(nq + 2 * nkv) * hd || (int64_t)pos0 + T > max_pos ||
        (int64_t)pos0 + T > (int64_t)table_len * block_tokens)
        return LYK_ERR_SHAPE;
    hipLaunchKernelGGL(chunk_rope_kv_kernel, dim3((unsigned)(nq + 2 * nkv), (unsigned)T), dim3(kRopeThreads), 0,
                       static_cast<hipStream_t>(stream), d_qkv, (int)ldq, pos0, nq, nkv, hd, d_cos, d_sin, d_q,
                       d_kcache, d_vcache, d_table, block_tokens, num_blocks);
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

int lyk_hip_chunk_attention(const float* d_q, const uint16_t* d_kcache, const uint16_t* d_vcache,
                            const int32_t* d_table, int table_len, int T, int pos0, int nq, int nkv, int hd,
                            int block_tokens, int num_blocks, uint16_t* d_out, int64_t ldo, void* stream) {
    if (!d_q || !d_kcache || !d_vcache || !d_table || !d_out) return LYK_ERR_INVALID_ARG;
    if (T < 1 || pos0 < 0 || nq < 1 || nkv < 1 || nq % nkv || num_blocks < 1 || table_len < 1)
        return LYK_ERR_INVALID_ARG;
    if ((hd != 64 && hd != 128) || block_tokens % 16 || ldo < (int64_t)nq * hd ||
        (int64_t)pos0 + T > (int64_t)table_len * block_tokens)
        return LYK_ERR_SHAPE;
    const dim3 grid((unsigned)((nq + kAttnWaves - 1) / kAttnWaves), (unsigned)((T + 15) / 16));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (hd == 128)
        hipLaunchKernelGGL(chunk_attention_kernel<128>, grid, dim3(kAttnWaves * 64), 0, st, d_q, T, pos0, nq, nkv,
                           d_kcache, d_vcache, d_table, block_tokens, num_blocks, d_out, (int)ldo);
    else
        hipLaunchKernelGGL(chunk_attention_kernel<64>, grid, dim3(kAttnWaves * 64), 0, st, d_q, T, pos0, nq, nkv,
                           d_kcache, d_vcache, d_table, block_tokens, num_blocks, d_out, (int)ldo);
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

}  // extern "C"
