/*
 * lykuro_hip.h -- the thin C ABI between the C++20 host model
 * (QwenHipModel, engine_amd/csrc/host) and the hand-written gfx950 kernels of
 * the hip backend.
 *
 * The reference engine has no C ABI on this path: its backend seam is the C++
 * class GenerativeModel (model/architectures/generative_model.h:40-105) and
 * its CUDA backend calls kernels from inside one translation unit
 * (backends/cuda/qwen_cuda_model.cu). Each entry point below replaces one
 * kernel family of that file; the citation names what it replaces.
 *
 * Conventions
 *   - Plain pointers and sizes only. Pointers named d_* are device pointers;
 *     `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *   - Every function returns 0 (LYK_OK) or a LYK_ERR_* code; nothing throws.
 *   - No entry point allocates device memory; scratch comes from the caller's
 *     workspace, sized by the matching *_workspace_bytes function and zeroed
 *     by the caller once, before first use. Every kernel returns the part it
 *     used to zero before it exits, so one workspace can serve every call on
 *     a stream; calls that overlap in time need separate workspaces.
 *   - fp16 values are passed as uint16_t bit patterns (IEEE binary16).
 *   - Results are deterministic: fixed-order reductions, no float atomics.
 */
#ifndef LYKURO_HIP_H
#define LYKURO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LYK_ABI_VERSION 1

enum {
    LYK_OK = 0,
    LYK_ERR_INVALID_ARG = 1,  /* null pointer, bad size or stride */
    LYK_ERR_SHAPE = 2,        /* shape outside what the kernel supports */
    LYK_ERR_WORKSPACE = 3,    /* workspace too small */
    LYK_ERR_LAUNCH = 4,       /* kernel launch failed */
    LYK_ERR_HIP = 5,          /* other HIP runtime error */
};

/* Packed weight layouts (defined by this backend; the reference keeps plain
 * row-major weights, qwen_cuda_model.cu:1070-1210).
 *
 * int4 ("q4"): symmetric, groups of 32 along K, one fp16 scale per group.
 *   Rows are cut into tiles of 64 (one row per lane of a wave). For tile t,
 *   group g, lane r the 16 bytes at qw[((t*Gp + g)*64 + r)*16] hold the 32
 *   codes of row 64t+r, k = 32g..32g+31, as nibbles q+8. In each 32-bit word
 *   w (k = 8d..8d+7 for word d) nibble j of the 8 sits at bit
 *   {0,16,4,20,8,24,12,28}[j], so one AND/OR with 0x000F000F / 0x00F000F0
 *   yields two fp16 values 1024+q+8 / 1024+16(q+8). Gp = groups rounded up to
 *   a multiple of 8. Scales: qs[((t*(Gp/8) + c)*64 + r)*8 + j] is the fp16
 *   scale of group 8c+j. Padding codes are q=0 (nibble 8).
 * int8 ("q8"): one fp16 scale per row; tiles of 64 rows; for tile t, block b
 *   of 16 consecutive k, lane r: 16 bytes at qw[((t*Bp + b)*64 + r)*16] hold
 *   the codes q+128 as unsigned bytes in k order. Bp = ceil(K/16) rounded up
 *   to a multiple of 8. Scales: qs[t*64 + r].
 * Paired ("SiLU-gate") packing: two matrices A, B of the same shape share
 *   tiles of 64 rows: rows 0-31 of tile t are A rows 32t.., rows 32-63 are B
 *   rows 32t.. (A = gate_proj, B = up_proj).
 */
#define LYK_TILE_ROWS 64
#define LYK_Q4_GROUP 32
#define LYK_Q8_BLOCK 16

/* Bytes of the packed weights and scales for an [n, k] matrix
 * (paired != 0: two [n, k] matrices packed as pairs). */
int lyk_q4_layout(int64_t n, int64_t k, int paired, uint64_t* weight_bytes,
                  uint64_t* scale_bytes);
int lyk_q8_layout(int64_t n, int64_t k, int paired, uint64_t* weight_bytes,
                  uint64_t* scale_bytes);

/* Host-side load-time quantizers (model/loader step; replaces
 * WeightBuffer::Quantize, qwen_cuda_model.cu:1133-1210, with this backend's
 * format). int4: s = fp16(absmax/7) per 32-group (1.0 for an all-zero group),
 * q = clamp(roundf(w/s), -8, 7); int8: s = fp16(absmax/127) per row,
 * q = clamp(roundf(w/s), -127, 127). codes row-major [n][k]; int4 scales
 * [n][ceil(k/32)], int8 scales [n]. Multithreaded over rows. */
int lyk_q4_quantize(const float* w, int64_t n, int64_t k, int8_t* codes,
                    uint16_t* scales);
int lyk_q8_quantize(const float* w, int64_t n, int64_t k, int8_t* codes,
                    uint16_t* scales);

/* Host-side repack of row-major codes/scales into the device layouts above
 * (into host buffers of the lyk_*_layout sizes; the caller uploads them).
 * b_codes/b_scales are the second matrix of a paired packing, else NULL. */
int lyk_q4_pack(const int8_t* codes, const uint16_t* scales,
                const int8_t* b_codes, const uint16_t* b_scales, int64_t n,
                int64_t k, void* qw, void* qs);
int lyk_q8_pack(const int8_t* codes, const uint16_t* scales,
                const int8_t* b_codes, const uint16_t* b_scales, int64_t n,
                int64_t k, void* qw, void* qs);

/* Tiled layouts of the fused decode step (lyk_hip_decode_step). Same codes,
 * nibble order and scales as above, cut for a chosen tile height tr in
 * {16, 32, 64} so that a matrix of few rows still spreads over every CU
 * without splitting rows across workgroups.
 *   Tile t holds tr rows (paired: rows 0..tr/2-1 from A, tr/2..tr-1 from B,
 *   matrix rows t*tr/2..). Lane l of a block covers tile row l % tr and
 *   sub-block s = l / tr of the block's 64/tr: block b of the tile gives lane
 *   l the 16 bytes of unit u = b*(64/tr) + s of that row, a unit being one
 *   32-code group (q4, same word order as above) or 16 codes (q8, bytes
 *   q+128). Blocks go 4 to a chunk; NB = ceil(units / (64/tr)) valid blocks
 *   per tile, NC = ceil(NB/4) chunks, NBp = 4*NC.
 *   q4 codes: qw[((t*NBp + b)*64 + l)*16], scales fp16
 *     qs[((t*NC + c)*64 + l)*4 + j] = scale of the lane's unit in block 4c+j.
 *   q8 codes: qw[((t*NBp + b)*64 + l)*16], scales qs[t*64 + l] = the fp16 row
 *     scale of the lane's row.
 * Padding (rows past n, units past k) is code 0 with scale 0. */
int lyk_q4_layout_tiled(int64_t n, int64_t k, int paired, int tile_rows,
                        uint64_t* weight_bytes, uint64_t* scale_bytes);
int lyk_q8_layout_tiled(int64_t n, int64_t k, int paired, int tile_rows,
                        uint64_t* weight_bytes, uint64_t* scale_bytes);
int lyk_q4_pack_tiled(const int8_t* codes, const uint16_t* scales,
                      const int8_t* b_codes, const uint16_t* b_scales, int64_t n,
                      int64_t k, int tile_rows, void* qw, void* qs);
int lyk_q8_pack_tiled(const int8_t* codes, const uint16_t* scales,
                      const int8_t* b_codes, const uint16_t* b_scales, int64_t n,
                      int64_t k, int tile_rows, void* qw, void* qs);
/* Host-side inverse of the tiled packing (tests): row-major codes and scales
 * (paired: the 2n rows A then B). */
int lyk_q4_unpack_tiled(const void* qw, const void* qs, int64_t n, int64_t k,
                        int paired, int tile_rows, int8_t* codes, uint16_t* scales);
int lyk_q8_unpack_tiled(const void* qw, const void* qs, int64_t n, int64_t k,
                        int paired, int tile_rows, int8_t* codes, uint16_t* scales);

/* Device-side inverse of the packing (for tests and diagnostics): writes the
 * row-major codes and scales of the matrix (paired: the 2n rows A then B). */
int lyk_hip_q4_unpack(const void* d_qw, const void* d_qs, int64_t n,
                      int64_t k, int paired, int8_t* d_codes,
                      uint16_t* d_scales, void* stream);
int lyk_hip_q8_unpack(const void* d_qw, const void* d_qs, int64_t n,
                      int64_t k, int paired, int8_t* d_codes,
                      uint16_t* d_scales, void* stream);
/* Device dequantization to row-major fp32, w = q * float(s) (exact). */
int lyk_hip_q4_dequant(const void* d_qw, const void* d_qs, int64_t n,
                       int64_t k, int paired, float* d_w, void* stream);
int lyk_hip_q8_dequant(const void* d_qw, const void* d_qs, int64_t n,
                       int64_t k, int paired, float* d_w, void* stream);

/* Weight-only dequant-GEMV, y[m] = W x[m] for m < M (M = 1..4).
 * Replaces MatVecEpi1Kernel / FusedQkv1Kernel / FusedGateUp1Kernel /
 * MatVecBatchKernel / MatVecEpilogueKernel (qwen_cuda_model.cu:533-578,
 * 615-819, 1268-1378) and the CPU MatVec (qwen_model.cpp:21-31).
 *   x: fp16 [M][ldx], ldx >= k rounded up to 32 (q4) or 16 (q8); entries
 *      between k and that bound must be 0.
 *   epilogue (per output row r of batch row m):
 *     LYK_EPI_STORE     y fp32 [M][ldy]: y = Wx (+ bias[r] when bias != NULL)
 *     LYK_EPI_ADD       y fp32 [M][ldy]: y += Wx   (residual add)
 *     LYK_EPI_STORE_F16 y fp16 [M][ldy]: y = fp16(Wx (+ bias))
 *     LYK_EPI_SILU_F16  paired packing; y fp16 [M][ldy]:
 *                       y = fp16(silu(A x) * (B x)), silu(g) = g/(1+exp(-g))
 *   splits: 0 = choose; else the number of waves sharing one row tile's K
 *           range (at most 4 per workgroup; beyond that several workgroups,
 *           whose partials the last to finish adds in a fixed order).
 *   workspace: lyk_hip_gemv_workspace_bytes(n, k, M, splits, paired, q8)
 *              bytes (0 when no split crosses workgroups). */
enum {
    LYK_EPI_STORE = 0,
    LYK_EPI_ADD = 1,
    LYK_EPI_STORE_F16 = 2,
    LYK_EPI_SILU_F16 = 3,
};
uint64_t lyk_hip_gemv_workspace_bytes(int64_t n, int64_t k, int m, int splits,
                                      int paired, int q8);
int lyk_hip_gemv_splits(int64_t n, int64_t k, int m, int paired, int q8);
int lyk_hip_gemv_q4(const void* d_qw, const void* d_qs, int64_t n, int64_t k,
                    const uint16_t* d_x, int64_t ldx, int m, int epilogue,
                    void* d_y, int64_t ldy, const float* d_bias, int splits,
                    void* d_workspace, uint64_t workspace_bytes, void* stream);
int lyk_hip_gemv_q8(const void* d_qw, const void* d_qs, int64_t n, int64_t k,
                    const uint16_t* d_x, int64_t ldx, int m, int epilogue,
                    void* d_y, int64_t ldy, const float* d_bias, int splits,
                    void* d_workspace, uint64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- decode
 * Paged KV cache: per layer, K and V pools of fp16 [num_blocks][nkv][bt][hd]
 * (bt = block_tokens). Token t of batch row m lives in block
 * table[m*table_stride + t/bt], slot t%bt. Positions d_pos[m] are the
 * 0-based position of each row's current token; its context is pos+1. */

/* xn[m] = fp16(h[m] * (1/sqrt(mean(h[m]^2) + eps)) * gamma): RMSNorm
 * (qwen_model.cpp:33-39; NormScaleKernel / RmsNormRowsKernel,
 * qwen_cuda_model.cu:182-201, 591-610, 921-944), output ready for a GEMV. */
int lyk_hip_rmsnorm_f16(const float* d_h, int64_t ldh, const float* d_gamma,
                        float eps, int m, int64_t n, uint16_t* d_xn, int64_t ldx,
                        void* stream);

/* h[m] = table[tokens[m]] (fp32 rows) and xn[m] = RMSNorm(h[m]) as above
 * (qwen_model.cpp:220-221, 235-236; GatherEmbedRowsKernel,
 * qwen_cuda_model.cu:910-919). */
int lyk_hip_embed_rmsnorm(const float* d_table, int64_t vocab,
                          const int32_t* d_tokens, int m, int64_t n, float* d_h,
                          int64_t ldh, const float* d_gamma, float eps,
                          uint16_t* d_xn, int64_t ldx, void* stream);

/* Rotate-half RoPE on the q and k parts of qkv fp32 [m][ldq] ([q | k | v],
 * nq and nkv heads of hd), q written to d_q fp32 [m][nq*hd], rotated k and v
 * appended to the paged caches as fp16 at each row's position. cos/sin are
 * fp32 [max_pos][hd/2] tables of cos(p*theta^(-2i/hd)) as the CPU computes
 * them (qwen_model.cpp:41-54, 239-253; RopeQkKernel + ScatterKv2Kernel,
 * qwen_cuda_model.cu:822-870). Rows whose position or block is out of range
 * are skipped. */
int lyk_hip_rope_kv_append(const float* d_qkv, int64_t ldq, int m, int nq,
                           int nkv, int hd, const int32_t* d_pos,
                           const float* d_cos, const float* d_sin, int max_pos,
                           float* d_q, uint16_t* d_kcache, uint16_t* d_vcache,
                           const int32_t* d_table, int table_stride,
                           int block_tokens, int num_blocks, void* stream);

/* GQA decode attention of each row's query (d_q fp32 [m][nq*hd]) over its
 * pos+1 cached tokens: out fp16 [m][ldo] = softmax(q k^T / sqrt(hd)) v per
 * head, kv head = head / (nq/nkv) (qwen_model.cpp:255-287;
 * BatchSplitAttentionKernel + BatchCombineAttentionKernel,
 * qwen_cuda_model.cu:401-527). Each kv head's context is cut into `splits`
 * ranges handled by separate workgroups and merged in split order. */
uint64_t lyk_hip_attn_workspace_bytes(int m, int nq, int nkv, int hd,
                                      int splits);
int lyk_hip_attn_decode(const float* d_q, const uint16_t* d_kcache,
                        const uint16_t* d_vcache, const int32_t* d_table,
                        int table_stride, const int32_t* d_pos, int m, int nq,
                        int nkv, int hd, int block_tokens, int num_blocks,
                        int splits, uint16_t* d_out, int64_t ldo,
                        void* d_workspace, uint64_t workspace_bytes,
                        void* stream);

/* Greedy token per row: the first index of the maximum logit, NaN never
 * winning (Sampler's greedy rule, sampler.cpp:48-53; ArgmaxStage1/2Kernel,
 * qwen_cuda_model.cu:1388-1458). Writes d_tokens[m]; optionally adds the
 * row's count of non-finite logits to d_nonfinite[m], adds 1 to
 * d_advance[m], and (m == 1 only) appends the token to d_history[*d_step]
 * and increments *d_step -- the on-device chaining of GreedyRun. */
uint64_t lyk_hip_argmax_workspace_bytes(int m, int64_t n);
int lyk_hip_argmax(const float* d_logits, int64_t ldl, int m, int64_t n,
                   int32_t* d_tokens, int32_t* d_nonfinite, int32_t* d_advance,
                   int32_t* d_history, int32_t* d_step, void* d_workspace,
                   uint64_t workspace_bytes, void* stream);

/* Prefill GEMM on the matrix cores over a chunk of T prompt rows: x fp16
 * [T][ldx] (ldx a multiple of 8) times W^T, W in the tiled layout above with
 * tile height tile_rows (q8: int8), fp32 sums whose products are exact (the
 * codes times fp16 x; int4 group scales and int8 row scales applied to the
 * sums). Epilogues, for j < n:
 *   LYK_GEMM_STORE       y fp32 [T][ldy]: y[t][j] = sum (+ d_bias[j])
 *   LYK_GEMM_ADD         y fp32 [T][ldy]: y[t][j] += sum (the residual)
 *   LYK_GEMM_SILU_PAIRS  W paired (gate rows A, up rows B, n each), y fp16
 *                        [T][ldy]: y[t][j] = fp16(SiLU(gate_j) * up_j)
 * Replaces GemmXWtKernel and the epilogue kernels of ForwardChunk
 * (backends/cuda/qwen_cuda_model.cu:878-908, 2398-2516). */
#define LYK_GEMM_STORE 0
#define LYK_GEMM_ADD 1
#define LYK_GEMM_SILU_PAIRS 2
int lyk_hip_gemm_q(const uint16_t* d_x, int64_t ldx, int64_t T, int64_t K,
                   const void* d_qw, const void* d_qs, int64_t n, int tile_rows,
                   int q8, int epilogue, const float* d_bias, void* d_y,
                   int64_t ldy, void* stream);

/* Chunk prefill, RoPE + KV append: T rows of one sequence's raw qkv sums
 * (fp32 [T][ldq], [q | k | v], bias included) at positions pos0 .. pos0+T-1;
 * q rotated into d_q fp32 [T][nq*hd], k rotated and v appended as fp16 to the
 * fused step's paged caches (K [blk][nkv][bt][hd], V [blk][nkv][hd][bt])
 * through d_table (table_len block ids). cos/sin as for
 * lyk_hip_rope_kv_append. Replaces ForwardChunk's RoPE and KV scatter
 * (backends/cuda/qwen_cuda_model.cu:822-870, 2398-2516). */
int lyk_hip_chunk_rope_kv(const float* d_qkv, int64_t ldq, int T, int pos0,
                          int nq, int nkv, int hd, const float* d_cos,
                          const float* d_sin, int max_pos, float* d_q,
                          uint16_t* d_kcache, uint16_t* d_vcache,
                          const int32_t* d_table, int table_len,
                          int block_tokens, int num_blocks, void* stream);
/* Chunk prefill, causal attention: the T queries of d_q (rows at positions
 * pos0..) over the cached keys 0..pos of each, out fp16 [T][ldo] =
 * softmax(q k^T / sqrt(hd)) v per head, kv head = head / (nq/nkv); hd 64 or
 * 128, block_tokens a multiple of 16. Replaces ChunkAttentionKernel
 * (backends/cuda/qwen_cuda_model.cu:981-1030). */
int lyk_hip_chunk_attention(const float* d_q, const uint16_t* d_kcache,
                            const uint16_t* d_vcache, const int32_t* d_table,
                            int table_len, int T, int pos0, int nq, int nkv,
                            int hd, int block_tokens, int num_blocks,
                            uint16_t* d_out, int64_t ldo, void* stream);

/* Temperature / top-k / top-p sampling per row, Sampler::Sample's rule
 * (core/generation/sampler.cpp:35-106; replaces the host sort the engine runs
 * on downloaded logits). temperature 0: the first index of the maximum; else
 * the stable descending order cut to top_k (0 = all), p_i =
 * exp(double(l_i - l_max) * (1.0f / temperature)), the shortest prefix whose
 * running sum of p_i / sum reaches top_p, and the first of it whose running
 * sum reaches u[r] * (its mass). u[r] in [0, 1): the row's draw, one
 * lyk_rng_canonical per non-greedy token. d_tokens[r] = the token, or -1
 * when the row holds a non-finite logit (the reference's kInferenceFailed).
 * m <= 4 rows of ldl floats, one workgroup each. */
uint64_t lyk_hip_sample_workspace_bytes(int m, int64_t n);
int lyk_hip_sample(const float* d_logits, int64_t ldl, int m, int64_t n,
                   float temperature, int32_t top_k, float top_p,
                   const double* u, int32_t* d_tokens, void* d_workspace,
                   uint64_t workspace_bytes, void* stream);
/* lyk_hip_sample without a caller workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The
 * scratch is a file-scope device array of 24 MiB (4 rows of up to 2^18
 * logits), one per GPU the library runs on, held until the process ends;
 * n > 2^18 returns LYK_ERR_SHAPE. Nothing is allocated or freed. Calls that
 * overlap in time on one GPU (different streams, no ordering between them)
 * share that scratch and race; calls on one stream are ordered and do not. */
int lyk_hip_sample_static(const float* d_logits, int64_t ldl, int m, int64_t n,
                          float temperature, int32_t top_k, float top_p,
                          const double* u, int32_t* d_tokens, void* stream);
/* The generator Sampler draws from (sampler.cpp:32-33): std::mt19937_64
 * seeded with the request's seed; lyk_rng_canonical returns the next
 * generate_canonical<double, 53> draw, the u of lyk_hip_sample. */
void* lyk_rng_new(uint64_t seed);
void lyk_rng_free(void* rng);
double lyk_rng_canonical(void* rng);

/* ---------------------------------------------------- fused decode step
 * One decode step of a Qwen2 model (embedding, every layer, final norm, LM
 * head, greedy argmax) as a single persistent cooperative launch of one
 * workgroup per CU; replaces the per-step kernel sequence of
 * QwenCudaModel::Decode / DecodeBatch / GreedyRun
 * (qwen_cuda_model.cu:2641-2776, 2778-3102), whose CPU counterpart is
 * QwenModel::Forward (qwen_model.cpp:216-331). Arithmetic per op is that of
 * the entry points above (same quantized formats, fp16 activations into each
 * GEMV, fp32 residual stream and softmax, fp16 KV cache).
 *
 * Weights: packed as above; qkv is one [(nq+2nkv)*hd, hidden] matrix, rows
 * [q | k | v] (bias the same), gate/up is a paired packing (A = gate,
 * B = up). The layer table is a device array. */
typedef struct lyk_step_layer {
    const void* qkv_w;
    const void* qkv_s;
    const float* qkv_bias;  /* fp32 [(nq+2nkv)*hd] */
    const void* o_w;
    const void* o_s;
    const void* gateup_w;
    const void* gateup_s;
    const void* down_w;
    const void* down_s;
    const float* input_norm;
    const float* post_norm;
    uint16_t* k_cache;      /* fp16 [num_blocks][nkv][block_tokens][hd] */
    uint16_t* v_cache;      /* fp16 [num_blocks][nkv][hd][block_tokens]: V is
                               stored transposed within each block, so runs of
                               consecutive tokens of one dim are contiguous (the
                               operand layout of the p.v matrix product) */
} lyk_step_layer;

typedef struct lyk_step_model {
    int32_t vocab_size, hidden_size, num_layers, num_heads, num_kv_heads, head_dim,
        intermediate_size;
    int32_t q8;              /* 0: int4 weights, 1: int8 weights */
    float rms_norm_eps;
    int32_t block_tokens, num_blocks;  /* block_tokens: a multiple of 16 */
    int32_t rope_positions;  /* rows of the cos/sin tables */
    /* Attention split of a row's context over workgroups: equal splits of
     * whole 16-token tiles, at least attn_split_tokens (a multiple of 16) long,
     * at most attn_max_splits (<= 64) of them; 0 selects the defaults (32, 32). */
    int32_t attn_split_tokens, attn_max_splits;
    /* Tile height (16, 32 or 64) each GEMV matrix was packed with
     * (lyk_q*_pack_tiled), in the order qkv, o, gate/up, down, LM head;
     * lyk_hip_step_tile_rows gives the one this device runs best. */
    int32_t tile_rows[5];
    /* Gate/up chunks per wave staged in LDS while the attention and O phases
     * run: 0 = as many as fit, -1 = none, n > 0 = at most n. */
    int32_t lds_prefetch;
    /* A step's waits for other workgroups' words give up after this many
     * microseconds (0: 2 s); the step then ends with the workspace error
     * word set. Small values force that failure path in tests. */
    uint32_t wait_limit_us;
    const float* embed;      /* fp32 [vocab][hidden] */
    const float* final_norm;
    const void* lm_head_w;
    const void* lm_head_s;
    const lyk_step_layer* layers;  /* device array [num_layers] */
    const float* rope_cos;   /* fp32 [rope_positions][hd/2] */
    const float* rope_sin;
} lyk_step_model;

enum {
    LYK_STEP_HIDDEN = 0,  /* KV append only (prompt tokens before the last) */
    LYK_STEP_LOGITS = 1,  /* + logits of every row */
    LYK_STEP_GREEDY = 2,  /* + on-device greedy token (m == 1) */
};

typedef struct lyk_step_io {
    int32_t m;                    /* batch rows, 1..4 */
    int32_t mode;
    int32_t* tokens;              /* device [m]; GREEDY: replaced by the chosen token */
    int32_t* positions;           /* device [m]; GREEDY: advanced by one */
    const int32_t* block_tables;  /* device [m][table_stride] */
    int32_t table_stride;
    float* logits;                /* device [m][ld_logits] (LOGITS, GREEDY) */
    int64_t ld_logits;
    int32_t* nonfinite;           /* GREEDY, optional: += non-finite logits */
    int32_t* history;             /* GREEDY, optional: history[*step] = token, */
    int32_t* step;                /*   ++*step (the GreedyRun chaining) */
    uint64_t* trace;              /* optional, grid * (4*phases + 2) values:
                                     s_memrealtime ticks (100 MHz) per workgroup
                                     w at [w*(4*phases+2) +]: entry [0], exit
                                     [1]; phase i entered [2+4i], inputs ready
                                     [3+4i], main loop done [4+4i], outputs
                                     written [5+4i] */
} lyk_step_io;

/* Workspace for steps of up to max_rows rows (0 if the geometry is
 * unsupported). Prepare it with lyk_hip_step_reset before the first step;
 * afterwards every step leaves it valid for the next on the same stream. */
uint64_t lyk_hip_step_workspace_bytes(const lyk_step_model* model, int max_rows);
/* Phases one step of `mode` runs (per layer QKV, attention, O, gate/up,
 * down; the LM head; the greedy argmax), and the workgroups of a launch:
 * the trace holds lyk_hip_step_grid() * (4*phases + 2) values. */
uint32_t lyk_hip_step_phases(const lyk_step_model* model, int mode);
int lyk_hip_step_grid(void);
/* Tile height to pack an [n, k] GEMV matrix with for the step on this device
 * (paired: gate/up; q8: int8 weights; normed_input: the matrix reads the
 * RMSNorm of the residual, as QKV, gate/up and the LM head do, so cutting
 * its tiles into K pieces saves no input traffic); 0 on invalid arguments. */
int lyk_hip_step_tile_rows(int64_t n, int64_t k, int paired, int q8, int normed_input);
/* Launches one step (stream-ordered, asynchronous). Positions must be
 * < rope_positions and have their blocks in the tables; the host checks
 * both. The launch arguments are kept in the workspace and uploaded only when
 * they change. A step whose grid could not complete (a wait exceeding ~2 s)
 * sets the workspace's error word and makes later steps exit at once: read it
 * with lyk_hip_step_error and, if set, call lyk_hip_step_reset. */
int lyk_hip_decode_step(const lyk_step_model* model, const lyk_step_io* io,
                        void* d_workspace, uint64_t workspace_bytes, int max_rows,
                        void* stream);
/* Zeroes the workspace (stream-ordered) and forgets its cached arguments. */
int lyk_hip_step_reset(void* d_workspace, uint64_t workspace_bytes, void* stream);
/* Launch tags. Every word one workgroup hands another carries the tag
 * (launches completed + 1) << 8 | layer, 32 bits: distinct and nonzero for
 * 2^24 - 1 launches of one workspace. lyk_hip_decode_step counts the launches
 * it queues on each workspace and zeroes the workspace (stream-ordered) before
 * the launch that would reach that count, so a long-running host never sees
 * a tag repeat. lyk_hip_step_launches returns the count since the last
 * zeroing; lyk_hip_step_set_launches zeroes the workspace and sets every
 * workgroup's counter and the host count to `launches` (<= 2^24 - 1) -- for
 * tests that cross the limit without running 2^24 steps. No counterpart in
 * the reference (its CUDA backend has no cross-workgroup dataflow). */
uint64_t lyk_hip_step_launches(const void* d_workspace);
int lyk_hip_step_set_launches(const lyk_step_model* model, int max_rows, void* d_workspace,
                              uint64_t workspace_bytes, uint64_t launches, void* stream);
/* Copies the error word (0 = no error) to *error_out and waits for it. */
int lyk_hip_step_error(const void* d_workspace, int32_t* error_out, void* stream);
int lyk_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* LYKURO_HIP_H */
