/*
 * CPU oracle for the Qwen2 decode path -- TEST INFRASTRUCTURE ONLY.
 *
 * This library restates, in plain C, the arithmetic of the reference engine's
 * CPU path so that the HIP backend can be checked against it. Nothing in the
 * product (engine_amd/) may link, load or call it; only tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py use it, and
 * only as the checker.
 *
 * What each part follows (paths relative to the reference tree):
 *   codecs         backends/cpu/cpu_backend.cpp:8-97
 *   MatVec         model/architectures/qwen/qwen_model.cpp:21-31
 *   RmsNorm        model/architectures/qwen/qwen_model.cpp:33-39
 *   ApplyRope      model/architectures/qwen/qwen_model.cpp:41-54
 *   ForwardToken   model/architectures/qwen/qwen_model.cpp:212-308
 *   Logits/finite  model/architectures/qwen/qwen_model.cpp:310-331
 *   Prefill/Decode model/architectures/qwen/qwen_model.cpp:333-360,398-412
 *   Sampler        core/generation/sampler.cpp:35-106 (mt19937_64 and
 *                  libstdc++'s uniform_real_distribution<double> restated)
 *   tiny weights   tests/testutil/tiny_model.cpp:14-24,52-116
 *   quantizers     rule of backends/cuda/qwen_cuda_model.cu:1136-1210 with
 *                  the build's format: int4 groups of 32 along K with fp16
 *                  scales, int8 per output row with fp16 scales.
 *
 * How each part is pinned (tests/test_oracle_*.py):
 *   codecs      dtype_test.cpp KATs + exhaustive 2^16 fp16/bf16 round trips
 *               + bit equality with the compiled reference (oracle/_ref)
 *   forward     golden_test.cpp:142-196 pinned logits and greedy sequences;
 *               bit equality with oracle/_ref on tiny and mid-size models
 *   sampler     sampler_test.cpp cases; token equality with oracle/_ref over
 *               many seeds; mt19937_64's published 10000th output
 *   quantizers  closed-form properties (|q|<=7 or 127, exact dequant,
 *               error <= s/2, absmax element maps to +-7/127) and brute force
 *               on small tiles
 *   normal gen  moments over 10^6 draws and bit equality with the product's
 *               generator
 */
#ifndef LYKURO_QWEN_ORACLE_H
#define LYKURO_QWEN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes: the numeric values of the reference's ErrorCode enum
 * (core/engine/error.h:12-43). */
enum {
    ORC_OK = 0,
    ORC_INVALID_REQUEST = 1,
    ORC_ARTIFACT_VERIFICATION_FAILED = 5,
    ORC_CONTEXT_LENGTH_EXCEEDED = 6,
    ORC_CAPACITY_EXHAUSTED = 8,
    ORC_INFERENCE_FAILED = 15,
    ORC_INTERNAL_ERROR = 17,
};

/* ---- codecs (cpu_backend.cpp:8-97) ---- */
float orc_bf16_to_f32(uint16_t v);
uint16_t orc_f32_to_bf16(float v);
float orc_f16_to_f32(uint16_t v);
uint16_t orc_f32_to_f16(float v);
void orc_f16_to_f32_array(const uint16_t* in, float* out, size_t n);
void orc_f32_to_f16_array(const float* in, uint16_t* out, size_t n);

/* ---- quantizers (format defined by this build) ----
 * int4: groups of 32 along K; scale s = fp16(absmax/7) (1.0 when the group is
 * all zero); q = clamp(roundf(w / s), -8, 7). The last group of a row may be
 * partial when K % 32 != 0. codes are one int8 per weight, row-major [N][K];
 * scales are fp16 bits, row-major [N][ceil(K/32)].
 * int8: one scale per output row, s = fp16(absmax/127); q = clamp(round, +-127).
 * Dequantization is q * float(s), exact in fp32. */
void orc_q4_quantize(const float* w, int64_t n, int64_t k, int8_t* codes,
                     uint16_t* scales);
void orc_q4_dequantize(const int8_t* codes, const uint16_t* scales, int64_t n,
                       int64_t k, float* w);
void orc_q8_quantize(const float* w, int64_t n, int64_t k, int8_t* codes,
                     uint16_t* scales);
void orc_q8_dequantize(const int8_t* codes, const uint16_t* scales, int64_t n,
                       int64_t k, float* w);
uint16_t orc_quant_scale_f16(float absmax, float qmax);

/* ---- primitives (qwen_model.cpp:21-54) ---- */
void orc_matvec(const float* w, const float* bias, const float* x,
                int64_t in_dim, int64_t out_dim, float* out);
/* Same per-row order, rows split over `threads` threads: bit-identical. */
void orc_matvec_mt(const float* w, const float* bias, const float* x,
                   int64_t in_dim, int64_t out_dim, float* out, int threads);
void orc_rmsnorm(const float* x, const float* weight, float eps, int64_t dim,
                 float* out);
void orc_rope(float* vec, uint32_t head_dim, uint32_t pos, float theta);
/* Decode attention of one query token over `context` cached positions, GQA.
 * q [heads*hd], keys/values [context][kv_heads*hd]; out [heads*hd]. */
void orc_attention(const float* q, const float* keys, const float* values,
                   uint32_t context, uint32_t heads, uint32_t kv_heads,
                   uint32_t head_dim, float* out);
/* Same, query heads split over `threads` threads: bit-identical. */
void orc_attention_mt(const float* q, const float* keys, const float* values,
                      uint32_t context, uint32_t heads, uint32_t kv_heads,
                      uint32_t head_dim, float* out, int threads);

/* ---- model (qwen_model.cpp:88-412) ---- */
typedef struct orc_config {
    uint32_t vocab_size, hidden_size, num_layers, num_heads, num_kv_heads,
        head_dim, intermediate_size, max_context_tokens;
    float rms_norm_eps, rope_theta;
    int32_t tie_word_embeddings;
} orc_config;

/* Tensor kinds, one per reference weight name (qwen_model.cpp:170-198). */
enum {
    ORC_T_EMBED = 0,      /* model.embed_tokens.weight [V,H] */
    ORC_T_INPUT_NORM,     /* layers.l.input_layernorm.weight [H] */
    ORC_T_Q_W,            /* self_attn.q_proj.weight [q_dim,H] */
    ORC_T_Q_B,
    ORC_T_K_W,
    ORC_T_K_B,
    ORC_T_V_W,
    ORC_T_V_B,
    ORC_T_O_W,            /* [H,q_dim] */
    ORC_T_POST_NORM,
    ORC_T_GATE_W,         /* [I,H] */
    ORC_T_UP_W,
    ORC_T_DOWN_W,         /* [H,I] */
    ORC_T_FINAL_NORM,     /* model.norm.weight [H] */
    ORC_T_LM_HEAD,        /* lm_head.weight [V,H], absent when tied */
    ORC_T_COUNT
};

typedef struct orc_model orc_model;
typedef struct orc_seq orc_seq;

orc_model* orc_model_new(const orc_config* c);
void orc_model_free(orc_model* m);
/* Pointer to the (zero-initialised, model-owned) fp32 storage of a tensor, or
 * NULL for a kind that does not exist (lm_head when tied). `layer` is ignored
 * for model-level tensors. */
float* orc_model_tensor(orc_model* m, int kind, uint32_t layer);
uint64_t orc_model_tensor_numel(const orc_model* m, int kind);
/* Worker threads for the matvecs and attention heads (results are identical
 * for any count). */
void orc_model_set_threads(orc_model* m, int threads);
/* fp16 mirror mode, a test bar rather than the reference: the forward above
 * with five values rounded to fp16 (RNE, orc_f32_to_f16) where the HIP decode
 * path stores them in fp16 -- the RMSNorm output feeding each matvec (QKV,
 * gate/up, LM head), the RoPE-rotated key and the value written to the cache,
 * the attention output feeding o_proj, and SiLU(gate)*up feeding down_proj.
 * Everything else is the reference's fp32 arithmetic, unchanged. Pinned by
 * tests/test_oracle.py against a composition of the pinned primitives with
 * the pinned codec at exactly those points. */
void orc_model_set_f16_mirror(orc_model* m, int on);
/* Noise-floor mode, also not the reference: the forward's matvecs add their
 * products in descending index order (bias first, as the reference does).
 * Comparing a run with its ascending twin measures how far the result moves
 * under a change of fp32 summation order alone -- the floor any other
 * correct implementation (a GPU's tree of partial sums) can be held to.
 * Pinned like the mirror mode, against the primitives on reversed inputs. */
void orc_model_set_descending_sums(orc_model* m, int on);

orc_seq* orc_seq_new(const orc_model* m, uint32_t max_tokens);
void orc_seq_free(orc_seq* s);
uint32_t orc_seq_length(const orc_seq* s);
int orc_prefill(const orc_model* m, orc_seq* s, const uint32_t* tokens,
                size_t n, float* logits);
int orc_decode(const orc_model* m, orc_seq* s, uint32_t token, float* logits);
/* Final hidden state of the last forward (before the final norm). */
const float* orc_seq_hidden(const orc_seq* s);

/* Tiny deterministic model of tests/testutil/tiny_model.cpp: LCG weights in
 * lexicographic tensor-name order, norms = 1.0, tied embeddings. */
void orc_fill_tiny_weights(orc_model* m, uint64_t seed);

/* ---- sampler (sampler.cpp:35-106) ---- */
typedef struct orc_sampler orc_sampler;
orc_sampler* orc_sampler_new(float temperature, float top_p, uint32_t top_k,
                             uint64_t seed);
void orc_sampler_free(orc_sampler* s);
int orc_sample(orc_sampler* s, const float* logits, size_t n, uint32_t* out);
/* Greedy rule alone: first index of the maximum. */
uint32_t orc_argmax(const float* logits, size_t n);

/* mt19937_64 (Matsumoto & Nishimura) and libstdc++'s canonical double. */
typedef struct orc_mt64 {
    uint64_t mt[312];
    int idx;
} orc_mt64;
void orc_mt64_seed(orc_mt64* g, uint64_t seed);
uint64_t orc_mt64_next(orc_mt64* g);
double orc_mt64_canonical(orc_mt64* g);

/* ---- synthetic weights ----
 * Seeded N(0, sigma^2) stream; value i of stream `stream_id` depends only on
 * (seed, stream_id, i). Restates the product generator (engine_amd host
 * library, lyk_synth_normal) so that both sides build identical weights. */
void orc_synth_normal(uint64_t seed, uint64_t stream_id, uint64_t first,
                      uint64_t count, float sigma, float* out);
/* Uniform integers in [0, n) for prompts, same construction. */
void orc_synth_tokens(uint64_t seed, uint64_t stream_id, uint64_t count,
                      uint32_t n, uint32_t* out);

#ifdef __cplusplus
}
#endif

#endif
