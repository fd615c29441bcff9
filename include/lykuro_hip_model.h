/*
 * lykuro_hip_model.h -- C entry points over QwenHipModel, the hip backend's
 * implementation of the engine's GenerativeModel interface
 * (model/architectures/generative_model.h:40-105).
 *
 * The engine itself links the C++ class (engine_amd/csrc/host/
 * qwen_hip_model.h); these functions expose the same operations with plain
 * pointers for callers that bind C (ctypes in the tests and bench, or any
 * FFI). Status returns are the numeric values of the engine's ErrorCode enum
 * (core/engine/error.h:12-43): 0 ok, 1 invalid_request, 4 unsupported_model,
 * 5 artifact_verification_failed, 6 context_length_exceeded,
 * 8 capacity_exhausted, 13 gpu_oom, 14 gpu_unhealthy, 15 inference_failed,
 * 17 internal_error.
 */
#ifndef LYKURO_HIP_MODEL_H
#define LYKURO_HIP_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Architecture fields of the model manifest (model/manifest/manifest.h:21-45). */
typedef struct lyk_model_config {
    uint32_t vocab_size, hidden_size, num_layers, num_heads, num_kv_heads, head_dim,
        intermediate_size, max_context_tokens;
    double rms_norm_eps, rope_theta;
    int32_t tie_word_embeddings;
    uint32_t eos_token_id;
} lyk_model_config;

/* HipModelOptions: quant 0 = int4 (groups of 32, fp16 scales), 1 = int8
 * (per row, fp16 scales); kv_pool_tokens 0 = 4x max context. */
typedef struct lyk_model_options {
    int32_t device_id;
    uint32_t kv_pool_tokens;
    uint32_t kv_block_tokens;  /* a multiple of 16 */
    int32_t quant;
    /* attention context split (lyk_step_model fields of the same names);
     * 0 selects the defaults */
    int32_t attn_split_tokens, attn_max_splits;
    /* GEMV tile heights (16/32/64) for qkv, o, gate/up, down, LM head;
     * 0 = lyk_hip_step_tile_rows' choice for this device */
    int32_t tile_rows[5];
    /* gate/up chunks per wave staged in LDS during attention: 0 = as many
     * as fit (the default), -1 = none, n > 0 = at most n */
    int32_t lds_prefetch;
    /* prompt rows per prefill chunk pass on the matrix cores: 0 = 2048 (the
     * default), -1 = none (every prompt token through the fused decode step),
     * n > 0 = n rows */
    int32_t prefill_chunk;
} lyk_model_options;

/* QwenHipModel::Load from a safetensors file (replaces QwenCudaModel::Load,
 * backends/cuda/qwen_cuda_model.h:51-55). NULL on failure, *status set. */
void* lyk_model_load_safetensors(const char* path, const lyk_model_config* config,
                                 const lyk_model_options* options, int32_t* status);
/* Load from the seeded synthetic source: every weight N(0, sigma^2) from
 * lyk_synth_normal(seed, kind*1000 + layer, ...), norms 1.0. */
void* lyk_model_load_synthetic(const lyk_model_config* config, uint64_t seed, float sigma,
                               const lyk_model_options* options, int32_t* status);
void lyk_model_free(void* model);
/* The loader's view of one tensor, without a device: opens the file with the
 * reader's checks (model/loader/safetensors.cpp:160-297: regular file, no
 * symlink, header bounds, dtype allow-list, rank <= 8, offsets tiling the
 * data) and widens F16/BF16 to fp32 as the loader does
 * (backends/cpu/cpu_backend.cpp:8-50). Writes min(max_count, elements)
 * floats to out and the element count to *count; returns the ErrorCode
 * value. */
int32_t lyk_model_read_tensor_f32(const char* path, const char* name, float* out, uint64_t max_count,
                                  uint64_t* count);

/* CreateSequence / CreateSequenceEx (generative_model.h:47-56). */
void* lyk_model_seq_new(void* model, uint32_t max_tokens, int32_t allow_prefix_cache,
                        const char* scope_key, int32_t* status);
void lyk_model_seq_free(void* seq);
uint32_t lyk_model_seq_length(const void* seq);
uint32_t lyk_model_seq_capacity(const void* seq);

/* Prefill / Decode (generative_model.h:60-66); logits_out has vocab_size
 * floats and is written when the call returns 0 or 15 (non-finite). */
int32_t lyk_model_prefill(void* model, void* seq, const uint32_t* tokens, size_t n,
                          float* logits_out);
int32_t lyk_model_decode(void* model, void* seq, uint32_t token, float* logits_out);
/* DecodeBatch (generative_model.h:68-87): logits_out [n][vocab_size],
 * per_item [n] statuses; the return is the overall status. */
int32_t lyk_model_decode_batch(void* model, void* const* seqs, const uint32_t* tokens, size_t n,
                               float* logits_out, int32_t* per_item);
/* GreedyRun (generative_model.h:98-104): up to max_new tokens into
 * out_tokens, *n_out set to the count produced. */
int32_t lyk_model_greedy_run(void* model, void* seq, uint32_t token, uint32_t max_new,
                             uint32_t* out_tokens, uint32_t* n_out);

uint32_t lyk_model_kv_blocks_total(const void* model);
uint32_t lyk_model_kv_blocks_free(const void* model);
uint64_t lyk_model_prefix_cache_hit_tokens(const void* model);
/* Bytes of packed GEMV weights (+ scales) streamed per decode token. */
uint64_t lyk_model_gemv_weight_bytes(const void* model);
/* Profiling: record the phase timeline of every step (lyk_step_io::trace);
 * lyk_model_step_trace copies that of the latest step (up to max values,
 * returns the count; 0 when tracing is off). */
int32_t lyk_model_set_step_tracing(void* model, int32_t on);
/* The hipStream_t (as void*) every device operation of the model runs on,
 * for callers that time it with events. */
void* lyk_model_stream(void* model);
size_t lyk_model_step_trace(void* model, uint64_t* out, size_t max);
/* Launch-tag epoch of the model's fused step (lyk_hip_step_launches /
 * lyk_hip_step_set_launches): launches since the workspace was last zeroed,
 * and a preset of that count for tests that cross the 2^24 - 1 limit. No
 * counterpart in the reference. */
uint64_t lyk_model_step_launches(const void* model);
/* Limit of the fused step's waits for other workgroups, in microseconds
 * (0: 2 s, the default). A step that exceeds it ends unfinished: the call
 * returns gpu_unhealthy (14), no sequence advances, and the next call runs
 * on a reset workspace. Small values exercise that path in tests. No
 * counterpart in the reference. */
void lyk_model_set_wait_limit(void* model, uint32_t microseconds);
int32_t lyk_model_set_step_launches(void* model, uint64_t launches);

/* Seeded N(0, sigma^2) stream: value i of stream `stream` depends only on
 * (seed, stream, i); Box-Muller on splitmix64 outputs. */
void lyk_synth_normal(uint64_t seed, uint64_t stream, uint64_t first, uint64_t count, float sigma,
                      float* out);

#ifdef __cplusplus
}
#endif

#endif /* LYKURO_HIP_MODEL_H */
