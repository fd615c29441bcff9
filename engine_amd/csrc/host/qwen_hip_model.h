// QwenHipModel: the MI355X `hip` backend of the Lykuro engine.
//
// Implements the engine's GenerativeModel interface
// (model/architectures/generative_model.h:40-105) for the
// approved_qwen_decoder_v1 architecture, with the same factory convention,
// error codes and ownership rules as the CUDA backend
// (backends/cuda/qwen_cuda_model.h:42-106), so `--backend hip` can be wired
// into the engine, CLI and servers without touching them.
//
// Weights are quantized at load (int4 in groups of 32 with fp16 scales, or
// int8 per output row with fp16 scales) and repacked into the tile layouts
// of include/lykuro_hip.h; GEMV inputs are fp16, the residual stream and
// logits fp32, the paged KV cache fp16. Each decode step (one token of up to
// four sequences) is one launch of the fused gfx950 step kernel behind the C
// ABI (lyk_hip_decode_step).
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "core/engine/error.h"
#include "model/architectures/generative_model.h"
#include "model/loader/safetensors.h"
#include "model/manifest/manifest.h"

namespace lykuro::nie {

enum class HipWeightQuant {
    kInt4,  // symmetric, groups of 32 along K, fp16 scale per group
    kInt8,  // symmetric, one fp16 scale per output row
};

struct HipModelOptions {
    int device_id = 0;
    // Total KV pool capacity in tokens (0 = 4x max context) and the paged
    // block granularity.
    uint32_t kv_pool_tokens = 0;
    uint32_t kv_block_tokens = 16;
    HipWeightQuant quantization = HipWeightQuant::kInt4;
    // Attention context split over workgroups (tokens per split at least, a
    // multiple of 16; splits at most, <= 32); 0 = the kernel's defaults.
    int attn_split_tokens = 0;
    int attn_max_splits = 0;
    // GEMV tile heights (16/32/64) for qkv, o, gate/up, down, LM head;
    // 0 = the device's choice (lyk_hip_step_tile_rows).
    int tile_rows[5] = {0, 0, 0, 0, 0};
    // Gate/up chunks per wave staged in LDS ahead of the gate/up phase:
    // 0 = as many as fit, -1 = none, n > 0 = at most n.
    int lds_prefetch = 0;
    // Prompt rows per prefill chunk pass (GEMMs on the matrix cores, causal
    // chunk attention): 0 = 2048, -1 = none (every prompt token through the
    // fused decode step), n > 0 = n rows.
    int prefill_chunk = 0;
};

// fp32 weights by reference tensor name. The safetensors file is one source;
// a seeded synthetic generator is another (benchmarks without checkpoints).
class WeightSource {
public:
    virtual ~WeightSource() = default;
    // Fills `out` with the tensor as fp32, or fails when it is missing or its
    // shape differs from `shape`.
    virtual Status Read(const std::string& name, const std::vector<uint64_t>& shape,
                        std::vector<float>& out) const = 0;
    // Number of tensors the source holds (the loader rejects extras).
    virtual size_t tensor_count() const = 0;
    // An offline-quantized [n, k] matrix stored as `base`.qweight and
    // `base`.qscale (the loader's own codes and fp16 scales: int4 groups of
    // 32, int8 per row); found = false when the source holds none.
    virtual Status ReadQuantized(const std::string& base, bool q8, int64_t n, int64_t k,
                                 std::vector<int8_t>& codes, std::vector<uint16_t>& scales, bool& found) const {
        (void)base, (void)q8, (void)n, (void)k, (void)codes, (void)scales;
        found = false;
        return Status::Ok();
    }
};

// A safetensors file as a weight source (F32 / F16 / BF16, widened to fp32
// with the reference's codecs).
class SafetensorsWeightSource final : public WeightSource {
public:
    explicit SafetensorsWeightSource(const SafetensorsFile& file) : file_(file) {}
    Status Read(const std::string& name, const std::vector<uint64_t>& shape,
                std::vector<float>& out) const override;
    size_t tensor_count() const override { return file_.header().tensors.size(); }
    Status ReadQuantized(const std::string& base, bool q8, int64_t n, int64_t k, std::vector<int8_t>& codes,
                         std::vector<uint16_t>& scales, bool& found) const override;

private:
    const SafetensorsFile& file_;
};

// Seeded N(0, sigma^2) weights (norms 1.0): value i of tensor (kind, layer)
// is element i of stream kind*1000+layer of the generator lyk_synth_normal.
class SyntheticWeightSource final : public WeightSource {
public:
    SyntheticWeightSource(uint64_t seed, float sigma, size_t tensors)
        : seed_(seed), sigma_(sigma), tensors_(tensors) {}
    Status Read(const std::string& name, const std::vector<uint64_t>& shape,
                std::vector<float>& out) const override;
    size_t tensor_count() const override { return tensors_; }

private:
    uint64_t seed_;
    float sigma_;
    size_t tensors_;
};

// Architecture parameters, derived and validated as QwenConfig::FromManifest
// does (model/architectures/qwen/qwen_model.cpp:88-124).
struct HipQwenConfig {
    uint32_t vocab_size = 0, hidden_size = 0, num_layers = 0, num_heads = 0, num_kv_heads = 0,
             head_dim = 0, intermediate_size = 0, max_context_tokens = 0;
    float rms_norm_eps = 1e-6f;
    float rope_theta = 10000.0f;
    bool tie_word_embeddings = false;
    std::vector<uint32_t> eos_token_ids;

    static Status FromManifest(const ModelManifest& manifest, HipQwenConfig& out);
};

class QwenHipModel : public GenerativeModel {
public:
    struct LoadResult {
        Status status;
        std::unique_ptr<QwenHipModel> model;
    };

    // Quantizes, repacks and uploads the verified weights to `device_id`.
    // Fails (unsupported_model / gpu_oom / gpu_unhealthy /
    // artifact_verification_failed) without partial residency.
    static LoadResult Load(const ModelManifest& manifest, const SafetensorsFile& weights,
                           const HipModelOptions& options);
    static LoadResult Load(const ModelManifest& manifest, const WeightSource& weights,
                           const HipModelOptions& options);

    ~QwenHipModel() override;
    QwenHipModel(const QwenHipModel&) = delete;
    QwenHipModel& operator=(const QwenHipModel&) = delete;

    const ModelLimits& limits() const override { return limits_; }
    Status CreateSequence(uint32_t max_tokens, std::unique_ptr<SequenceState>& out) override;
    Status CreateSequenceEx(uint32_t max_tokens, const SequenceOptions& options,
                            std::unique_ptr<SequenceState>& out) override;
    Status Prefill(SequenceState& state, const std::vector<uint32_t>& tokens,
                   std::vector<float>& logits) override;
    Status Decode(SequenceState& state, uint32_t token, std::vector<float>& logits) override;
    Status DecodeBatch(std::vector<DecodeBatchItem>& items, std::vector<Status>& per_item) override;
    bool SupportsGreedyRun() const override { return true; }
    Status GreedyRun(SequenceState& state, uint32_t token, uint32_t max_new,
                     std::vector<uint32_t>& out_tokens) override;

    const HipQwenConfig& config() const { return config_; }

    // Paged-KV / prefix-cache introspection (tests, capacity metrics).
    uint32_t kv_blocks_total() const;
    uint32_t kv_blocks_free() const;
    uint64_t prefix_cache_hit_tokens() const;
    // Bytes of quantized GEMV weights streamed per decode token.
    uint64_t gemv_weight_bytes() const;
    // Phase timeline of the fused step (profiling): when on, every step
    // records device timestamps (see lyk_step_io::trace); StepTrace returns
    // those of the most recent step.
    Status SetStepTracing(bool on);
    // The HIP stream (hipStream_t) all device work of the model runs on.
    void* stream() const;
    Status StepTrace(std::vector<uint64_t>& ticks);
    // Launches of the fused step since its workspace was last zeroed, and a
    // way to preset that count (tests of the launch-tag epoch; see
    // lyk_hip_step_set_launches).
    uint64_t step_launches() const;
    Status SetStepLaunches(uint64_t launches);
    // Limit of a step's waits for other workgroups (microseconds, 0 = 2 s);
    // past it the step ends unfinished and the call reports kGpuUnhealthy.
    void SetWaitLimit(uint32_t microseconds);

    struct Impl;

private:
    QwenHipModel() = default;

    HipQwenConfig config_;
    ModelLimits limits_;
    int device_id_ = 0;
    std::unique_ptr<Impl> impl_;
};

}  // namespace lykuro::nie
