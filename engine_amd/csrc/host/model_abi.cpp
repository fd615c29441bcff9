// C entry points over QwenHipModel (include/lykuro_hip_model.h).
#include <cmath>
#include <algorithm>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "lykuro_hip_model.h"
#include "qwen_hip_model.h"

using namespace lykuro::nie;

namespace {

struct SeqHandle {
    std::unique_ptr<SequenceState> state;
};

ModelManifest ToManifest(const lyk_model_config& c) {
    ModelManifest m;
    m.schema_version = "1";
    m.model_family = "qwen";
    m.architecture = "approved_qwen_decoder_v1";
    m.weight_format = "safetensors";
    m.vocab_size = c.vocab_size;
    m.hidden_size = c.hidden_size;
    m.num_layers = c.num_layers;
    m.num_attention_heads = c.num_heads;
    m.num_key_value_heads = c.num_kv_heads;
    m.head_dim = c.head_dim;
    m.intermediate_size = c.intermediate_size;
    m.max_context_tokens = c.max_context_tokens;
    m.rms_norm_eps = c.rms_norm_eps;
    m.rope_theta = c.rope_theta;
    m.tie_word_embeddings = c.tie_word_embeddings != 0;
    m.eos_token_ids = {c.eos_token_id};
    return m;
}

HipModelOptions ToOptions(const lyk_model_options* o) {
    HipModelOptions opt;
    if (o == nullptr) return opt;
    opt.device_id = o->device_id;
    opt.kv_pool_tokens = o->kv_pool_tokens;
    if (o->kv_block_tokens) opt.kv_block_tokens = o->kv_block_tokens;
    opt.quantization = o->quant == 1 ? HipWeightQuant::kInt8 : HipWeightQuant::kInt4;
    opt.attn_split_tokens = o->attn_split_tokens;
    opt.attn_max_splits = o->attn_max_splits;
    for (int i = 0; i < 5; ++i) opt.tile_rows[i] = o->tile_rows[i];
    opt.lds_prefetch = o->lds_prefetch;
    opt.prefill_chunk = o->prefill_chunk;
    return opt;
}

int32_t Code(const Status& s) { return int32_t(s.code()); }

void* Finish(QwenHipModel::LoadResult r, int32_t* status) {
    if (status) *status = Code(r.status);
    return r.status.ok() ? r.model.release() : nullptr;
}

QwenHipModel* M(void* p) { return static_cast<QwenHipModel*>(p); }
SequenceState* S(void* p) { return static_cast<SeqHandle*>(p)->state.get(); }

}  // namespace

extern "C" {

void* lyk_model_load_safetensors(const char* path, const lyk_model_config* config,
                                 const lyk_model_options* options, int32_t* status) {
    if (!path || !config) {
        if (status) *status = int32_t(ErrorCode::kInvalidRequest);
        return nullptr;
    }
    SafetensorsFile file;
    Status s = file.Open(path);
    if (!s.ok()) {
        if (status) *status = Code(s);
        return nullptr;
    }
    return Finish(QwenHipModel::Load(ToManifest(*config), file, ToOptions(options)), status);
}

void* lyk_model_load_synthetic(const lyk_model_config* config, uint64_t seed, float sigma,
                               const lyk_model_options* options, int32_t* status) {
    if (!config) {
        if (status) *status = int32_t(ErrorCode::kInvalidRequest);
        return nullptr;
    }
    const size_t tensors = 2 + size_t(config->num_layers) * 12 + (config->tie_word_embeddings ? 0 : 1);
    SyntheticWeightSource src(seed, sigma, tensors);
    return Finish(QwenHipModel::Load(ToManifest(*config), src, ToOptions(options)), status);
}

int32_t lyk_model_read_tensor_f32(const char* path, const char* name, float* out, uint64_t max_count,
                                  uint64_t* count) {
    if (!path || !name) return int32_t(ErrorCode::kInvalidRequest);
    SafetensorsFile file;
    Status s = file.Open(path);
    if (!s.ok()) return Code(s);
    const TensorInfo* info = file.FindTensor(name);
    if (info == nullptr) return int32_t(ErrorCode::kArtifactVerificationFailed);
    std::vector<float> v;
    s = SafetensorsWeightSource(file).Read(name, info->shape, v);
    if (!s.ok()) return Code(s);
    if (count) *count = v.size();
    if (out) std::memcpy(out, v.data(), std::min<uint64_t>(max_count, v.size()) * 4);
    return 0;
}

void lyk_model_free(void* model) { delete M(model); }

void* lyk_model_seq_new(void* model, uint32_t max_tokens, int32_t allow_prefix_cache,
                        const char* scope_key, int32_t* status) {
    auto h = std::make_unique<SeqHandle>();
    SequenceOptions opt;
    opt.allow_prefix_cache = allow_prefix_cache != 0;
    if (scope_key) opt.scope_key = scope_key;
    Status s = M(model)->CreateSequenceEx(max_tokens, opt, h->state);
    if (status) *status = Code(s);
    return s.ok() ? h.release() : nullptr;
}

void lyk_model_seq_free(void* seq) { delete static_cast<SeqHandle*>(seq); }
uint32_t lyk_model_seq_length(const void* seq) {
    return static_cast<const SeqHandle*>(seq)->state->length();
}
uint32_t lyk_model_seq_capacity(const void* seq) {
    return static_cast<const SeqHandle*>(seq)->state->capacity();
}

int32_t lyk_model_prefill(void* model, void* seq, const uint32_t* tokens, size_t n, float* logits_out) {
    std::vector<uint32_t> t(tokens, tokens + n);
    std::vector<float> logits;
    Status s = M(model)->Prefill(*S(seq), t, logits);
    if (!logits.empty() && logits_out) std::memcpy(logits_out, logits.data(), logits.size() * 4);
    return Code(s);
}

int32_t lyk_model_decode(void* model, void* seq, uint32_t token, float* logits_out) {
    std::vector<float> logits;
    Status s = M(model)->Decode(*S(seq), token, logits);
    if (!logits.empty() && logits_out) std::memcpy(logits_out, logits.data(), logits.size() * 4);
    return Code(s);
}

int32_t lyk_model_decode_batch(void* model, void* const* seqs, const uint32_t* tokens, size_t n,
                               float* logits_out, int32_t* per_item) {
    const size_t V = M(model)->limits().vocab_size;
    std::vector<std::vector<float>> logits(n);
    std::vector<GenerativeModel::DecodeBatchItem> items(n);
    for (size_t i = 0; i < n; ++i) items[i] = {S(seqs[i]), tokens[i], &logits[i]};
    std::vector<Status> st;
    Status s = M(model)->DecodeBatch(items, st);
    for (size_t i = 0; i < n; ++i) {
        if (per_item) per_item[i] = i < st.size() ? Code(st[i]) : Code(s);
        if (logits_out && logits[i].size() == V) std::memcpy(logits_out + i * V, logits[i].data(), V * 4);
    }
    return Code(s);
}

int32_t lyk_model_greedy_run(void* model, void* seq, uint32_t token, uint32_t max_new,
                             uint32_t* out_tokens, uint32_t* n_out) {
    std::vector<uint32_t> out;
    Status s = M(model)->GreedyRun(*S(seq), token, max_new, out);
    if (out_tokens) std::memcpy(out_tokens, out.data(), out.size() * 4);
    if (n_out) *n_out = uint32_t(out.size());
    return Code(s);
}

uint32_t lyk_model_kv_blocks_total(const void* model) {
    return static_cast<const QwenHipModel*>(model)->kv_blocks_total();
}
uint32_t lyk_model_kv_blocks_free(const void* model) {
    return static_cast<const QwenHipModel*>(model)->kv_blocks_free();
}
uint64_t lyk_model_prefix_cache_hit_tokens(const void* model) {
    return static_cast<const QwenHipModel*>(model)->prefix_cache_hit_tokens();
}
uint64_t lyk_model_gemv_weight_bytes(const void* model) {
    return static_cast<const QwenHipModel*>(model)->gemv_weight_bytes();
}
void* lyk_model_stream(void* model) { return M(model)->stream(); }
int32_t lyk_model_set_step_tracing(void* model, int32_t on) {
    return Code(M(model)->SetStepTracing(on != 0));
}
void lyk_model_set_wait_limit(void* model, uint32_t microseconds) { M(model)->SetWaitLimit(microseconds); }
uint64_t lyk_model_step_launches(const void* model) {
    return static_cast<const QwenHipModel*>(model)->step_launches();
}
int32_t lyk_model_set_step_launches(void* model, uint64_t launches) {
    return Code(M(model)->SetStepLaunches(launches));
}
size_t lyk_model_step_trace(void* model, uint64_t* out, size_t max) {
    std::vector<uint64_t> t;
    if (!M(model)->StepTrace(t).ok()) return 0;
    const size_t n = std::min(max, t.size());
    if (out) std::memcpy(out, t.data(), n * 8);
    return n;
}

}  // extern "C"
