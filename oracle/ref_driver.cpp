// C entry points around the reference engine's own CPU path, compiled from
// its sources where they lie (oracle/Makefile, target `ref`). TEST
// INFRASTRUCTURE ONLY: the result, oracle/_ref/libqwen_ref.so, is used by
// tests/ to pin the C restatement in qwen_oracle.c and by bench.py as the
// CPU baseline ("kind": "reference"). It is never loaded by the product.
//
// Wraps: QwenModel::Load/CreateSequence/Prefill/Decode
// (model/architectures/qwen/qwen_model.cpp:145-412), SafetensorsFile::Open
// (model/loader/safetensors.cpp:230-284), Sampler::Sample
// (core/generation/sampler.cpp:35-106) and the codecs
// (backends/cpu/cpu_backend.cpp:8-97).

#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "backends/cpu/cpu_backend.h"
#include "core/generation/sampler.h"
#include "model/architectures/qwen/qwen_model.h"
#include "model/loader/safetensors.h"

using namespace lykuro::nie;

namespace {

struct RefModel {
    SafetensorsFile file;
    std::unique_ptr<QwenModel> model;
};

struct RefSeq {
    std::unique_ptr<SequenceState> state;
};

}  // namespace

extern "C" {

float ref_f16_to_f32(uint16_t v) { return Fp16ToFloat(v); }
uint16_t ref_f32_to_f16(float v) { return FloatToFp16(v); }
float ref_bf16_to_f32(uint16_t v) { return Bf16ToFloat(v); }
uint16_t ref_f32_to_bf16(float v) { return FloatToBf16(v); }

// Opens a safetensors file and loads the reference model with a manifest
// built from the given fields. Returns NULL and sets *code on failure.
void* ref_model_load(const char* path, uint32_t vocab, uint32_t hidden,
                     uint32_t layers, uint32_t heads, uint32_t kv_heads,
                     uint32_t head_dim, uint32_t inter, uint32_t max_ctx,
                     double eps, double theta, int tied, uint32_t eos,
                     int32_t* code) {
    auto m = std::make_unique<RefModel>();
    Status s = m->file.Open(path);
    if (!s.ok()) {
        *code = int32_t(s.code());
        return nullptr;
    }
    ModelManifest man;
    man.vocab_size = vocab;
    man.hidden_size = hidden;
    man.num_layers = layers;
    man.num_attention_heads = heads;
    man.num_key_value_heads = kv_heads;
    man.head_dim = head_dim;
    man.intermediate_size = inter;
    man.max_context_tokens = max_ctx;
    man.rms_norm_eps = eps;
    man.rope_theta = theta;
    man.tie_word_embeddings = tied != 0;
    man.eos_token_ids = {eos};
    auto r = QwenModel::Load(man, m->file);
    *code = int32_t(r.status.code());
    if (!r.status.ok()) return nullptr;
    m->model = std::move(r.model);
    return m.release();
}

void ref_model_free(void* m) { delete static_cast<RefModel*>(m); }

void* ref_seq_new(void* m, uint32_t max_tokens) {
    auto* rm = static_cast<RefModel*>(m);
    auto s = std::make_unique<RefSeq>();
    if (!rm->model->CreateSequence(max_tokens, s->state).ok()) return nullptr;
    return s.release();
}

void ref_seq_free(void* s) { delete static_cast<RefSeq*>(s); }

int32_t ref_prefill(void* m, void* s, const uint32_t* tokens, size_t n,
                    float* logits_out) {
    auto* rm = static_cast<RefModel*>(m);
    std::vector<uint32_t> toks(tokens, tokens + n);
    std::vector<float> logits;
    Status st =
        rm->model->Prefill(*static_cast<RefSeq*>(s)->state, toks, logits);
    if (st.ok()) std::memcpy(logits_out, logits.data(), logits.size() * 4);
    return int32_t(st.code());
}

int32_t ref_decode(void* m, void* s, uint32_t token, float* logits_out) {
    auto* rm = static_cast<RefModel*>(m);
    std::vector<float> logits;
    Status st =
        rm->model->Decode(*static_cast<RefSeq*>(s)->state, token, logits);
    if (st.ok()) std::memcpy(logits_out, logits.data(), logits.size() * 4);
    return int32_t(st.code());
}

void* ref_sampler_new(float temperature, float top_p, uint32_t top_k,
                      uint64_t seed) {
    SamplingParams p;
    p.temperature = temperature;
    p.top_p = top_p;
    p.top_k = top_k;
    p.seed = seed;
    return new Sampler(p);
}

void ref_sampler_free(void* s) { delete static_cast<Sampler*>(s); }

int32_t ref_sample(void* s, const float* logits, size_t n, uint32_t* out) {
    std::vector<float> l(logits, logits + n);
    return int32_t(static_cast<Sampler*>(s)->Sample(l, *out).code());
}

}  // extern "C"
