// The validated model manifest, restated with the reference's field names
// (model/manifest/manifest.h:15-54) so the hip backend's Load takes the same
// argument the engine passes to every backend.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace lykuro::nie {

struct ManifestFile {
    std::string path;
    std::string sha256;
    uint64_t size_bytes = 0;
};

struct ModelManifest {
    std::string schema_version;
    std::string artifact_id;
    std::string model_family;
    std::string architecture;
    std::string model_version;
    std::string weight_format;
    std::string precision;
    uint32_t vocab_size = 0;
    uint32_t hidden_size = 0;
    uint32_t num_layers = 0;
    uint32_t num_attention_heads = 0;
    uint32_t num_key_value_heads = 0;
    uint32_t head_dim = 0;
    uint32_t max_context_tokens = 0;
    uint32_t intermediate_size = 0;
    double rms_norm_eps = 0.0;
    double rope_theta = 0.0;
    bool tie_word_embeddings = false;
    std::vector<uint32_t> eos_token_ids;
    std::string tokenizer_type;
    std::string chat_template_id;
    std::vector<ManifestFile> files;
    std::string license_review_id;
    std::vector<std::string> certified_profiles;
    std::string created_at;
};

}  // namespace lykuro::nie
