// The engine's model-level backend interface, restated so the hip backend
// compiles on its own; identical in names, signatures and contract to the
// reference seam (model/architectures/generative_model.h:19-105), which the
// engine (core/engine/engine.cpp:378-396, 491-501) and the CLI / HTTP
// generator (cmd/native-engine/generator.cpp:321-384) call.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "core/engine/error.h"

namespace lykuro::nie {

// Per-sequence state (KV cache and backend data), released by destruction.
class SequenceState {
public:
    virtual ~SequenceState() = default;
    virtual uint32_t length() const = 0;
    virtual uint32_t capacity() const = 0;
};

struct ModelLimits {
    uint32_t vocab_size = 0;
    uint32_t max_context_tokens = 0;
    std::vector<uint32_t> eos_token_ids;
};

// Prefix reuse is opt-in per request and scoped by scope_key.
struct SequenceOptions {
    bool allow_prefix_cache = false;
    std::string scope_key;
};

class GenerativeModel {
public:
    virtual ~GenerativeModel() = default;

    virtual const ModelLimits& limits() const = 0;

    virtual Status CreateSequence(uint32_t max_tokens, std::unique_ptr<SequenceState>& out) = 0;

    virtual Status CreateSequenceEx(uint32_t max_tokens, const SequenceOptions&,
                                    std::unique_ptr<SequenceState>& out) {
        return CreateSequence(max_tokens, out);
    }

    // Runs the prompt; returns last-position logits (host fp32). Non-finite
    // logits fail with inference_failed.
    virtual Status Prefill(SequenceState& state, const std::vector<uint32_t>& tokens,
                           std::vector<float>& logits) = 0;

    // Appends one token and returns logits for the next position.
    virtual Status Decode(SequenceState& state, uint32_t token, std::vector<float>& logits) = 0;

    struct DecodeBatchItem {
        SequenceState* state = nullptr;
        uint32_t token = 0;
        std::vector<float>* logits = nullptr;
    };

    // One pass for several sequences. An item's sequence advances only when
    // its per_item status is ok; on a non-ok overall return no sequence
    // advanced.
    virtual Status DecodeBatch(std::vector<DecodeBatchItem>& items, std::vector<Status>& per_item) {
        per_item.resize(items.size());
        for (size_t i = 0; i < items.size(); ++i)
            per_item[i] = Decode(*items[i].state, items[i].token, *items[i].logits);
        return Status::Ok();
    }

    // Optional greedy fast path: up to max_new decode steps inside the
    // backend with the greedy rule (argmax, ties to the lowest index).
    virtual bool SupportsGreedyRun() const { return false; }
    virtual Status GreedyRun(SequenceState& /*state*/, uint32_t /*token*/, uint32_t /*max_new*/,
                             std::vector<uint32_t>& /*out_tokens*/) {
        return Status(ErrorCode::kInternalError, "greedy run unsupported", "model");
    }
};

}  // namespace lykuro::nie
