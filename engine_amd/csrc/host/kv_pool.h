// Paged KV block pool of the hip backend (host side).
//
// Behaviour follows the reference engine's CUDA backend pool and prefix
// cache (backends/cuda/qwen_cuda_model.cu:1637-1749, 2545-2608): block ids
// index every layer's K/V pool; sequences take blocks on demand and give
// them back when destroyed; a prompt's full blocks can be published under a
// chain key seeded with the request's scope key, stay resident after their
// last user lets go, and are reclaimed least-recently-released first when no
// free block is left.
//
// Design: every block has a reference count. Blocks no one references are
// either on the free stack (never published) or on an intrusive
// doubly-linked list of reclaimable published blocks, ordered by release
// time, so taking a block, looking one up and letting one go are O(1).
#pragma once

#include <cstdint>
#include <optional>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace lykuro::nie::hip {

class KvBlockPool {
public:
    KvBlockPool(uint32_t num_blocks, uint32_t block_tokens);

    uint32_t block_tokens() const { return block_tokens_; }
    uint32_t num_blocks() const { return uint32_t(slots_.size()); }
    // Blocks a sequence could take now: free plus reclaimable published ones.
    uint32_t available() const { return uint32_t(free_.size()) + reclaimable_; }

    // A block with one reference: a free one, else the published block
    // released longest ago (which leaves the cache). nullopt when every
    // block is referenced.
    std::optional<int32_t> Take();
    // One reference fewer; at zero the block becomes free, or reclaimable
    // when published.
    void Drop(int32_t block);
    // The block published under `key`, with one more reference.
    std::optional<int32_t> Find(uint64_t key);
    // Publishes a referenced block under `key`. The first block published
    // under a key keeps it; a block is published at most once.
    void Publish(uint64_t key, int32_t block);

private:
    static constexpr int32_t kNone = -1;
    struct Slot {
        uint32_t refs = 0;
        bool published = false;
        uint64_t key = 0;
        int32_t prev = kNone, next = kNone;   // reclaimable list links
    };
    void Unlink(int32_t b);
    void Append(int32_t b);

    uint32_t block_tokens_;
    std::vector<Slot> slots_;
    std::vector<int32_t> free_;                  // stack of never-published free blocks
    int32_t oldest_ = kNone, newest_ = kNone;    // reclaimable list ends
    uint32_t reclaimable_ = 0;
    std::unordered_map<uint64_t, int32_t> by_key_;
};

// Chain keys of a prompt's full blocks: key b covers tokens [0, (b+1)*bt) and
// the scope key, so equal prefixes in different scopes never share blocks.
// FNV-1a (64-bit) over the scope key's bytes, then each block's token ids as
// 32-bit little-endian values, continuing the same state.
std::vector<uint64_t> PrefixChainKeys(std::string_view scope, const uint32_t* tokens, size_t count,
                                      uint32_t block_tokens);

}  // namespace lykuro::nie::hip
