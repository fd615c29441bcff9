#include "kv_pool.h"

namespace lykuro::nie::hip {

KvBlockPool::KvBlockPool(uint32_t num_blocks, uint32_t block_tokens)
    : block_tokens_(block_tokens), slots_(num_blocks) {
    // block 0 is handed out first
    free_.reserve(num_blocks);
    for (uint32_t i = num_blocks; i-- > 0;) free_.push_back(int32_t(i));
}

void KvBlockPool::Unlink(int32_t b) {
    Slot& s = slots_[b];
    (s.prev == kNone ? oldest_ : slots_[s.prev].next) = s.next;
    (s.next == kNone ? newest_ : slots_[s.next].prev) = s.prev;
    s.prev = s.next = kNone;
    --reclaimable_;
}

void KvBlockPool::Append(int32_t b) {
    Slot& s = slots_[b];
    s.prev = newest_;
    s.next = kNone;
    (newest_ == kNone ? oldest_ : slots_[newest_].next) = b;
    newest_ = b;
    ++reclaimable_;
}

std::optional<int32_t> KvBlockPool::Take() {
    int32_t b;
    if (!free_.empty()) {
        b = free_.back();
        free_.pop_back();
    } else if (oldest_ != kNone) {
        b = oldest_;
        Unlink(b);
        by_key_.erase(slots_[b].key);
        slots_[b].published = false;
    } else {
        return std::nullopt;
    }
    slots_[b].refs = 1;
    return b;
}

void KvBlockPool::Drop(int32_t block) {
    Slot& s = slots_[block];
    if (s.refs == 0 || --s.refs > 0) return;
    if (s.published) Append(block);
    else free_.push_back(block);
}

std::optional<int32_t> KvBlockPool::Find(uint64_t key) {
    const auto it = by_key_.find(key);
    if (it == by_key_.end()) return std::nullopt;
    Slot& s = slots_[it->second];
    if (s.refs++ == 0) Unlink(it->second);
    return it->second;
}

void KvBlockPool::Publish(uint64_t key, int32_t block) {
    Slot& s = slots_[block];
    if (s.published || s.refs == 0) return;
    if (!by_key_.emplace(key, block).second) return;
    s.published = true;
    s.key = key;
}

std::vector<uint64_t> PrefixChainKeys(std::string_view scope, const uint32_t* tokens, size_t count,
                                      uint32_t block_tokens) {
    constexpr uint64_t kBasis = 0xcbf29ce484222325ull, kPrime = 0x100000001b3ull;
    uint64_t state = kBasis;
    auto mix = [&state](uint8_t byte) { state = (state ^ byte) * kPrime; };
    for (char c : scope) mix(uint8_t(c));
    std::vector<uint64_t> keys;
    const size_t blocks = block_tokens ? count / block_tokens : 0;
    keys.reserve(blocks);
    for (size_t b = 0; b < blocks; ++b) {
        for (size_t i = b * block_tokens; i < (b + 1) * block_tokens; ++i)
            for (int byte = 0; byte < 4; ++byte) mix(uint8_t(tokens[i] >> (8 * byte)));
        keys.push_back(state);
    }
    return keys;
}

}  // namespace lykuro::nie::hip
