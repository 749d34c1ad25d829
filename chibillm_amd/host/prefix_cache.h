// Byte-bounded LRU of prefix checkpoints keyed by exact token sequences (the
// behaviour of src/prefix_cache.cc:11-73): find() returns the longest cached
// *proper* prefix of a prompt (a suffix must remain to produce logits) and
// moves it to the front; insert() evicts from the back until the new entry
// fits. An entry's size is its tokens (4 B each) plus its checkpoint's
// size_bytes(); with hip_model_state's shared checkpoints that is the KV
// pages the entry keeps alive.
//
// Entries are found by an index on a hash of their tokens, and a prompt's
// longest cached prefix by hashing only the prefix lengths present in the
// cache, longest first: a lookup costs O(distinct lengths x prompt) token
// reads whatever the number of entries.
#pragma once

#include <cstdint>
#include <functional>
#include <list>
#include <map>
#include <memory>
#include <span>
#include <unordered_map>
#include <vector>

#include "model_state.h"

namespace chibillm {

class prefix_cache {
public:
    explicit prefix_cache(std::size_t capacity_bytes) noexcept
        : capacity_(capacity_bytes)
    {}

    const model_checkpoint* find(std::span<const token_id> prompt);
    bool contains(std::span<const token_id> prefix) const noexcept;
    bool fits(std::size_t token_count, std::size_t state_bytes) const noexcept;
    void make_room(std::size_t token_count, std::size_t state_bytes) noexcept;
    void insert(std::span<const token_id> prefix, std::unique_ptr<model_checkpoint> state);

    std::size_t size_bytes() const noexcept { return bytes_; }
    std::size_t entry_count() const noexcept { return recency_.size(); }

private:
    struct entry {
        std::vector<token_id> tokens;
        std::uint64_t key; // hash of tokens
        std::unique_ptr<model_checkpoint> state;
        std::size_t bytes() const noexcept
        {
            return tokens.size() * sizeof(token_id) + state->size_bytes();
        }
    };
    using position = std::list<entry>::iterator;

    position locate(std::span<const token_id> tokens, std::uint64_t key) const noexcept;
    void evict_oldest() noexcept;

    std::size_t capacity_;
    std::size_t bytes_ = 0;
    std::list<entry> recency_;                              // most recently used first
    std::unordered_multimap<std::uint64_t, position> index_; // by hash of the tokens
    std::map<std::size_t, std::size_t, std::greater<>> lengths_; // entry length -> entries
};

} // namespace chibillm
