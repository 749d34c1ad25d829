// Byte-bounded LRU of prefix checkpoints keyed by exact token sequences (the
// behaviour of src/prefix_cache.cc:11-73): find() returns the longest cached
// *proper* prefix of a prompt (a suffix must remain to produce logits) and
// moves it to the front; insert() evicts from the back until the new entry
// fits. An entry's size is its tokens (4 B each) plus its checkpoint's
// size_bytes(); with hip_model_state's shared checkpoints that is the KV
// pages the entry keeps alive.
#pragma once

#include <list>
#include <memory>
#include <span>
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
    std::size_t entry_count() const noexcept { return entries_.size(); }

private:
    struct entry {
        std::vector<token_id> tokens;
        std::unique_ptr<model_checkpoint> state;
        std::size_t bytes() const noexcept
        {
            return tokens.size() * sizeof(token_id) + state->size_bytes();
        }
    };

    std::size_t capacity_;
    std::size_t bytes_ = 0;
    std::list<entry> entries_; // most recently used first
};

} // namespace chibillm
