// Fixed-size page allocator (the behaviour of src/block_manager.cc:5-64): a FIFO
// free list that starts 0..N-1, reservations pop from its front, releases push
// to its back. Pages carry reference counts so that a prefix can be shared by
// several sequences and checkpoints: with nothing shared every count is 1 and
// the allocator behaves exactly like the reference's (same ids, same order).
#pragma once

#include <cstddef>
#include <cstdint>
#include <deque>
#include <unordered_map>
#include <vector>

#include "model_state.h"

namespace chibillm {

enum class block_manager_errc {
    invalid_block_count,
    invalid_block_size,
    too_many_blocks,
};

[[nodiscard]] inline std::string_view
error_name(block_manager_errc code) noexcept
{
    static constexpr std::array<std::string_view, 3> names {
        "block_manager.invalid_block_count",
        "block_manager.invalid_block_size",
        "block_manager.too_many_blocks",
    };
    const auto i = static_cast<std::size_t>(code);
    return i < names.size() ? names[i] : "block_manager.unknown_error";
}

class block_manager final : public model_state {
public:
    static result<block_manager, block_manager_errc> make(std::size_t block_count,
                                                          std::size_t block_size);
    block_manager(block_manager&&) noexcept = default;
    block_manager& operator=(block_manager&&) noexcept = default;

    std::size_t block_count() const noexcept { return count_; }
    std::size_t block_size() const noexcept override { return size_; }
    std::size_t free_block_count() const noexcept { return free_.size(); }
    std::size_t used_block_count() const noexcept { return count_ - free_.size(); }

    sequence_resources resources(seq_id id) const noexcept override;
    result<void, state_error> reserve(seq_id id, std::size_t tokens) override;
    // Drops one reference from each of the sequence's pages; pages reaching
    // zero return to the back of the free list in table order.
    void release(seq_id id) noexcept override;

    // ---- sharing ------------------------------------------------------------
    std::uint32_t refcount(block_id block) const noexcept;
    // Adds a reference to each page (all must be allocated).
    result<void, state_error> retain(std::span<const block_id> blocks);
    // Drops a reference from each page, as release() does for a table.
    void drop(std::span<const block_id> blocks) noexcept;
    // The sequence's table becomes `prefix` (each page gains a reference)
    // followed by the pages it already owns.
    result<void, state_error> share_prefix(seq_id id, std::span<const block_id> prefix);
    // Replaces the sequence's page at `index` by a fresh private page (one
    // reference) and drops the old one: the table edit of a copy-on-write.
    // Returns the new page; the caller copies the data.
    result<block_id, state_error> fork(seq_id id, std::size_t index);

private:
    block_manager(std::size_t count, std::size_t size);
    block_id take() noexcept;
    void unref(block_id block) noexcept;

    std::size_t count_;
    std::size_t size_;
    std::deque<block_id> free_;
    std::vector<std::uint32_t> refs_;
    std::unordered_map<seq_id, std::vector<block_id>> tables_;
};

} // namespace chibillm
