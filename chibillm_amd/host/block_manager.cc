#include "block_manager.h"

#include <limits>

namespace chibillm {

result<block_manager, block_manager_errc>
block_manager::make(std::size_t count, std::size_t size)
{
    if (count == 0)
        return fail(block_manager_errc::invalid_block_count);
    if (size == 0)
        return fail(block_manager_errc::invalid_block_size);
    if (count - 1 > std::numeric_limits<block_id>::max())
        return fail(block_manager_errc::too_many_blocks);
    return block_manager(count, size);
}

block_manager::block_manager(std::size_t count, std::size_t size)
    : count_(count)
    , size_(size)
    , refs_(count, 0)
{
    for (std::size_t b = 0; b < count; ++b)
        free_.push_back(static_cast<block_id>(b));
}

sequence_resources
block_manager::resources(seq_id id) const noexcept
{
    const auto it = tables_.find(id);
    if (it == tables_.end())
        return {};
    return { it->second };
}

block_id
block_manager::take() noexcept
{
    const block_id b = free_.front();
    free_.pop_front();
    refs_[b] = 1;
    return b;
}

void
block_manager::unref(block_id block) noexcept
{
    if (refs_[block] && --refs_[block] == 0)
        free_.push_back(block);
}

result<void, state_error>
block_manager::reserve(seq_id id, std::size_t tokens)
{
    if (tokens == 0)
        return fail(state_errc::invalid_reservation);
    const std::size_t needed = (tokens - 1) / size_ + 1;
    const auto it = tables_.find(id);
    const std::size_t have = it == tables_.end() ? 0 : it->second.size();
    if (needed <= have)
        return {};
    if (needed - have > free_.size())
        return fail(state_errc::capacity_exhausted);
    auto& table = tables_[id];
    table.reserve(needed);
    while (table.size() < needed)
        table.push_back(take());
    return {};
}

void
block_manager::release(seq_id id) noexcept
{
    const auto it = tables_.find(id);
    if (it == tables_.end())
        return;
    for (const block_id b : it->second)
        unref(b);
    tables_.erase(it);
}

std::uint32_t
block_manager::refcount(block_id block) const noexcept
{
    return block < refs_.size() ? refs_[block] : 0;
}

result<void, state_error>
block_manager::retain(std::span<const block_id> blocks)
{
    for (const block_id b : blocks)
        if (b >= count_ || refs_[b] == 0)
            return fail(state_errc::invalid_reservation);
    for (const block_id b : blocks)
        ++refs_[b];
    return {};
}

void
block_manager::drop(std::span<const block_id> blocks) noexcept
{
    for (const block_id b : blocks)
        if (b < count_)
            unref(b);
}

result<void, state_error>
block_manager::share_prefix(seq_id id, std::span<const block_id> prefix)
{
    CL_TRY(retain(prefix));
    auto& table = tables_[id];
    table.insert(table.begin(), prefix.begin(), prefix.end());
    return {};
}

result<block_id, state_error>
block_manager::fork(seq_id id, std::size_t index)
{
    const auto it = tables_.find(id);
    if (it == tables_.end() || index >= it->second.size())
        return fail(state_errc::invalid_reservation);
    if (free_.empty())
        return fail(state_errc::capacity_exhausted);
    const block_id fresh = take();
    const block_id old = it->second[index];
    it->second[index] = fresh;
    unref(old);
    return fresh;
}

} // namespace chibillm
