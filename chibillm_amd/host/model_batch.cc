#include "model_batch.h"

#include <algorithm>
#include <limits>
#include <unordered_set>

namespace chibillm {

std::size_t
model_batch::sample_count() const noexcept
{
    return static_cast<std::size_t>(std::count_if(
        items.begin(), items.end(), [](const auto& item) { return item.logits_index.has_value(); }));
}

result<model_batch, model_batch_errc>
build_model_batch(const scheduled_batch& scheduled, const scheduler& engine)
{
    if (scheduled.empty())
        return fail(model_batch_errc::empty_batch);
    if (scheduled.phase != batch_phase::prefill && scheduled.phase != batch_phase::decode)
        return fail(model_batch_errc::invalid_sequence_state);
    const seq_status expected =
        scheduled.phase == batch_phase::prefill ? seq_status::waiting : seq_status::running;
    constexpr std::size_t max_position = std::numeric_limits<position_id>::max();

    // validate everything before building any output
    std::unordered_set<seq_id> seen;
    seen.reserve(scheduled.items.size());
    for (const scheduled_item& item : scheduled.items) {
        if (item.token_count == 0)
            return fail(model_batch_errc::zero_token_count);
        if (!seen.insert(item.id).second)
            return fail(model_batch_errc::duplicate_sequence_id);
        const seq* s = engine.find_sequence(item.id);
        if (!s)
            return fail(model_batch_errc::unknown_sequence);
        if (s->status() != expected)
            return fail(model_batch_errc::invalid_sequence_state);
        if (item.token_count != s->scheduled_token_count())
            return fail(model_batch_errc::scheduled_token_count_mismatch);
        const std::size_t first = s->processed_token_count();
        if (first > s->token_count() || item.token_count > s->token_count() - first)
            return fail(model_batch_errc::token_range_out_of_bounds);
        if (first > max_position || item.token_count - 1 > max_position - first)
            return fail(model_batch_errc::position_out_of_range);
    }

    model_batch out { scheduled.id, scheduled.phase, engine.state().block_size(), {}, {}, {} };
    out.tokens.reserve(scheduled.token_count());
    out.positions.reserve(scheduled.token_count());
    out.items.reserve(scheduled.items.size());
    for (const scheduled_item& item : scheduled.items) {
        const seq& s = *engine.find_sequence(item.id);
        const std::size_t offset = out.tokens.size();
        const std::size_t first = s.processed_token_count();
        const auto slice = s.tokens().subspan(first, item.token_count);
        out.tokens.insert(out.tokens.end(), slice.begin(), slice.end());
        for (std::size_t i = 0; i < item.token_count; ++i)
            out.positions.push_back(static_cast<position_id>(first + i));
        const auto table = engine.state().resources(item.id).blocks;
        out.items.push_back({ item.id, offset, item.token_count,
                              item.sample ? std::optional(offset + item.token_count - 1)
                                          : std::nullopt,
                              std::vector<block_id>(table.begin(), table.end()) });
    }
    return out;
}

result<paged_batch_metadata, model_batch_errc>
prepare_paged_batch(const model_batch& batch, std::size_t max_positions, std::size_t block_count,
                    std::size_t block_size)
{
    if (batch.empty())
        return fail(model_batch_errc::empty_batch);
    if (!block_size || !block_count || batch.tokens.size() != batch.positions.size()
        || batch.kv_block_size != block_size)
        return fail(model_batch_errc::inconsistent_batch);
    constexpr std::uint64_t u32_max = std::numeric_limits<std::uint32_t>::max();
    paged_batch_metadata md;
    md.slots.reserve(batch.tokens.size());
    md.table_offsets.reserve(batch.tokens.size());
    md.table_lengths.reserve(batch.tokens.size());
    md.logits_indices.reserve(batch.items.size());
    std::size_t next_row = 0;
    for (const model_batch_item& item : batch.items) {
        const bool logits_ok = !item.logits_index
            || (*item.logits_index >= item.token_offset
                && *item.logits_index < item.token_offset + item.token_count);
        if (item.token_count == 0 || item.token_offset != next_row
            || item.token_count > batch.tokens.size() - next_row || !logits_ok
            || item.block_table.empty() || md.block_table.size() > u32_max
            || item.block_table.size() > u32_max - md.block_table.size())
            return fail(model_batch_errc::inconsistent_batch);
        const auto table_offset = static_cast<std::uint32_t>(md.block_table.size());
        const auto table_length = static_cast<std::uint32_t>(item.block_table.size());
        for (const block_id b : item.block_table) {
            if (b >= block_count)
                return fail(model_batch_errc::inconsistent_batch);
            md.block_table.push_back(b);
        }
        for (std::size_t row = item.token_offset; row < item.token_offset + item.token_count; ++row) {
            const std::size_t pos = batch.positions[row];
            if (pos >= max_positions || pos / block_size >= item.block_table.size())
                return fail(model_batch_errc::inconsistent_batch);
            const std::uint64_t slot =
                (std::uint64_t)item.block_table[pos / block_size] * block_size + pos % block_size;
            if (slot > u32_max)
                return fail(model_batch_errc::inconsistent_batch);
            md.slots.push_back(static_cast<std::uint32_t>(slot));
            md.table_offsets.push_back(table_offset);
            md.table_lengths.push_back(table_length);
        }
        if (item.logits_index)
            md.logits_indices.push_back(*item.logits_index);
        next_row += item.token_count;
    }
    if (next_row != batch.tokens.size())
        return fail(model_batch_errc::inconsistent_batch);
    return md;
}

} // namespace chibillm
