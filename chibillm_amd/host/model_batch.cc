// Model batches: the backend's copy of a scheduled batch, and the paged
// metadata the device path needs from it. The contract (the interface of
// src/model_batch.h:13-92, pinned by the model_batch tests in tests/cpp):
//
// build_model_batch refuses, before producing anything: an empty batch; an
// item with no tokens, a repeated sequence, an unknown one, one not in the
// phase's state (waiting for prefill, running for decode), one whose
// scheduled count differs from the item's, or whose tokens or positions would
// leave the sequence or the u32 position range. It then lays the items'
// unprocessed tokens end to end in batch order, each at its position
// (processed + i), with a copy of the sequence's block table, and marks the
// last row of each sampling item as its logits row.
//
// prepare_paged_batch turns a model batch into the arrays the KV path takes:
// the items' block tables concatenated, and per row its slot
// table[pos / bs] * bs + pos % bs, its item's offset into the concatenated
// table and that table's length, plus the logits rows. Everything that does
// not line up (rows out of order or not all covered, a logits row outside its
// item, an empty table or one entry past the pool, a position past its table
// or max_positions, a slot or table beyond u32) is inconsistent_batch.
#include "model_batch.h"

#include <algorithm>
#include <limits>
#include <unordered_set>

namespace chibillm {

std::size_t
model_batch::sample_count() const noexcept
{
    std::size_t n = 0;
    for (const model_batch_item& item : items)
        n += item.logits_index.has_value();
    return n;
}

namespace {

// What build_model_batch takes from the scheduler for one item.
struct item_source {
    const seq* sequence;
    std::size_t first; // position of the item's first token
};

std::optional<model_batch_errc>
item_fault(const scheduled_item& item, const seq* s, seq_status wanted)
{
    constexpr std::size_t last_position = std::numeric_limits<position_id>::max();
    if (!s)
        return model_batch_errc::unknown_sequence;
    if (s->status() != wanted)
        return model_batch_errc::invalid_sequence_state;
    if (s->scheduled_token_count() != item.token_count)
        return model_batch_errc::scheduled_token_count_mismatch;
    const std::size_t first = s->processed_token_count();
    if (first > s->token_count() || s->token_count() - first < item.token_count)
        return model_batch_errc::token_range_out_of_bounds;
    if (first > last_position || item.token_count - 1 > last_position - first)
        return model_batch_errc::position_out_of_range;
    return std::nullopt;
}

} // namespace

result<model_batch, model_batch_errc>
build_model_batch(const scheduled_batch& scheduled, const scheduler& engine)
{
    if (scheduled.empty())
        return fail(model_batch_errc::empty_batch);
    seq_status wanted;
    switch (scheduled.phase) {
    case batch_phase::prefill:
        wanted = seq_status::waiting;
        break;
    case batch_phase::decode:
        wanted = seq_status::running;
        break;
    default:
        return fail(model_batch_errc::invalid_sequence_state);
    }

    // pass 1: every item checked and resolved, nothing built yet
    std::vector<item_source> sources;
    sources.reserve(scheduled.items.size());
    std::unordered_set<seq_id> ids;
    std::size_t rows = 0;
    for (const scheduled_item& item : scheduled.items) {
        if (item.token_count == 0)
            return fail(model_batch_errc::zero_token_count);
        if (!ids.insert(item.id).second)
            return fail(model_batch_errc::duplicate_sequence_id);
        const seq* s = engine.find_sequence(item.id);
        if (const auto fault = item_fault(item, s, wanted))
            return fail(*fault);
        sources.push_back({ s, s->processed_token_count() });
        rows += item.token_count;
    }

    // pass 2: rows laid end to end in batch order
    model_batch out { scheduled.id, scheduled.phase, engine.state().block_size(), {}, {}, {} };
    out.tokens.resize(rows);
    out.positions.resize(rows);
    out.items.reserve(scheduled.items.size());
    std::size_t row = 0;
    for (std::size_t i = 0; i < scheduled.items.size(); ++i) {
        const scheduled_item& item = scheduled.items[i];
        const auto [s, first] = sources[i];
        const auto unprocessed = s->tokens().subspan(first, item.token_count);
        std::copy(unprocessed.begin(), unprocessed.end(), out.tokens.begin() + row);
        for (std::size_t t = 0; t < item.token_count; ++t)
            out.positions[row + t] = static_cast<position_id>(first + t);
        const auto table = engine.state().resources(item.id).blocks;
        model_batch_item built { item.id, row, item.token_count, std::nullopt,
                                 std::vector<block_id>(table.begin(), table.end()) };
        if (item.sample)
            built.logits_index = row + item.token_count - 1;
        out.items.push_back(std::move(built));
        row += item.token_count;
    }
    return out;
}

result<paged_batch_metadata, model_batch_errc>
prepare_paged_batch(const model_batch& batch, std::size_t max_positions, std::size_t block_count,
                    std::size_t block_size)
{
    if (batch.empty())
        return fail(model_batch_errc::empty_batch);
    constexpr std::uint64_t u32_limit = std::numeric_limits<std::uint32_t>::max();
    const auto inconsistent = [] { return fail(model_batch_errc::inconsistent_batch); };
    if (block_size == 0 || block_count == 0 || batch.kv_block_size != block_size
        || batch.positions.size() != batch.tokens.size())
        return inconsistent();
    const std::size_t rows = batch.tokens.size();

    // pass 1: the items tile the rows in order, and the tables fit u32
    std::uint64_t entries = 0;
    std::size_t covered = 0;
    for (const model_batch_item& item : batch.items) {
        const bool tiles = item.token_count != 0 && item.token_offset == covered
            && item.token_count <= rows - covered;
        const bool logits_inside = !item.logits_index
            || (*item.logits_index >= item.token_offset
                && *item.logits_index - item.token_offset < item.token_count);
        if (!tiles || !logits_inside || item.block_table.empty() || entries > u32_limit
            || item.block_table.size() > u32_limit - entries)
            return inconsistent();
        entries += item.block_table.size();
        covered += item.token_count;
    }
    if (covered != rows)
        return inconsistent();

    // pass 2: fill the arrays by index
    paged_batch_metadata md;
    md.block_table.resize(entries);
    md.slots.resize(rows);
    md.table_offsets.resize(rows);
    md.table_lengths.resize(rows);
    std::size_t at = 0;
    for (const model_batch_item& item : batch.items) {
        const auto& table = item.block_table;
        if (std::any_of(table.begin(), table.end(), [&](block_id b) { return b >= block_count; }))
            return inconsistent();
        std::copy(table.begin(), table.end(), md.block_table.begin() + at);
        for (std::size_t r = item.token_offset; r < item.token_offset + item.token_count; ++r) {
            const std::size_t position = batch.positions[r];
            const std::size_t page = position / block_size;
            if (position >= max_positions || page >= table.size())
                return inconsistent();
            const std::uint64_t slot =
                static_cast<std::uint64_t>(table[page]) * block_size + position % block_size;
            if (slot > u32_limit)
                return inconsistent();
            md.slots[r] = static_cast<std::uint32_t>(slot);
            md.table_offsets[r] = static_cast<std::uint32_t>(at);
            md.table_lengths[r] = static_cast<std::uint32_t>(table.size());
        }
        if (item.logits_index)
            md.logits_indices.push_back(*item.logits_index);
        at += table.size();
    }
    return md;
}

} // namespace chibillm
