// Backend-owned snapshot of a scheduled batch and the paged metadata derived
// from it (src/model_batch.h:13-92): flattened tokens/positions, per-item
// block tables, and prepare_paged_batch's slot mapping
// slot = table[pos / bs] * bs + pos % bs (src/model_batch.cc:178-185) plus
// each row's table offset/length into one flat table. These arrays are what
// ckv_tables_upload sends to the device.
#pragma once

#include <optional>
#include <vector>

#include "scheduler.h"

namespace chibillm {

using position_id = std::uint32_t;

struct model_batch_item {
    seq_id id;
    std::size_t token_offset; // range in model_batch::tokens / positions
    std::size_t token_count;
    std::optional<std::size_t> logits_index; // flattened row sampled for this sequence
    std::vector<block_id> block_table;       // copied: independent of scheduler state
};

struct model_batch {
    batch_id id;
    batch_phase phase;
    std::size_t kv_block_size;
    std::vector<token_id> tokens;
    std::vector<position_id> positions;
    std::vector<model_batch_item> items;

    [[nodiscard]] bool empty() const noexcept { return items.empty(); }
    [[nodiscard]] std::size_t sequence_count() const noexcept { return items.size(); }
    [[nodiscard]] std::size_t token_count() const noexcept { return tokens.size(); }
    [[nodiscard]] std::size_t sample_count() const noexcept;
};

enum class model_batch_errc : std::uint8_t {
    empty_batch,
    inconsistent_batch,
    zero_token_count,
    duplicate_sequence_id,
    unknown_sequence,
    invalid_sequence_state,
    scheduled_token_count_mismatch,
    token_range_out_of_bounds,
    position_out_of_range,
};

[[nodiscard]] inline std::string_view
error_name(model_batch_errc code) noexcept
{
    static constexpr std::array<std::string_view, 9> names {
        "model_batch.empty_batch",
        "model_batch.inconsistent_batch",
        "model_batch.zero_token_count",
        "model_batch.duplicate_sequence_id",
        "model_batch.unknown_sequence",
        "model_batch.invalid_sequence_state",
        "model_batch.scheduled_token_count_mismatch",
        "model_batch.token_range_out_of_bounds",
        "model_batch.position_out_of_range",
    };
    const auto i = static_cast<std::size_t>(code);
    return i < names.size() ? names[i] : "model_batch.unknown_error";
}

struct paged_batch_metadata {
    std::vector<std::uint32_t> slots;
    std::vector<std::uint32_t> block_table;
    std::vector<std::uint32_t> table_offsets;
    std::vector<std::uint32_t> table_lengths;
    std::vector<std::size_t> logits_indices;
};

result<paged_batch_metadata, model_batch_errc> prepare_paged_batch(const model_batch& batch,
                                                                   std::size_t max_positions,
                                                                   std::size_t block_count,
                                                                   std::size_t block_size);

[[nodiscard]] result<model_batch, model_batch_errc>
build_model_batch(const scheduled_batch& scheduled, const scheduler& engine);

} // namespace chibillm
