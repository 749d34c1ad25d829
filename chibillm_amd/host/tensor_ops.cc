#include "tensor_ops.h"

#include <cmath>
#include <cstring>
#include <initializer_list>

#include "model_batch.h"

namespace chibillm {

namespace {

struct tensor_layout {
    const device_tensor& tensor;
    std::size_t rank;
    dtype type;
};

// every rank before any dtype (src/tensor/validation.h:15-28)
result<void, tensor_op_error>
validate_layouts(std::initializer_list<tensor_layout> layouts)
{
    for (const auto& l : layouts)
        if (l.tensor.rank() != l.rank)
            return fail(tensor_op_errc::invalid_rank);
    for (const auto& l : layouts)
        if (l.tensor.type != l.type)
            return fail(tensor_op_errc::unsupported_dtype);
    return {};
}

dtype
cache_dtype(const hip_kv_cache& cache) noexcept
{
    switch (cache.type()) {
    case kv_dtype::f32:
        return dtype::f32;
    case kv_dtype::bf16:
        return dtype::bf16;
    default:
        return dtype::f16;
    }
}

failure<tensor_op_error>
from_ckv(const hip_kv_cache& cache, int rc)
{
    const std::string detail = ckv_last_error(cache.context().get());
    if (rc >= 100 && rc < 129)
        return fail(tensor_op_error { static_cast<tensor_op_errc>(rc - 100), detail });
    return fail(tensor_op_error { tensor_op_errc::backend_failure,
                                  std::string(ckv_error_name(rc)) + ": " + detail });
}

result<std::size_t, tensor_op_error>
validate_attention(const hip_kv_cache& cache, const device_tensor& queries, std::size_t layer,
                   std::size_t q_heads, const device_tensor& output)
{
    const dtype t = cache_dtype(cache);
    CL_TRY(validate_layouts({ { queries, 2, t }, { output, 2, t } }));
    const std::size_t rows = queries.dims[0];
    const std::size_t features = queries.dims[1];
    if (output.dims[0] != rows || output.dims[1] != features)
        return fail(tensor_op_errc::output_shape_mismatch);
    if (q_heads == 0)
        return fail(tensor_op_errc::invalid_head_count);
    if (features % q_heads != 0)
        return fail(tensor_op_errc::invalid_head_dimension);
    if (features / q_heads != cache.head_dimension())
        return fail(tensor_op_errc::cache_head_dimension_mismatch);
    if (q_heads % cache.kv_head_count() != 0)
        return fail(tensor_op_errc::invalid_kv_head_mapping);
    if (layer >= cache.layer_count())
        return fail(tensor_op_errc::cache_layer_out_of_range);
    return rows;
}

result<std::size_t, tensor_op_error>
validate_store(const hip_kv_cache& cache, const device_tensor& keys, const device_tensor& values,
               std::size_t layer)
{
    const dtype t = cache_dtype(cache);
    CL_TRY(validate_layouts({ { keys, 2, t }, { values, 2, t } }));
    if (values.dims != keys.dims)
        return fail(tensor_op_errc::input_shape_mismatch);
    if (keys.dims[1] != cache.elements_per_token())
        return fail(tensor_op_errc::cache_feature_count_mismatch);
    if (layer >= cache.layer_count())
        return fail(tensor_op_errc::cache_layer_out_of_range);
    return keys.dims[0];
}

float
attention_scale(const hip_kv_cache& cache) noexcept
{
    return 1.0f / std::sqrt(static_cast<float>(cache.head_dimension()));
}

} // namespace

result<void, tensor_op_error>
upload_attention_metadata(hip_kv_cache& cache, attention_metadata md)
{
    const std::size_t rows = md.positions.size();
    if (md.block_table_offsets.size() != rows || md.block_table_lengths.size() != rows)
        return fail(tensor_op_errc::block_table_metadata_count_mismatch);
    if (!md.slots.empty() && md.slots.size() != rows)
        return fail(tensor_op_errc::cache_slot_count_mismatch);
    const int rc = ckv_tables_upload(cache.pool(), md.block_table.data(), md.block_table.size(),
                                     md.block_table_offsets.data(), md.block_table_lengths.data(),
                                     md.positions.data(),
                                     md.slots.empty() ? nullptr : md.slots.data(), rows);
    if (rc)
        return from_ckv(cache, rc);
    return {};
}

device_tables::device_tables(hip_kv_cache& cache, std::size_t max_sequences, std::size_t cap)
    : cache_(&cache)
    , cap_(cap)
    , sent_(max_sequences)
{
    free_rows_.reserve(max_sequences);
    for (std::size_t r = max_sequences; r-- > 0;)
        free_rows_.push_back(static_cast<std::uint32_t>(r));
}

result<device_tables, tensor_op_error>
device_tables::make(hip_kv_cache& cache, std::size_t max_sequences, std::size_t pages_per_sequence)
{
    const int rc = ckv_seq_tables_reserve(cache.pool(), max_sequences, pages_per_sequence);
    if (rc)
        return from_ckv(cache, rc);
    return device_tables(cache, max_sequences, pages_per_sequence);
}

void
device_tables::release(seq_id id) noexcept
{
    const auto it = row_of_.find(id);
    if (it == row_of_.end())
        return;
    // the row's entries stay on the device and are overwritten by its next owner
    sent_[it->second].clear();
    free_rows_.push_back(it->second);
    row_of_.erase(it);
}

result<void, tensor_op_error>
device_tables::upload(const model_batch& batch, std::size_t max_positions, bool with_slots)
{
    const std::size_t bs = cache_->block_size();
    seq_.clear();
    index_.clear();
    block_.clear();
    len_seq_.clear();
    length_.clear();
    item_row_.clear();
    item_first_.clear();
    item_count_.clear();
    // the shape checks of prepare_paged_batch (src/model_batch.cc:148-185),
    // on items: rows covered in order, consecutive positions, each position
    // inside its item's table
    std::size_t expected = 0;
    for (const auto& item : batch.items) {
        if (!item.token_count || item.token_offset != expected
            || item.token_count > batch.positions.size() - expected)
            return fail(tensor_op_errc::position_count_mismatch);
        const std::uint32_t first = batch.positions[item.token_offset];
        for (std::size_t j = 1; j < item.token_count; ++j)
            if (batch.positions[item.token_offset + j] != first + j)
                return fail(tensor_op_errc::position_count_mismatch);
        const std::size_t last = static_cast<std::size_t>(first) + item.token_count - 1;
        if (last >= max_positions || last / bs >= item.block_table.size()
            || item.block_table.size() > cap_)
            return fail(tensor_op_errc::block_table_range_out_of_bounds);
        expected += item.token_count;
    }
    if (expected != batch.positions.size())
        return fail(tensor_op_errc::position_count_mismatch);

    // rows for new sequences, then the table deltas
    std::vector<seq_id> taken; // rows given out by this call, returned on failure
    auto undo = [&] {
        for (const seq_id id : taken)
            release(id);
    };
    for (const auto& item : batch.items) {
        auto it = row_of_.find(item.id);
        if (it == row_of_.end()) {
            if (free_rows_.empty()) {
                undo();
                return fail(tensor_op_errc::block_table_range_out_of_bounds);
            }
            it = row_of_.emplace(item.id, free_rows_.back()).first;
            free_rows_.pop_back();
            taken.push_back(item.id);
        }
        const std::uint32_t row = it->second;
        const auto& table = item.block_table;
        const auto& sent = sent_[row];
        // tables mostly grow at the end: compare the common part in one pass
        const std::size_t common = std::min(sent.size(), table.size());
        std::size_t i = 0;
        if (common
            && std::memcmp(sent.data(), table.data(), common * sizeof(block_id)) == 0)
            i = common;
        for (; i < table.size(); ++i)
            if (i >= sent.size() || sent[i] != table[i]) {
                seq_.push_back(row);
                index_.push_back(static_cast<std::uint32_t>(i));
                block_.push_back(table[i]);
            }
        if (table.size() != sent.size()) {
            len_seq_.push_back(row);
            length_.push_back(static_cast<std::uint32_t>(table.size()));
        }
        item_row_.push_back(row);
        item_first_.push_back(batch.positions[item.token_offset]);
        item_count_.push_back(static_cast<std::uint32_t>(item.token_count));
    }
    int rc = ckv_seq_tables_update(cache_->pool(), seq_.data(), index_.data(), block_.data(),
                                   seq_.size(), len_seq_.data(), length_.data(), len_seq_.size());
    if (rc) {
        undo();
        return from_ckv(*cache_, rc);
    }
    entries_sent_ += seq_.size();
    for (std::size_t k = 0; k < seq_.size(); ++k) { // the mirror takes the sent entries
        auto& sent = sent_[seq_[k]];
        if (index_[k] >= sent.size())
            sent.resize(index_[k] + 1);
        sent[index_[k]] = block_[k];
    }
    for (std::size_t k = 0; k < len_seq_.size(); ++k)
        sent_[len_seq_[k]].resize(length_[k]);
    rc = ckv_batch_upload(cache_->pool(), item_row_.data(), item_first_.data(),
                          item_count_.data(), item_row_.size(), with_slots ? 1 : 0);
    if (rc)
        return from_ckv(*cache_, rc);
    return {};
}

result<void, tensor_op_error>
store_kv(hip_kv_cache& cache, const device_tensor& keys, const device_tensor& values,
         std::size_t layer)
{
    std::size_t rows = 0;
    CL_TRY_ASSIGN(rows, validate_store(cache, keys, values, layer));
    const int rc = ckv_append(cache.pool(), layer, keys.data, values.data, rows);
    if (rc)
        return from_ckv(cache, rc);
    return {};
}

result<void, tensor_op_error>
paged_attention(hip_kv_cache& cache, const device_tensor& queries, std::size_t layer,
                std::size_t q_heads, device_tensor& output)
{
    std::size_t rows = 0;
    CL_TRY_ASSIGN(rows, validate_attention(cache, queries, layer, q_heads, output));
    const int rc = ckv_attention(cache.pool(), layer, queries.data, q_heads,
                                 attention_scale(cache), output.data, rows);
    if (rc)
        return from_ckv(cache, rc);
    return {};
}

result<void, tensor_op_error>
store_kv_and_attend(hip_kv_cache& cache, const device_tensor& keys, const device_tensor& values,
                    const device_tensor& queries, std::size_t layer, std::size_t q_heads,
                    device_tensor& output)
{
    std::size_t rows = 0;
    CL_TRY_ASSIGN(rows, validate_store(cache, keys, values, layer));
    std::size_t q_rows = 0;
    CL_TRY_ASSIGN(q_rows, validate_attention(cache, queries, layer, q_heads, output));
    if (q_rows != rows)
        return fail(tensor_op_errc::position_count_mismatch);
    const int rc = ckv_append_decode(cache.pool(), layer, keys.data, values.data, queries.data,
                                     q_heads, attention_scale(cache), output.data, rows);
    if (rc)
        return from_ckv(cache, rc);
    return {};
}

namespace {

// The gate is shaped and typed like the output ([rows, q_heads * head_dim]).
result<void, tensor_op_error>
validate_gate(const hip_kv_cache& cache, const device_tensor& gate, const device_tensor& output)
{
    CL_TRY(validate_layouts({ { gate, 2, cache_dtype(cache) } }));
    if (gate.dims != output.dims)
        return fail(tensor_op_errc::input_shape_mismatch);
    return {};
}

} // namespace

result<void, tensor_op_error>
paged_attention_gated(hip_kv_cache& cache, const device_tensor& queries,
                      const device_tensor& gate, std::size_t layer, std::size_t q_heads,
                      device_tensor& output)
{
    std::size_t rows = 0;
    CL_TRY_ASSIGN(rows, validate_attention(cache, queries, layer, q_heads, output));
    CL_TRY(validate_gate(cache, gate, output));
    const int rc = ckv_attention_gated(cache.pool(), layer, queries.data, q_heads,
                                       attention_scale(cache), gate.data, output.data, rows);
    if (rc)
        return from_ckv(cache, rc);
    return {};
}

result<void, tensor_op_error>
store_kv_and_attend_gated(hip_kv_cache& cache, const device_tensor& keys,
                          const device_tensor& values, const device_tensor& queries,
                          const device_tensor& gate, std::size_t layer, std::size_t q_heads,
                          device_tensor& output)
{
    std::size_t rows = 0;
    CL_TRY_ASSIGN(rows, validate_store(cache, keys, values, layer));
    std::size_t q_rows = 0;
    CL_TRY_ASSIGN(q_rows, validate_attention(cache, queries, layer, q_heads, output));
    if (q_rows != rows)
        return fail(tensor_op_errc::position_count_mismatch);
    CL_TRY(validate_gate(cache, gate, output));
    const int rc = ckv_append_decode_gated(cache.pool(), layer, keys.data, values.data,
                                           queries.data, q_heads, attention_scale(cache),
                                           gate.data, output.data, rows);
    if (rc)
        return from_ckv(cache, rc);
    return {};
}

result<void, tensor_op_error>
sigmoid_mul(hip_kv_cache& cache, const device_tensor& gate, const device_tensor& input,
            device_tensor& output)
{
    // validate_elementwise_output (src/tensor/tensor_ops.cc:17-43): layouts,
    // then the input shapes, then the output's
    const dtype t = cache_dtype(cache);
    CL_TRY(validate_layouts({ { gate, 2, t }, { input, 2, t }, { output, 2, t } }));
    if (input.dims != gate.dims)
        return fail(tensor_op_errc::input_shape_mismatch);
    if (output.dims != gate.dims)
        return fail(tensor_op_errc::output_shape_mismatch);
    const int rc = ckv_sigmoid_mul(cache.context().get(), static_cast<int>(cache.type()),
                                   gate.data, input.data, output.data, gate.element_count());
    if (rc)
        return from_ckv(cache, rc);
    return {};
}

result<void, tensor_op_error>
rope(hip_kv_cache& cache, const device_tensor& input, std::size_t head_count, float theta,
     device_tensor& output, std::size_t rotary_dimension)
{
    const dtype t = cache_dtype(cache);
    CL_TRY(validate_layouts({ { input, 2, t }, { output, 2, t } }));
    if (output.dims != input.dims)
        return fail(tensor_op_errc::output_shape_mismatch);
    if (head_count && input.dims[1] != head_count * cache.head_dimension())
        return fail(tensor_op_errc::invalid_head_dimension);
    // position count, head count, rotary width and theta are checked by
    // libckv; the output shape and feature count (which it cannot see) are
    // checked here first, so when several are wrong at once the shape error
    // wins where the reference would report the count
    const int rc = ckv_rope(cache.pool(), input.data, output.data, head_count, theta,
                            rotary_dimension, input.dims[0]);
    if (rc)
        return from_ckv(cache, rc);
    return {};
}

result<void, tensor_op_error>
store_kv_rotated(hip_kv_cache& cache, const device_tensor& keys, const device_tensor& values,
                 std::size_t layer, float theta, std::size_t rotary_dimension)
{
    std::size_t rows = 0;
    CL_TRY_ASSIGN(rows, validate_store(cache, keys, values, layer));
    const int rc = ckv_rope_append(cache.pool(), layer, keys.data, values.data, theta,
                                   rotary_dimension, rows);
    if (rc)
        return from_ckv(cache, rc);
    return {};
}

} // namespace chibillm
