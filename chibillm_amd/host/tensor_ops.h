// The KV-path ops of the tensor layer (src/tensor/tensor_ops.h:160-178,
// src/tensor/attention.h:6-78) over non-owning device tensor views, with the
// reference's validation order (all ranks, then dtypes, then shapes, then
// bounds; src/tensor/validation.h:15-28) and error codes. Batch metadata is
// uploaded once per step (upload_attention_metadata) and used by every layer.
#pragma once

#include <cstdint>
#include <span>
#include <unordered_map>
#include <vector>

#include "hip_kv_cache.h"

namespace chibillm {

// src/tensor/types.h:90-95, plus f16
enum class dtype : std::uint8_t {
    f32,
    bf16,
    i32,
    u32,
    f16,
};

// A device array with a shape; does not own its memory.
struct device_tensor {
    void* data = nullptr;
    dtype type = dtype::f32;
    std::vector<std::size_t> dims;

    std::size_t rank() const noexcept { return dims.size(); }
    std::size_t element_count() const noexcept
    {
        std::size_t n = 1;
        for (std::size_t d : dims)
            n *= d;
        return n;
    }
};

enum class tensor_op_errc : std::uint8_t {
    tensor_creation_failed,
    allocation_failed,
    empty_tokens,
    empty_logits_indices,
    invalid_hidden_states,
    logits_index_out_of_range,
    token_id_overflow,
    invalid_rank,
    unsupported_dtype,
    input_shape_mismatch,
    inner_dimension_mismatch,
    output_shape_mismatch,
    token_out_of_range,
    invalid_epsilon,
    position_count_mismatch,
    invalid_head_count,
    invalid_head_dimension,
    invalid_rope_theta,
    cache_slot_count_mismatch,
    cache_feature_count_mismatch,
    cache_layer_out_of_range,
    cache_slot_out_of_range,
    block_table_metadata_count_mismatch,
    block_table_range_out_of_bounds,
    cache_block_out_of_range,
    cache_head_dimension_mismatch,
    invalid_kv_head_mapping,
    backend_failure,
    unsupported_aliasing,
};

[[nodiscard]] inline std::string_view
error_name(tensor_op_errc code) noexcept
{
    // the ckv status of code c is c + 100 and carries the same name
    const char* name = ckv_error_name(static_cast<int>(code) + 100);
    return std::string_view(name).starts_with("tensor_op.") ? name : "tensor_op.unknown_error";
}

using tensor_op_error = error<tensor_op_errc>;

// The five arrays of attention_metadata (src/tensor/attention.h:6-12).
struct attention_metadata {
    std::span<const std::uint32_t> positions;
    std::span<const std::uint32_t> slots; // may be empty when no append follows
    std::span<const std::uint32_t> block_table;
    std::span<const std::uint32_t> block_table_offsets;
    std::span<const std::uint32_t> block_table_lengths;
};

// Validates on the host and uploads (src/tensor/attention.cc:8-29, :110-137).
result<void, tensor_op_error> upload_attention_metadata(hip_kv_cache& cache,
                                                        attention_metadata metadata);

struct model_batch;

// prepare_paged_batch + upload_attention_metadata with the tables kept on the
// device (src/model_batch.cc:127-204, src/tensor/attention.cc:8-29): every
// live sequence owns a row of the pool's sequence-table arena, upload() sends
// only the table entries that changed since the sequence's previous batch and
// one (sequence row, first position, token count) triple per item, and the
// device expands the per-row offsets, lengths, positions and slots. The
// result is the metadata prepare_paged_batch would upload for the same batch.
class device_tables {
public:
    static result<device_tables, tensor_op_error> make(hip_kv_cache& cache,
                                                       std::size_t max_sequences,
                                                       std::size_t pages_per_sequence);

    // The batch's items must cover its rows in order with consecutive
    // positions (as the scheduler builds them); positions must stay below
    // max_positions. Errors: position_count_mismatch (rows not covered or
    // not consecutive), block_table_range_out_of_bounds (a position past the
    // item's table, max_positions, a table longer than pages_per_sequence or
    // more live sequences than max_sequences), cache_block_out_of_range.
    result<void, tensor_op_error> upload(const model_batch& batch, std::size_t max_positions,
                                         bool with_slots);
    // Frees the sequence's row (model_state::release). Unknown ids are harmless.
    void release(seq_id id) noexcept;

    std::size_t live_sequences() const noexcept { return row_of_.size(); }
    // Table entries sent to the device so far (the deltas).
    std::size_t entries_sent() const noexcept { return entries_sent_; }

private:
    device_tables(hip_kv_cache& cache, std::size_t max_sequences, std::size_t cap);

    hip_kv_cache* cache_;
    std::size_t cap_;
    std::unordered_map<seq_id, std::uint32_t> row_of_;
    std::vector<std::uint32_t> free_rows_;
    std::vector<std::vector<block_id>> sent_; // per row: the table the device holds
    std::size_t entries_sent_ = 0;
    // per-upload staging, kept to avoid reallocation
    std::vector<std::uint32_t> seq_, index_, block_, len_seq_, length_;
    std::vector<std::uint32_t> item_row_, item_first_, item_count_;
};

// keys/values: [rows, kv_heads * head_dim] of the cache dtype (src/tensor/tensor_ops.cc:412-463).
result<void, tensor_op_error> store_kv(hip_kv_cache& cache, const device_tensor& keys,
                                       const device_tensor& values, std::size_t layer);

// queries/output: [rows, q_heads * head_dim] of the cache dtype; scale
// 1/sqrt(head_dim) (src/tensor/attention.cc:188-254). Selection as the
// reference: query tiles (prefill form) when a run of rows shares a tile.
result<void, tensor_op_error> paged_attention(hip_kv_cache& cache, const device_tensor& queries,
                                              std::size_t layer, std::size_t query_head_count,
                                              device_tensor& output);

// store_kv then paged_attention of decode rows in one pass where possible
// (ckv_append_decode): the pair run_attention issues per layer
// (src/qwen/qwen_layer.cc:32-50).
result<void, tensor_op_error> store_kv_and_attend(hip_kv_cache& cache, const device_tensor& keys,
                                                  const device_tensor& values,
                                                  const device_tensor& queries, std::size_t layer,
                                                  std::size_t query_head_count,
                                                  device_tensor& output);

// The attention output's consumer in Qwen3.5 layers (src/qwen/qwen_layer.cc:183-206):
// paged_attention then sigmoid_mul(gate, attended, attended), with the gate
// applied in the attention epilogue. gate: [rows, q_heads * head_dim] of the
// cache dtype (input_shape_mismatch otherwise), checked after the attention.
result<void, tensor_op_error> paged_attention_gated(hip_kv_cache& cache,
                                                    const device_tensor& queries,
                                                    const device_tensor& gate, std::size_t layer,
                                                    std::size_t query_head_count,
                                                    device_tensor& output);
result<void, tensor_op_error> store_kv_and_attend_gated(hip_kv_cache& cache,
                                                        const device_tensor& keys,
                                                        const device_tensor& values,
                                                        const device_tensor& queries,
                                                        const device_tensor& gate,
                                                        std::size_t layer,
                                                        std::size_t query_head_count,
                                                        device_tensor& output);
// sigmoid_mul (src/tensor/tensor_ops.h:131-135): output = input * sigmoid(gate),
// rank-2 tensors of the cache dtype; output may be input.
result<void, tensor_op_error> sigmoid_mul(hip_kv_cache& cache, const device_tensor& gate,
                                          const device_tensor& input, device_tensor& output);

// rope (src/tensor/tensor_ops.cc:356-410) on [rows, heads * head_dim] rows of
// the cache dtype and head dimension at the uploaded positions; input may be
// output. rotary_dimension 0 means the whole head.
result<void, tensor_op_error> rope(hip_kv_cache& cache, const device_tensor& input,
                                   std::size_t head_count, float theta, device_tensor& output,
                                   std::size_t rotary_dimension = 0);

// rope of the key rows fused into store_kv (ckv_rope_append): the
// apply_rope + store_kv pair of src/qwen/qwen_layer.cc:20-30, :43.
result<void, tensor_op_error> store_kv_rotated(hip_kv_cache& cache, const device_tensor& keys,
                                               const device_tensor& values, std::size_t layer,
                                               float theta, std::size_t rotary_dimension = 0);

} // namespace chibillm
