#include "tensor_ops.h"

#include <cmath>
#include <initializer_list>

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
