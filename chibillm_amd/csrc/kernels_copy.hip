// Bit-exact data movement kernels: slot-mapped KV append, gather through a
// block table, page copies (copy-on-write) and packed checkpoints.
//
// All of them move whole K/V rows (kv_heads*head_dim elements, 2 KiB for
// Qwen3 bf16 shapes). A wave owns one row and moves it with the widest
// vector type the row length allows (128-bit when the row is a multiple of
// 16 bytes), so every store is a coalesced 1 KiB wave transaction.
#include "ckv_internal.h"

namespace ckv {
namespace {

constexpr uint32_t rows_per_block = 4; // one wave per row, 256 threads

template <typename V>
__device__ __forceinline__ void copy_row(char* __restrict__ dst, const char* __restrict__ src,
                                         uint32_t n_vec, uint32_t lane)
{
    V* d = reinterpret_cast<V*>(dst);
    const V* s = reinterpret_cast<const V*>(src);
    for (uint32_t i = lane; i < n_vec; i += 64)
        d[i] = s[i];
}

// src/metal/kernels/attention.metal:3-33: cache row (layer*slot_count + slot)
// := input row; rows whose slot is outside the cache are skipped.
template <typename V>
__global__ __launch_bounds__(256) void store_kv_kernel(pool_view p, const uint32_t* __restrict__ slots,
                                                       uint32_t layer, const char* __restrict__ keys,
                                                       const char* __restrict__ values, uint32_t rows)
{
    const uint32_t row = blockIdx.x * rows_per_block + (threadIdx.x >> 6);
    if (row >= rows)
        return;
    const uint32_t slot_count = p.blocks * p.block_size;
    const uint32_t slot = slots[row];
    if (slot >= slot_count)
        return;
    const uint64_t row_bytes = (uint64_t)p.features * p.elem_size;
    const uint64_t target = ((uint64_t)layer * slot_count + slot) * row_bytes;
    const uint32_t n_vec = (uint32_t)(row_bytes / sizeof(V));
    const uint32_t lane = threadIdx.x & 63;
    copy_row<V>(static_cast<char*>(p.keys) + target, keys + row * row_bytes, n_vec, lane);
    copy_row<V>(static_cast<char*>(p.values) + target, values + row * row_bytes, n_vec, lane);
}

// Token t of a sequence lives at slot table[t / bs] * bs + t % bs.
template <typename V>
__global__ __launch_bounds__(256) void gather_kernel(pool_view p, const uint32_t* __restrict__ table,
                                                     uint32_t layer, uint32_t n_tokens,
                                                     char* __restrict__ out_keys,
                                                     char* __restrict__ out_values)
{
    const uint32_t t = blockIdx.x * rows_per_block + (threadIdx.x >> 6);
    if (t >= n_tokens)
        return;
    const uint32_t slot_count = p.blocks * p.block_size;
    const uint32_t slot = table[t / p.block_size] * p.block_size + t % p.block_size;
    const uint64_t row_bytes = (uint64_t)p.features * p.elem_size;
    const uint64_t source = ((uint64_t)layer * slot_count + slot) * row_bytes;
    const uint32_t n_vec = (uint32_t)(row_bytes / sizeof(V));
    const uint32_t lane = threadIdx.x & 63;
    copy_row<V>(out_keys + t * row_bytes, static_cast<const char*>(p.keys) + source, n_vec, lane);
    copy_row<V>(out_values + t * row_bytes, static_cast<const char*>(p.values) + source, n_vec,
                lane);
}

// One block per (pair, layer); blockIdx.y selects keys or values.
template <typename V>
__global__ __launch_bounds__(256) void copy_blocks_kernel(pool_view p, uint32_t layers,
                                                          const uint32_t* __restrict__ pairs,
                                                          uint32_t n)
{
    const uint32_t pair = blockIdx.x / layers;
    const uint32_t layer = blockIdx.x % layers;
    if (pair >= n)
        return;
    const uint64_t page_bytes = (uint64_t)p.block_size * p.features * p.elem_size;
    const uint64_t layer_base = (uint64_t)layer * p.blocks;
    char* base = static_cast<char*>(blockIdx.y ? p.values : p.keys);
    const V* src = reinterpret_cast<const V*>(base + (layer_base + pairs[2 * pair]) * page_bytes);
    V* dst = reinterpret_cast<V*>(base + (layer_base + pairs[2 * pair + 1]) * page_bytes);
    const uint32_t n_vec = (uint32_t)(page_bytes / sizeof(V));
    for (uint32_t i = threadIdx.x; i < n_vec; i += blockDim.x)
        dst[i] = src[i];
}

// src/metal/metal_kv_cache.cc:14-35: packed row (layer*tokens + t) <-> the
// paged row of token t of `blocks`.
template <typename V>
__global__ __launch_bounds__(256) void checkpoint_kernel(pool_view p, uint32_t layers,
                                                         const uint32_t* __restrict__ blocks,
                                                         uint32_t tokens, char* packed_keys,
                                                         char* packed_values, bool unpack)
{
    const uint64_t r = (uint64_t)blockIdx.x * rows_per_block + (threadIdx.x >> 6);
    if (r >= (uint64_t)layers * tokens)
        return;
    const uint32_t layer = (uint32_t)(r / tokens);
    const uint32_t t = (uint32_t)(r % tokens);
    const uint32_t slot_count = p.blocks * p.block_size;
    const uint32_t slot = blocks[t / p.block_size] * p.block_size + t % p.block_size;
    const uint64_t row_bytes = (uint64_t)p.features * p.elem_size;
    char* paged_k = static_cast<char*>(p.keys) + ((uint64_t)layer * slot_count + slot) * row_bytes;
    char* paged_v = static_cast<char*>(p.values) + ((uint64_t)layer * slot_count + slot) * row_bytes;
    char* pk = packed_keys + r * row_bytes;
    char* pv = packed_values + r * row_bytes;
    const uint32_t n_vec = (uint32_t)(row_bytes / sizeof(V));
    const uint32_t lane = threadIdx.x & 63;
    if (unpack) {
        copy_row<V>(paged_k, pk, n_vec, lane);
        copy_row<V>(paged_v, pv, n_vec, lane);
    } else {
        copy_row<V>(pk, paged_k, n_vec, lane);
        copy_row<V>(pv, paged_v, n_vec, lane);
    }
}

__global__ __launch_bounds__(256) void table_patch_kernel(uint32_t* __restrict__ table,
                                                          const uint32_t* __restrict__ pairs,
                                                          uint32_t n)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        table[pairs[2 * i]] = pairs[2 * i + 1];
}

__global__ __launch_bounds__(256) void fill_kernel(uint32_t* __restrict__ dst, uint32_t value,
                                                   uint32_t n)
{
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        dst[i] = value;
}

// One thread per row; the row's item is found by binary search over the
// items' first rows (ascending).
__global__ __launch_bounds__(256) void expand_batch_kernel(
    const uint32_t* __restrict__ items, uint32_t n_items, uint32_t rows,
    const uint32_t* __restrict__ seq_table, uint32_t cap, uint32_t block_size, bool with_slots,
    uint32_t* __restrict__ offsets, uint32_t* __restrict__ lengths,
    uint32_t* __restrict__ positions, uint32_t* __restrict__ slots)
{
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows)
        return;
    const uint32_t* seq = items;
    const uint32_t* first = items + n_items;
    const uint32_t* row_start = items + 3 * n_items;
    const uint32_t* length = items + 4 * n_items;
    uint32_t lo = 0, hi = n_items - 1; // last item whose first row <= r
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1) / 2;
        if (row_start[mid] <= r)
            lo = mid;
        else
            hi = mid - 1;
    }
    const uint32_t position = first[lo] + (r - row_start[lo]);
    const uint32_t base = seq[lo] * cap;
    offsets[r] = base;
    lengths[r] = length[lo];
    positions[r] = position;
    if (with_slots)
        slots[r] = seq_table[base + position / block_size] * block_size + position % block_size;
}

// Widest vector that divides the row and the given pointers' alignment.
int vector_width(uint64_t bytes, std::initializer_list<const void*> pointers)
{
    uint64_t mask = bytes;
    for (const void* ptr : pointers)
        mask |= reinterpret_cast<uintptr_t>(ptr);
    if (mask % 16 == 0)
        return 16;
    if (mask % 4 == 0)
        return 4;
    return 2;
}

uint32_t grid_rows(uint64_t rows)
{
    return (uint32_t)((rows + rows_per_block - 1) / rows_per_block);
}

} // namespace

hipError_t launch_store_kv(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                           const void* keys, const void* values, uint32_t rows)
{
    if (!rows)
        return hipSuccess;
    const uint64_t row_bytes = (uint64_t)p.features * p.elem_size;
    const auto k = static_cast<const char*>(keys);
    const auto v = static_cast<const char*>(values);
    const dim3 grid(grid_rows(rows)), block(64 * rows_per_block);
    switch (vector_width(row_bytes, { keys, values, p.keys, p.values })) {
    case 16:
        store_kv_kernel<uint4><<<grid, block, 0, s>>>(p, m.slots, layer, k, v, rows);
        break;
    case 4:
        store_kv_kernel<uint32_t><<<grid, block, 0, s>>>(p, m.slots, layer, k, v, rows);
        break;
    default:
        store_kv_kernel<uint16_t><<<grid, block, 0, s>>>(p, m.slots, layer, k, v, rows);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_gather(hipStream_t s, const pool_view& p, const uint32_t* table,
                         uint32_t layer, uint32_t n_tokens, void* out_keys, void* out_values)
{
    if (!n_tokens)
        return hipSuccess;
    const uint64_t row_bytes = (uint64_t)p.features * p.elem_size;
    const auto ok = static_cast<char*>(out_keys);
    const auto ov = static_cast<char*>(out_values);
    const dim3 grid(grid_rows(n_tokens)), block(64 * rows_per_block);
    switch (vector_width(row_bytes, { out_keys, out_values, p.keys, p.values })) {
    case 16:
        gather_kernel<uint4><<<grid, block, 0, s>>>(p, table, layer, n_tokens, ok, ov);
        break;
    case 4:
        gather_kernel<uint32_t><<<grid, block, 0, s>>>(p, table, layer, n_tokens, ok, ov);
        break;
    default:
        gather_kernel<uint16_t><<<grid, block, 0, s>>>(p, table, layer, n_tokens, ok, ov);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_copy_blocks(hipStream_t s, const pool_view& p, uint32_t layers,
                              const uint32_t* pairs, uint32_t n)
{
    if (!n)
        return hipSuccess;
    const uint64_t page_bytes = (uint64_t)p.block_size * p.features * p.elem_size;
    const dim3 grid(n * layers, 2), block(256);
    switch (vector_width(page_bytes, { p.keys, p.values })) {
    case 16:
        copy_blocks_kernel<uint4><<<grid, block, 0, s>>>(p, layers, pairs, n);
        break;
    case 4:
        copy_blocks_kernel<uint32_t><<<grid, block, 0, s>>>(p, layers, pairs, n);
        break;
    default:
        copy_blocks_kernel<uint16_t><<<grid, block, 0, s>>>(p, layers, pairs, n);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_checkpoint(hipStream_t s, const pool_view& p, uint32_t layers,
                             const uint32_t* blocks, uint32_t tokens, void* packed_keys,
                             void* packed_values, bool unpack)
{
    if (!tokens)
        return hipSuccess;
    const uint64_t row_bytes = (uint64_t)p.features * p.elem_size;
    const auto pk = static_cast<char*>(packed_keys);
    const auto pv = static_cast<char*>(packed_values);
    const dim3 grid(grid_rows((uint64_t)layers * tokens)), block(64 * rows_per_block);
    switch (vector_width(row_bytes, { packed_keys, packed_values, p.keys, p.values })) {
    case 16:
        checkpoint_kernel<uint4><<<grid, block, 0, s>>>(p, layers, blocks, tokens, pk, pv, unpack);
        break;
    case 4:
        checkpoint_kernel<uint32_t><<<grid, block, 0, s>>>(p, layers, blocks, tokens, pk, pv,
                                                           unpack);
        break;
    default:
        checkpoint_kernel<uint16_t><<<grid, block, 0, s>>>(p, layers, blocks, tokens, pk, pv,
                                                           unpack);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_table_patch(hipStream_t s, uint32_t* table, const uint32_t* pairs, uint32_t n)
{
    if (!n)
        return hipSuccess;
    table_patch_kernel<<<(n + 255) / 256, 256, 0, s>>>(table, pairs, n);
    return hipGetLastError();
}

hipError_t launch_fill(hipStream_t s, uint32_t* dst, uint32_t value, uint32_t n)
{
    if (!n)
        return hipSuccess;
    const uint32_t blocks = std::min<uint32_t>((n + 255) / 256, 4096);
    fill_kernel<<<blocks, 256, 0, s>>>(dst, value, n);
    return hipGetLastError();
}

hipError_t launch_expand_batch(hipStream_t s, const uint32_t* items, uint32_t n_items,
                               uint32_t rows, const uint32_t* seq_table, uint32_t cap,
                               uint32_t block_size, bool with_slots, uint32_t* offsets,
                               uint32_t* lengths, uint32_t* positions, uint32_t* slots)
{
    if (!rows || !n_items)
        return hipSuccess;
    expand_batch_kernel<<<(rows + 255) / 256, 256, 0, s>>>(items, n_items, rows, seq_table, cap,
                                                           block_size, with_slots, offsets,
                                                           lengths, positions, slots);
    return hipGetLastError();
}

} // namespace ckv
