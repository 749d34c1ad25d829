// Device KV pool of the paged cache (the role of metal_kv_cache,
// src/metal/metal_kv_cache.h:16-122): keys and values
// [layer, block, token_in_block, kv_head, feature] in HBM through libckv, with
// the reference's geometry checks, element offsets and packed checkpoints.
#pragma once

#include <memory>
#include <span>
#include <string>

#include "ckv.h"
#include "model_state.h"

namespace chibillm {

enum class kv_dtype : int {
    f32 = CKV_F32,
    bf16 = CKV_BF16,
    f16 = CKV_F16,
};

[[nodiscard]] inline std::size_t
element_bytes(kv_dtype t) noexcept
{
    return t == kv_dtype::f32 ? 4 : 2;
}

// Status of a libckv call with its name and the context's detail text.
struct ckv_failure {
    int code;
    std::string detail;
};

[[nodiscard]] inline std::string
describe_error(const ckv_failure& f)
{
    return std::string(ckv_error_name(f.code)) + (f.detail.empty() ? "" : ": " + f.detail);
}

// Owns a ckv_context: one device and the stream all KV work is ordered on.
class hip_context {
public:
    static result<hip_context, ckv_failure> make(int device = 0);
    hip_context(hip_context&& other) noexcept;
    hip_context& operator=(hip_context&& other) noexcept;
    hip_context(const hip_context&) = delete;
    hip_context& operator=(const hip_context&) = delete;
    ~hip_context();

    ckv_context* get() const noexcept { return ctx_; }
    result<void, ckv_failure> sync() const;
    ckv_failure last(int code) const { return { code, ckv_last_error(ctx_) }; }

private:
    explicit hip_context(ckv_context* ctx) noexcept
        : ctx_(ctx)
    {}
    ckv_context* ctx_ = nullptr;
};

// Move-only device allocation.
class device_buffer {
public:
    static result<device_buffer, ckv_failure> make(const hip_context& ctx, std::size_t bytes);
    device_buffer() = default;
    device_buffer(device_buffer&& other) noexcept;
    device_buffer& operator=(device_buffer&& other) noexcept;
    device_buffer(const device_buffer&) = delete;
    device_buffer& operator=(const device_buffer&) = delete;
    ~device_buffer();

    void* data() const noexcept { return ptr_; }
    std::size_t size_bytes() const noexcept { return bytes_; }
    result<void, ckv_failure> upload(const void* host, std::size_t bytes);
    result<void, ckv_failure> download(void* host, std::size_t bytes) const;

private:
    ckv_context* ctx_ = nullptr;
    void* ptr_ = nullptr;
    std::size_t bytes_ = 0;
};

// Move-only pinned host allocation (ckv_host_alloc); freeing it waits for the
// context stream, so queued copies from or to it finish first.
class host_buffer {
public:
    static result<host_buffer, ckv_failure> make(const hip_context& ctx, std::size_t bytes);
    host_buffer() = default;
    host_buffer(host_buffer&& other) noexcept;
    host_buffer& operator=(host_buffer&& other) noexcept;
    host_buffer(const host_buffer&) = delete;
    host_buffer& operator=(const host_buffer&) = delete;
    ~host_buffer();

    void* data() const noexcept { return ptr_; }
    std::size_t size_bytes() const noexcept { return bytes_; }

private:
    ckv_context* ctx_ = nullptr;
    void* ptr_ = nullptr;
    std::size_t bytes_ = 0;
};

struct kv_cache_config {
    std::size_t layer_count;
    std::size_t block_count;
    std::size_t block_size;
    std::size_t kv_head_count;
    std::size_t head_dimension;
};

enum class kv_cache_errc : std::uint8_t {
    invalid_layer_count,
    invalid_block_count,
    invalid_block_size,
    invalid_kv_head_count,
    invalid_head_dimension,
    layout_size_overflow,
    allocation_failed,
    layer_out_of_range,
    block_out_of_range,
    token_offset_out_of_range,
    kv_head_out_of_range,
    head_feature_out_of_range,
};

[[nodiscard]] inline std::string_view
error_name(kv_cache_errc code) noexcept
{
    static constexpr std::array<std::string_view, 12> names {
        "kv_cache.invalid_layer_count",    "kv_cache.invalid_block_count",
        "kv_cache.invalid_block_size",     "kv_cache.invalid_kv_head_count",
        "kv_cache.invalid_head_dimension", "kv_cache.layout_size_overflow",
        "kv_cache.allocation_failed",      "kv_cache.layer_out_of_range",
        "kv_cache.block_out_of_range",     "kv_cache.token_offset_out_of_range",
        "kv_cache.kv_head_out_of_range",   "kv_cache.head_feature_out_of_range",
    };
    const auto i = static_cast<std::size_t>(code);
    return i < names.size() ? names[i] : "kv_cache.unknown_error";
}

using kv_cache_error = error<kv_cache_errc>;

// Packed [layer, token, kv_head, feature] copy of a prefix, independent of
// page ids (src/metal/metal_kv_cache.h:24-40), held in device memory.
struct kv_cache_checkpoint : model_checkpoint {
    kv_cache_checkpoint(kv_cache_config c, std::size_t tokens)
        : model_checkpoint(tokens)
        , config(c)
    {}
    kv_cache_config config;
    device_buffer keys;
    device_buffer values;
    std::size_t size_bytes() const noexcept override
    {
        return keys.size_bytes() + values.size_bytes();
    }
};

// The same packed data in pinned host memory (ckv_checkpoint_export): where the
// reference keeps its checkpoints (host byte vectors, src/metal/metal_kv_cache.h:24-40),
// so a prefix outlives its pages without holding HBM.
struct host_kv_checkpoint : model_checkpoint {
    host_kv_checkpoint(kv_cache_config c, std::size_t tokens)
        : model_checkpoint(tokens)
        , config(c)
    {}
    kv_cache_config config;
    host_buffer keys;
    host_buffer values;
    std::size_t size_bytes() const noexcept override
    {
        return keys.size_bytes() + values.size_bytes();
    }
};

class hip_kv_cache {
public:
    [[nodiscard]] static result<hip_kv_cache, kv_cache_error>
    make(const hip_context& ctx, kv_cache_config config, kv_dtype type = kv_dtype::bf16);

    hip_kv_cache(hip_kv_cache&& other) noexcept;
    hip_kv_cache& operator=(hip_kv_cache&& other) noexcept;
    hip_kv_cache(const hip_kv_cache&) = delete;
    hip_kv_cache& operator=(const hip_kv_cache&) = delete;
    ~hip_kv_cache();

    const kv_cache_config& config() const noexcept { return config_; }
    kv_dtype type() const noexcept { return type_; }
    std::size_t layer_count() const noexcept { return config_.layer_count; }
    std::size_t block_count() const noexcept { return config_.block_count; }
    std::size_t block_size() const noexcept { return config_.block_size; }
    std::size_t kv_head_count() const noexcept { return config_.kv_head_count; }
    std::size_t head_dimension() const noexcept { return config_.head_dimension; }
    std::size_t elements_per_token() const noexcept
    {
        return config_.kv_head_count * config_.head_dimension;
    }
    std::size_t elements_per_block() const noexcept
    {
        return config_.block_size * elements_per_token();
    }
    std::size_t elements_per_layer() const noexcept
    {
        return config_.block_count * elements_per_block();
    }
    std::size_t element_count() const noexcept { return config_.layer_count * elements_per_layer(); }
    // Bytes of one page across all layers, keys and values.
    std::size_t page_bytes_all_layers() const noexcept
    {
        return 2 * config_.layer_count * elements_per_block() * element_bytes(type_);
    }

    [[nodiscard]] result<std::size_t, kv_cache_error> element_offset(std::size_t layer,
                                                                     std::size_t block,
                                                                     std::size_t token_offset,
                                                                     std::size_t kv_head,
                                                                     std::size_t feature) const
        noexcept;

    ckv_pool* pool() const noexcept { return pool_; }
    const hip_context& context() const noexcept { return *ctx_; }
    void* keys() const noexcept;
    void* values() const noexcept;

    // Packed checkpoints with the reference's semantics (metal_kv_cache.cc:205-253):
    // only the first `tokens` tokens are copied, the tail page partially.
    std::size_t checkpoint_bytes(std::size_t tokens) const noexcept;
    result<std::unique_ptr<kv_cache_checkpoint>, state_error>
    checkpoint(std::span<const block_id> blocks, std::size_t tokens) const;
    result<void, state_error> restore(std::span<const block_id> blocks,
                                      const kv_cache_checkpoint& saved);
    // The packed prefix to and from pinned host memory. Both are queued on the
    // context stream; the checkpoint's buffers wait for it before they are freed.
    result<std::unique_ptr<host_kv_checkpoint>, state_error>
    export_prefix(std::span<const block_id> blocks, std::size_t tokens) const;
    result<void, state_error> import_prefix(std::span<const block_id> blocks,
                                            const host_kv_checkpoint& saved);
    // Page copies on the device, all layers, keys and values.
    result<void, state_error> copy_pages(std::span<const block_id> from,
                                         std::span<const block_id> to);

private:
    hip_kv_cache(const hip_context* ctx, ckv_pool* pool, kv_cache_config config, kv_dtype type)
        : ctx_(ctx)
        , pool_(pool)
        , config_(config)
        , type_(type)
    {}
    const hip_context* ctx_ = nullptr;
    ckv_pool* pool_ = nullptr;
    kv_cache_config config_ {};
    kv_dtype type_ = kv_dtype::bf16;
};

} // namespace chibillm
