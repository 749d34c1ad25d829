#include "hip_kv_cache.h"

#include <limits>
#include <utility>

namespace chibillm {

// ---- hip_context ----------------------------------------------------------------

result<hip_context, ckv_failure>
hip_context::make(int device)
{
    ckv_context* ctx = nullptr;
    const int rc = ckv_context_create(device, &ctx);
    if (rc)
        return fail(ckv_failure { rc, "context creation" });
    return hip_context(ctx);
}

hip_context::hip_context(hip_context&& other) noexcept
    : ctx_(std::exchange(other.ctx_, nullptr))
{}

hip_context&
hip_context::operator=(hip_context&& other) noexcept
{
    if (this != &other) {
        if (ctx_)
            ckv_context_destroy(ctx_);
        ctx_ = std::exchange(other.ctx_, nullptr);
    }
    return *this;
}

hip_context::~hip_context()
{
    if (ctx_)
        ckv_context_destroy(ctx_);
}

result<void, ckv_failure>
hip_context::sync() const
{
    const int rc = ckv_sync(ctx_);
    if (rc)
        return fail(last(rc));
    return {};
}

// ---- device_buffer ----------------------------------------------------------------

result<device_buffer, ckv_failure>
device_buffer::make(const hip_context& ctx, std::size_t bytes)
{
    device_buffer b;
    const int rc = ckv_device_alloc(ctx.get(), bytes, &b.ptr_);
    if (rc)
        return fail(ctx.last(rc));
    b.ctx_ = ctx.get();
    b.bytes_ = bytes;
    return b;
}

device_buffer::device_buffer(device_buffer&& other) noexcept
    : ctx_(std::exchange(other.ctx_, nullptr))
    , ptr_(std::exchange(other.ptr_, nullptr))
    , bytes_(std::exchange(other.bytes_, 0))
{}

device_buffer&
device_buffer::operator=(device_buffer&& other) noexcept
{
    if (this != &other) {
        if (ptr_)
            ckv_device_free(ctx_, ptr_);
        ctx_ = std::exchange(other.ctx_, nullptr);
        ptr_ = std::exchange(other.ptr_, nullptr);
        bytes_ = std::exchange(other.bytes_, 0);
    }
    return *this;
}

device_buffer::~device_buffer()
{
    if (ptr_)
        ckv_device_free(ctx_, ptr_);
}

result<void, ckv_failure>
device_buffer::upload(const void* host, std::size_t bytes)
{
    const int rc = ckv_copy_to_device(ctx_, ptr_, host, bytes);
    if (rc)
        return fail(ckv_failure { rc, ckv_last_error(ctx_) });
    return {};
}

result<void, ckv_failure>
device_buffer::download(void* host, std::size_t bytes) const
{
    const int rc = ckv_copy_to_host(ctx_, host, ptr_, bytes);
    if (rc)
        return fail(ckv_failure { rc, ckv_last_error(ctx_) });
    return {};
}

result<host_buffer, ckv_failure>
host_buffer::make(const hip_context& ctx, std::size_t bytes)
{
    host_buffer b;
    const int rc = ckv_host_alloc(ctx.get(), bytes, &b.ptr_);
    if (rc)
        return fail(ctx.last(rc));
    b.ctx_ = ctx.get();
    b.bytes_ = bytes;
    return b;
}

host_buffer::host_buffer(host_buffer&& other) noexcept
    : ctx_(std::exchange(other.ctx_, nullptr))
    , ptr_(std::exchange(other.ptr_, nullptr))
    , bytes_(std::exchange(other.bytes_, 0))
{}

host_buffer&
host_buffer::operator=(host_buffer&& other) noexcept
{
    if (this != &other) {
        if (ptr_)
            ckv_host_free(ctx_, ptr_);
        ctx_ = std::exchange(other.ctx_, nullptr);
        ptr_ = std::exchange(other.ptr_, nullptr);
        bytes_ = std::exchange(other.bytes_, 0);
    }
    return *this;
}

host_buffer::~host_buffer()
{
    if (ptr_)
        ckv_host_free(ctx_, ptr_);
}

// ---- hip_kv_cache ------------------------------------------------------------------

result<hip_kv_cache, kv_cache_error>
hip_kv_cache::make(const hip_context& ctx, kv_cache_config c, kv_dtype type)
{
    ckv_pool* pool = nullptr;
    const int rc = ckv_pool_create(ctx.get(), c.layer_count, c.block_count, c.block_size,
                                   c.kv_head_count, c.head_dimension, static_cast<int>(type), &pool);
    if (rc >= 200 && rc < 212)
        return fail(kv_cache_error { static_cast<kv_cache_errc>(rc - 200), ckv_last_error(ctx.get()) });
    if (rc)
        return fail(kv_cache_error { kv_cache_errc::allocation_failed,
                                     describe_error(ctx.last(rc)) });
    return hip_kv_cache(&ctx, pool, c, type);
}

hip_kv_cache::hip_kv_cache(hip_kv_cache&& other) noexcept
    : ctx_(other.ctx_)
    , pool_(std::exchange(other.pool_, nullptr))
    , config_(other.config_)
    , type_(other.type_)
{}

hip_kv_cache&
hip_kv_cache::operator=(hip_kv_cache&& other) noexcept
{
    if (this != &other) {
        if (pool_)
            ckv_pool_destroy(pool_);
        ctx_ = other.ctx_;
        pool_ = std::exchange(other.pool_, nullptr);
        config_ = other.config_;
        type_ = other.type_;
    }
    return *this;
}

hip_kv_cache::~hip_kv_cache()
{
    if (pool_)
        ckv_pool_destroy(pool_);
}

void*
hip_kv_cache::keys() const noexcept
{
    void* k = nullptr;
    ckv_pool_buffers(pool_, &k, nullptr, nullptr);
    return k;
}

void*
hip_kv_cache::values() const noexcept
{
    void* v = nullptr;
    ckv_pool_buffers(pool_, nullptr, &v, nullptr);
    return v;
}

result<std::size_t, kv_cache_error>
hip_kv_cache::element_offset(std::size_t layer, std::size_t block, std::size_t token_offset,
                             std::size_t kv_head, std::size_t feature) const noexcept
{
    std::size_t offset = 0;
    const int rc = ckv_element_offset(pool_, layer, block, token_offset, kv_head, feature, &offset);
    if (rc)
        return fail(static_cast<kv_cache_errc>(rc - 200));
    return offset;
}

std::size_t
hip_kv_cache::checkpoint_bytes(std::size_t tokens) const noexcept
{
    // src/metal/metal_kv_cache.cc:205-212, at this cache's element size
    if (!tokens || tokens > block_count() * block_size())
        return 0;
    const std::size_t bytes = tokens * elements_per_token() * layer_count() * element_bytes(type_);
    return bytes <= std::numeric_limits<std::size_t>::max() / 2 ? 2 * bytes : 0;
}

result<std::unique_ptr<kv_cache_checkpoint>, state_error>
hip_kv_cache::checkpoint(std::span<const block_id> blocks, std::size_t tokens) const
{
    const std::size_t bytes = checkpoint_bytes(tokens);
    if (!bytes)
        return fail(state_errc::invalid_reservation);
    auto saved = std::make_unique<kv_cache_checkpoint>(config_, tokens);
    auto k = device_buffer::make(*ctx_, bytes / 2);
    auto v = device_buffer::make(*ctx_, bytes / 2);
    if (!k || !v)
        return fail(state_errc::allocation_failed);
    saved->keys = std::move(*k);
    saved->values = std::move(*v);
    const int rc = ckv_checkpoint_pack(pool_, blocks.data(), blocks.size(), tokens,
                                       saved->keys.data(), saved->values.data());
    if (rc == CKV_E_STATE_INVALID_RESERVATION)
        return fail(state_errc::invalid_reservation);
    if (rc)
        return fail(state_errc::backend_failure, ctx_->last(rc), "checkpoint pack");
    return saved;
}

result<void, state_error>
hip_kv_cache::restore(std::span<const block_id> blocks, const kv_cache_checkpoint& saved)
{
    const bool same_geometry = saved.config.layer_count == layer_count()
        && saved.config.kv_head_count == kv_head_count()
        && saved.config.head_dimension == head_dimension();
    const std::size_t bytes = checkpoint_bytes(saved.token_count);
    if (!same_geometry || !bytes || saved.keys.size_bytes() != bytes / 2
        || saved.values.size_bytes() != bytes / 2)
        return fail(state_errc::invalid_reservation);
    const int rc = ckv_checkpoint_unpack(pool_, blocks.data(), blocks.size(), saved.token_count,
                                         saved.keys.data(), saved.values.data());
    if (rc == CKV_E_STATE_INVALID_RESERVATION)
        return fail(state_errc::invalid_reservation);
    if (rc)
        return fail(state_errc::backend_failure, ctx_->last(rc), "checkpoint unpack");
    return {};
}

result<std::unique_ptr<host_kv_checkpoint>, state_error>
hip_kv_cache::export_prefix(std::span<const block_id> blocks, std::size_t tokens) const
{
    const std::size_t bytes = checkpoint_bytes(tokens);
    if (!bytes)
        return fail(state_errc::invalid_reservation);
    auto saved = std::make_unique<host_kv_checkpoint>(config_, tokens);
    auto k = host_buffer::make(*ctx_, bytes / 2);
    auto v = host_buffer::make(*ctx_, bytes / 2);
    if (!k || !v)
        return fail(state_errc::allocation_failed);
    saved->keys = std::move(*k);
    saved->values = std::move(*v);
    const int rc = ckv_checkpoint_export(pool_, blocks.data(), blocks.size(), tokens,
                                         saved->keys.data(), saved->values.data());
    if (rc == CKV_E_STATE_INVALID_RESERVATION)
        return fail(state_errc::invalid_reservation);
    if (rc)
        return fail(state_errc::backend_failure, ctx_->last(rc), "checkpoint export");
    return saved;
}

result<void, state_error>
hip_kv_cache::import_prefix(std::span<const block_id> blocks, const host_kv_checkpoint& saved)
{
    const bool same_geometry = saved.config.layer_count == layer_count()
        && saved.config.kv_head_count == kv_head_count()
        && saved.config.head_dimension == head_dimension();
    const std::size_t bytes = checkpoint_bytes(saved.token_count);
    if (!same_geometry || !bytes || saved.keys.size_bytes() != bytes / 2
        || saved.values.size_bytes() != bytes / 2)
        return fail(state_errc::invalid_reservation);
    const int rc = ckv_checkpoint_import(pool_, blocks.data(), blocks.size(), saved.token_count,
                                         saved.keys.data(), saved.values.data());
    if (rc == CKV_E_STATE_INVALID_RESERVATION)
        return fail(state_errc::invalid_reservation);
    if (rc)
        return fail(state_errc::backend_failure, ctx_->last(rc), "checkpoint import");
    return {};
}

result<void, state_error>
hip_kv_cache::copy_pages(std::span<const block_id> from, std::span<const block_id> to)
{
    if (from.size() != to.size())
        return fail(state_errc::invalid_reservation);
    const int rc = ckv_copy_blocks(pool_, from.data(), to.data(), from.size());
    if (rc)
        return fail(state_errc::backend_failure, ctx_->last(rc), "page copy");
    return {};
}

} // namespace chibillm
