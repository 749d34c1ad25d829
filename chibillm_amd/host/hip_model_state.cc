#include "hip_model_state.h"

namespace chibillm {

result<std::unique_ptr<hip_model_state>, state_error>
hip_model_state::make(const hip_context& ctx, kv_cache_config config, kv_dtype type,
                      prefix_sharing sharing)
{
    auto pages = block_manager::make(config.block_count, config.block_size);
    if (!pages)
        return fail(state_errc::invalid_reservation, pages.error(), "block allocator");
    auto cache = hip_kv_cache::make(ctx, config, type);
    if (!cache)
        return fail(state_errc::backend_failure, cache.error(), "KV cache");
    return std::unique_ptr<hip_model_state>(new hip_model_state(
        std::make_shared<block_manager>(std::move(*pages)), std::move(*cache), sharing));
}

result<void, state_error>
hip_model_state::reserve(seq_id id, std::size_t tokens)
{
    auto reserved = pages_->reserve(id, tokens);
    if (reserved || reserved.error().code != state_errc::capacity_exhausted || !spill_)
        return reserved;
    const std::size_t bs = pages_->block_size();
    const std::size_t required = tokens ? 1 + (tokens - 1) / bs : 0;
    const std::size_t held = pages_->resources(id).blocks.size();
    if (required <= held || !spill_for(required - held))
        return reserved;
    return pages_->reserve(id, tokens);
}

bool
hip_model_state::spill_for(std::size_t pages) noexcept
try {
    // passes until no checkpoint frees a page: spilling one checkpoint can
    // leave an older one (a shorter prefix of the same pages) the only holder
    for (bool progress = true; progress && pages_->free_block_count() < pages;) {
        progress = false;
        for (shared_prefix_checkpoint* saved : *live_) {
            if (pages_->free_block_count() >= pages)
                break;
            if (saved->is_spilled())
                continue;
            // only pages that nothing else references come free
            std::size_t freed = 0;
            for (const block_id b : saved->pages)
                freed += pages_->refcount(b) == 1;
            if (!freed)
                continue;
            // the export is queued before any later write of the freed pages
            auto exported = cache_.export_prefix(saved->pages, saved->token_count);
            if (!exported)
                return false;
            saved->spilled = std::move(*exported);
            pages_->drop(saved->pages);
            saved->pages.clear();
            ++spills_;
            spilled_pages_ += freed;
            progress = true;
        }
    }
    return pages_->free_block_count() >= pages;
} catch (const std::bad_alloc&) {
    return false;
}

std::size_t
hip_model_state::checkpoint_bytes(std::size_t tokens) const noexcept
{
    if (sharing_ != prefix_sharing::shared_pages)
        return cache_.checkpoint_bytes(tokens);
    if (!tokens || tokens > cache_.block_count() * cache_.block_size())
        return 0;
    // the pages a shared checkpoint keeps alive
    return (1 + (tokens - 1) / cache_.block_size()) * cache_.page_bytes_all_layers();
}

result<std::unique_ptr<model_checkpoint>, state_error>
hip_model_state::checkpoint(seq_id id, std::size_t tokens) const
{
    const auto table = resources(id).blocks;
    if (sharing_ == prefix_sharing::packed_copy) {
        auto saved = cache_.checkpoint(table, tokens);
        if (!saved)
            return fail(saved.error());
        return std::unique_ptr<model_checkpoint>(std::move(*saved));
    }
    if (sharing_ == prefix_sharing::host_copy) {
        auto saved = cache_.export_prefix(table, tokens);
        if (!saved)
            return fail(saved.error());
        return std::unique_ptr<model_checkpoint>(std::move(*saved));
    }
    const std::size_t bytes = checkpoint_bytes(tokens);
    if (!bytes)
        return fail(state_errc::invalid_reservation);
    const std::size_t needed = 1 + (tokens - 1) / cache_.block_size();
    if (table.size() < needed)
        return fail(state_errc::invalid_reservation);
    std::vector<block_id> held(table.begin(), table.begin() + needed);
    CL_TRY(pages_->retain(held));
    return std::unique_ptr<model_checkpoint>(
        std::make_unique<shared_prefix_checkpoint>(pages_, live_, std::move(held), tokens, bytes));
}

result<void, state_error>
hip_model_state::restore(seq_id id, const model_checkpoint& saved)
{
    const host_kv_checkpoint* host = dynamic_cast<const host_kv_checkpoint*>(&saved);
    if (const auto* shared = dynamic_cast<const shared_prefix_checkpoint*>(&saved)) {
        if (!shared->is_spilled())
            return restore_shared(id, *shared);
        host = shared->spilled.get();
    }
    if (host) { // reserve, copy in from host memory
        CL_TRY(reserve(id, host->token_count));
        return cache_.import_prefix(resources(id).blocks, *host);
    }
    const auto* packed = dynamic_cast<const kv_cache_checkpoint*>(&saved);
    if (!packed)
        return fail(state_errc::invalid_reservation);
    // the reference path (src/metal/metal_model_state.h:60-68): reserve, copy in
    CL_TRY(reserve(id, packed->token_count));
    return cache_.restore(resources(id).blocks, *packed);
}

result<void, state_error>
hip_model_state::restore_shared(seq_id id, const shared_prefix_checkpoint& saved)
{
    const std::size_t bs = cache_.block_size();
    const auto own = resources(id).blocks;
    // a fresh reservation holds exactly the one page admission reserved
    if (saved.owner != pages_ || own.size() != 1 || saved.pages.empty())
        return fail(state_errc::invalid_reservation);
    const block_id fresh = own[0];
    const std::size_t full = saved.token_count / bs;
    const bool partial_tail = saved.token_count % bs != 0;
    if (partial_tail) {
        // copy-on-write of the shared tail page into the sequence's own page,
        // which follows the shared full pages in its table
        const block_id tail = saved.pages[full];
        CL_TRY(cache_.copy_pages(std::span(&tail, 1), std::span(&fresh, 1)));
        ++cow_copies_;
    }
    // the own page now covers positions [full * bs, (full + 1) * bs)
    return pages_->share_prefix(id, std::span(saved.pages).first(full));
}

} // namespace chibillm
