// model_state over the device KV pool (the class that replaces
// metal_model_state, src/metal/metal_model_state.h:6-84): a refcounted
// block_manager for the pages and a hip_kv_cache for their contents.
//
// Prefix checkpoints come in two forms:
//  - shared (default, new): the checkpoint takes a reference on the prefix's
//    pages; restoring it gives the new sequence the same physical full pages
//    and a private copy of a partial tail page (copy-on-write on the device).
//    Nothing else is copied and full pages are never written again: every new
//    token lands at a position past the prefix.
//  - packed: the reference's behaviour (metal_kv_cache::checkpoint/restore):
//    the prefix is copied out to a packed buffer and copied back into the new
//    sequence's own pages.
#pragma once

#include <memory>

#include "block_manager.h"
#include "hip_kv_cache.h"
#include "tensor_ops.h"

namespace chibillm {

enum class prefix_sharing {
    shared_pages,
    packed_copy,
};

// A prefix held as references on physical pages.
struct shared_prefix_checkpoint : model_checkpoint {
    shared_prefix_checkpoint(std::shared_ptr<block_manager> owner, std::vector<block_id> pages,
                             std::size_t tokens, std::size_t bytes)
        : model_checkpoint(tokens)
        , owner(std::move(owner))
        , pages(std::move(pages))
        , bytes(bytes)
    {}
    ~shared_prefix_checkpoint() override { owner->drop(pages); }
    std::size_t size_bytes() const noexcept override { return bytes; }

    std::shared_ptr<block_manager> owner;
    std::vector<block_id> pages; // ceil(tokens / block_size) pages, one reference each
    std::size_t bytes;           // KV bytes those pages hold, all layers
};

class hip_model_state final : public model_state {
public:
    static result<std::unique_ptr<hip_model_state>, state_error>
    make(const hip_context& ctx, kv_cache_config config, kv_dtype type = kv_dtype::bf16,
         prefix_sharing sharing = prefix_sharing::shared_pages);

    result<void, state_error> reserve(seq_id id, std::size_t tokens) override
    {
        return pages_->reserve(id, tokens);
    }
    void release(seq_id id) noexcept override
    {
        pages_->release(id);
        if (tables_)
            tables_->release(id);
    }
    std::size_t block_size() const noexcept override { return pages_->block_size(); }
    sequence_resources resources(seq_id id) const noexcept override
    {
        return pages_->resources(id);
    }

    std::size_t checkpoint_bytes(std::size_t tokens) const noexcept override;
    result<std::unique_ptr<model_checkpoint>, state_error> checkpoint(seq_id id,
                                                                      std::size_t tokens) const override;
    result<void, state_error> restore(seq_id id, const model_checkpoint& saved) override;

    // Keeps the sequences' block tables on the device (device_tables); the
    // rows of released sequences are returned to it.
    result<void, tensor_op_error> enable_device_tables(std::size_t max_sequences,
                                                       std::size_t pages_per_sequence)
    {
        auto made = device_tables::make(cache_, max_sequences, pages_per_sequence);
        if (!made)
            return fail(made.error());
        tables_ = std::make_unique<device_tables>(std::move(*made));
        return {};
    }
    device_tables* tables() noexcept { return tables_.get(); }

    hip_kv_cache& cache() noexcept { return cache_; }
    const hip_kv_cache& cache() const noexcept { return cache_; }
    const block_manager& pages() const noexcept { return *pages_; }
    prefix_sharing sharing() const noexcept { return sharing_; }
    // Page copies made by restores of shared checkpoints (copy-on-write count).
    std::size_t cow_copies() const noexcept { return cow_copies_; }

private:
    hip_model_state(std::shared_ptr<block_manager> pages, hip_kv_cache cache,
                    prefix_sharing sharing)
        : pages_(std::move(pages))
        , cache_(std::move(cache))
        , sharing_(sharing)
    {}
    result<void, state_error> restore_shared(seq_id id, const shared_prefix_checkpoint& saved);

    std::shared_ptr<block_manager> pages_;
    hip_kv_cache cache_;
    prefix_sharing sharing_;
    std::size_t cow_copies_ = 0;
    std::unique_ptr<device_tables> tables_;
};

} // namespace chibillm
