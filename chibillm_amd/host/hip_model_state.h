// model_state over the device KV pool (the class that replaces
// metal_model_state, src/metal/metal_model_state.h:6-84): a refcounted
// block_manager for the pages and a hip_kv_cache for their contents.
//
// Prefix checkpoints come in three forms:
//  - shared (default, new): the checkpoint takes a reference on the prefix's
//    pages; restoring it gives the new sequence the same physical full pages
//    and a private copy of a partial tail page (copy-on-write on the device).
//    Nothing else is copied and full pages are never written again: every new
//    token lands at a position past the prefix. When a reservation finds the
//    pool exhausted, shared checkpoints that alone hold pages are spilled,
//    oldest first: the prefix is exported to pinned host memory in the packed
//    layout and the pages are released. A spilled checkpoint restores like a
//    packed one.
//  - packed: the reference's behaviour (metal_kv_cache::checkpoint/restore):
//    the prefix is copied out to a packed device buffer and copied back into
//    the new sequence's own pages.
//  - host: the packed copy kept in pinned host memory, where the reference
//    keeps its checkpoints (host byte vectors): no HBM is held by the cache.
#pragma once

#include <list>
#include <memory>

#include "block_manager.h"
#include "hip_kv_cache.h"
#include "tensor_ops.h"

namespace chibillm {

enum class prefix_sharing {
    shared_pages,
    packed_copy,
    host_copy,
};

struct shared_prefix_checkpoint;
// The live shared checkpoints, oldest first: the candidates for a spill.
using shared_checkpoint_list = std::list<shared_prefix_checkpoint*>;

// A prefix held as references on physical pages, or, once spilled, as a
// packed copy in host memory.
struct shared_prefix_checkpoint : model_checkpoint {
    shared_prefix_checkpoint(std::shared_ptr<block_manager> owner,
                             std::shared_ptr<shared_checkpoint_list> live,
                             std::vector<block_id> pages, std::size_t tokens, std::size_t bytes)
        : model_checkpoint(tokens)
        , owner(std::move(owner))
        , live(std::move(live))
        , pages(std::move(pages))
        , bytes(bytes)
    {
        where = this->live->insert(this->live->end(), this);
    }
    ~shared_prefix_checkpoint() override
    {
        owner->drop(pages); // empty once spilled
        live->erase(where);
    }
    std::size_t size_bytes() const noexcept override { return bytes; }
    bool is_spilled() const noexcept { return spilled != nullptr; }

    std::shared_ptr<block_manager> owner;
    std::shared_ptr<shared_checkpoint_list> live;
    shared_checkpoint_list::iterator where;
    std::vector<block_id> pages; // ceil(tokens / block_size) pages, one reference each
    std::size_t bytes;           // KV bytes those pages hold, all layers
    std::unique_ptr<host_kv_checkpoint> spilled; // the prefix after a spill
};

class hip_model_state final : public model_state {
public:
    static result<std::unique_ptr<hip_model_state>, state_error>
    make(const hip_context& ctx, kv_cache_config config, kv_dtype type = kv_dtype::bf16,
         prefix_sharing sharing = prefix_sharing::shared_pages);

    // A reservation the pool cannot hold spills shared checkpoints first.
    result<void, state_error> reserve(seq_id id, std::size_t tokens) override;
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
    // Shared checkpoints moved to host memory to free pages, and the pages freed.
    std::size_t spills() const noexcept { return spills_; }
    std::size_t spilled_pages() const noexcept { return spilled_pages_; }
    // Spilling is on by default; off, an exhausted pool fails the reservation.
    void set_spill(bool on) noexcept { spill_ = on; }

private:
    hip_model_state(std::shared_ptr<block_manager> pages, hip_kv_cache cache,
                    prefix_sharing sharing)
        : pages_(std::move(pages))
        , cache_(std::move(cache))
        , sharing_(sharing)
    {}
    result<void, state_error> restore_shared(seq_id id, const shared_prefix_checkpoint& saved);
    // Spills shared checkpoints, oldest first, until `pages` pages are free.
    bool spill_for(std::size_t pages) noexcept;

    std::shared_ptr<block_manager> pages_;
    hip_kv_cache cache_;
    prefix_sharing sharing_;
    std::size_t cow_copies_ = 0;
    std::unique_ptr<device_tables> tables_;
    std::shared_ptr<shared_checkpoint_list> live_ = std::make_shared<shared_checkpoint_list>();
    bool spill_ = true;
    std::size_t spills_ = 0, spilled_pages_ = 0;
};

} // namespace chibillm
