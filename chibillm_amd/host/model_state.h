// Backend state behind the scheduler (the contract of src/model_state.h:10-100):
// per-sequence page reservations, optional prefix checkpoints and a batch
// transaction. Implemented by block_manager (pages only) and hip_model_state
// (pages + the device KV pool).
#pragma once

#include <memory>
#include <span>

#include "error.h"
#include "result.h"
#include "seq.h"

namespace chibillm {

struct model_batch;

enum class state_errc {
    capacity_exhausted,
    invalid_reservation,
    backend_failure,
    allocation_failed,
};

[[nodiscard]] inline std::string_view
error_name(state_errc code) noexcept
{
    static constexpr std::array<std::string_view, 4> names {
        "state.capacity_exhausted",
        "state.invalid_reservation",
        "state.backend_failure",
        "state.allocation_failed",
    };
    const auto i = static_cast<std::size_t>(code);
    return i < names.size() ? names[i] : "state.unknown_error";
}

using state_error = error<state_errc>;

// Non-owning; valid until the next reserve/release of that sequence.
struct sequence_resources {
    std::span<const block_id> blocks;
};

// An immutable, backend-owned image of the state after an exact token prefix.
struct model_checkpoint {
    explicit model_checkpoint(std::size_t tokens) noexcept
        : token_count(tokens)
    {}
    virtual ~model_checkpoint() = default;
    const std::size_t token_count;
    virtual std::size_t size_bytes() const noexcept = 0;
};

class model_state {
public:
    virtual ~model_state() = default;
    // Capacity for at least token_count tokens; smaller requests keep what exists.
    virtual result<void, state_error> reserve(seq_id id, std::size_t token_count) = 0;
    // Unknown ids are harmless.
    virtual void release(seq_id id) noexcept = 0;

    // Zero: checkpoints unsupported or the prefix out of range.
    virtual std::size_t checkpoint_bytes(std::size_t) const noexcept { return 0; }
    virtual result<std::unique_ptr<model_checkpoint>, state_error> checkpoint(seq_id,
                                                                              std::size_t) const
    {
        return std::unique_ptr<model_checkpoint> {};
    }
    // Into a fresh reservation, between batches.
    virtual result<void, state_error> restore(seq_id, const model_checkpoint&)
    {
        return fail(state_errc::invalid_reservation);
    }

    virtual std::size_t block_size() const noexcept { return 0; }
    virtual sequence_resources resources(seq_id) const noexcept { return {}; }

    // A failed batch must leave the pre-batch state for the retry.
    virtual result<void, state_error> begin_batch(const model_batch&) { return {}; }
    virtual void commit_batch() noexcept {}
    virtual void abort_batch() noexcept {}
};

} // namespace chibillm
