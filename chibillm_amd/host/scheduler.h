// Continuous-batching scheduler (the interface and behaviour of
// src/scheduler.h:20-210 and src/scheduler.cc): admission against a page
// budget, alternation between a prefill turn and a decode round over the
// running sequences, chunked prefill split at uncached checkpoint boundaries,
// commit / abort / cancel of the one batch in flight, and prefix checkpoints
// published into a prefix_cache.
#pragma once

#include <deque>
#include <memory>
#include <optional>
#include <span>
#include <unordered_map>
#include <vector>

#include "block_manager.h"
#include "prefix_cache.h"
#include "seq.h"

namespace chibillm {

using batch_id = std::uint64_t;

enum class batch_phase : std::uint8_t {
    prefill,
    decode,
};

struct scheduler_config {
    std::size_t max_sequences { 4 };
    std::size_t max_batch_tokens { 128 };
    std::size_t kv_block_count { 256 };
    std::size_t kv_block_size { 16 };
    // applied only when other sequences compete for the batch
    std::size_t prefill_chunk_tokens { 64 };
    std::size_t prefix_cache_bytes { 128 * 1024 * 1024 };
    std::size_t prefix_cache_min_tokens { 64 };
};

enum class admission_result : std::uint8_t {
    admitted,
    deferred,
    too_large,
};

struct sequence_update {
    seq_id id;
    token_id token;
    finish_reason reason;
};

struct scheduled_item {
    seq_id id;
    std::size_t token_count;
    bool sample { true };
};

struct scheduled_batch {
    batch_id id;
    batch_phase phase;
    std::vector<scheduled_item> items;

    [[nodiscard]] bool empty() const noexcept { return items.empty(); }
    [[nodiscard]] std::size_t token_count() const noexcept;
};

enum class scheduler_errc : std::uint8_t {
    invalid_max_sequences,
    invalid_max_batch_tokens,
    invalid_kv_block_count,
    invalid_kv_block_size,
    duplicate_sequence_id,
    invalid_sequence_state,
    unknown_sequence,
    batch_in_flight,
    no_batch_in_flight,
    batch_id_mismatch,
    result_count_mismatch,
    no_runnable_sequences,
    cache_capacity_exhausted,
    block_manager_failure,
    sequence_failure,
    invalid_prefill_chunk_tokens,
    admission_deferred,
    sequence_exceeds_cache_capacity,
};

[[nodiscard]] inline std::string_view
error_name(scheduler_errc code) noexcept
{
    static constexpr std::array<std::string_view, 18> names {
        "scheduler.invalid_max_sequences",    "scheduler.invalid_max_batch_tokens",
        "scheduler.invalid_kv_block_count",   "scheduler.invalid_kv_block_size",
        "scheduler.duplicate_sequence_id",    "scheduler.invalid_sequence_state",
        "scheduler.unknown_sequence",         "scheduler.batch_in_flight",
        "scheduler.no_batch_in_flight",       "scheduler.batch_id_mismatch",
        "scheduler.result_count_mismatch",    "scheduler.no_runnable_sequences",
        "scheduler.cache_capacity_exhausted", "scheduler.block_manager_failure",
        "scheduler.sequence_failure",         "scheduler.invalid_prefill_chunk_tokens",
        "scheduler.admission_deferred",       "scheduler.sequence_exceeds_cache_capacity",
    };
    const auto i = static_cast<std::size_t>(code);
    return i < names.size() ? names[i] : "scheduler.unknown_error";
}

using scheduler_error = error<scheduler_errc>;

class scheduler {
public:
    // Without a state, a block_manager of kv_block_count x kv_block_size is used.
    [[nodiscard]] static result<scheduler, scheduler_error>
    make(scheduler_config config, token_id eos_token, std::unique_ptr<model_state> state = {});

    scheduler(const scheduler&) = delete;
    scheduler& operator=(const scheduler&) = delete;
    scheduler(scheduler&&) noexcept = default;
    scheduler& operator=(scheduler&&) noexcept = default;

    [[nodiscard]] const scheduler_config& config() const noexcept { return config_; }
    [[nodiscard]] std::size_t sequence_count() const noexcept { return members_.size(); }
    [[nodiscard]] std::size_t waiting_count() const noexcept { return waiting_.size(); }
    [[nodiscard]] std::size_t running_count() const noexcept { return running_.size(); }
    [[nodiscard]] bool has_in_flight_batch() const noexcept { return active_.has_value(); }
    // Finished sequences stay queryable until remove().
    [[nodiscard]] bool is_finished() const noexcept;
    [[nodiscard]] const seq* find_sequence(seq_id id) const noexcept;
    [[nodiscard]] const model_state& state() const noexcept { return *state_; }
    [[nodiscard]] model_state& state() noexcept { return *state_; }
    [[nodiscard]] const prefix_cache& prefixes() const noexcept { return prefixes_; }

    [[nodiscard]] bool fits_cache(const seq& sequence) const noexcept;
    // Only `admitted` moves from the sequence; the caller keeps deferred and
    // too-large requests. Valid only between batches.
    [[nodiscard]] result<admission_result, scheduler_error> try_add(seq& sequence);
    // Strict admission: deferral and oversize become errors.
    [[nodiscard]] result<void, scheduler_error> add(seq sequence);

    // Reserves one prefill or decode batch.
    [[nodiscard]] result<scheduled_batch, scheduler_error> schedule();
    result<void, scheduler_error> begin_execution(const model_batch& batch);
    // Commits the batch; samples apply to the items that sample, in order.
    [[nodiscard]] result<std::vector<sequence_update>, scheduler_error>
    complete(batch_id id, std::span<const token_id> sampled_tokens);
    // Cancels the reservation in flight; pages stay reserved for the retry.
    [[nodiscard]] result<void, scheduler_error> abort(batch_id id);

    [[nodiscard]] result<void, scheduler_error> cancel(seq_id id);
    [[nodiscard]] result<void, scheduler_error> remove(seq_id id);

private:
    // A sequence the scheduler holds (live or finished) and the pages it was
    // admitted against; they are committed while it is waiting or running.
    struct member {
        seq sequence;
        std::size_t budget;
    };
    // One item of a batch before any reservation: how many tokens, and
    // whether they end the sequence's unprocessed tokens (it then samples).
    struct planned {
        seq_id id;
        std::size_t tokens;
        bool samples;
    };

    scheduler(scheduler_config config, token_id eos, std::unique_ptr<model_state> state);
    member* find_member(seq_id id) noexcept;
    std::optional<std::size_t> page_budget(const seq& sequence) const noexcept;
    result<void, scheduler_error> open_state(seq& sequence);
    bool restore_checkpoint(seq_id id, const model_checkpoint& saved) noexcept;
    result<std::vector<planned>, scheduler_error> plan(bool prefill, std::size_t limit) const;
    std::size_t checkpoint_cut(const seq& sequence, std::size_t tokens) const noexcept;
    result<void, scheduler_error> reserve(const std::vector<planned>& items, scheduled_batch& batch);
    result<void, scheduler_error> settle(seq_id id, member& m, token_id sample, bool prefill);
    void leave(seq_id id, member& m) noexcept;
    void unschedule(const scheduled_batch& batch) noexcept;
    bool worth_caching(std::size_t count) const noexcept;
    void publish_prefix(const seq& sequence) noexcept;
    void check_invariants() const noexcept;

    scheduler_config config_;
    token_id eos_;
    std::unique_ptr<model_state> state_;
    prefix_cache prefixes_; // declared after state_: destroyed first
    std::unordered_map<seq_id, member> members_;
    std::deque<seq_id> waiting_;
    std::deque<seq_id> running_;
    std::size_t committed_pages_ = 0; // the budgets of the waiting and running members
    // running members still to serve in the current decode round (they are the
    // first decode_left_ of running_); 0 outside a round, the prefill turn
    std::size_t decode_left_ = 0;
    std::optional<scheduled_batch> active_;
    bool transaction_open_ = false;
    batch_id next_batch_ = 1;
};

} // namespace chibillm
