#include "scheduler.h"

#include <algorithm>
#include <cassert>
#include <limits>
#include <new>
#include <string>

#include "model_batch.h"

namespace chibillm {

namespace {
// Pages a sequence may ever need: prompt plus max_new_tokens - 1 outputs (the
// final sample ends the sequence without another forward pass).
std::optional<std::size_t>
cache_budget(const seq& s, std::size_t block_size) noexcept
{
    const std::size_t prompt = s.prompt_token_count();
    const std::size_t outputs = s.params().max_new_tokens - 1;
    if (outputs > std::numeric_limits<std::size_t>::max() - prompt)
        return std::nullopt;
    return 1 + (prompt + outputs - 1) / block_size;
}
} // namespace

std::size_t
scheduled_batch::token_count() const noexcept
{
    std::size_t n = 0;
    for (const auto& item : items)
        n += item.token_count;
    return n;
}

result<scheduler, scheduler_error>
scheduler::make(scheduler_config config, token_id eos_token, std::unique_ptr<model_state> state)
{
    if (config.max_sequences == 0)
        return fail(scheduler_errc::invalid_max_sequences);
    if (config.max_batch_tokens == 0)
        return fail(scheduler_errc::invalid_max_batch_tokens);
    if (config.prefill_chunk_tokens == 0)
        return fail(scheduler_errc::invalid_prefill_chunk_tokens);
    if (!state) {
        if (config.kv_block_count == 0)
            return fail(scheduler_errc::invalid_kv_block_count);
        if (config.kv_block_size == 0)
            return fail(scheduler_errc::invalid_kv_block_size);
        auto pages = block_manager::make(config.kv_block_count, config.kv_block_size);
        if (!pages)
            return fail(scheduler_errc::block_manager_failure, pages.error());
        state = std::make_unique<block_manager>(std::move(*pages));
    }
    if (state->block_size()) {
        if (config.kv_block_count == 0)
            return fail(scheduler_errc::invalid_kv_block_count);
        if (config.kv_block_size != state->block_size())
            return fail(scheduler_errc::invalid_kv_block_size);
    }
    return scheduler(config, eos_token, std::move(state));
}

scheduler::scheduler(scheduler_config config, token_id eos, std::unique_ptr<model_state> state)
    : config_(config)
    , eos_(eos)
    , state_(std::move(state))
    , prefixes_(config.prefix_cache_bytes)
{
    check_invariants();
}

bool
scheduler::is_finished() const noexcept
{
    return waiting_.empty() && running_.empty() && !active_;
}

const seq*
scheduler::find_sequence(seq_id id) const noexcept
{
    const auto it = sequences_.find(id);
    return it == sequences_.end() ? nullptr : &it->second;
}

seq*
scheduler::mutable_sequence(seq_id id) noexcept
{
    const auto it = sequences_.find(id);
    return it == sequences_.end() ? nullptr : &it->second;
}

bool
scheduler::fits_cache(const seq& sequence) const noexcept
{
    if (!state_->block_size())
        return true;
    const auto pages = cache_budget(sequence, state_->block_size());
    return pages && *pages <= config_.kv_block_count;
}

result<void, scheduler_error>
scheduler::add(seq sequence)
{
    auto admitted = try_add(sequence);
    if (!admitted)
        return fail(admitted.error());
    if (*admitted == admission_result::deferred)
        return fail(scheduler_errc::admission_deferred);
    if (*admitted == admission_result::too_large)
        return fail(scheduler_errc::sequence_exceeds_cache_capacity);
    return {};
}

result<admission_result, scheduler_error>
scheduler::try_add(seq& sequence)
{
    if (active_)
        return fail(scheduler_errc::batch_in_flight);
    const seq_id id = sequence.id();
    if (sequences_.count(id))
        return fail(scheduler_errc::duplicate_sequence_id);
    const bool pristine = sequence.status() == seq_status::waiting
        && sequence.scheduled_token_count() == 0 && sequence.processed_token_count() == 0
        && sequence.token_count() == sequence.prompt_token_count();
    if (!pristine)
        return fail(scheduler_errc::invalid_sequence_state);
    if (!fits_cache(sequence))
        return admission_result::too_large;
    if (waiting_.size() + running_.size() >= config_.max_sequences)
        return admission_result::deferred;

    // every admitted sequence holds its whole page budget against the pool
    if (const std::size_t bs = state_->block_size()) {
        std::size_t committed = 0;
        for (const auto* queue : { &waiting_, &running_ })
            for (const seq_id other : *queue)
                committed += *cache_budget(*find_sequence(other), bs);
        assert(committed <= config_.kv_block_count);
        if (*cache_budget(sequence, bs) > config_.kv_block_count - committed)
            return admission_result::deferred;
    }

    // per-sequence state is created here so a failure affects only this request
    auto reserved = state_->reserve(id, 1);
    if (!reserved) {
        state_->release(id);
        return fail(scheduler_errc::block_manager_failure, reserved.error(), "admit sequence");
    }
    if (const model_checkpoint* cached = prefixes_.find(sequence.prompt_tokens())) {
        bool restored = false;
        try {
            restored = state_->restore(id, *cached).has_value();
        } catch (const std::bad_alloc&) {
        }
        if (restored) {
            auto applied = sequence.restore_prefix(cached->token_count);
            assert(applied);
            (void)applied;
        } else {
            // a failed restore falls back to a cold prefill
            state_->release(id);
            reserved = state_->reserve(id, 1);
            if (!reserved) {
                state_->release(id);
                return fail(scheduler_errc::block_manager_failure, reserved.error(),
                            "admit sequence");
            }
        }
    }
    sequences_.emplace(id, std::move(sequence));
    waiting_.push_back(id);
    check_invariants();
    return admission_result::admitted;
}

result<void, scheduler_error>
scheduler::select(scheduled_batch& batch, std::deque<seq_id>& queue, std::size_t item_limit)
{
    const bool prefill = batch.phase == batch_phase::prefill;
    const bool contended = waiting_.size() > 1 || !running_.empty();
    const std::size_t quantum = prefill && contended ? config_.prefill_chunk_tokens
                                                     : config_.max_batch_tokens;
    const std::size_t max_items = std::min(item_limit, config_.max_sequences);
    batch.items.reserve(max_items);
    std::size_t used = 0;
    for (const seq_id id : queue) {
        if (batch.items.size() >= max_items || used >= config_.max_batch_tokens)
            break;
        seq* s = mutable_sequence(id);
        assert(s);
        const std::size_t available = s->schedulable_token_count();
        if (available == 0 || (!prefill && available != 1))
            return fail(scheduler_errc::invalid_sequence_state);
        std::size_t count = std::min({ available, quantum, config_.max_batch_tokens - used });
        if (prefill) {
            // stop the chunk at the first checkpoint worth caching
            const std::size_t start = s->processed_token_count();
            for (const std::size_t boundary : s->checkpoints()) {
                if (boundary > start && boundary < start + count && cacheable_prefix(boundary)
                    && !prefixes_.contains(s->prompt_tokens().first(boundary))) {
                    count = boundary - start;
                    break;
                }
            }
        }
        auto capacity = state_->reserve(id, s->processed_token_count() + count);
        if (!capacity) {
            if (capacity.error() == state_errc::capacity_exhausted)
                return fail(scheduler_errc::cache_capacity_exhausted, capacity.error());
            return fail(scheduler_errc::block_manager_failure, capacity.error(),
                        "reserve sequence " + std::to_string(id));
        }
        auto scheduled = s->schedule_tokens(count);
        if (!scheduled)
            return fail(scheduler_errc::sequence_failure, scheduled.error(), "reserve tokens");
        batch.items.push_back({ id, count, count == available });
        used += count;
    }
    return {};
}

result<scheduled_batch, scheduler_error>
scheduler::schedule()
{
    if (active_)
        return fail(scheduler_errc::batch_in_flight);
    if (waiting_.empty() && running_.empty())
        return fail(scheduler_errc::no_runnable_sequences);
    if (std::holds_alternative<prefill_turn>(turn_) && waiting_.empty())
        turn_ = decode_round { running_.size() };
    const auto* round = std::get_if<decode_round>(&turn_);
    scheduled_batch batch { next_batch_, round ? batch_phase::decode : batch_phase::prefill, {} };
    auto& queue = round ? running_ : waiting_;
    auto selected = select(batch, queue, round ? round->remaining : queue.size());
    if (!selected) {
        rollback_reservations(batch);
        return fail(selected.error());
    }
    if (batch.empty())
        return fail(scheduler_errc::no_runnable_sequences);
    active_ = batch;
    ++next_batch_;
    check_invariants();
    return batch;
}

result<void, scheduler_error>
scheduler::begin_execution(const model_batch& batch)
{
    if (!active_)
        return fail(scheduler_errc::no_batch_in_flight);
    if (active_->id != batch.id)
        return fail(scheduler_errc::batch_id_mismatch);
    if (transaction_open_)
        return fail(scheduler_errc::batch_in_flight);
    transaction_open_ = true;
    auto begun = state_->begin_batch(batch);
    if (!begun)
        return fail(scheduler_errc::block_manager_failure, begun.error(),
                    "begin model state transaction");
    return {};
}

result<std::vector<sequence_update>, scheduler_error>
scheduler::complete(batch_id id, std::span<const token_id> sampled)
{
    if (!active_)
        return fail(scheduler_errc::no_batch_in_flight);
    const scheduled_batch& batch = *active_;
    if (id != batch.id)
        return fail(scheduler_errc::batch_id_mismatch);
    const auto samples = static_cast<std::size_t>(
        std::count_if(batch.items.begin(), batch.items.end(), [](const auto& i) { return i.sample; }));
    if (sampled.size() != samples)
        return fail(scheduler_errc::result_count_mismatch);

    if (transaction_open_) {
        state_->commit_batch();
        transaction_open_ = false;
    }
    const bool prefill = batch.phase == batch_phase::prefill;
    std::vector<sequence_update> updates;
    updates.reserve(samples);
    std::size_t next_sample = 0;
    for (const scheduled_item& item : batch.items) {
        seq* s = mutable_sequence(item.id);
        assert(s);
        auto committed = s->commit_scheduled_tokens();
        if (!committed)
            return fail(scheduler_errc::sequence_failure, committed.error());
        if (prefill)
            cache_prefix(*s);
        auto& source = prefill ? waiting_ : running_;
        assert(!source.empty() && source.front() == item.id);
        source.pop_front();
        if (!item.sample) { // an unfinished prompt goes to the back of the line
            waiting_.push_back(item.id);
            continue;
        }
        if (prefill) {
            auto running = s->mark_running();
            if (!running)
                return fail(scheduler_errc::sequence_failure, running.error());
        }
        // the sample is the next unprocessed token: the one-token cache gap
        auto appended = s->append_token(sampled[next_sample++]);
        if (!appended)
            return fail(scheduler_errc::sequence_failure, appended.error());
        const finish_reason stop = s->evaluate_stop(eos_);
        if (stop != finish_reason::none) {
            auto finished = s->finish(stop);
            if (!finished)
                return fail(scheduler_errc::sequence_failure, finished.error());
            state_->release(item.id);
        } else {
            running_.push_back(item.id);
        }
        updates.push_back({ item.id, s->last_token(), s->reason() });
    }
    if (prefill) {
        if (!running_.empty())
            turn_ = decode_round { running_.size() };
    } else {
        auto& round = std::get<decode_round>(turn_);
        round.remaining -= batch.items.size();
        if (round.remaining == 0)
            turn_ = prefill_turn {};
    }
    active_.reset();
    check_invariants();
    return updates;
}

result<void, scheduler_error>
scheduler::abort(batch_id id)
{
    if (!active_)
        return fail(scheduler_errc::no_batch_in_flight);
    if (id != active_->id)
        return fail(scheduler_errc::batch_id_mismatch);
    if (transaction_open_) {
        state_->abort_batch();
        transaction_open_ = false;
    }
    rollback_reservations(*active_);
    active_.reset();
    check_invariants();
    return {};
}

result<void, scheduler_error>
scheduler::cancel(seq_id id)
{
    if (active_)
        return fail(scheduler_errc::batch_in_flight);
    seq* s = mutable_sequence(id);
    if (!s)
        return fail(scheduler_errc::unknown_sequence);
    if (s->is_finished())
        return {};
    const bool running = s->status() == seq_status::running;
    auto& queue = running ? running_ : waiting_;
    const auto where = std::find(queue.begin(), queue.end(), id);
    if (where == queue.end())
        return fail(scheduler_errc::invalid_sequence_state);
    if (running) {
        // a sequence not yet visited in this decode round shortens the round
        if (auto* round = std::get_if<decode_round>(&turn_)) {
            if (static_cast<std::size_t>(where - queue.begin()) < round->remaining
                && --round->remaining == 0)
                turn_ = prefill_turn {};
        }
    }
    queue.erase(where);
    auto finished = s->finish(finish_reason::cancelled);
    if (!finished)
        return fail(scheduler_errc::sequence_failure, finished.error());
    state_->release(id);
    check_invariants();
    return {};
}

result<void, scheduler_error>
scheduler::remove(seq_id id)
{
    if (active_)
        return fail(scheduler_errc::batch_in_flight);
    const auto it = sequences_.find(id);
    if (it == sequences_.end())
        return fail(scheduler_errc::unknown_sequence);
    if (!it->second.is_finished())
        return fail(scheduler_errc::invalid_sequence_state);
    sequences_.erase(it);
    check_invariants();
    return {};
}

void
scheduler::cache_prefix(const seq& s) noexcept
try {
    const std::size_t count = s.processed_token_count();
    const auto boundaries = s.checkpoints();
    if (!std::binary_search(boundaries.begin(), boundaries.end(), count)
        || !cacheable_prefix(count))
        return;
    const auto tokens = s.prompt_tokens().first(count);
    if (prefixes_.contains(tokens))
        return;
    prefixes_.make_room(count, state_->checkpoint_bytes(count));
    auto saved = state_->checkpoint(s.id(), count);
    if (saved)
        prefixes_.insert(tokens, std::move(*saved));
} catch (const std::bad_alloc&) {
    // checkpoints are optional: generation continues without one
}

bool
scheduler::cacheable_prefix(std::size_t count) const noexcept
{
    return count >= config_.prefix_cache_min_tokens
        && prefixes_.fits(count, state_->checkpoint_bytes(count));
}

void
scheduler::rollback_reservations(const scheduled_batch& batch) noexcept
{
    for (const scheduled_item& item : batch.items) {
        seq* s = mutable_sequence(item.id);
        assert(s && s->scheduled_token_count() == item.token_count);
        if (s)
            s->cancel_scheduled_tokens();
    }
}

void
scheduler::check_invariants() const noexcept
{
    assert(config_.max_sequences > 0 && config_.max_batch_tokens > 0);
    assert(config_.prefill_chunk_tokens > 0 && state_);
    assert(waiting_.size() + running_.size() <= config_.max_sequences);
    if (const auto* round = std::get_if<decode_round>(&turn_)) {
        assert(round->remaining > 0 && round->remaining <= running_.size());
        (void)round;
    }
}

} // namespace chibillm
