// The continuous-batching scheduler. Its contract, as the scheduler tests in
// tests/cpp pin it (the behaviour of src/scheduler.h:20-210):
//
// Admission (try_add), between batches only, of a sequence that has done
// nothing yet: too_large when its lifetime page budget (prompt plus
// max_new_tokens - 1 samples; the last sample is never processed) exceeds the
// pool; deferred when max_sequences are live or the pool's uncommitted pages
// cannot hold the budget. An admitted sequence commits its whole budget until
// it finishes, gets its model state (one token reserved) and, when the prefix
// cache holds a proper prefix of its prompt, starts from that checkpoint.
//
// Batches (schedule): the scheduler alternates a prefill turn (one batch from
// the waiting queue) with a decode round (every running sequence once, in
// queue order, over as many batches as the limits need); with nothing
// waiting it keeps to decode rounds, and a round in progress finishes before
// the next prefill. A prefill item takes the sequence's schedulable tokens up
// to the batch budget, and, when others compete for the batch, up to
// prefill_chunk_tokens; it stops early at a checkpoint boundary whose prefix
// is worth caching and not cached yet. A decode item is one token. Pages for
// every item are reserved before the batch is returned.
//
// Completion (complete) commits the scheduled tokens in batch order: prefill
// items publish a checkpoint when they end on a boundary; an item that does
// not sample goes to the back of the waiting queue; one that samples appends
// its sample (a prefill item first becomes running), then either finishes on
// EOS or the length limit (its pages released, its budget returned) or joins
// the back of the running queue. abort() undoes the batch's scheduling but
// keeps its pages for the retry; cancel() finishes a live sequence.
#include "scheduler.h"

#include <algorithm>
#include <cassert>
#include <limits>
#include <new>
#include <string>

#include "model_batch.h"

namespace chibillm {

std::size_t
scheduled_batch::token_count() const noexcept
{
    std::size_t total = 0;
    for (const scheduled_item& item : items)
        total += item.token_count;
    return total;
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
    // a paged state (its own, or a default block_manager) must agree with the
    // geometry the admission budget is computed from
    const bool own_pages = !state;
    if (own_pages || state->block_size() != 0) {
        if (config.kv_block_count == 0)
            return fail(scheduler_errc::invalid_kv_block_count);
        const std::size_t page = own_pages ? config.kv_block_size : state->block_size();
        if (config.kv_block_size == 0 || config.kv_block_size != page)
            return fail(scheduler_errc::invalid_kv_block_size);
    }
    if (own_pages) {
        auto pages = block_manager::make(config.kv_block_count, config.kv_block_size);
        if (!pages)
            return fail(scheduler_errc::block_manager_failure, pages.error());
        state = std::make_unique<block_manager>(std::move(*pages));
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
    return !active_ && waiting_.empty() && running_.empty();
}

scheduler::member*
scheduler::find_member(seq_id id) noexcept
{
    const auto at = members_.find(id);
    return at == members_.end() ? nullptr : &at->second;
}

const seq*
scheduler::find_sequence(seq_id id) const noexcept
{
    const auto at = members_.find(id);
    return at == members_.end() ? nullptr : &at->second.sequence;
}

// ---- admission -----------------------------------------------------------------

std::optional<std::size_t>
scheduler::page_budget(const seq& s) const noexcept
{
    const std::size_t page = state_->block_size();
    if (page == 0)
        return 0; // an unpaged state: nothing to commit
    const std::size_t prompt = s.prompt_token_count();
    const std::size_t samples = s.params().max_new_tokens - 1; // max_new_tokens >= 1
    if (samples > std::numeric_limits<std::size_t>::max() - prompt)
        return std::nullopt;
    const std::size_t tokens = prompt + samples; // >= 1
    return tokens / page + (tokens % page != 0);
}

bool
scheduler::fits_cache(const seq& sequence) const noexcept
{
    const auto budget = page_budget(sequence);
    return budget && (state_->block_size() == 0 || *budget <= config_.kv_block_count);
}

bool
scheduler::restore_checkpoint(seq_id id, const model_checkpoint& saved) noexcept
{
    try {
        return state_->restore(id, saved).has_value();
    } catch (const std::bad_alloc&) {
        return false;
    }
}

result<void, scheduler_error>
scheduler::open_state(seq& s)
{
    const seq_id id = s.id();
    // one token of state per sequence from its admission; a failure leaves no trace
    auto first_page = [&]() -> result<void, scheduler_error> {
        auto got = state_->reserve(id, 1);
        if (got)
            return {};
        state_->release(id);
        return fail(scheduler_errc::block_manager_failure, got.error(), "admit sequence");
    };
    if (auto opened = first_page(); !opened)
        return opened;
    const model_checkpoint* cached = prefixes_.find(s.prompt_tokens());
    if (!cached)
        return {};
    if (restore_checkpoint(id, *cached)) {
        [[maybe_unused]] auto restored = s.restore_prefix(cached->token_count);
        assert(restored);
        return {};
    }
    // the checkpoint could not be restored: the sequence starts cold
    state_->release(id);
    return first_page();
}

result<admission_result, scheduler_error>
scheduler::try_add(seq& sequence)
{
    if (active_)
        return fail(scheduler_errc::batch_in_flight);
    if (members_.contains(sequence.id()))
        return fail(scheduler_errc::duplicate_sequence_id);
    const bool untouched = sequence.status() == seq_status::waiting
        && sequence.processed_token_count() == 0 && sequence.scheduled_token_count() == 0
        && sequence.completion_token_count() == 0;
    if (!untouched)
        return fail(scheduler_errc::invalid_sequence_state);
    if (!fits_cache(sequence))
        return admission_result::too_large;
    const std::size_t budget = *page_budget(sequence);
    if (waiting_.size() + running_.size() >= config_.max_sequences)
        return admission_result::deferred;
    if (state_->block_size() != 0 && budget > config_.kv_block_count - committed_pages_)
        return admission_result::deferred;
    if (auto opened = open_state(sequence); !opened)
        return fail(opened.error());
    const seq_id id = sequence.id();
    members_.emplace(id, member { std::move(sequence), budget });
    waiting_.push_back(id);
    committed_pages_ += budget;
    check_invariants();
    return admission_result::admitted;
}

result<void, scheduler_error>
scheduler::add(seq sequence)
{
    auto outcome = try_add(sequence);
    if (!outcome)
        return fail(outcome.error());
    switch (*outcome) {
    case admission_result::admitted:
        return {};
    case admission_result::deferred:
        return fail(scheduler_errc::admission_deferred);
    case admission_result::too_large:
        break;
    }
    return fail(scheduler_errc::sequence_exceeds_cache_capacity);
}

// ---- batches ------------------------------------------------------------------------

bool
scheduler::worth_caching(std::size_t count) const noexcept
{
    return count >= config_.prefix_cache_min_tokens
        && prefixes_.fits(count, state_->checkpoint_bytes(count));
}

std::size_t
scheduler::checkpoint_cut(const seq& s, std::size_t tokens) const noexcept
{
    const std::size_t from = s.processed_token_count();
    const auto prompt = s.prompt_tokens();
    for (const std::size_t boundary : s.checkpoints()) {
        if (boundary <= from)
            continue;
        if (boundary >= from + tokens)
            break; // boundaries are sorted
        if (worth_caching(boundary) && !prefixes_.contains(prompt.first(boundary)))
            return boundary - from;
    }
    return tokens;
}

result<std::vector<scheduler::planned>, scheduler_error>
scheduler::plan(bool prefill, std::size_t limit) const
{
    const auto& queue = prefill ? waiting_ : running_;
    const bool competing = waiting_.size() > 1 || !running_.empty();
    const std::size_t per_item = prefill && competing ? config_.prefill_chunk_tokens
                                                      : config_.max_batch_tokens;
    const std::size_t max_items = std::min(limit, config_.max_sequences);
    std::vector<planned> items;
    std::size_t budget = config_.max_batch_tokens;
    for (auto it = queue.begin(); it != queue.end() && items.size() < max_items && budget > 0;
         ++it) {
        const seq& s = members_.at(*it).sequence;
        const std::size_t open = s.schedulable_token_count();
        if (open == 0 || (!prefill && open != 1))
            return fail(scheduler_errc::invalid_sequence_state);
        std::size_t take = std::min({ open, per_item, budget });
        if (prefill)
            take = checkpoint_cut(s, take);
        items.push_back({ *it, take, take == open });
        budget -= take;
    }
    return items;
}

void
scheduler::unschedule(const scheduled_batch& batch) noexcept
{
    for (const scheduled_item& item : batch.items)
        if (member* m = find_member(item.id))
            m->sequence.cancel_scheduled_tokens();
}

result<void, scheduler_error>
scheduler::reserve(const std::vector<planned>& items, scheduled_batch& batch)
{
    for (const planned& p : items) {
        seq& s = members_.at(p.id).sequence;
        auto room = state_->reserve(p.id, s.processed_token_count() + p.tokens);
        if (!room) {
            unschedule(batch); // pages already reserved stay with their sequences
            if (room.error() == state_errc::capacity_exhausted)
                return fail(scheduler_errc::cache_capacity_exhausted, room.error());
            return fail(scheduler_errc::block_manager_failure, room.error(),
                        "reserve sequence " + std::to_string(p.id));
        }
        if (auto booked = s.schedule_tokens(p.tokens); !booked) {
            unschedule(batch);
            return fail(scheduler_errc::sequence_failure, booked.error(), "reserve tokens");
        }
        batch.items.push_back({ p.id, p.tokens, p.samples });
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
    if (decode_left_ == 0 && waiting_.empty())
        decode_left_ = running_.size(); // a new decode round: everyone running, once
    const bool prefill = decode_left_ == 0;
    auto items = plan(prefill, prefill ? waiting_.size() : decode_left_);
    if (!items)
        return fail(items.error());
    if (items->empty())
        return fail(scheduler_errc::no_runnable_sequences);
    scheduled_batch batch { next_batch_, prefill ? batch_phase::prefill : batch_phase::decode, {} };
    batch.items.reserve(items->size());
    if (auto reserved = reserve(*items, batch); !reserved)
        return fail(reserved.error());
    ++next_batch_;
    active_ = batch;
    check_invariants();
    return batch;
}

result<void, scheduler_error>
scheduler::begin_execution(const model_batch& batch)
{
    if (!active_)
        return fail(scheduler_errc::no_batch_in_flight);
    if (batch.id != active_->id)
        return fail(scheduler_errc::batch_id_mismatch);
    if (transaction_open_)
        return fail(scheduler_errc::batch_in_flight);
    transaction_open_ = true;
    if (auto begun = state_->begin_batch(batch); !begun)
        return fail(scheduler_errc::block_manager_failure, begun.error(),
                    "begin model state transaction");
    return {};
}

// ---- completion --------------------------------------------------------------------

void
scheduler::publish_prefix(const seq& s) noexcept
{
    const std::size_t count = s.processed_token_count();
    const auto boundaries = s.checkpoints();
    if (!std::binary_search(boundaries.begin(), boundaries.end(), count) || !worth_caching(count))
        return;
    const auto prefix = s.prompt_tokens().first(count);
    if (prefixes_.contains(prefix))
        return;
    try {
        prefixes_.make_room(count, state_->checkpoint_bytes(count));
        if (auto saved = state_->checkpoint(s.id(), count))
            prefixes_.insert(prefix, std::move(*saved));
    } catch (const std::bad_alloc&) {
        // a checkpoint is an optimisation: the sequence goes on without one
    }
}

void
scheduler::leave(seq_id id, member& m) noexcept
{
    state_->release(id);
    committed_pages_ -= m.budget;
}

result<void, scheduler_error>
scheduler::settle(seq_id id, member& m, token_id sample, bool prefill)
{
    seq& s = m.sequence;
    if (prefill)
        if (auto running = s.mark_running(); !running)
            return fail(scheduler_errc::sequence_failure, running.error());
    // the sample becomes the unprocessed token of the one-token cache gap
    if (auto appended = s.append_token(sample); !appended)
        return fail(scheduler_errc::sequence_failure, appended.error());
    const finish_reason stop = s.evaluate_stop(eos_);
    if (stop == finish_reason::none) {
        running_.push_back(id);
        return {};
    }
    if (auto finished = s.finish(stop); !finished)
        return fail(scheduler_errc::sequence_failure, finished.error());
    leave(id, m);
    return {};
}

result<std::vector<sequence_update>, scheduler_error>
scheduler::complete(batch_id id, std::span<const token_id> sampled)
{
    if (!active_)
        return fail(scheduler_errc::no_batch_in_flight);
    if (id != active_->id)
        return fail(scheduler_errc::batch_id_mismatch);
    const scheduled_batch& batch = *active_;
    const auto sampling = static_cast<std::size_t>(std::count_if(
        batch.items.begin(), batch.items.end(), [](const scheduled_item& i) { return i.sample; }));
    if (sampled.size() != sampling)
        return fail(scheduler_errc::result_count_mismatch);

    if (std::exchange(transaction_open_, false))
        state_->commit_batch();
    const bool prefill = batch.phase == batch_phase::prefill;
    std::deque<seq_id>& served_from = prefill ? waiting_ : running_;
    std::vector<sequence_update> updates;
    updates.reserve(sampling);
    auto sample = sampled.begin();
    for (const scheduled_item& item : batch.items) {
        member& m = members_.at(item.id);
        if (auto committed = m.sequence.commit_scheduled_tokens(); !committed)
            return fail(scheduler_errc::sequence_failure, committed.error());
        if (prefill)
            publish_prefix(m.sequence);
        assert(!served_from.empty() && served_from.front() == item.id);
        served_from.pop_front();
        if (!item.sample) {
            waiting_.push_back(item.id); // the rest of its prompt waits its turn
            continue;
        }
        if (auto settled = settle(item.id, m, *sample++, prefill); !settled)
            return fail(settled.error());
        updates.push_back({ item.id, m.sequence.last_token(), m.sequence.reason() });
    }
    // a prefill turn hands over to a decode round of everyone running; a
    // decode batch serves the round's first members
    decode_left_ = prefill ? running_.size() : decode_left_ - batch.items.size();
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
    if (std::exchange(transaction_open_, false))
        state_->abort_batch();
    unschedule(*active_);
    active_.reset();
    check_invariants();
    return {};
}

result<void, scheduler_error>
scheduler::cancel(seq_id id)
{
    if (active_)
        return fail(scheduler_errc::batch_in_flight);
    member* m = find_member(id);
    if (!m)
        return fail(scheduler_errc::unknown_sequence);
    if (m->sequence.is_finished())
        return {};
    const bool running = m->sequence.status() == seq_status::running;
    std::deque<seq_id>& queue = running ? running_ : waiting_;
    const auto at = std::find(queue.begin(), queue.end(), id);
    if (at == queue.end())
        return fail(scheduler_errc::invalid_sequence_state);
    // a member the current decode round has not served yet leaves the round
    if (running && static_cast<std::size_t>(at - queue.begin()) < decode_left_)
        --decode_left_;
    queue.erase(at);
    if (auto finished = m->sequence.finish(finish_reason::cancelled); !finished)
        return fail(scheduler_errc::sequence_failure, finished.error());
    leave(id, *m);
    check_invariants();
    return {};
}

result<void, scheduler_error>
scheduler::remove(seq_id id)
{
    if (active_)
        return fail(scheduler_errc::batch_in_flight);
    const auto at = members_.find(id);
    if (at == members_.end())
        return fail(scheduler_errc::unknown_sequence);
    if (!at->second.sequence.is_finished())
        return fail(scheduler_errc::invalid_sequence_state);
    members_.erase(at);
    check_invariants();
    return {};
}

void
scheduler::check_invariants() const noexcept
{
    assert(state_ && config_.max_sequences > 0 && config_.max_batch_tokens > 0);
    assert(config_.prefill_chunk_tokens > 0);
    assert(waiting_.size() + running_.size() <= config_.max_sequences);
    assert(decode_left_ <= running_.size());
    assert(state_->block_size() == 0 || committed_pages_ <= config_.kv_block_count);
}

} // namespace chibillm
