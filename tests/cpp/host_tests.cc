// CPU tests of the C++ host layer: the reference's own unit tests for the
// sequence, page allocator, scheduler, batch builder, prefix cache and engine
// (tests/*_test.cc in the chibillm tree, cited per case), restated against
// this implementation, plus the refcount invariants sharing adds. No GPU call.
#include <algorithm>
#include <array>
#include <limits>
#include <numeric>
#include <unordered_map>

#include "check.h"
#include "inference_engine.h"
#include "model_batch.h"
#include "prefix_cache.h"

using namespace chibillm;

namespace {

template <typename R, typename C>
bool
error_is(const R& r, C code)
{
    return !r.has_value() && r.error() == code;
}

const block_manager&
pages_of(const scheduler& s)
{
    return dynamic_cast<const block_manager&>(s.state());
}

scheduler_config
small_config()
{
    scheduler_config c;
    c.max_sequences = 4;
    c.max_batch_tokens = 8;
    c.kv_block_count = 8;
    c.kv_block_size = 2;
    return c;
}

void
commit_all(scheduler& s, const scheduled_batch& batch)
{
    std::vector<token_id> samples;
    for (const auto& item : batch.items)
        if (item.sample)
            samples.push_back(42);
    REQUIRE(s.complete(batch.id, samples));
}

seq
make_seq(seq_id id, std::vector<token_id> prompt, std::size_t max_new, bool ignore_eos = false)
{
    auto s = seq::make(id, std::move(prompt), generation_params { max_new, ignore_eos });
    REQUIRE(s);
    return std::move(*s);
}

} // namespace

// ---- seq (tests/seq_test.cc) ---------------------------------------------------------

TEST("seq: a sequence owns its prompt and starts waiting")
{
    auto s = seq::make(7, { 1, 2, 3 }, generation_params {});
    REQUIRE(s);
    CHECK(s->id() == 7);
    CHECK(s->status() == seq_status::waiting && s->reason() == finish_reason::none);
    CHECK(s->token_count() == 3 && s->prompt_token_count() == 3);
    CHECK(s->completion_token_count() == 0 && s->processed_token_count() == 0);
    CHECK(s->scheduled_token_count() == 0 && s->last_token() == 3);
    CHECK(s->prompt_tokens().size() == 3 && s->completion_tokens().empty());
}

TEST("seq: a restored prefix keeps prompt accounting and leaves tokens to execute")
{
    auto s = seq::make(1, { 1, 2, 3, 4 }, generation_params {}, { 3, 1 });
    REQUIRE(s);
    CHECK(s->checkpoints()[0] == 1 && s->checkpoints()[1] == 3);
    CHECK_FALSE(s->restore_prefix(0));
    CHECK_FALSE(s->restore_prefix(4));
    REQUIRE(s->restore_prefix(3));
    CHECK(s->cached_token_count() == 3 && s->prompt_token_count() == 4);
    CHECK(s->completion_token_count() == 0 && s->schedulable_token_count() == 1);
    CHECK_FALSE(s->restore_prefix(2));
    CHECK_FALSE(seq::make(2, { 1, 2 }, generation_params {}, { 2 }));
    CHECK_FALSE(seq::make(2, { 1, 2 }, generation_params {}, { 0 }));
    CHECK_FALSE(seq::make(2, { 1, 2 }, generation_params {}, { 1, 1 }));
}

TEST("seq: invalid construction arguments return specific errors")
{
    CHECK(error_is(seq::make(1, {}, generation_params {}), seq_errc::empty_prompt));
    CHECK(error_is(seq::make(1, { 1 }, generation_params { 0 }), seq_errc::invalid_max_new_tokens));
}

TEST("seq: prefill and decode maintain the one-token cache gap")
{
    auto s = make_seq(1, { 10, 20, 30 }, 64);
    REQUIRE(s.schedule_tokens(3));
    CHECK(s.unprocessed_token_count() == 3 && s.schedulable_token_count() == 0);
    REQUIRE(s.commit_scheduled_tokens());
    REQUIRE(s.mark_running());
    REQUIRE(s.append_token(40));
    CHECK(s.token_count() == 4 && s.completion_token_count() == 1);
    CHECK(s.processed_token_count() == 3 && s.unprocessed_token_count() == 1);
    CHECK(s.completion_tokens().front() == 40);
    REQUIRE(s.schedule_tokens(1));
    REQUIRE(s.commit_scheduled_tokens());
    CHECK(s.processed_token_count() == 4);
}

TEST("seq: a second scheduling reservation cannot overwrite the first")
{
    auto s = make_seq(1, { 1, 2, 3 }, 64);
    REQUIRE(s.schedule_tokens(2));
    CHECK(error_is(s.schedule_tokens(1), seq_errc::work_already_scheduled));
    CHECK(s.scheduled_token_count() == 2);
    s.cancel_scheduled_tokens();
    CHECK(s.scheduled_token_count() == 0 && s.processed_token_count() == 0);
}

TEST("seq: lifecycle transitions reject invalid source states")
{
    auto s = make_seq(1, { 1, 2 }, 64);
    CHECK(error_is(s.mark_running(), seq_errc::invalid_state_transition));
    CHECK(error_is(s.append_token(3), seq_errc::invalid_state_transition));
    REQUIRE(s.schedule_tokens(2));
    CHECK(error_is(s.mark_running(), seq_errc::work_already_scheduled));
    REQUIRE(s.commit_scheduled_tokens());
    REQUIRE(s.mark_running());
    CHECK(error_is(s.mark_running(), seq_errc::invalid_state_transition));
    REQUIRE(s.append_token(3));
    CHECK(error_is(s.append_token(4), seq_errc::invalid_state_transition));
    REQUIRE(s.schedule_tokens(1));
    REQUIRE(s.commit_scheduled_tokens());
}

TEST("seq: EOS and length limits are evaluated after appending")
{
    constexpr token_id eos = 99;
    auto a = make_seq(1, { 1 }, 64);
    CHECK(a.evaluate_stop(eos) == finish_reason::none);
    REQUIRE(a.schedule_tokens(1));
    REQUIRE(a.commit_scheduled_tokens());
    REQUIRE(a.mark_running());
    REQUIRE(a.append_token(eos));
    CHECK(a.evaluate_stop(eos) == finish_reason::eos);
    auto b = make_seq(2, { 1 }, 2, true);
    REQUIRE(b.schedule_tokens(1));
    REQUIRE(b.commit_scheduled_tokens());
    REQUIRE(b.mark_running());
    REQUIRE(b.append_token(eos));
    CHECK(b.evaluate_stop(eos) == finish_reason::none);
    REQUIRE(b.schedule_tokens(1));
    REQUIRE(b.commit_scheduled_tokens());
    REQUIRE(b.append_token(5));
    CHECK(b.evaluate_stop(eos) == finish_reason::len_limit);
}

TEST("seq: finished sequences cannot be revived or mutated")
{
    auto s = make_seq(1, { 1 }, 64);
    CHECK(error_is(s.finish(finish_reason::none), seq_errc::invalid_finish_reason));
    REQUIRE(s.finish(finish_reason::cancelled));
    CHECK(s.is_finished() && s.reason() == finish_reason::cancelled);
    CHECK(error_is(s.schedule_tokens(1), seq_errc::already_finished));
    CHECK(error_is(s.append_token(2), seq_errc::already_finished));
}

// ---- block_manager (tests/block_manager_test.cc) --------------------------------------

TEST("block_manager: paged state validates geometry")
{
    CHECK(error_is(block_manager::make(0, 16), block_manager_errc::invalid_block_count));
    CHECK(error_is(block_manager::make(4, 0), block_manager_errc::invalid_block_size));
    CHECK(error_is(
        block_manager::make(static_cast<std::size_t>(std::numeric_limits<block_id>::max()) + 2, 16),
        block_manager_errc::too_many_blocks));
}

TEST("block_manager: reservations grow at block boundaries and release FIFO")
{
    auto s = block_manager::make(4, 2);
    REQUIRE(s);
    REQUIRE(s->reserve(1, 3));
    CHECK(s->resources(1).blocks.size() == 2 && s->free_block_count() == 2);
    REQUIRE(s->reserve(1, 4));
    CHECK(s->free_block_count() == 2);
    REQUIRE(s->reserve(1, 5));
    CHECK(s->resources(1).blocks.size() == 3);
    REQUIRE(s->reserve(2, 2));
    CHECK(s->resources(2).blocks[0] == 3);
    s->release(1);
    CHECK(s->resources(1).blocks.empty() && s->free_block_count() == 3);
    s->release(1);
    CHECK(s->free_block_count() == 3);
    REQUIRE(s->reserve(3, 1));
    CHECK(s->resources(3).blocks[0] == 0 && s->resources(2).blocks[0] == 3);
}

TEST("block_manager: failed reservations leave existing allocations intact")
{
    auto s = block_manager::make(2, 2);
    REQUIRE(s);
    REQUIRE(s->reserve(1, 2));
    CHECK(error_is(s->reserve(2, 3), state_errc::capacity_exhausted));
    CHECK(s->resources(2).blocks.empty());
    CHECK(error_is(s->reserve(1, 5), state_errc::capacity_exhausted));
    CHECK(s->resources(1).blocks.size() == 1 && s->free_block_count() == 1);
    CHECK(error_is(s->reserve(2, 0), state_errc::invalid_reservation));
}

TEST("block_manager: shared pages are freed only by their last reference")
{
    auto s = block_manager::make(6, 4);
    REQUIRE(s);
    REQUIRE(s->reserve(1, 10)); // pages 0 1 2
    REQUIRE(s->reserve(2, 1));  // page 3
    const std::vector<block_id> prefix { 0, 1 };
    REQUIRE(s->share_prefix(2, prefix)); // table of 2: 0 1 3
    const auto t2 = s->resources(2).blocks;
    CHECK(t2.size() == 3 && t2[0] == 0 && t2[1] == 1 && t2[2] == 3);
    CHECK(s->refcount(0) == 2 && s->refcount(1) == 2 && s->refcount(2) == 1);
    s->release(1);
    CHECK(s->free_block_count() == 3); // page 2 freed; 0 and 1 still held by 2
    CHECK(s->refcount(0) == 1 && s->refcount(2) == 0);
    REQUIRE(s->retain(std::vector<block_id> { 1 }));
    s->release(2);
    CHECK(s->refcount(1) == 1 && s->free_block_count() == 5);
    s->drop(std::vector<block_id> { 1 });
    CHECK(s->free_block_count() == 6);
    // invariant: pages with references + free pages = pool, each page once
    CHECK(error_is(s->retain(std::vector<block_id> { 0 }), state_errc::invalid_reservation));
    CHECK(error_is(s->share_prefix(9, std::vector<block_id> { 4 }), state_errc::invalid_reservation));
}

TEST("block_manager: fork gives a sequence a private page in place of a shared one")
{
    auto s = block_manager::make(4, 2);
    REQUIRE(s);
    REQUIRE(s->reserve(1, 4)); // 0 1
    REQUIRE(s->reserve(2, 1)); // 2
    REQUIRE(s->share_prefix(2, std::vector<block_id> { 0, 1 }));
    auto fresh = s->fork(2, 1);
    REQUIRE(fresh);
    CHECK(*fresh == 3);
    const auto t = s->resources(2).blocks;
    CHECK(t[0] == 0 && t[1] == 3 && t[2] == 2);
    CHECK(s->refcount(1) == 1 && s->refcount(3) == 1);
    CHECK(error_is(s->fork(2, 7), state_errc::invalid_reservation));
    CHECK(error_is(s->fork(1, 0), state_errc::capacity_exhausted));
}

TEST("block_manager: without sharing the allocation order equals a plain FIFO")
{
    // random reserve / release traffic against a model of the reference's deque
    auto s = block_manager::make(64, 4);
    REQUIRE(s);
    std::deque<block_id> model;
    for (block_id b = 0; b < 64; ++b)
        model.push_back(b);
    std::unordered_map<seq_id, std::vector<block_id>> tables;
    std::uint64_t x = 12345;
    auto next = [&] { return x = x * 6364136223846793005ULL + 1442695040888963407ULL; };
    for (int step = 0; step < 4000; ++step) {
        const seq_id id = (next() >> 33) % 12;
        if ((next() >> 40) % 4 == 0) {
            s->release(id);
            for (block_id b : tables[id])
                model.push_back(b);
            tables.erase(id);
        } else {
            const std::size_t tokens = 1 + (next() >> 35) % 40;
            const std::size_t need = (tokens - 1) / 4 + 1;
            auto& t = tables[id];
            const bool fits = need <= t.size() || need - t.size() <= model.size();
            CHECK(s->reserve(id, tokens).has_value() == fits);
            while (fits && t.size() < need) {
                t.push_back(model.front());
                model.pop_front();
            }
        }
        const auto got = s->resources(id).blocks;
        const auto& want = tables[id];
        CHECK(std::equal(got.begin(), got.end(), want.begin(), want.end()));
        CHECK(s->free_block_count() == model.size());
    }
}

// ---- scheduler (tests/scheduler_test.cc) ----------------------------------------------

TEST("scheduler: construction validates limits and exposes cache geometry")
{
    auto c = small_config();
    c.max_sequences = 0;
    CHECK(error_is(scheduler::make(c, 99), scheduler_errc::invalid_max_sequences));
    c = small_config();
    c.max_batch_tokens = 0;
    CHECK(error_is(scheduler::make(c, 99), scheduler_errc::invalid_max_batch_tokens));
    c = small_config();
    c.prefill_chunk_tokens = 0;
    CHECK(error_is(scheduler::make(c, 99), scheduler_errc::invalid_prefill_chunk_tokens));
    c = small_config();
    c.kv_block_count = 0;
    CHECK(error_is(scheduler::make(c, 99), scheduler_errc::invalid_kv_block_count));
    c = small_config();
    c.kv_block_size = 0;
    CHECK(error_is(scheduler::make(c, 99), scheduler_errc::invalid_kv_block_size));
    auto s = scheduler::make(small_config(), 99);
    REQUIRE(s);
    CHECK(s->sequence_count() == 0 && s->waiting_count() == 0 && s->running_count() == 0);
    CHECK(s->is_finished());
    CHECK(pages_of(*s).block_count() == 8 && pages_of(*s).block_size() == 2);
}

TEST("scheduler: completion without an active batch is rejected")
{
    auto s = scheduler::make(small_config(), 99);
    REQUIRE(s);
    CHECK(error_is(s->complete(1, std::array<token_id, 1> { 42 }), scheduler_errc::no_batch_in_flight));
    CHECK_FALSE(s->has_in_flight_batch());
}

TEST("scheduler: add admits one pristine waiting sequence and rejects a duplicate ID")
{
    auto s = scheduler::make(small_config(), 99);
    REQUIRE(s);
    REQUIRE(s->add(make_seq(10, { 1, 2 }, 4)));
    CHECK(s->sequence_count() == 1 && s->waiting_count() == 1 && s->running_count() == 0);
    CHECK(s->find_sequence(10) != nullptr);
    CHECK(error_is(s->add(make_seq(10, { 8 }, 4)), scheduler_errc::duplicate_sequence_id));
    CHECK(s->sequence_count() == 1 && s->waiting_count() == 1);
}

TEST("scheduler: prefill can be chunked and only the final chunk appends a sample")
{
    auto c = small_config();
    c.max_batch_tokens = 2;
    auto s = scheduler::make(c, 99);
    REQUIRE(s);
    REQUIRE(s->add(make_seq(1, { 10, 20, 30 }, 4)));
    auto first = s->schedule();
    REQUIRE(first);
    CHECK(first->phase == batch_phase::prefill && first->items.size() == 1);
    CHECK(first->items[0].token_count == 2);
    CHECK(error_is(s->schedule(), scheduler_errc::batch_in_flight));
    REQUIRE(s->complete(first->id, std::array<token_id, 0> {}));
    const seq* q = s->find_sequence(1);
    CHECK(q->processed_token_count() == 2 && q->token_count() == 3);
    CHECK(q->status() == seq_status::waiting);
    auto last = s->schedule();
    REQUIRE(last);
    CHECK(last->phase == batch_phase::prefill && last->items[0].token_count == 1);
    REQUIRE(s->complete(last->id, std::array<token_id, 1> { 40 }));
    q = s->find_sequence(1);
    CHECK(q->status() == seq_status::running && q->processed_token_count() == 3);
    CHECK(q->completion_token_count() == 1 && q->last_token() == 40);
    CHECK(s->waiting_count() == 0 && s->running_count() == 1);
}

TEST("scheduler: decode commits the old sample and creates the next one-token cache gap")
{
    auto s = scheduler::make(small_config(), 99);
    REQUIRE(s);
    REQUIRE(s->add(make_seq(1, { 10, 20 }, 4)));
    auto prefill = s->schedule();
    REQUIRE(prefill);
    REQUIRE(s->complete(prefill->id, std::array<token_id, 1> { 30 }));
    CHECK(s->find_sequence(1)->token_count() == 3);
    CHECK(s->find_sequence(1)->processed_token_count() == 2);
    auto decode = s->schedule();
    REQUIRE(decode);
    CHECK(decode->phase == batch_phase::decode && decode->items[0].token_count == 1);
    REQUIRE(s->complete(decode->id, std::array<token_id, 1> { 40 }));
    const seq* q = s->find_sequence(1);
    CHECK(q->token_count() == 4 && q->processed_token_count() == 3);
    CHECK(q->unprocessed_token_count() == 1 && q->last_token() == 40);
}

TEST("scheduler: sequences finish on EOS or length limit and release cache blocks")
{
    for (const auto& [max_new, sample, why] :
         { std::tuple { std::size_t(4), token_id(99), finish_reason::eos },
           std::tuple { std::size_t(1), token_id(42), finish_reason::len_limit } }) {
        auto s = scheduler::make(small_config(), 99);
        REQUIRE(s);
        REQUIRE(s->add(make_seq(1, { 10, 20 }, max_new)));
        auto prefill = s->schedule();
        REQUIRE(prefill);
        REQUIRE(s->complete(prefill->id, std::array<token_id, 1> { sample }));
        const seq* q = s->find_sequence(1);
        CHECK(q->status() == seq_status::finished && q->reason() == why);
        CHECK(s->state().resources(1).blocks.empty());
        CHECK(pages_of(*s).used_block_count() == 0 && s->is_finished());
    }
}

TEST("scheduler: cancel releases a running sequence and allows it to be retired")
{
    auto s = scheduler::make(small_config(), 99);
    REQUIRE(s);
    REQUIRE(s->add(make_seq(1, { 10, 20 }, 4)));
    auto prefill = s->schedule();
    REQUIRE(prefill);
    REQUIRE(s->complete(prefill->id, std::array<token_id, 1> { 30 }));
    CHECK(pages_of(*s).used_block_count() == 1);
    REQUIRE(s->cancel(1));
    CHECK(s->find_sequence(1)->reason() == finish_reason::cancelled);
    CHECK(pages_of(*s).used_block_count() == 0 && s->is_finished());
    REQUIRE(s->remove(1));
    CHECK(s->find_sequence(1) == nullptr && s->sequence_count() == 0);
}

TEST("scheduler: completion validation leaves an in-flight reservation untouched")
{
    auto s = scheduler::make(small_config(), 99);
    REQUIRE(s);
    REQUIRE(s->add(make_seq(1, { 10 }, 4)));
    auto batch = s->schedule();
    REQUIRE(batch);
    CHECK(error_is(s->complete(batch->id, std::array<token_id, 0> {}),
                   scheduler_errc::result_count_mismatch));
    CHECK(s->has_in_flight_batch());
    CHECK(s->find_sequence(1)->scheduled_token_count() == 1);
    CHECK(s->find_sequence(1)->processed_token_count() == 0);
}

TEST("scheduler: abort validates active batch and restores reservations")
{
    auto s = scheduler::make(small_config(), 99);
    REQUIRE(s);
    REQUIRE(s->add(make_seq(1, { 10, 20, 30 }, 4)));
    auto batch = s->schedule();
    REQUIRE(batch);
    CHECK(pages_of(*s).used_block_count() == 2);
    CHECK(error_is(s->abort(batch->id + 1), scheduler_errc::batch_id_mismatch));
    CHECK(s->has_in_flight_batch());
    REQUIRE(s->abort(batch->id));
    CHECK_FALSE(s->has_in_flight_batch());
    CHECK(s->waiting_count() == 1 && s->running_count() == 0);
    CHECK(pages_of(*s).used_block_count() == 2);
    CHECK(s->find_sequence(1)->processed_token_count() == 0);
    CHECK(s->find_sequence(1)->scheduled_token_count() == 0);
    CHECK(s->state().resources(1).blocks.size() == 2);
    auto retry = s->schedule();
    REQUIRE(retry);
    CHECK(retry->items.size() == 1 && retry->items[0].id == batch->items[0].id);
    CHECK(retry->items[0].token_count == batch->items[0].token_count);
}

TEST("scheduler: new prefill waits for an existing decode round")
{
    auto s = scheduler::make(small_config(), 99);
    REQUIRE(s);
    REQUIRE(s->add(make_seq(1, { 10 }, 4)));
    auto first = s->schedule();
    REQUIRE(first);
    REQUIRE(s->complete(first->id, std::array<token_id, 1> { 11 }));
    REQUIRE(s->add(make_seq(2, { 20 }, 4)));
    auto next = s->schedule();
    REQUIRE(next);
    CHECK(next->phase == batch_phase::decode && next->items.size() == 1 && next->items[0].id == 1);
    REQUIRE(s->complete(next->id, std::array<token_id, 1> { 12 }));
    next = s->schedule();
    REQUIRE(next);
    CHECK(next->phase == batch_phase::prefill && next->items[0].id == 2);
}

TEST("scheduler: an oversized request is rejected without allocating or consuming it")
{
    auto c = small_config();
    c.kv_block_count = 1;
    auto s = scheduler::make(c, 99);
    REQUIRE(s);
    auto q = make_seq(1, { 10, 20, 30 }, 4);
    auto admitted = s->try_add(q);
    REQUIRE(admitted);
    CHECK(*admitted == admission_result::too_large);
    CHECK(q.prompt_token_count() == 3 && !s->has_in_flight_batch());
    CHECK(pages_of(*s).used_block_count() == 0 && s->find_sequence(1) == nullptr);
    CHECK(s->state().resources(1).blocks.empty() && q.status() == seq_status::waiting);
}

TEST("scheduler: contended prompt chunks rotate only after successful completion")
{
    auto c = small_config();
    c.kv_block_count = 32;
    c.max_batch_tokens = 2;
    c.prefill_chunk_tokens = 1;
    auto s = scheduler::make(c, 99);
    REQUIRE(s);
    for (seq_id id : { 1, 2, 3, 4 })
        REQUIRE(s->add(make_seq(id, std::vector<token_id>(5, 10), 2)));
    auto batch = s->schedule();
    REQUIRE(batch);
    REQUIRE(batch->items.size() == 2);
    CHECK(batch->items[0].id == 1 && batch->items[1].id == 2 && batch->items[0].token_count == 1);
    REQUIRE(s->abort(batch->id));
    auto retry = s->schedule();
    REQUIRE(retry);
    CHECK(retry->items[0].id == 1 && retry->items[1].id == 2);
    commit_all(*s, *retry);
    batch = s->schedule();
    REQUIRE(batch);
    CHECK(batch->items[0].id == 3 && batch->items[1].id == 4);
    commit_all(*s, *batch);
    for (seq_id id : { 1, 2, 3, 4 })
        CHECK(s->find_sequence(id)->processed_token_count() == 1);
}

TEST("scheduler: a new arrival can shorten an aborted prefill retry without shrinking its pages")
{
    auto c = small_config();
    c.max_batch_tokens = 4;
    c.prefill_chunk_tokens = 1;
    auto s = scheduler::make(c, 99);
    REQUIRE(s);
    REQUIRE(s->add(make_seq(1, std::vector<token_id>(5, 10), 2)));
    auto batch = s->schedule();
    REQUIRE(batch);
    CHECK(batch->items[0].token_count == 4);
    REQUIRE(s->abort(batch->id));
    REQUIRE(s->add(make_seq(2, { 10 }, 1)));
    batch = s->schedule();
    REQUIRE(batch);
    REQUIRE(batch->items.size() == 2);
    CHECK(batch->items[0].token_count == 1);
    CHECK(s->state().resources(1).blocks.size() == 2);
    commit_all(*s, *batch);
    CHECK(s->find_sequence(1)->processed_token_count() == 1);
    CHECK(s->find_sequence(2)->is_finished());
    batch = s->schedule();
    REQUIRE(batch);
    CHECK(batch->items[0].token_count == 4);
    commit_all(*s, *batch);
    CHECK(s->find_sequence(1)->processed_token_count() == 5);
}

TEST("scheduler: a short newcomer and an existing stream advance beside a long prompt")
{
    auto c = small_config();
    c.kv_block_count = 32;
    c.max_batch_tokens = 4;
    c.prefill_chunk_tokens = 2;
    auto s = scheduler::make(c, 99);
    REQUIRE(s);
    REQUIRE(s->add(make_seq(1, { 10 }, 12)));
    auto batch = s->schedule();
    REQUIRE(batch);
    commit_all(*s, *batch);
    REQUIRE(s->add(make_seq(2, std::vector<token_id>(20, 10), 2)));
    REQUIRE(s->add(make_seq(3, { 10, 20 }, 4)));
    for (std::size_t round = 0; round < 3; ++round) {
        batch = s->schedule();
        REQUIRE(batch);
        CHECK(batch->phase == batch_phase::decode);
        commit_all(*s, *batch);
        CHECK(s->find_sequence(1)->completion_token_count() == round + 2);
        batch = s->schedule();
        REQUIRE(batch);
        CHECK(batch->phase == batch_phase::prefill);
        commit_all(*s, *batch);
        CHECK(s->find_sequence(2)->processed_token_count() == (round + 1) * 2);
        CHECK(s->find_sequence(3)->completion_token_count() >= 1);
    }
}

TEST("scheduler: small decode batches cover a whole round despite retries and cancellation")
{
    for (int variant = 0; variant < 2; ++variant) {
        auto c = small_config();
        c.kv_block_count = 64;
        c.max_batch_tokens = 1;
        auto s = scheduler::make(c, 99);
        REQUIRE(s);
        for (seq_id id : { 1, 2, 3 })
            REQUIRE(s->add(make_seq(id, { 10 }, 10)));
        while (s->waiting_count()) {
            auto b = s->schedule();
            REQUIRE(b);
            commit_all(*s, *b);
        }
        REQUIRE(s->add(make_seq(4, { 20, 30 }, 2)));
        auto batch = s->schedule();
        REQUIRE(batch);
        CHECK(batch->phase == batch_phase::decode && batch->items[0].id == 1);
        commit_all(*s, *batch);
        if (variant == 0) { // cancel an unvisited round member
            REQUIRE(s->cancel(2));
        } else { // cancel a member already visited this round
            REQUIRE(s->cancel(1));
            batch = s->schedule();
            REQUIRE(batch);
            CHECK(batch->phase == batch_phase::decode && batch->items[0].id == 2);
            commit_all(*s, *batch);
        }
        batch = s->schedule();
        REQUIRE(batch);
        CHECK(batch->phase == batch_phase::decode && batch->items[0].id == 3);
        REQUIRE(s->abort(batch->id));
        batch = s->schedule();
        REQUIRE(batch);
        CHECK(batch->phase == batch_phase::decode && batch->items[0].id == 3);
        commit_all(*s, *batch);
        batch = s->schedule();
        REQUIRE(batch);
        CHECK(batch->phase == batch_phase::prefill && batch->items[0].id == 4);
    }
}

TEST("scheduler: admission commits future pages once and releases the budget at early EOS")
{
    auto c = small_config();
    c.kv_block_count = 4;
    auto s = scheduler::make(c, 99);
    REQUIRE(s);
    auto first = make_seq(1, { 10, 20, 30 }, 4); // 3 pages
    auto second = make_seq(2, { 10 }, 2);        // 1 page
    auto pending = make_seq(3, { 10 }, 1);       // 1 page
    CHECK(s->try_add(first).value() == admission_result::admitted);
    CHECK(s->try_add(second).value() == admission_result::admitted);
    CHECK(pages_of(*s).used_block_count() == 2);
    CHECK(s->try_add(pending).value() == admission_result::deferred);
    CHECK(pending.tokens().size() == 1 && pending.tokens()[0] == 10);
    CHECK(s->find_sequence(3) == nullptr);
    auto batch = s->schedule();
    REQUIRE(batch);
    REQUIRE(s->complete(batch->id, std::array<token_id, 2> { 99, 42 }));
    CHECK(s->find_sequence(1)->reason() == finish_reason::eos);
    CHECK(s->try_add(pending).value() == admission_result::admitted);
    REQUIRE(s->cancel(2));
    REQUIRE(s->cancel(3));
    CHECK(pages_of(*s).used_block_count() == 0);
}

TEST("scheduler: admission accounts for page boundaries and the unprocessed terminal sample")
{
    for (const auto& [prompt, output] : { std::pair { 1u, 2u }, std::pair { 2u, 1u } }) {
        auto c = small_config();
        c.kv_block_count = 1;
        auto s = scheduler::make(c, 99);
        REQUIRE(s);
        REQUIRE(s->add(make_seq(1, std::vector<token_id>(prompt, 10), output)));
        while (!s->is_finished()) {
            auto batch = s->schedule();
            REQUIRE(batch);
            CHECK(pages_of(*s).used_block_count() == 1);
            commit_all(*s, *batch);
        }
        CHECK(s->find_sequence(1)->completion_token_count() == output);
        CHECK(pages_of(*s).used_block_count() == 0);
    }
    auto s = scheduler::make(small_config(), 99);
    REQUIRE(s);
    auto overflow = make_seq(1, { 10, 20, 30 }, std::numeric_limits<std::size_t>::max());
    CHECK(s->try_add(overflow).value() == admission_result::too_large);
}

TEST("scheduler: sequence slots and cache commitments are reusable after cancellation")
{
    auto c = small_config();
    c.max_sequences = 1;
    auto s = scheduler::make(c, 99);
    REQUIRE(s);
    REQUIRE(s->add(make_seq(1, { 10 }, 4)));
    auto next = make_seq(2, { 20 }, 4);
    CHECK(s->try_add(next).value() == admission_result::deferred);
    REQUIRE(s->cancel(1));
    CHECK(s->try_add(next).value() == admission_result::admitted);
    CHECK(s->find_sequence(1)->is_finished());
    REQUIRE(s->cancel(2));
}

namespace {
struct failing_state final : model_state {
    block_manager pages;
    bool fail_next = true;
    explicit failing_state(block_manager p)
        : pages(std::move(p))
    {}
    std::size_t block_size() const noexcept override { return pages.block_size(); }
    sequence_resources resources(seq_id id) const noexcept override { return pages.resources(id); }
    result<void, state_error> reserve(seq_id id, std::size_t count) override
    {
        auto got = pages.reserve(id, count);
        if (!got)
            return got;
        if (std::exchange(fail_next, false))
            return fail(state_errc::allocation_failed);
        return {};
    }
    void release(seq_id id) noexcept override { pages.release(id); }
};
} // namespace

TEST("scheduler: failed state creation rolls back admission and leaves the request retryable")
{
    auto pages = block_manager::make(8, 2);
    REQUIRE(pages);
    auto storage = std::make_unique<failing_state>(std::move(*pages));
    const failing_state* state = storage.get();
    auto s = scheduler::make(small_config(), 99, std::move(storage));
    REQUIRE(s);
    auto q = make_seq(1, { 10, 20 }, 2);
    CHECK(error_is(s->try_add(q), scheduler_errc::block_manager_failure));
    CHECK(state->pages.used_block_count() == 0 && s->find_sequence(1) == nullptr);
    CHECK(q.token_count() == 2);
    CHECK(s->try_add(q).value() == admission_result::admitted);
    REQUIRE(s->cancel(1));
    CHECK(state->pages.used_block_count() == 0);
}

// ---- model_batch (tests/model_batch_test.cc) -------------------------------------------

TEST("model_batch: builds chunked prefill and subsequent decode batches")
{
    auto c = small_config();
    c.max_batch_tokens = 2;
    auto s = scheduler::make(c, 99);
    REQUIRE(s);
    REQUIRE(s->add(make_seq(1, { 10, 20, 30 }, 4)));
    auto first = s->schedule();
    REQUIRE(first);
    auto b = build_model_batch(*first, *s);
    REQUIRE(b);
    CHECK(b->id == first->id && b->phase == batch_phase::prefill && b->kv_block_size == 2);
    CHECK((b->tokens == std::vector<token_id> { 10, 20 }));
    CHECK((b->positions == std::vector<position_id> { 0, 1 }));
    REQUIRE(b->items.size() == 1);
    CHECK(b->items[0].id == 1 && b->items[0].token_offset == 0 && b->items[0].token_count == 2);
    CHECK(!b->items[0].logits_index.has_value() && b->items[0].block_table.size() == 1);
    CHECK(s->find_sequence(1)->processed_token_count() == 0);
    CHECK(s->find_sequence(1)->scheduled_token_count() == 2);
    REQUIRE(s->complete(first->id, std::array<token_id, 0> {}));
    auto second = s->schedule();
    REQUIRE(second);
    b = build_model_batch(*second, *s);
    REQUIRE(b);
    CHECK((b->tokens == std::vector<token_id> { 30 }));
    CHECK((b->positions == std::vector<position_id> { 2 }));
    CHECK(b->items[0].token_offset == 0 && b->items[0].token_count == 1);
    CHECK(b->items[0].logits_index == std::optional<std::size_t>(0));
    REQUIRE(s->complete(second->id, std::array<token_id, 1> { 40 }));
    auto decode = s->schedule();
    REQUIRE(decode);
    b = build_model_batch(*decode, *s);
    REQUIRE(b);
    CHECK(b->phase == batch_phase::decode);
    CHECK((b->tokens == std::vector<token_id> { 40 }));
    CHECK((b->positions == std::vector<position_id> { 3 }));
    CHECK(b->items[0].logits_index == std::optional<std::size_t>(0));
    CHECK(b->items[0].block_table.size() == 2);
}

TEST("model_batch: ragged prefill is flattened in scheduled order")
{
    auto c = small_config();
    c.max_sequences = 2;
    c.max_batch_tokens = 3;
    auto s = scheduler::make(c, 99);
    REQUIRE(s);
    REQUIRE(s->add(make_seq(1, { 10, 11 }, 4)));
    REQUIRE(s->add(make_seq(2, { 20, 21 }, 4)));
    auto scheduled = s->schedule();
    REQUIRE(scheduled);
    auto b = build_model_batch(*scheduled, *s);
    REQUIRE(b);
    CHECK((b->tokens == std::vector<token_id> { 10, 11, 20 }));
    CHECK((b->positions == std::vector<position_id> { 0, 1, 0 }));
    REQUIRE(b->items.size() == 2);
    CHECK(b->items[0].id == 1 && b->items[0].token_offset == 0 && b->items[0].token_count == 2);
    CHECK(b->items[0].logits_index == std::optional<std::size_t>(1));
    CHECK(b->items[1].id == 2 && b->items[1].token_offset == 2 && b->items[1].token_count == 1);
    CHECK(!b->items[1].logits_index.has_value());
    auto updates = s->complete(scheduled->id, std::array<token_id, 1> { 42 });
    REQUIRE(updates);
    CHECK(updates->size() == 1 && updates->front().id == 1);
    CHECK(s->find_sequence(2)->completion_token_count() == 0);
    CHECK(s->find_sequence(2)->processed_token_count() == 1);
}

TEST("model_batch: rejects invalid scheduled batches")
{
    auto s = scheduler::make(small_config(), 99);
    REQUIRE(s);
    const scheduled_batch empty { 1, batch_phase::prefill, {} };
    CHECK(error_is(build_model_batch(empty, *s), model_batch_errc::empty_batch));
    REQUIRE(s->add(make_seq(1, { 10 }, 4)));
    auto scheduled = s->schedule();
    REQUIRE(scheduled);
    auto mismatched = *scheduled;
    ++mismatched.items[0].token_count;
    CHECK(error_is(build_model_batch(mismatched, *s), model_batch_errc::scheduled_token_count_mismatch));
    auto duplicated = *scheduled;
    duplicated.items.push_back(duplicated.items.front());
    CHECK(error_is(build_model_batch(duplicated, *s), model_batch_errc::duplicate_sequence_id));
    CHECK(s->find_sequence(1)->processed_token_count() == 0);
    CHECK(s->find_sequence(1)->scheduled_token_count() == 1);
}

TEST("model_batch: prepare_paged_batch slots follow the tables")
{
    // slot = table[pos / bs] * bs + pos % bs (src/model_batch.cc:178-185)
    model_batch b { 1, batch_phase::prefill, 4, { 1, 2, 3, 4, 5, 6 }, { 3, 4, 5, 0, 1, 2 }, {} };
    b.items.push_back({ 7, 0, 3, 2, { 9, 2 } });
    b.items.push_back({ 8, 3, 3, std::nullopt, { 5 } });
    auto md = prepare_paged_batch(b, 4096, 10, 4);
    REQUIRE(md);
    CHECK((md->slots == std::vector<std::uint32_t> { 39, 8, 9, 20, 21, 22 }));
    CHECK((md->block_table == std::vector<std::uint32_t> { 9, 2, 5 }));
    CHECK((md->table_offsets == std::vector<std::uint32_t> { 0, 0, 0, 2, 2, 2 }));
    CHECK((md->table_lengths == std::vector<std::uint32_t> { 2, 2, 2, 1, 1, 1 }));
    CHECK((md->logits_indices == std::vector<std::size_t> { 2 }));
    CHECK(error_is(prepare_paged_batch(b, 4096, 9, 4), model_batch_errc::inconsistent_batch));
    CHECK(error_is(prepare_paged_batch(b, 5, 10, 4), model_batch_errc::inconsistent_batch));
    b.positions[3] = 4; // beyond the one-page table of item 8
    CHECK(error_is(prepare_paged_batch(b, 4096, 10, 4), model_batch_errc::inconsistent_batch));
}

// ---- prefix cache and engine (tests/prefix_cache_test.cc, tests/inference_engine_test.cc) ---

namespace {

struct token_checkpoint final : model_checkpoint {
    explicit token_checkpoint(std::vector<token_id> data)
        : model_checkpoint(data.size())
        , tokens(std::move(data))
    {}
    std::vector<token_id> tokens;
    std::size_t size_bytes() const noexcept override { return tokens.size() * sizeof(token_id); }
};

// A toy recurrent backend: every sample depends on the whole processed prefix.
struct token_state final : model_state {
    std::unordered_map<seq_id, std::vector<token_id>> tokens, backup;
    bool reject_restore = false;
    bool reject_checkpoint = false;

    result<void, state_error> reserve(seq_id id, std::size_t) override
    {
        tokens.try_emplace(id);
        return {};
    }
    void release(seq_id id) noexcept override { tokens.erase(id); }
    std::size_t checkpoint_bytes(std::size_t n) const noexcept override
    {
        return n * sizeof(token_id);
    }
    result<std::unique_ptr<model_checkpoint>, state_error> checkpoint(seq_id id,
                                                                      std::size_t n) const override
    {
        if (reject_checkpoint || tokens.at(id).size() != n)
            return fail(state_errc::backend_failure);
        return std::unique_ptr<model_checkpoint>(std::make_unique<token_checkpoint>(tokens.at(id)));
    }
    result<void, state_error> restore(seq_id id, const model_checkpoint& saved) override
    {
        if (std::exchange(reject_restore, false))
            return fail(state_errc::backend_failure);
        tokens.at(id) = dynamic_cast<const token_checkpoint&>(saved).tokens;
        return {};
    }
    result<void, state_error> begin_batch(const model_batch&) override
    {
        backup = tokens;
        return {};
    }
    void commit_batch() noexcept override { backup.clear(); }
    void abort_batch() noexcept override { tokens = std::move(backup); }
};

struct checkpoint_runner final : model_runner {
    mutable token_state* storage = nullptr;
    bool fail_next = false;
    std::size_t prefill_tokens = 0;

    const model_info& info() const noexcept override
    {
        static const model_info value { "checkpoint-test", 256, -1 };
        return value;
    }
    result<std::unique_ptr<model_state>, model_runner_error> make_state(scheduler_config) const override
    {
        auto state = std::make_unique<token_state>();
        storage = state.get();
        return std::unique_ptr<model_state>(std::move(state));
    }
    result<std::vector<token_id>, model_runner_error> execute(const model_batch& batch,
                                                              model_state&) override
    {
        if (batch.phase == batch_phase::prefill)
            prefill_tokens += batch.tokens.size();
        std::vector<token_id> samples;
        for (const auto& item : batch.items) {
            auto& history = storage->tokens.at(item.id);
            for (std::size_t i = item.token_offset; i < item.token_offset + item.token_count; ++i) {
                CHECK(batch.positions[i] == history.size());
                history.push_back(batch.tokens[i]);
            }
            if (item.logits_index)
                samples.push_back(1 + std::accumulate(history.begin(), history.end(), 0) % 10);
        }
        if (std::exchange(fail_next, false))
            return fail(model_runner_errc::backend_failure);
        return samples;
    }
};

scheduler_config
prefix_config()
{
    scheduler_config c;
    c.max_sequences = 2;
    c.max_batch_tokens = 16;
    c.kv_block_count = 16;
    c.kv_block_size = 2;
    c.prefix_cache_bytes = 256;
    c.prefix_cache_min_tokens = 1;
    return c;
}

std::vector<token_id>
run_to_end(inference_engine& engine, seq_id id)
{
    while (!engine.is_finished()) {
        auto stepped = engine.step();
        REQUIRE(stepped);
    }
    const auto done = engine.find_sequence(id)->completion_tokens();
    return { done.begin(), done.end() };
}

void
add_prompt(inference_engine& engine, seq_id id, std::vector<token_id> tokens,
           std::vector<std::size_t> boundaries = { 3 })
{
    auto s = seq::make(id, std::move(tokens), generation_params { 3 }, std::move(boundaries));
    REQUIRE(s);
    REQUIRE(engine.add(std::move(*s)));
}

} // namespace

TEST("prefix_cache: LRU uses the longest exact proper prefix and bounds payload bytes")
{
    prefix_cache cache(32);
    const std::vector<token_id> a { 1, 2 }, b { 3, 4 }, c { 5, 6 };
    cache.insert(a, std::make_unique<token_checkpoint>(a));
    cache.insert(b, std::make_unique<token_checkpoint>(b));
    CHECK(cache.size_bytes() == 32);
    CHECK(cache.find(a) == nullptr); // cached state has no logits: a suffix must remain
    REQUIRE(cache.find(std::vector<token_id> { 1, 2, 7 })); // touch a
    cache.insert(c, std::make_unique<token_checkpoint>(c));
    CHECK(cache.find(std::vector<token_id> { 3, 4, 7 }) == nullptr);
    REQUIRE(cache.find(std::vector<token_id> { 1, 2, 7 }));
    REQUIRE(cache.find(std::vector<token_id> { 5, 6, 7 }));
    CHECK_FALSE(cache.fits(1, 32));
    CHECK_FALSE(cache.fits(std::numeric_limits<std::size_t>::max(), 1));
    const std::vector<token_id> long_prefix { 1, 2, 3, 4, 5 };
    cache.insert(long_prefix, std::make_unique<token_checkpoint>(long_prefix));
    CHECK(cache.size_bytes() == 32);
    prefix_cache nested(64);
    const std::vector<token_id> short_prefix { 1 };
    nested.insert(a, std::make_unique<token_checkpoint>(a));
    nested.insert(short_prefix, std::make_unique<token_checkpoint>(short_prefix));
    const model_checkpoint* best = nested.find(std::vector<token_id> { 1, 2, 8 });
    REQUIRE(best);
    CHECK(best->token_count == 2);
}

TEST("prefix_cache: repeated and branching prompts restore private state and skip prefill")
{
    checkpoint_runner runner;
    auto engine = inference_engine::make(prefix_config(), runner);
    REQUIRE(engine);
    add_prompt(*engine, 1, { 1, 2, 3, 4, 5 });
    const auto expected = run_to_end(*engine, 1);
    CHECK(runner.prefill_tokens == 5);
    REQUIRE(engine->remove(1));
    add_prompt(*engine, 1, { 1, 2, 3, 4, 5 });
    CHECK(engine->find_sequence(1)->cached_token_count() == 3);
    CHECK(run_to_end(*engine, 1) == expected);
    CHECK(runner.prefill_tokens == 7);
    REQUIRE(engine->remove(1));
    add_prompt(*engine, 2, { 1, 2, 3, 8 });
    add_prompt(*engine, 3, { 1, 2, 3, 9 });
    CHECK(engine->find_sequence(2)->cached_token_count() == 3);
    CHECK(engine->find_sequence(3)->cached_token_count() == 3);
    const auto branch = run_to_end(*engine, 2);
    const auto other = engine->find_sequence(3)->completion_tokens();
    const std::vector<token_id> other_tokens(other.begin(), other.end());
    checkpoint_runner cold_runner;
    auto cold_config = prefix_config();
    cold_config.prefix_cache_bytes = 0;
    auto cold = inference_engine::make(cold_config, cold_runner);
    REQUIRE(cold);
    add_prompt(*cold, 2, { 1, 2, 3, 8 });
    add_prompt(*cold, 3, { 1, 2, 3, 9 });
    CHECK(run_to_end(*cold, 2) == branch);
    const auto cold_other = cold->find_sequence(3)->completion_tokens();
    CHECK(std::equal(cold_other.begin(), cold_other.end(), other_tokens.begin(), other_tokens.end()));
}

TEST("prefix_cache: failed batches publish no checkpoints and restored state remains retryable")
{
    checkpoint_runner runner;
    auto engine = inference_engine::make(prefix_config(), runner);
    REQUIRE(engine);
    add_prompt(*engine, 1, { 1, 2, 3, 4 });
    runner.fail_next = true;
    CHECK_FALSE(engine->step());
    CHECK(runner.storage->tokens.at(1).empty());
    REQUIRE(engine->cancel(1));
    REQUIRE(engine->remove(1));
    add_prompt(*engine, 2, { 1, 2, 3, 4 });
    CHECK(engine->find_sequence(2)->cached_token_count() == 0);
    const auto expected = run_to_end(*engine, 2);
    REQUIRE(engine->remove(2));
    add_prompt(*engine, 3, { 1, 2, 3, 4 });
    CHECK(engine->find_sequence(3)->cached_token_count() == 3);
    runner.fail_next = true;
    CHECK_FALSE(engine->step());
    CHECK((runner.storage->tokens.at(3) == std::vector<token_id> { 1, 2, 3 }));
    CHECK(run_to_end(*engine, 3) == expected);
    REQUIRE(engine->remove(3));
    runner.storage->reject_restore = true;
    add_prompt(*engine, 4, { 1, 2, 3, 4 });
    CHECK(engine->find_sequence(4)->cached_token_count() == 0);
    CHECK(run_to_end(*engine, 4) == expected);
}

TEST("prefix_cache: disabled, short, oversized and unavailable checkpoints do not split prefill")
{
    for (int mode = 0; mode < 4; ++mode) {
        auto settings = prefix_config();
        if (mode == 0)
            settings.prefix_cache_bytes = 0;
        if (mode == 1)
            settings.prefix_cache_min_tokens = 64;
        if (mode == 2)
            settings.prefix_cache_bytes = 1;
        checkpoint_runner runner;
        auto engine = inference_engine::make(settings, runner);
        REQUIRE(engine);
        runner.storage->reject_checkpoint = mode == 3;
        add_prompt(*engine, 1, { 1, 2, 3, 4 });
        if (mode < 3) {
            auto first = engine->step();
            REQUIRE(first);
            CHECK(first->size() == 1);
        }
        run_to_end(*engine, 1);
        add_prompt(*engine, 2, { 1, 2, 3, 4 });
        CHECK(engine->find_sequence(2)->cached_token_count() == 0);
        run_to_end(*engine, 2);
    }
}

namespace {

// Returns `token` (or the model's EOS when negative) for every sampled item
// (tests/fake_model_runner.cc:60-96).
struct constant_runner final : model_runner {
    explicit constant_runner(token_id t)
        : token(t)
    {}
    token_id token;
    const model_info& info() const noexcept override
    {
        static const model_info value { "fake", 16, 99 };
        return value;
    }
    result<std::vector<token_id>, model_runner_error> execute(const model_batch& batch,
                                                              model_state&) override
    {
        if (batch.empty())
            return fail(model_runner_errc::empty_batch);
        for (const auto& item : batch.items) {
            const bool bad_logits = item.logits_index
                && (*item.logits_index < item.token_offset
                    || *item.logits_index >= item.token_offset + item.token_count);
            if (item.token_count == 0 || item.token_offset > batch.tokens.size()
                || item.token_count > batch.tokens.size() - item.token_offset || bad_logits)
                return fail(model_runner_errc::inconsistent_batch);
        }
        return std::vector<token_id>(batch.sample_count(), token < 0 ? info().eos_token : token);
    }
};

struct stub_runner final : model_runner {
    explicit stub_runner(result<std::vector<token_id>, model_runner_error> r)
        : response(std::move(r))
    {}
    result<std::vector<token_id>, model_runner_error> response;
    const model_info& info() const noexcept override
    {
        static const model_info value { "test", 16, 99 };
        return value;
    }
    result<std::vector<token_id>, model_runner_error> execute(const model_batch&, model_state&) override
    {
        return response;
    }
};

scheduler_config
engine_config()
{
    scheduler_config c;
    c.max_sequences = 4;
    c.max_batch_tokens = 2;
    c.kv_block_count = 8;
    c.kv_block_size = 2;
    return c;
}

} // namespace

TEST("engine: fake runner rejects malformed model batches")
{
    constant_runner runner { 42 };
    auto state = runner.make_state(engine_config());
    REQUIRE(state);
    const model_batch empty { 1, batch_phase::prefill, 2, {}, {}, {} };
    CHECK(error_is(runner.execute(empty, **state), model_runner_errc::empty_batch));
}

TEST("engine: runs chunked prefill and decode until the length limit")
{
    constant_runner runner { 42 };
    auto engine = inference_engine::make(engine_config(), runner);
    REQUIRE(engine);
    REQUIRE(engine->add(make_seq(1, { 10, 20, 30 }, 3)));
    std::size_t steps = 0, updates = 0;
    while (!engine->is_finished()) {
        auto u = engine->step();
        REQUIRE(u);
        updates += u->size();
        ++steps;
    }
    CHECK(steps == 4 && updates == 3);
    const seq* done = engine->find_sequence(1);
    CHECK(done->status() == seq_status::finished && done->reason() == finish_reason::len_limit);
    REQUIRE(done->completion_token_count() == 3);
    CHECK(done->completion_tokens()[0] == 42 && done->completion_tokens()[2] == 42);
}

TEST("engine: takes the EOS token from the model")
{
    constant_runner runner { -1 };
    auto engine = inference_engine::make(engine_config(), runner);
    REQUIRE(engine);
    REQUIRE(engine->add(make_seq(1, { 10 }, 3)));
    auto updates = engine->step();
    REQUIRE(updates);
    REQUIRE(updates->size() == 1);
    CHECK(updates->front().token == runner.info().eos_token);
    CHECK(updates->front().reason == finish_reason::eos);
    CHECK(engine->is_finished() && engine->find_sequence(1)->completion_token_count() == 1);
}

TEST("engine: runner failures abort the scheduler reservation")
{
    auto check_failure = [](result<std::vector<token_id>, model_runner_error> response,
                            inference_engine_errc expected, std::string_view detail) {
        stub_runner runner(std::move(response));
        auto engine = inference_engine::make(engine_config(), runner);
        REQUIRE(engine);
        REQUIRE(engine->add(make_seq(1, { 10 }, 4)));
        auto stepped = engine->step();
        REQUIRE_FALSE(stepped);
        CHECK(stepped.error() == expected);
        CHECK(describe_error(stepped.error()).find(detail) != std::string::npos);
        CHECK_FALSE(engine->has_in_flight_batch());
        const seq* q = engine->find_sequence(1);
        CHECK(q->processed_token_count() == 0 && q->scheduled_token_count() == 0);
        CHECK(q->status() == seq_status::waiting);
    };
    check_failure(fail(model_runner_errc::backend_failure, "GPU command failed", "layer 2"),
                  inference_engine_errc::model_execution_failed, "layer 2: GPU command failed");
    check_failure(std::vector<token_id> {}, inference_engine_errc::runner_result_count_mismatch,
                  "expected 1 samples, received 0");
}

TEST("engine: creation and lifecycle errors retain their causes")
{
    constant_runner runner { 42 };
    auto c = engine_config();
    c.kv_block_count = 0;
    auto invalid = inference_engine::make(c, runner);
    REQUIRE_FALSE(invalid);
    CHECK(invalid.error() == inference_engine_errc::scheduler_creation_failed);
    CHECK(describe_error(invalid.error()).find("block_manager.invalid_block_count") != std::string::npos);
    auto engine = inference_engine::make(engine_config(), runner);
    REQUIRE(engine);
    auto removed = engine->remove(123);
    REQUIRE_FALSE(removed);
    CHECK(removed.error() == inference_engine_errc::sequence_remove_failed);
    CHECK(describe_error(removed.error()).find("scheduler.unknown_sequence") != std::string::npos);
}
