// seq: the token history of one request and its progress through prefill and
// decode. Every mutating operation is written as a list of preconditions,
// each with the error it reports, checked in the listed order; the first
// violated one is the result and nothing changes. The contract (the
// interface of src/seq.h:12-150, pinned by the seq tests in tests/cpp):
//
//  - tokens = prompt | completion; processed <= processed + scheduled <= tokens;
//  - a waiting sequence becomes running once every token is processed; a
//    running sequence takes one sampled token at a time, only when nothing is
//    scheduled and every token is processed (the one-token cache gap is then
//    the new sample);
//  - finishing needs a reason other than none and no scheduled work, and is
//    final; scheduling reserves 1..schedulable tokens, once, until committed
//    (processed += scheduled) or cancelled;
//  - restore_prefix marks a proper prefix of the prompt as processed (and
//    cached) on a sequence that has done nothing yet;
//  - checkpoint boundaries are distinct positions strictly inside the prompt,
//    kept sorted; none given means the proper prefix prompt - 1.
#include "seq.h"

#include <algorithm>
#include <cassert>
#include <initializer_list>
#include <utility>

namespace chibillm {

namespace {

struct precondition {
    bool violated;
    seq_errc error;
};

// The error of the first violated precondition, or success.
result<void, seq_errc>
check(std::initializer_list<precondition> list)
{
    for (const precondition& p : list)
        if (p.violated)
            return fail(p.error);
    return {};
}

// Boundaries sorted, each in (0, prompt) and distinct; none means prompt - 1
// (no boundary at all for a one-token prompt).
result<std::vector<std::size_t>, seq_errc>
normalise_checkpoints(std::vector<std::size_t> boundaries, std::size_t prompt)
{
    if (boundaries.empty()) {
        if (prompt > 1)
            boundaries.push_back(prompt - 1);
        return boundaries;
    }
    std::sort(boundaries.begin(), boundaries.end());
    std::size_t previous = 0; // boundaries are > 0, so 0 never repeats a valid one
    for (const std::size_t b : boundaries) {
        if (b == previous || b >= prompt)
            return fail(seq_errc::invalid_cached_prefix);
        previous = b;
    }
    return boundaries;
}

} // namespace

seq::seq(seq_id id, std::vector<token_id> prompt, generation_params params)
    : id_(id)
    , tokens_(std::move(prompt))
    , prompt_size_(tokens_.size())
    , params_(params)
{}

result<seq, seq_errc>
seq::make(seq_id id, std::vector<token_id> prompt, generation_params params,
          std::vector<std::size_t> checkpoints)
{
    if (auto bad = check({ { prompt.empty(), seq_errc::empty_prompt },
                           { params.max_new_tokens == 0, seq_errc::invalid_max_new_tokens } });
        !bad)
        return fail(bad.error());
    auto boundaries = normalise_checkpoints(std::move(checkpoints), prompt.size());
    if (!boundaries)
        return fail(boundaries.error());
    seq made(id, std::move(prompt), params);
    made.checkpoints_ = std::move(*boundaries);
    made.check_invariants();
    return made;
}

std::span<const token_id>
seq::prompt_tokens() const noexcept
{
    return { tokens_.data(), prompt_size_ };
}

std::span<const token_id>
seq::completion_tokens() const noexcept
{
    return { tokens_.data() + prompt_size_, tokens_.size() - prompt_size_ };
}

result<void, seq_errc>
seq::restore_prefix(std::size_t count)
{
    const bool untouched = status_ == seq_status::waiting && processed_ == 0 && scheduled_ == 0
        && tokens_.size() == prompt_size_;
    if (auto bad = check({ { !untouched || count == 0 || count >= prompt_size_,
                             seq_errc::invalid_cached_prefix } });
        !bad)
        return bad;
    processed_ = cached_ = count;
    check_invariants();
    return {};
}

result<void, seq_errc>
seq::append_token(token_id token)
{
    if (auto bad = check({ { is_finished(), seq_errc::already_finished },
                           { status_ != seq_status::running, seq_errc::invalid_state_transition },
                           { scheduled_ != 0, seq_errc::work_already_scheduled },
                           { processed_ != tokens_.size(), seq_errc::invalid_state_transition } });
        !bad)
        return bad;
    tokens_.push_back(token);
    check_invariants();
    return {};
}

result<void, seq_errc>
seq::mark_running()
{
    if (auto bad = check({ { is_finished(), seq_errc::already_finished },
                           { status_ != seq_status::waiting, seq_errc::invalid_state_transition },
                           { scheduled_ != 0, seq_errc::work_already_scheduled },
                           { processed_ != tokens_.size(), seq_errc::invalid_state_transition } });
        !bad)
        return bad;
    status_ = seq_status::running;
    check_invariants();
    return {};
}

result<void, seq_errc>
seq::finish(finish_reason why)
{
    if (auto bad = check({ { is_finished(), seq_errc::already_finished },
                           { why == finish_reason::none, seq_errc::invalid_finish_reason },
                           { scheduled_ != 0, seq_errc::work_already_scheduled } });
        !bad)
        return bad;
    status_ = seq_status::finished;
    reason_ = why;
    check_invariants();
    return {};
}

result<void, seq_errc>
seq::schedule_tokens(std::size_t count)
{
    if (auto bad = check({ { is_finished(), seq_errc::already_finished },
                           { scheduled_ != 0, seq_errc::work_already_scheduled },
                           { count == 0, seq_errc::zero_scheduled_tokens },
                           { count > schedulable_token_count(),
                             seq_errc::too_many_scheduled_tokens } });
        !bad)
        return bad;
    scheduled_ = count;
    check_invariants();
    return {};
}

result<void, seq_errc>
seq::commit_scheduled_tokens()
{
    if (auto bad = check({ { is_finished(), seq_errc::already_finished },
                           { scheduled_ == 0, seq_errc::no_work_scheduled } });
        !bad)
        return bad;
    processed_ += std::exchange(scheduled_, 0);
    check_invariants();
    return {};
}

void
seq::cancel_scheduled_tokens() noexcept
{
    scheduled_ = 0;
}

finish_reason
seq::evaluate_stop(token_id eos) const noexcept
{
    const std::size_t produced = completion_token_count();
    if (produced == 0)
        return finish_reason::none;
    // an end-of-sequence sample wins over reaching the length limit with it
    if (tokens_.back() == eos && !params_.ignore_eos)
        return finish_reason::eos;
    return produced >= params_.max_new_tokens ? finish_reason::len_limit : finish_reason::none;
}

void
seq::check_invariants() const noexcept
{
    assert(prompt_size_ > 0 && prompt_size_ <= tokens_.size());
    assert(scheduled_ <= tokens_.size() - processed_);
    assert(is_finished() == (reason_ != finish_reason::none));
    assert(!is_finished() || scheduled_ == 0);
}

} // namespace chibillm
