#include "seq.h"

#include <algorithm>
#include <cassert>

namespace chibillm {

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
    if (prompt.empty())
        return fail(seq_errc::empty_prompt);
    if (params.max_new_tokens == 0)
        return fail(seq_errc::invalid_max_new_tokens);
    if (checkpoints.empty() && prompt.size() > 1)
        checkpoints.push_back(prompt.size() - 1);
    std::sort(checkpoints.begin(), checkpoints.end());
    const bool out_of_range = !checkpoints.empty()
        && (checkpoints.front() == 0 || checkpoints.back() >= prompt.size());
    const bool repeated =
        std::adjacent_find(checkpoints.begin(), checkpoints.end()) != checkpoints.end();
    if (out_of_range || repeated)
        return fail(seq_errc::invalid_cached_prefix);
    seq s(id, std::move(prompt), params);
    s.checkpoints_ = std::move(checkpoints);
    s.check_invariants();
    return s;
}

std::span<const token_id>
seq::prompt_tokens() const noexcept
{
    return std::span<const token_id>(tokens_).first(prompt_size_);
}

std::span<const token_id>
seq::completion_tokens() const noexcept
{
    return std::span<const token_id>(tokens_).subspan(prompt_size_);
}

result<void, seq_errc>
seq::restore_prefix(std::size_t count)
{
    const bool pristine = status_ == seq_status::waiting && processed_ == 0 && scheduled_ == 0
        && completion_token_count() == 0;
    if (!pristine || count == 0 || count >= prompt_size_)
        return fail(seq_errc::invalid_cached_prefix);
    processed_ = count;
    cached_ = count;
    check_invariants();
    return {};
}

result<void, seq_errc>
seq::append_token(token_id token)
{
    if (status_ == seq_status::finished)
        return fail(seq_errc::already_finished);
    if (status_ != seq_status::running)
        return fail(seq_errc::invalid_state_transition);
    if (scheduled_ != 0)
        return fail(seq_errc::work_already_scheduled);
    if (processed_ != tokens_.size())
        return fail(seq_errc::invalid_state_transition);
    tokens_.push_back(token);
    check_invariants();
    return {};
}

result<void, seq_errc>
seq::mark_running()
{
    if (status_ == seq_status::finished)
        return fail(seq_errc::already_finished);
    if (status_ != seq_status::waiting)
        return fail(seq_errc::invalid_state_transition);
    if (scheduled_ != 0)
        return fail(seq_errc::work_already_scheduled);
    if (processed_ != tokens_.size())
        return fail(seq_errc::invalid_state_transition);
    status_ = seq_status::running;
    check_invariants();
    return {};
}

result<void, seq_errc>
seq::finish(finish_reason why)
{
    if (status_ == seq_status::finished)
        return fail(seq_errc::already_finished);
    if (why == finish_reason::none)
        return fail(seq_errc::invalid_finish_reason);
    if (scheduled_ != 0)
        return fail(seq_errc::work_already_scheduled);
    status_ = seq_status::finished;
    reason_ = why;
    check_invariants();
    return {};
}

result<void, seq_errc>
seq::schedule_tokens(std::size_t count)
{
    if (status_ == seq_status::finished)
        return fail(seq_errc::already_finished);
    if (scheduled_ != 0)
        return fail(seq_errc::work_already_scheduled);
    if (count == 0)
        return fail(seq_errc::zero_scheduled_tokens);
    if (count > schedulable_token_count())
        return fail(seq_errc::too_many_scheduled_tokens);
    scheduled_ = count;
    check_invariants();
    return {};
}

result<void, seq_errc>
seq::commit_scheduled_tokens()
{
    if (status_ == seq_status::finished)
        return fail(seq_errc::already_finished);
    if (scheduled_ == 0)
        return fail(seq_errc::no_work_scheduled);
    processed_ += scheduled_;
    scheduled_ = 0;
    check_invariants();
    return {};
}

void
seq::cancel_scheduled_tokens() noexcept
{
    scheduled_ = 0;
    check_invariants();
}

finish_reason
seq::evaluate_stop(token_id eos) const noexcept
{
    if (completion_token_count() == 0)
        return finish_reason::none;
    if (!params_.ignore_eos && last_token() == eos)
        return finish_reason::eos;
    if (completion_token_count() >= params_.max_new_tokens)
        return finish_reason::len_limit;
    return finish_reason::none;
}

void
seq::check_invariants() const noexcept
{
    assert(!tokens_.empty() && prompt_size_ > 0 && prompt_size_ <= tokens_.size());
    assert(processed_ + scheduled_ <= tokens_.size());
    assert((status_ == seq_status::finished) == (reason_ != finish_reason::none));
    assert(status_ != seq_status::finished || scheduled_ == 0);
}

} // namespace chibillm
