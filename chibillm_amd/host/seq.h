// One request's token history and its progress through prefill and decode
// (the interface of src/seq.h:12-150). Tokens are [prompt | completion];
// `processed` tokens are in the KV cache, `scheduled` tokens belong to the
// batch in flight, and there is always a one-token gap between a running
// sequence's last sample and the cache.
#pragma once

#include <cstddef>
#include <cstdint>
#include <span>
#include <vector>

#include "error.h"
#include "result.h"

namespace chibillm {

using token_id = std::int32_t;
using seq_id = std::uint64_t;
using block_id = std::uint32_t;

enum class seq_status {
    waiting, // needs prefill
    running, // ready for one-token decode
    finished,
};

enum class finish_reason {
    none,
    eos,
    len_limit,
    cancelled,
};

enum class seq_errc : std::uint8_t {
    empty_prompt,
    invalid_max_new_tokens,
    already_finished,
    invalid_state_transition,
    invalid_finish_reason,
    zero_scheduled_tokens,
    work_already_scheduled,
    too_many_scheduled_tokens,
    no_work_scheduled,
    invalid_cached_prefix,
};

[[nodiscard]] inline std::string_view
error_name(seq_errc code) noexcept
{
    static constexpr std::array<std::string_view, 10> names {
        "seq.empty_prompt",           "seq.invalid_max_new_tokens",
        "seq.already_finished",       "seq.invalid_state_transition",
        "seq.invalid_finish_reason",  "seq.zero_scheduled_tokens",
        "seq.work_already_scheduled", "seq.too_many_scheduled_tokens",
        "seq.no_work_scheduled",      "seq.invalid_cached_prefix",
    };
    const auto i = static_cast<std::size_t>(code);
    return i < names.size() ? names[i] : "seq.unknown_error";
}

struct generation_params {
    std::size_t max_new_tokens { 64 };
    bool ignore_eos { false };
};

class seq {
public:
    // An empty checkpoint list defaults to the proper prompt prefix
    // prompt_size - 1 (src/seq.cc:32-33); boundaries must lie in (0, prompt).
    [[nodiscard]] static result<seq, seq_errc> make(seq_id id, std::vector<token_id> prompt,
                                                    generation_params params,
                                                    std::vector<std::size_t> checkpoints = {});

    seq(const seq&) = delete;
    seq& operator=(const seq&) = delete;
    seq(seq&&) noexcept = default;
    seq& operator=(seq&&) noexcept = default;

    [[nodiscard]] seq_id id() const noexcept { return id_; }
    [[nodiscard]] seq_status status() const noexcept { return status_; }
    [[nodiscard]] finish_reason reason() const noexcept { return reason_; }
    [[nodiscard]] bool is_finished() const noexcept { return status_ == seq_status::finished; }

    [[nodiscard]] std::span<const token_id> tokens() const noexcept { return tokens_; }
    [[nodiscard]] std::span<const token_id> prompt_tokens() const noexcept;
    [[nodiscard]] std::span<const token_id> completion_tokens() const noexcept;
    [[nodiscard]] token_id last_token() const noexcept { return tokens_.back(); }
    [[nodiscard]] std::size_t token_count() const noexcept { return tokens_.size(); }
    [[nodiscard]] std::size_t prompt_token_count() const noexcept { return prompt_size_; }
    [[nodiscard]] std::size_t completion_token_count() const noexcept
    {
        return tokens_.size() - prompt_size_;
    }

    // A sampled token becomes the next unprocessed token of a running sequence.
    [[nodiscard]] result<void, seq_errc> append_token(token_id token);
    [[nodiscard]] result<void, seq_errc> mark_running();
    [[nodiscard]] result<void, seq_errc> finish(finish_reason why);

    [[nodiscard]] std::size_t processed_token_count() const noexcept { return processed_; }
    [[nodiscard]] std::size_t cached_token_count() const noexcept { return cached_; }
    [[nodiscard]] std::span<const std::size_t> checkpoints() const noexcept { return checkpoints_; }
    // Marks a restored proper prefix of the prompt as processed.
    [[nodiscard]] result<void, seq_errc> restore_prefix(std::size_t count);

    [[nodiscard]] std::size_t scheduled_token_count() const noexcept { return scheduled_; }
    [[nodiscard]] std::size_t unprocessed_token_count() const noexcept
    {
        return tokens_.size() - processed_;
    }
    [[nodiscard]] std::size_t schedulable_token_count() const noexcept
    {
        return tokens_.size() - processed_ - scheduled_;
    }
    [[nodiscard]] result<void, seq_errc> schedule_tokens(std::size_t count);
    [[nodiscard]] result<void, seq_errc> commit_scheduled_tokens();
    void cancel_scheduled_tokens() noexcept;

    [[nodiscard]] const generation_params& params() const noexcept { return params_; }
    // EOS takes precedence over the length limit.
    [[nodiscard]] finish_reason evaluate_stop(token_id eos) const noexcept;

private:
    seq(seq_id id, std::vector<token_id> prompt, generation_params params);
    void check_invariants() const noexcept;

    seq_id id_;
    seq_status status_ = seq_status::waiting;
    finish_reason reason_ = finish_reason::none;
    std::vector<token_id> tokens_;
    std::size_t prompt_size_;
    std::size_t processed_ = 0;
    std::size_t cached_ = 0;
    std::vector<std::size_t> checkpoints_;
    std::size_t scheduled_ = 0;
    generation_params params_;
};

} // namespace chibillm
