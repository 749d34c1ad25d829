// Model-family adapter the engine drives (src/model_runner.h:14-88, reduced to
// what the KV path needs: geometry/EOS, state creation and batch execution).
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "model_batch.h"

namespace chibillm {

struct model_info {
    std::string id;
    std::size_t max_context_tokens;
    token_id eos_token;
};

// src/model_runner.h:18-36 (chat and tokenizer codes kept for numbering)
enum class model_runner_errc : std::uint8_t {
    empty_batch,
    inconsistent_batch,
    invalid_chat,
    tokenizer_failure,
    backend_failure,
};

[[nodiscard]] inline std::string_view
error_name(model_runner_errc code) noexcept
{
    static constexpr std::array<std::string_view, 5> names {
        "model_runner.empty_batch",     "model_runner.inconsistent_batch",
        "model_runner.invalid_chat",    "model_runner.tokenizer_failure",
        "model_runner.backend_failure",
    };
    const auto i = static_cast<std::size_t>(code);
    return i < names.size() ? names[i] : "model_runner.unknown_error";
}

using model_runner_error = error<model_runner_errc>;

class model_runner {
public:
    virtual ~model_runner() = default;
    virtual const model_info& info() const noexcept = 0;
    // Default: a page allocator alone (src/model_runner.cc:85-92).
    virtual result<std::unique_ptr<model_state>, model_runner_error>
    make_state(scheduler_config config) const
    {
        auto pages = block_manager::make(config.kv_block_count, config.kv_block_size);
        if (!pages)
            return fail(model_runner_errc::backend_failure, pages.error(), "block allocator");
        return std::unique_ptr<model_state>(std::make_unique<block_manager>(std::move(*pages)));
    }
    // One sampled token per item with a logits index, in item order.
    virtual result<std::vector<token_id>, model_runner_error> execute(const model_batch& batch,
                                                                      model_state& state) = 0;
};

} // namespace chibillm
