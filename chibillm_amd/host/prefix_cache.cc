#include "prefix_cache.h"

#include <algorithm>

namespace chibillm {

namespace {
bool
same_tokens(std::span<const token_id> a, std::span<const token_id> b) noexcept
{
    return a.size() == b.size() && std::equal(a.begin(), a.end(), b.begin());
}
} // namespace

const model_checkpoint*
prefix_cache::find(std::span<const token_id> prompt)
{
    auto best = entries_.end();
    for (auto it = entries_.begin(); it != entries_.end(); ++it) {
        const std::size_t n = it->tokens.size();
        const bool proper = n < prompt.size();
        const bool longer = best == entries_.end() || n > best->tokens.size();
        if (proper && longer && same_tokens(it->tokens, prompt.first(n)))
            best = it;
    }
    if (best == entries_.end())
        return nullptr;
    entries_.splice(entries_.begin(), entries_, best);
    return entries_.front().state.get();
}

bool
prefix_cache::contains(std::span<const token_id> prefix) const noexcept
{
    return std::any_of(entries_.begin(), entries_.end(),
                       [&](const entry& e) { return same_tokens(e.tokens, prefix); });
}

bool
prefix_cache::fits(std::size_t tokens, std::size_t state_bytes) const noexcept
{
    return state_bytes != 0 && state_bytes <= capacity_
        && tokens <= (capacity_ - state_bytes) / sizeof(token_id);
}

void
prefix_cache::make_room(std::size_t tokens, std::size_t state_bytes) noexcept
{
    if (!fits(tokens, state_bytes))
        return;
    const std::size_t needed = tokens * sizeof(token_id) + state_bytes;
    while (bytes_ > capacity_ - needed) {
        bytes_ -= entries_.back().bytes();
        entries_.pop_back();
    }
}

void
prefix_cache::insert(std::span<const token_id> prefix, std::unique_ptr<model_checkpoint> state)
{
    if (!state || state->token_count != prefix.size() || !fits(prefix.size(), state->size_bytes())
        || contains(prefix))
        return;
    make_room(prefix.size(), state->size_bytes());
    entries_.push_front({ { prefix.begin(), prefix.end() }, std::move(state) });
    bytes_ += entries_.front().bytes();
}

} // namespace chibillm
