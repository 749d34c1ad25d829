#include "prefix_cache.h"

#include <algorithm>

namespace chibillm {

namespace {

// FNV-1a over the tokens' bytes, extended one token at a time, so that the
// keys of every prefix of a prompt come from one pass over it.
constexpr std::uint64_t fnv_basis = 0xcbf29ce484222325ull;
constexpr std::uint64_t fnv_prime = 0x100000001b3ull;

std::uint64_t
extend(std::uint64_t key, token_id token) noexcept
{
    auto bits = static_cast<std::uint32_t>(token);
    for (int byte = 0; byte < 4; ++byte, bits >>= 8)
        key = (key ^ (bits & 0xFFu)) * fnv_prime;
    return key;
}

std::uint64_t
key_of(std::span<const token_id> tokens) noexcept
{
    std::uint64_t key = fnv_basis;
    for (const token_id t : tokens)
        key = extend(key, t);
    return key;
}

} // namespace

prefix_cache::position
prefix_cache::locate(std::span<const token_id> tokens, std::uint64_t key) const noexcept
{
    const auto [first, last] = index_.equal_range(key);
    for (auto it = first; it != last; ++it) {
        const auto& held = it->second->tokens;
        if (held.size() == tokens.size() && std::equal(held.begin(), held.end(), tokens.begin()))
            return it->second;
    }
    return const_cast<std::list<entry>&>(recency_).end();
}

const model_checkpoint*
prefix_cache::find(std::span<const token_id> prompt)
{
    if (lengths_.empty() || prompt.size() < 2)
        return nullptr;
    // keys of the prompt's proper prefixes, by length
    std::vector<std::uint64_t> keys(prompt.size());
    std::uint64_t key = fnv_basis;
    for (std::size_t n = 1; n < prompt.size(); ++n) {
        key = extend(key, prompt[n - 1]);
        keys[n] = key;
    }
    // lengths_ runs longest first: the first hit is the longest cached prefix
    for (auto it = lengths_.lower_bound(prompt.size() - 1); it != lengths_.end(); ++it) {
        const std::size_t n = it->first;
        const position hit = locate(prompt.first(n), keys[n]);
        if (hit != recency_.end()) {
            recency_.splice(recency_.begin(), recency_, hit); // iterators stay valid
            return hit->state.get();
        }
    }
    return nullptr;
}

bool
prefix_cache::contains(std::span<const token_id> prefix) const noexcept
{
    return locate(prefix, key_of(prefix)) != recency_.end();
}

bool
prefix_cache::fits(std::size_t tokens, std::size_t state_bytes) const noexcept
{
    // an entry must carry state and fit the budget on its own
    if (state_bytes == 0 || state_bytes > capacity_)
        return false;
    return tokens <= (capacity_ - state_bytes) / sizeof(token_id);
}

void
prefix_cache::evict_oldest() noexcept
{
    const entry& victim = recency_.back();
    const auto [first, last] = index_.equal_range(victim.key);
    for (auto it = first; it != last; ++it)
        if (&*it->second == &victim) {
            index_.erase(it);
            break;
        }
    if (auto n = lengths_.find(victim.tokens.size()); n != lengths_.end() && --n->second == 0)
        lengths_.erase(n);
    bytes_ -= victim.bytes();
    recency_.pop_back();
}

void
prefix_cache::make_room(std::size_t tokens, std::size_t state_bytes) noexcept
{
    if (!fits(tokens, state_bytes))
        return;
    const std::size_t budget = capacity_ - (tokens * sizeof(token_id) + state_bytes);
    while (bytes_ > budget)
        evict_oldest();
}

void
prefix_cache::insert(std::span<const token_id> prefix, std::unique_ptr<model_checkpoint> state)
{
    if (!state || state->token_count != prefix.size())
        return;
    const std::size_t state_bytes = state->size_bytes();
    const std::uint64_t key = key_of(prefix);
    if (!fits(prefix.size(), state_bytes) || locate(prefix, key) != recency_.end())
        return;
    make_room(prefix.size(), state_bytes);
    recency_.push_front(entry { { prefix.begin(), prefix.end() }, key, std::move(state) });
    index_.emplace(key, recency_.begin());
    ++lengths_[prefix.size()];
    bytes_ += recency_.front().bytes();
}

} // namespace chibillm
