// Typed error codes with an optional detail string, the convention of the
// reference's src/error.h:13-68: control flow switches on `code`, `detail`
// carries the lower layer's description.
#pragma once

#include <array>
#include <string>
#include <string_view>
#include <type_traits>
#include <utility>

namespace chibillm {

template <typename Code>
struct error {
    Code code;
    std::string detail;

    error(Code c) noexcept
        : code(c)
    {}

    error(Code c, std::string d)
        : code(c)
        , detail(std::move(d))
    {}

    [[nodiscard]] bool
    operator==(Code other) const noexcept
    {
        return code == other;
    }
};

template <typename Code>
    requires std::is_enum_v<Code>
[[nodiscard]] std::string
describe_error(Code code)
{
    return std::string(error_name(code));
}

template <typename Code>
[[nodiscard]] std::string
describe_error(const error<Code>& e)
{
    std::string text = describe_error(e.code);
    if (!e.detail.empty())
        text += ": " + e.detail;
    return text;
}

[[nodiscard]] inline std::string
describe_error(std::string_view message)
{
    return std::string(message);
}

// Prefixes a stage name to the detail.
template <typename Code>
[[nodiscard]] error<Code>
at_stage(error<Code> e, std::string_view stage)
{
    e.detail = e.detail.empty() ? std::string(stage) : std::string(stage) + ": " + e.detail;
    return e;
}

} // namespace chibillm
