// result<T, E>: a value or an error, with the call-site shape of the
// reference's std::expected alias (src/result.h:10-48): has_value(),
// operator bool, operator*, operator->, error(), fail(...), CL_TRY and
// CL_TRY_ASSIGN. Written here because neither libstdc++ 11 nor the ROCm
// clang setup provides <expected>.
#pragma once

#include <optional>
#include <string_view>
#include <type_traits>
#include <utility>
#include <variant>

#include "error.h"

namespace chibillm {

// The error half of a result under construction; converts to any result
// whose error type can be built from E.
template <typename E>
struct failure {
    E value;
};

template <typename E>
[[nodiscard]] failure<std::decay_t<E>>
fail(E&& e)
{
    return failure<std::decay_t<E>> { std::forward<E>(e) };
}

// Translates a code at a boundary, keeping the cause (and stage) as detail.
template <typename Code, typename Cause>
[[nodiscard]] failure<error<Code>>
fail(Code code, const Cause& cause, std::string_view stage = {})
{
    std::string detail = describe_error(cause);
    if (!stage.empty())
        detail = std::string(stage) + ": " + detail;
    return failure<error<Code>> { error<Code> { code, std::move(detail) } };
}

template <typename T, typename E>
class [[nodiscard]] result {
public:
    using value_type = T;
    using error_type = E;

    result(const T& v)
        : state_(std::in_place_index<0>, v)
    {}

    result(T&& v)
        : state_(std::in_place_index<0>, std::move(v))
    {}

    template <typename U>
        requires std::is_constructible_v<T, U&&> && (!std::is_same_v<std::decay_t<U>, result>)
        && (!std::is_same_v<std::decay_t<U>, T>)
    result(U&& v)
        : state_(std::in_place_index<0>, T(std::forward<U>(v)))
    {}

    template <typename F>
        requires std::is_constructible_v<E, F>
    result(failure<F> f)
        : state_(std::in_place_index<1>, E(std::move(f.value)))
    {}

    [[nodiscard]] bool has_value() const noexcept { return state_.index() == 0; }
    explicit operator bool() const noexcept { return has_value(); }

    T& operator*() & { return std::get<0>(state_); }
    const T& operator*() const& { return std::get<0>(state_); }
    T&& operator*() && { return std::get<0>(std::move(state_)); }
    T* operator->() { return &std::get<0>(state_); }
    const T* operator->() const { return &std::get<0>(state_); }
    T& value() & { return std::get<0>(state_); }
    const T& value() const& { return std::get<0>(state_); }

    E& error() & { return std::get<1>(state_); }
    const E& error() const& { return std::get<1>(state_); }

private:
    std::variant<T, E> state_;
};

template <typename E>
class [[nodiscard]] result<void, E> {
public:
    using value_type = void;
    using error_type = E;

    result() noexcept = default;

    template <typename F>
        requires std::is_constructible_v<E, F>
    result(failure<F> f)
        : error_(E(std::move(f.value)))
    {}

    [[nodiscard]] bool has_value() const noexcept { return !error_.has_value(); }
    explicit operator bool() const noexcept { return has_value(); }
    void operator*() const noexcept {}

    E& error() & { return *error_; }
    const E& error() const& { return *error_; }

private:
    std::optional<E> error_;
};

} // namespace chibillm

// Returns the error of an expected-like expression from the enclosing function.
#define CL_TRY(expression)                                                                         \
    do {                                                                                           \
        auto cl_try_result = (expression);                                                         \
        if (!cl_try_result)                                                                        \
            return ::chibillm::fail(cl_try_result.error());                                        \
    } while (false)

// Assigns the value of an expected-like expression or returns its error.
#define CL_TRY_ASSIGN(destination, expression)                                                     \
    do {                                                                                           \
        auto cl_try_result = (expression);                                                         \
        if (!cl_try_result)                                                                        \
            return ::chibillm::fail(cl_try_result.error());                                        \
        destination = std::move(*cl_try_result);                                                   \
    } while (false)
