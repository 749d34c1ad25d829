// A small test harness for the C++ host tests: TEST("name") registers a case,
// CHECK records a failure and continues, REQUIRE stops the case. main() runs
// every case (or those whose name contains argv[1]) and exits non-zero if any
// check failed.
#pragma once

#include <cstdio>
#include <cstring>
#include <exception>
#include <functional>
#include <string>
#include <vector>

namespace check {

struct test_case {
    const char* name;
    std::function<void()> body;
};

inline std::vector<test_case>& registry()
{
    static std::vector<test_case> cases;
    return cases;
}

inline int& failures()
{
    static int count = 0;
    return count;
}

struct stop_case {};

struct registrar {
    registrar(const char* name, std::function<void()> body)
    {
        registry().push_back({ name, std::move(body) });
    }
};

inline void report(const char* file, int line, const char* expr)
{
    ++failures();
    std::fprintf(stderr, "  FAILED %s:%d: %s\n", file, line, expr);
}

} // namespace check

#define CHECK_CAT2(a, b) a##b
#define CHECK_CAT(a, b) CHECK_CAT2(a, b)
#define TEST(name)                                                                                 \
    static void CHECK_CAT(test_body_, __LINE__)();                                                 \
    static ::check::registrar CHECK_CAT(test_reg_, __LINE__)(name, CHECK_CAT(test_body_, __LINE__)); \
    static void CHECK_CAT(test_body_, __LINE__)()

#define CHECK(expr)                                                                                \
    do {                                                                                           \
        if (!static_cast<bool>(expr))                                                              \
            ::check::report(__FILE__, __LINE__, #expr);                                            \
    } while (false)
#define CHECK_FALSE(expr) CHECK(!static_cast<bool>(expr))
#define REQUIRE(expr)                                                                              \
    do {                                                                                           \
        if (!static_cast<bool>(expr)) {                                                            \
            ::check::report(__FILE__, __LINE__, #expr);                                            \
            throw ::check::stop_case {};                                                           \
        }                                                                                          \
    } while (false)
#define REQUIRE_FALSE(expr) REQUIRE(!static_cast<bool>(expr))

int main(int argc, char** argv)
{
    const char* filter = argc > 1 ? argv[1] : nullptr;
    int run = 0;
    for (const auto& c : ::check::registry()) {
        if (filter && !std::strstr(c.name, filter))
            continue;
        const int before = ::check::failures();
        ++run;
        try {
            c.body();
        } catch (const ::check::stop_case&) {
        } catch (const std::exception& e) {
            ::check::report(__FILE__, __LINE__, e.what());
        }
        std::printf("%s %s\n", ::check::failures() == before ? "ok  " : "FAIL", c.name);
        std::fflush(stdout);
    }
    std::printf("%d cases, %d failed checks\n", run, ::check::failures());
    return ::check::failures() ? 1 : 0;
}
