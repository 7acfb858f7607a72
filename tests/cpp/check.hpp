// check.hpp — minimal assertion harness for the C++ tests (gtest is not
// available offline).  Each CHECK failure prints file:line and counts; main()
// returns the failure count.
#pragma once

#include <cstdio>
#include <functional>
#include <string>
#include <vector>

namespace check {

inline int& failures() {
    static int n = 0;
    return n;
}

struct Case {
    const char* name;
    std::function<void()> fn;
};

inline std::vector<Case>& cases() {
    static std::vector<Case> c;
    return c;
}

struct Register {
    Register(const char* name, std::function<void()> fn) { cases().push_back({name, std::move(fn)}); }
};

inline int run_all() {
    for (auto& c : cases()) {
        const int before = failures();
        c.fn();
        std::printf("[%s] %s\n", failures() == before ? "PASS" : "FAIL", c.name);
    }
    std::printf("%d failure(s) in %zu case(s)\n", failures(), cases().size());
    return failures();
}

}  // namespace check

#define TEST_CASE(name)                                              \
    static void name();                                              \
    static check::Register reg_##name(#name, name);                  \
    static void name()

#define CHECK(cond)                                                               \
    do {                                                                          \
        if (!(cond)) {                                                            \
            std::printf("  %s:%d: CHECK(%s) failed\n", __FILE__, __LINE__, #cond); \
            ++check::failures();                                                  \
        }                                                                         \
    } while (0)

#define CHECK_EQ(a, b)                                                                          \
    do {                                                                                        \
        auto _a = (a);                                                                          \
        auto _b = (b);                                                                          \
        if (!(_a == _b)) {                                                                      \
            std::printf("  %s:%d: CHECK_EQ(%s, %s) failed: %lld vs %lld\n", __FILE__, __LINE__, #a, #b, \
                        (long long)_a, (long long)_b);                                          \
            ++check::failures();                                                                \
        }                                                                                       \
    } while (0)
