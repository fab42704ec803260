// Minimal test runner for the C++ tests (Catch2-like macros; Catch2 is not
// available in this environment).  Usage: velomind_tests [tag-filter]
// where the filter is "[tag]" (only tests with the tag) or "~[tag]"
// (tests without it).  Exit status is the number of failed tests.
#pragma once

#include <cmath>
#include <cstdio>
#include <exception>
#include <functional>
#include <sstream>
#include <string>
#include <vector>

namespace vmtest {

struct Case {
    const char* name;
    const char* tags;
    void (*fn)();
};

inline std::vector<Case>& registry() {
    static std::vector<Case> cases;
    return cases;
}

struct Registrar {
    Registrar(const char* name, const char* tags, void (*fn)()) { registry().push_back({name, tags, fn}); }
};

struct Failure : std::exception {
    std::string msg;
    explicit Failure(std::string m) : msg(std::move(m)) {}
    const char* what() const noexcept override { return msg.c_str(); }
};

struct Skip : std::exception {
    std::string msg;
    explicit Skip(std::string m) : msg(std::move(m)) {}
};

inline int& check_failures() {
    static int n = 0;
    return n;
}

inline std::string where(const char* file, int line) { return std::string(file) + ":" + std::to_string(line); }

}  // namespace vmtest

#define VMT_CAT2(a, b) a##b
#define VMT_CAT(a, b) VMT_CAT2(a, b)
#define TEST_CASE(NAME, TAGS)                                                                     \
    static void VMT_CAT(vmt_fn_, __LINE__)();                                                     \
    static ::vmtest::Registrar VMT_CAT(vmt_reg_, __LINE__)(NAME, TAGS, &VMT_CAT(vmt_fn_, __LINE__)); \
    static void VMT_CAT(vmt_fn_, __LINE__)()

#define REQUIRE(EXPR)                                                                             \
    do {                                                                                          \
        if (!(EXPR)) throw ::vmtest::Failure(::vmtest::where(__FILE__, __LINE__) + ": REQUIRE(" #EXPR ")"); \
    } while (0)

#define CHECK(EXPR)                                                                               \
    do {                                                                                          \
        if (!(EXPR)) {                                                                            \
            std::printf("  %s: CHECK(%s) failed\n", ::vmtest::where(__FILE__, __LINE__).c_str(), #EXPR); \
            ++::vmtest::check_failures();                                                         \
        }                                                                                         \
    } while (0)

#define REQUIRE_THROWS_AS(EXPR, TYPE)                                                             \
    do {                                                                                          \
        bool vmt_caught = false;                                                                  \
        try {                                                                                     \
            (void)(EXPR);                                                                         \
        } catch (const TYPE&) {                                                                   \
            vmt_caught = true;                                                                    \
        } catch (...) {                                                                           \
        }                                                                                         \
        if (!vmt_caught)                                                                          \
            throw ::vmtest::Failure(::vmtest::where(__FILE__, __LINE__) + ": expected " #TYPE " from " #EXPR); \
    } while (0)

#define REQUIRE_NOTHROW(EXPR)                                                                     \
    do {                                                                                          \
        try {                                                                                     \
            (void)(EXPR);                                                                         \
        } catch (const std::exception& e) {                                                       \
            throw ::vmtest::Failure(::vmtest::where(__FILE__, __LINE__) + ": unexpected exception: " + e.what()); \
        }                                                                                         \
    } while (0)

#define SKIP(MSG) throw ::vmtest::Skip(MSG)

#define VMT_MAIN()                                                                                \
    int main(int argc, char** argv) {                                                             \
        std::string filter = argc > 1 ? argv[1] : "";                                             \
        bool negate = !filter.empty() && filter[0] == '~';                                        \
        std::string tag = negate ? filter.substr(1) : filter;                                     \
        int failed = 0, passed = 0, skipped = 0;                                                  \
        for (const auto& c : ::vmtest::registry()) {                                              \
            const bool has = !tag.empty() && std::string(c.tags).find(tag) != std::string::npos;  \
            if (!tag.empty() && has == negate) continue;                                          \
            std::printf("[ RUN  ] %s %s\n", c.name, c.tags);                                      \
            std::fflush(stdout);                                                                  \
            const int before = ::vmtest::check_failures();                                        \
            try {                                                                                 \
                c.fn();                                                                           \
                if (::vmtest::check_failures() != before) throw ::vmtest::Failure("CHECK failures"); \
                ++passed;                                                                         \
                std::printf("[  OK  ] %s\n", c.name);                                             \
            } catch (const ::vmtest::Skip& s) {                                                   \
                ++skipped;                                                                        \
                std::printf("[ SKIP ] %s: %s\n", c.name, s.msg.c_str());                          \
            } catch (const std::exception& e) {                                                   \
                ++failed;                                                                         \
                std::printf("[ FAIL ] %s: %s\n", c.name, e.what());                               \
            }                                                                                     \
            std::fflush(stdout);                                                                  \
        }                                                                                         \
        std::printf("%d passed, %d failed, %d skipped\n", passed, failed, skipped);               \
        return failed;                                                                            \
    }
