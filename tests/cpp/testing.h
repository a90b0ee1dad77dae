// testing.h -- minimal test registry for the C++ unit tests (no external deps).
// Each TEST registers a function; main() lists (--list) or runs the named
// tests (all when none are named) and exits with the number of failures.
#pragma once
#include <cmath>
#include <cstdio>
#include <functional>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace t {
struct Case {
    std::string name;
    std::function<void()> fn;
};
inline std::vector<Case>& cases() {
    static std::vector<Case> c;
    return c;
}
struct Reg {
    Reg(const char* n, std::function<void()> f) { cases().push_back({n, std::move(f)}); }
};
struct Failure : std::runtime_error {
    using std::runtime_error::runtime_error;
};
}  // namespace t

#define TEST(name)                                   \
    static void test_##name();                       \
    static t::Reg reg_##name(#name, test_##name);    \
    static void test_##name()

#define CHECK(cond)                                                                                    \
    do {                                                                                               \
        if (!(cond)) {                                                                                 \
            std::ostringstream os_;                                                                    \
            os_ << __FILE__ << ":" << __LINE__ << ": CHECK(" #cond ") failed";                        \
            throw t::Failure(os_.str());                                                               \
        }                                                                                              \
    } while (0)

#define CHECK_EQ(a, b)                                                                                 \
    do {                                                                                               \
        auto va_ = (a);                                                                                \
        auto vb_ = (b);                                                                                \
        if (!(va_ == vb_)) {                                                                           \
            std::ostringstream os_;                                                                    \
            os_ << __FILE__ << ":" << __LINE__ << ": CHECK_EQ(" #a ", " #b ") failed: " << va_ << " vs " << vb_; \
            throw t::Failure(os_.str());                                                               \
        }                                                                                              \
    } while (0)

inline int run_tests(int argc, char** argv) {
    std::vector<std::string> want;
    for (int i = 1; i < argc; ++i) {
        std::string a = argv[i];
        if (a == "--list") {
            for (auto& c : t::cases()) std::printf("%s\n", c.name.c_str());
            return 0;
        }
        want.push_back(a);
    }
    int failures = 0, ran = 0;
    for (auto& c : t::cases()) {
        if (!want.empty()) {
            bool sel = false;
            for (auto& w : want) sel |= (w == c.name);
            if (!sel) continue;
        } else if (c.name.rfind("gpu_", 0) == 0) {
            continue;  // GPU tests run only when named
        }
        ++ran;
        try {
            c.fn();
            std::printf("PASS %s\n", c.name.c_str());
        } catch (const std::exception& e) {
            ++failures;
            std::printf("FAIL %s: %s\n", c.name.c_str(), e.what());
        }
        std::fflush(stdout);
    }
    if (ran == 0 && !want.empty()) {
        std::printf("no test matched\n");
        return 1;
    }
    return failures;
}
