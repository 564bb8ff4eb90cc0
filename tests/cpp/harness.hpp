// Minimal test harness shared by the C++ test binaries: TEST(name) registers
// a case, CHECK(cond) fails it, and run_cases() implements
//   <binary> --list        print every case name
//   <binary> NAME...       run the named cases (all when none given)
#pragma once

#include <cstdio>
#include <cstring>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

namespace harness {

struct Case {
    const char *name;
    std::function<void()> fn;
};
inline std::vector<Case> &registry() {
    static std::vector<Case> r;
    return r;
}
struct Register {
    Register(const char *n, std::function<void()> f) { registry().push_back({n, std::move(f)}); }
};
struct Failure : std::runtime_error {
    using std::runtime_error::runtime_error;
};

template <class E = std::exception, class F>
std::string expect_throw(F f) {
    try {
        f();
    } catch (const E &e) {
        return e.what();
    }
    throw Failure("expected an exception");
}

inline int run_cases(int argc, char **argv) {
    if (argc == 2 && std::strcmp(argv[1], "--list") == 0) {
        for (const auto &c : registry()) std::printf("%s\n", c.name);
        return 0;
    }
    int failed = 0, ran = 0;
    for (const auto &c : registry()) {
        bool wanted = argc == 1;
        for (int i = 1; i < argc; ++i) wanted = wanted || std::strcmp(argv[i], c.name) == 0;
        if (!wanted) continue;
        ++ran;
        try {
            c.fn();
            std::printf("PASS %s\n", c.name);
        } catch (const std::exception &e) {
            ++failed;
            std::printf("FAIL %s: %s\n", c.name, e.what());
        }
        std::fflush(stdout);
    }
    if (ran == 0) {
        std::printf("no such case\n");
        return 2;
    }
    return failed ? 1 : 0;
}

}  // namespace harness

#define TEST(name)                                           \
    static void name();                                      \
    static harness::Register reg_##name(#name, name);        \
    static void name()

#define CHECK(cond)                                                                                            \
    do {                                                                                                       \
        if (!(cond)) throw harness::Failure(std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " #cond); \
    } while (0)
