#pragma once
// A small self-registering test harness for the C++ test programs (no external framework).
#include <cstdio>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

namespace vktest {

struct Entry {
    const char* name;
    std::function<void()> fn;
};

inline std::vector<Entry>& entries() {
    static std::vector<Entry> all;
    return all;
}

struct Add {
    Add(const char* name, std::function<void()> fn) { entries().push_back({name, std::move(fn)}); }
};

inline int run() {
    int failures = 0;
    for (const auto& e : entries()) {
        try {
            e.fn();
            std::printf("ok    %s\n", e.name);
        } catch (const std::exception& ex) {
            ++failures;
            std::printf("FAIL  %s: %s\n", e.name, ex.what());
        }
        std::fflush(stdout);
    }
    std::printf("%zu cases, %d failed\n", entries().size(), failures);
    return failures ? 1 : 0;
}

[[noreturn]] inline void fail_at(const char* file, int line, const std::string& what) {
    throw std::runtime_error(std::string(file) + ":" + std::to_string(line) + ": " + what);
}

}  // namespace vktest

#define VKT_JOIN2(a, b) a##b
#define VKT_JOIN(a, b) VKT_JOIN2(a, b)
#define CASE(name)                                                                          \
    static void VKT_JOIN(case_, __LINE__)();                                                \
    static const vktest::Add VKT_JOIN(add_, __LINE__)(name, &VKT_JOIN(case_, __LINE__));    \
    static void VKT_JOIN(case_, __LINE__)()
#define EXPECT(cond) \
    do {             \
        if (!(cond)) vktest::fail_at(__FILE__, __LINE__, "expected " #cond); \
    } while (0)
#define EXPECT_THROWS(stmt)                                                          \
    do {                                                                             \
        bool thrown_ = false;                                                        \
        try {                                                                        \
            stmt;                                                                    \
        } catch (const std::exception&) {                                            \
            thrown_ = true;                                                          \
        }                                                                            \
        if (!thrown_) vktest::fail_at(__FILE__, __LINE__, "no exception from " #stmt); \
    } while (0)
