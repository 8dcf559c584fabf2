// Minimal checks for the C++ drop-in tests: a failed CHECK prints the
// condition and location and exits non-zero (independent of NDEBUG).
#pragma once

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <string>

#define CHECK(cond)                                                                       \
    do {                                                                                  \
        if (!(cond)) {                                                                    \
            std::fprintf(stderr, "CHECK failed: %s at %s:%d\n", #cond, __FILE__, __LINE__); \
            std::exit(1);                                                                 \
        }                                                                                 \
    } while (0)

// Runs f and requires an exception of type E whose what() contains `needle`.
template <typename E, typename F>
void expect_throw(const char * needle, F && f, const char * file = __builtin_FILE(), int line = __builtin_LINE()) {
    try {
        f();
    } catch (const E & e) {
        if (needle && std::strstr(e.what(), needle) == nullptr) {
            std::fprintf(stderr, "%s:%d: wrong message \"%s\" (want \"%s\")\n", file, line, e.what(), needle);
            std::exit(1);
        }
        return;
    } catch (const std::exception & e) {
        std::fprintf(stderr, "%s:%d: wrong exception type: %s\n", file, line, e.what());
        std::exit(1);
    }
    std::fprintf(stderr, "%s:%d: no exception (want \"%s\")\n", file, line, needle ? needle : "");
    std::exit(1);
}

inline bool bit_equal(const float * a, const float * b, std::size_t n) {
    return std::memcmp(a, b, n * sizeof(float)) == 0;
}
