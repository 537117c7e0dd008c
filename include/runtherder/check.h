// Fail-fast argument checks with the reference engine's behaviour: print the
// failed condition and a reason to stderr, then exit(EXIT_FAILURE)
// (reference include/runtherder/check.h:8-23).
#pragma once

#include <cstdio>
#include <cstdlib>

namespace runtherder {

[[noreturn]] inline void check_failed(const char* cond, const char* reason,
                                      const char* file, int line) {
    std::fprintf(stderr, "runtherder check failed at %s:%d\n  condition: %s\n  reason:    %s\n",
                 file, line, cond, reason);
    std::exit(EXIT_FAILURE);
}

}  // namespace runtherder

#define RUNTHERDER_CHECK(cond, msg)                                         \
    do {                                                                    \
        if (!(cond)) [[unlikely]] {                                         \
            ::runtherder::check_failed(#cond, (msg), __FILE__, __LINE__);   \
        }                                                                   \
    } while (0)
