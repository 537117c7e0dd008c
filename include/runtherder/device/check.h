// HIP error and C-ABI status checks, fail-fast like the reference's
// RUNTHERDER_CUDA_CHECK (reference include/runtherder/device/check.cuh:11-26).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include <rth_attn.h>
#include <runtherder/check.h>

namespace runtherder::device {

inline void check_hip(hipError_t err, const char* expr, const char* file, int line) {
    if (err != hipSuccess) [[unlikely]] {
        std::fprintf(stderr, "HIP error at %s:%d -- %s\n  %s\n", file, line,
                     hipGetErrorString(err), expr);
        std::exit(EXIT_FAILURE);
    }
}

inline void check_rth(int rc, const char* expr, const char* file, int line) {
    if (rc != RTH_OK) [[unlikely]] {
        std::fprintf(stderr, "runtherder check failed at %s:%d\n  call:      %s\n  reason:    %s\n",
                     file, line, expr, rth_last_error_string());
        std::exit(EXIT_FAILURE);
    }
}

}  // namespace runtherder::device

#define RUNTHERDER_HIP_CHECK(expr) ::runtherder::device::check_hip((expr), #expr, __FILE__, __LINE__)
#define RUNTHERDER_RTH_CHECK(expr) ::runtherder::device::check_rth((expr), #expr, __FILE__, __LINE__)
