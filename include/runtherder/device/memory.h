// Owning device buffers (reference include/runtherder/device/memory.cuh:11-35),
// allocated with hipMalloc and released with hipFree.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <memory>

#include <runtherder/device/check.h>

namespace runtherder::device {

struct HipFree {
    template <typename T>
    void operator()(T* p) const noexcept {
        if (p != nullptr) {
            (void)hipFree(p);
        }
    }
};

template <typename T>
using DeviceUniquePtr = std::unique_ptr<T[], HipFree>;

// count == 0 yields an empty pointer and no allocation.
template <typename T>
[[nodiscard]] inline DeviceUniquePtr<T> make_device_unique(std::size_t count) {
    if (count == 0) {
        return DeviceUniquePtr<T>{};
    }
    T* p = nullptr;
    RUNTHERDER_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&p), count * sizeof(T)));
    return DeviceUniquePtr<T>{p};
}

}  // namespace runtherder::device
