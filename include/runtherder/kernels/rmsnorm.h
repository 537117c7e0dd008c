// RMSNorm free function with the reference signature (reference
// include/runtherder/kernels/rmsnorm.cuh:14-22), forwarding to the C ABI.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include <rth_attn.h>
#include <runtherder/device/check.h>

namespace runtherder::kernels {

// y = (x / rms(x)) * g per row of x [num_tokens, hidden_dim]; y may alias x.
inline void rmsnorm_bf16_forward(__hip_bfloat16*       y,
                                 const __hip_bfloat16* x,
                                 const __hip_bfloat16* g,
                                 int                   num_tokens,
                                 int                   hidden_dim,
                                 float                 eps,
                                 hipStream_t           stream = nullptr) {
    RUNTHERDER_RTH_CHECK(rth_rmsnorm_bf16(reinterpret_cast<std::uint16_t*>(y),
                                          reinterpret_cast<const std::uint16_t*>(x),
                                          reinterpret_cast<const std::uint16_t*>(g), num_tokens,
                                          hidden_dim, eps, stream));
}

}  // namespace runtherder::kernels
