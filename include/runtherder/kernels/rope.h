// RoPE free function with the reference signature (reference
// include/runtherder/kernels/rope.cuh:16-25), forwarding to the C ABI.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include <rth_attn.h>
#include <runtherder/device/check.h>

namespace runtherder::kernels {

// In place rotate-half RoPE on q [seq_len, num_q_heads, head_dim] and
// k [seq_len, num_kv_heads, head_dim]; token t rotates by positions[t] with the
// per pair frequencies inv_freq [head_dim / 2] (plain or scaled by the caller).
inline void rope_bf16(__hip_bfloat16* q,
                      __hip_bfloat16* k,
                      const int*      positions,
                      const float*    inv_freq,
                      int             seq_len,
                      int             num_q_heads,
                      int             num_kv_heads,
                      int             head_dim,
                      hipStream_t     stream = nullptr) {
    RUNTHERDER_RTH_CHECK(rth_rope_bf16(reinterpret_cast<std::uint16_t*>(q),
                                       reinterpret_cast<std::uint16_t*>(k), positions, inv_freq,
                                       seq_len, num_q_heads, num_kv_heads, head_dim, stream));
}

}  // namespace runtherder::kernels
