// Causal flash prefill with the reference signature (reference
// include/runtherder/kernels/flash_prefill.cuh:26-39), forwarding to the C ABI.
// Scores: the E4M3 K codes and a two-part E4M3 split of q on the scaled fp8
// MFMA (exact products); P V: f16 P and f16(code * v_scale); the accumulation
// and softmax are fp32. flash_prefill_split_bf16 (no reference counterpart)
// serves a few tokens after a long cache as split-K decode.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_fp8.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include <rth_attn.h>
#include <runtherder/device/check.h>

namespace runtherder::kernels {

inline void flash_prefill_bf16(__hip_bfloat16*       out,
                               const __hip_bfloat16* q,
                               const __hip_fp8_e4m3* k,
                               const __hip_fp8_e4m3* v,
                               const float*          k_scale,
                               const float*          v_scale,
                               int                   n_new,
                               const int*            cache_len,
                               int                   num_q_heads,
                               int                   num_kv_heads,
                               int                   head_dim,
                               float                 scale,
                               hipStream_t           stream = nullptr) {
    RUNTHERDER_RTH_CHECK(rth_attn_prefill(
        reinterpret_cast<std::uint16_t*>(out), reinterpret_cast<const std::uint16_t*>(q),
        reinterpret_cast<const std::uint8_t*>(k), reinterpret_cast<const std::uint8_t*>(v),
        k_scale, v_scale, n_new, cache_len, num_q_heads, num_kv_heads, head_dim, scale,
        stream));
}

// No reference counterpart: the same attention split over the keys
// (rth_attn_prefill_split): up to 80 tokens as split-K decode over (token
// block, kv head) units, beyond as the flash prefill over num_splits key runs
// per (row block, q head); partial holds flash_split_scratch_floats(n_new *
// num_q_heads, head_dim, num_splits) floats.
inline void flash_prefill_split_bf16(__hip_bfloat16*       out,
                                     const __hip_bfloat16* q,
                                     const __hip_fp8_e4m3* k,
                                     const __hip_fp8_e4m3* v,
                                     const float*          k_scale,
                                     const float*          v_scale,
                                     float*                partial,
                                     int                   num_splits,
                                     int                   n_new,
                                     const int*            cache_len,
                                     int                   num_q_heads,
                                     int                   num_kv_heads,
                                     int                   head_dim,
                                     float                 scale,
                                     hipStream_t           stream = nullptr) {
    RUNTHERDER_RTH_CHECK(rth_attn_prefill_split(
        reinterpret_cast<std::uint16_t*>(out), reinterpret_cast<const std::uint16_t*>(q),
        reinterpret_cast<const std::uint8_t*>(k), reinterpret_cast<const std::uint8_t*>(v),
        k_scale, v_scale, partial, num_splits, n_new, cache_len, num_q_heads, num_kv_heads,
        head_dim, scale, stream));
}

}  // namespace runtherder::kernels
