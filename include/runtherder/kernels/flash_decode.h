// Split-K flash decode with the reference signature (reference
// include/runtherder/kernels/flash_decode.cuh:16-59), forwarding to the C ABI.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_fp8.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include <rth_attn.h>
#include <runtherder/device/check.h>

namespace runtherder::kernels {

// Floats of decode scratch for max_splits splits: Hq*S m, then Hq*S l, then
// Hq*S*D acc values, one contiguous slab (same formula as the reference, and as
// rth_split_scratch_floats; usable in constant expressions as the reference's).
[[nodiscard]] constexpr std::size_t flash_split_scratch_floats(int num_q_heads, int head_dim,
                                                               int max_splits) {
    const std::size_t heads  = static_cast<std::size_t>(num_q_heads);
    const std::size_t splits = static_cast<std::size_t>(max_splits);
    const std::size_t dim    = static_cast<std::size_t>(head_dim);
    return heads * splits * 2 + heads * splits * dim;
}

// One query token attends *cache_len + 1 keys in num_splits key ranges merged by
// log-sum-exp. The split reassociates the float accumulation and can differ
// from a serial accumulation in the last bits, not in value.
inline void flash_decode_split_bf16(__hip_bfloat16*       out,
                                    const __hip_bfloat16* q,
                                    const __hip_fp8_e4m3* k,
                                    const __hip_fp8_e4m3* v,
                                    const float*          k_scale,
                                    const float*          v_scale,
                                    float*                partial,
                                    int                   num_splits,
                                    const int*            cache_len,
                                    int                   num_q_heads,
                                    int                   num_kv_heads,
                                    int                   head_dim,
                                    float                 scale,
                                    hipStream_t           stream = nullptr) {
    RUNTHERDER_RTH_CHECK(rth_attn_decode_split(
        reinterpret_cast<std::uint16_t*>(out), reinterpret_cast<const std::uint16_t*>(q),
        reinterpret_cast<const std::uint8_t*>(k), reinterpret_cast<const std::uint8_t*>(v),
        k_scale, v_scale, partial, num_splits, cache_len, num_q_heads, num_kv_heads, head_dim,
        scale, stream));
}

// KVCache::append of one token at row *cache_len followed by
// flash_decode_split_bf16 over *cache_len + 1 keys, as one call (no reference
// counterpart). k, v, k_scale, v_scale are the layer's writable cache slabs;
// k_new, v_new are [num_kv_heads, head_dim] bf16.
inline void flash_decode_append_split_bf16(__hip_bfloat16*       out,
                                           const __hip_bfloat16* q,
                                           __hip_fp8_e4m3*       k,
                                           __hip_fp8_e4m3*       v,
                                           float*                k_scale,
                                           float*                v_scale,
                                           const __hip_bfloat16* k_new,
                                           const __hip_bfloat16* v_new,
                                           float*                partial,
                                           int                   num_splits,
                                           const int*            cache_len,
                                           int                   num_q_heads,
                                           int                   num_kv_heads,
                                           int                   head_dim,
                                           float                 scale,
                                           hipStream_t           stream = nullptr) {
    RUNTHERDER_RTH_CHECK(rth_attn_decode_append_split(
        reinterpret_cast<std::uint16_t*>(out), reinterpret_cast<const std::uint16_t*>(q),
        reinterpret_cast<std::uint8_t*>(k), reinterpret_cast<std::uint8_t*>(v), k_scale, v_scale,
        reinterpret_cast<const std::uint16_t*>(k_new), reinterpret_cast<const std::uint16_t*>(v_new),
        partial, num_splits, cache_len, num_q_heads, num_kv_heads, head_dim, scale, stream));
}

}  // namespace runtherder::kernels
