// KV quantization free functions with the reference signatures (reference
// include/runtherder/kernels/quantization.cuh:50-66), forwarding to the C ABI.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_fp8.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include <rth_attn.h>
#include <runtherder/device/check.h>

namespace runtherder::kernels {

// q = x / scale with scale = row amax / 448, one row per quant group; rows land
// at *at_pos * rows_per_pos onward. at_pos is device resident and unchecked.
inline void quantize_kv_fp8(__hip_fp8_e4m3*       q,
                            float*                scale,
                            const __hip_bfloat16* x,
                            const int*            at_pos,
                            int                   rows_per_pos,
                            int                   num_rows,
                            int                   head_dim,
                            hipStream_t           stream = nullptr) {
    RUNTHERDER_RTH_CHECK(rth_kv_quantize_fp8(reinterpret_cast<std::uint8_t*>(q), scale,
                                             reinterpret_cast<const std::uint16_t*>(x),
                                             at_pos, rows_per_pos, num_rows, head_dim,
                                             stream));
}

// Per value inverse of quantize_kv_fp8 (host side: decodes the E4M3 byte).
[[nodiscard]] inline float dequantize_kv_fp8(__hip_fp8_e4m3 q, float scale) {
    return static_cast<float>(q) * scale;
}

}  // namespace runtherder::kernels
