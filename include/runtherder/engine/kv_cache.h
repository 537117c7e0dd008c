// Single-sequence contiguous E4M3 KV cache (reference
// include/runtherder/engine/kv_cache.h:23-104): K and V slabs
// [num_layers, max_seq_len, num_kv_heads, head_dim], scale slabs
// [num_layers, max_seq_len, num_kv_heads] fp32. The caller owns the write
// position. append() quantizes K and V of one layer in a single launch.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_fp8.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include <rth_attn.h>
#include <runtherder/attention/kv_view.h>
#include <runtherder/check.h>
#include <runtherder/device/check.h>
#include <runtherder/device/memory.h>

namespace runtherder::engine {

class KVCache {
public:
    KVCache(int num_layers, int max_seq_len, int num_kv_heads, int head_dim)
        : num_layers_(num_layers),
          max_seq_len_(max_seq_len),
          num_kv_heads_(num_kv_heads),
          head_dim_(head_dim),
          layer_stride_(static_cast<std::size_t>(max_seq_len) * num_kv_heads * head_dim),
          scale_layer_stride_(static_cast<std::size_t>(max_seq_len) * num_kv_heads) {
        RUNTHERDER_CHECK(num_layers >= 1, "KVCache num_layers must be >= 1");
        RUNTHERDER_CHECK(max_seq_len >= 1, "KVCache max_seq_len must be >= 1");
        RUNTHERDER_CHECK(num_kv_heads >= 1, "KVCache num_kv_heads must be >= 1");
        RUNTHERDER_CHECK(head_dim >= 1, "KVCache head_dim must be >= 1");
        const std::size_t n  = static_cast<std::size_t>(num_layers) * layer_stride_;
        const std::size_t ns = static_cast<std::size_t>(num_layers) * scale_layer_stride_;
        k_       = device::make_device_unique<__hip_fp8_e4m3>(n);
        v_       = device::make_device_unique<__hip_fp8_e4m3>(n);
        k_scale_ = device::make_device_unique<float>(ns);
        v_scale_ = device::make_device_unique<float>(ns);
    }

    KVCache(KVCache&&) noexcept            = default;
    KVCache& operator=(KVCache&&) noexcept = default;
    KVCache(const KVCache&)                = delete;
    KVCache& operator=(const KVCache&)     = delete;

    // Quantizes n_new keys and values ([n_new, num_kv_heads, head_dim] bf16)
    // into `layer` at rows *at_pos .. *at_pos + n_new - 1. at_pos is device
    // resident and unchecked against max_seq_len.
    void append(int layer, const __hip_bfloat16* k, const __hip_bfloat16* v, int n_new,
                const int* at_pos, hipStream_t stream) {
        RUNTHERDER_CHECK(layer >= 0 && layer < num_layers_, "KVCache append layer out of range");
        RUNTHERDER_CHECK(n_new >= 1, "KVCache append n_new must be >= 1");
        RUNTHERDER_CHECK(at_pos != nullptr, "KVCache append at_pos must not be null");
        const std::size_t dst  = static_cast<std::size_t>(layer) * layer_stride_;
        const std::size_t sdst = static_cast<std::size_t>(layer) * scale_layer_stride_;
        RUNTHERDER_RTH_CHECK(rth_kv_append_fp8(
            reinterpret_cast<std::uint8_t*>(k_.get() + dst),
            reinterpret_cast<std::uint8_t*>(v_.get() + dst), k_scale_.get() + sdst,
            v_scale_.get() + sdst, reinterpret_cast<const std::uint16_t*>(k),
            reinterpret_cast<const std::uint16_t*>(v), at_pos, n_new, num_kv_heads_, head_dim_,
            stream));
    }

    // rope_bf16(q, k) followed by append(layer, k, v, ...) in one launch (no
    // reference counterpart; the caller sequence it replaces is reference
    // src/model/supported/llama/llama3.cu:228-232). q is rotated in place;
    // the cache receives the rotated K bytes the two-step sequence would
    // write; k itself is left unrotated. head_dim in {64, 128, 256}.
    void append_rope(int layer, __hip_bfloat16* q, const __hip_bfloat16* k,
                     const __hip_bfloat16* v, int n_new, const int* positions,
                     const float* inv_freq, const int* at_pos, int num_q_heads,
                     hipStream_t stream) {
        RUNTHERDER_CHECK(layer >= 0 && layer < num_layers_, "KVCache append layer out of range");
        RUNTHERDER_CHECK(n_new >= 1, "KVCache append n_new must be >= 1");
        RUNTHERDER_CHECK(at_pos != nullptr, "KVCache append at_pos must not be null");
        const std::size_t dst  = static_cast<std::size_t>(layer) * layer_stride_;
        const std::size_t sdst = static_cast<std::size_t>(layer) * scale_layer_stride_;
        RUNTHERDER_RTH_CHECK(rth_rope_append_fp8(
            reinterpret_cast<std::uint16_t*>(q), reinterpret_cast<std::uint8_t*>(k_.get() + dst),
            reinterpret_cast<std::uint8_t*>(v_.get() + dst), k_scale_.get() + sdst,
            v_scale_.get() + sdst, reinterpret_cast<const std::uint16_t*>(k),
            reinterpret_cast<const std::uint16_t*>(v), positions, inv_freq, at_pos, n_new,
            num_q_heads, num_kv_heads_, head_dim_, stream));
    }

    // Qwen3 order in one launch (no reference counterpart; the caller
    // sequence it replaces is reference src/model/supported/llama/
    // qwen3.cu:189-200): per-head RMSNorm of q and k with gains q_norm,
    // k_norm [head_dim], RoPE, append. q is updated in place; k is read only.
    void append_qk_norm_rope(int layer, __hip_bfloat16* q, const __hip_bfloat16* k,
                             const __hip_bfloat16* v, int n_new, const __hip_bfloat16* q_norm,
                             const __hip_bfloat16* k_norm, float eps, const int* positions,
                             const float* inv_freq, const int* at_pos, int num_q_heads,
                             hipStream_t stream) {
        RUNTHERDER_CHECK(layer >= 0 && layer < num_layers_, "KVCache append layer out of range");
        RUNTHERDER_CHECK(n_new >= 1, "KVCache append n_new must be >= 1");
        RUNTHERDER_CHECK(at_pos != nullptr, "KVCache append at_pos must not be null");
        const std::size_t dst  = static_cast<std::size_t>(layer) * layer_stride_;
        const std::size_t sdst = static_cast<std::size_t>(layer) * scale_layer_stride_;
        RUNTHERDER_RTH_CHECK(rth_qk_norm_rope_append_fp8(
            reinterpret_cast<std::uint16_t*>(q), reinterpret_cast<std::uint8_t*>(k_.get() + dst),
            reinterpret_cast<std::uint8_t*>(v_.get() + dst), k_scale_.get() + sdst,
            v_scale_.get() + sdst, reinterpret_cast<const std::uint16_t*>(k),
            reinterpret_cast<const std::uint16_t*>(v),
            reinterpret_cast<const std::uint16_t*>(q_norm),
            reinterpret_cast<const std::uint16_t*>(k_norm), eps, positions, inv_freq, at_pos,
            n_new, num_q_heads, num_kv_heads_, head_dim_, stream));
    }

    [[nodiscard]] attention::KVView view(int layer) const {
        RUNTHERDER_CHECK(layer >= 0 && layer < num_layers_, "KVCache view layer out of range");
        const std::size_t base  = static_cast<std::size_t>(layer) * layer_stride_;
        const std::size_t sbase = static_cast<std::size_t>(layer) * scale_layer_stride_;
        return attention::KVView{k_.get() + base, v_.get() + base, k_scale_.get() + sbase,
                                 v_scale_.get() + sbase};
    }

    // The writable slabs of `layer`, for AdaptiveAttention's fused decode
    // steps (which store the new token into them).
    [[nodiscard]] attention::KVSlabs slabs(int layer) {
        RUNTHERDER_CHECK(layer >= 0 && layer < num_layers_, "KVCache slabs layer out of range");
        const std::size_t base  = static_cast<std::size_t>(layer) * layer_stride_;
        const std::size_t sbase = static_cast<std::size_t>(layer) * scale_layer_stride_;
        return attention::KVSlabs{k_.get() + base, v_.get() + base, k_scale_.get() + sbase,
                                  v_scale_.get() + sbase};
    }

    [[nodiscard]] int max_seq_len() const noexcept { return max_seq_len_; }

private:
    device::DeviceUniquePtr<__hip_fp8_e4m3> k_;
    device::DeviceUniquePtr<__hip_fp8_e4m3> v_;
    device::DeviceUniquePtr<float>          k_scale_;
    device::DeviceUniquePtr<float>          v_scale_;
    int         num_layers_;
    int         max_seq_len_;
    int         num_kv_heads_;
    int         head_dim_;
    std::size_t layer_stride_;        // max_seq_len * num_kv_heads * head_dim
    std::size_t scale_layer_stride_;  // max_seq_len * num_kv_heads
};

}  // namespace runtherder::engine
