// Paged FP8 KV cache (no counterpart in the reference, whose README plans
// paged attention): per layer, num_blocks physical blocks of block_size
// positions. The caller owns the block table (device int array mapping
// logical block -> physical block) and passes it to append() and view();
// views carry it, so AttentionBackend::run keeps its signature.
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

class PagedKVCache {
public:
    // block_size: a power of two >= 32.
    PagedKVCache(int num_layers, int num_blocks, int block_size, int num_kv_heads, int head_dim)
        : num_layers_(num_layers), num_blocks_(num_blocks), block_size_(block_size),
          num_kv_heads_(num_kv_heads), head_dim_(head_dim) {
        RUNTHERDER_CHECK(num_layers >= 1 && num_blocks >= 1 && num_kv_heads >= 1 &&
                             head_dim >= 1,
                         "PagedKVCache dimensions must be >= 1");
        RUNTHERDER_CHECK(block_size >= 32 && (block_size & (block_size - 1)) == 0,
                         "PagedKVCache block_size must be a power of two >= 32");
        const std::size_t rows = static_cast<std::size_t>(num_blocks) * block_size * num_kv_heads;
        layer_stride_       = rows * head_dim;
        scale_layer_stride_ = rows;
        k_       = device::make_device_unique<__hip_fp8_e4m3>(layer_stride_ * num_layers);
        v_       = device::make_device_unique<__hip_fp8_e4m3>(layer_stride_ * num_layers);
        k_scale_ = device::make_device_unique<float>(scale_layer_stride_ * num_layers);
        v_scale_ = device::make_device_unique<float>(scale_layer_stride_ * num_layers);
    }

    // Quantizes n_new keys and values into logical positions *at_pos ..
    // *at_pos + n_new - 1 of `layer`, through block_table.
    void append(int layer, const __hip_bfloat16* k, const __hip_bfloat16* v, int n_new,
                const int* at_pos, const int* block_table, hipStream_t stream) {
        RUNTHERDER_CHECK(layer >= 0 && layer < num_layers_, "KVCache append layer out of range");
        RUNTHERDER_CHECK(n_new >= 1, "KVCache append n_new must be >= 1");
        const std::size_t dst  = static_cast<std::size_t>(layer) * layer_stride_;
        const std::size_t sdst = static_cast<std::size_t>(layer) * scale_layer_stride_;
        RUNTHERDER_RTH_CHECK(rth_kv_append_fp8_paged(
            reinterpret_cast<std::uint8_t*>(k_.get() + dst),
            reinterpret_cast<std::uint8_t*>(v_.get() + dst), k_scale_.get() + sdst,
            v_scale_.get() + sdst, reinterpret_cast<const std::uint16_t*>(k),
            reinterpret_cast<const std::uint16_t*>(v), at_pos, n_new, num_kv_heads_, head_dim_,
            block_table, block_size_, stream));
    }

    [[nodiscard]] attention::KVView view(int layer, const int* block_table) const {
        RUNTHERDER_CHECK(layer >= 0 && layer < num_layers_, "KVCache view layer out of range");
        const std::size_t base  = static_cast<std::size_t>(layer) * layer_stride_;
        const std::size_t sbase = static_cast<std::size_t>(layer) * scale_layer_stride_;
        return attention::KVView{k_.get() + base, v_.get() + base, k_scale_.get() + sbase,
                                 v_scale_.get() + sbase, block_table, block_size_};
    }

    [[nodiscard]] attention::KVSlabs slabs(int layer, const int* block_table) {
        RUNTHERDER_CHECK(layer >= 0 && layer < num_layers_, "KVCache slabs layer out of range");
        const std::size_t base  = static_cast<std::size_t>(layer) * layer_stride_;
        const std::size_t sbase = static_cast<std::size_t>(layer) * scale_layer_stride_;
        return attention::KVSlabs{k_.get() + base, v_.get() + base, k_scale_.get() + sbase,
                                  v_scale_.get() + sbase, block_table, block_size_};
    }

    [[nodiscard]] int block_size() const noexcept { return block_size_; }
    [[nodiscard]] int num_blocks() const noexcept { return num_blocks_; }

private:
    int         num_layers_, num_blocks_, block_size_, num_kv_heads_, head_dim_;
    std::size_t layer_stride_       = 0;
    std::size_t scale_layer_stride_ = 0;
    device::DeviceUniquePtr<__hip_fp8_e4m3> k_;
    device::DeviceUniquePtr<__hip_fp8_e4m3> v_;
    device::DeviceUniquePtr<float>          k_scale_;
    device::DeviceUniquePtr<float>          v_scale_;
};

}  // namespace runtherder::engine
