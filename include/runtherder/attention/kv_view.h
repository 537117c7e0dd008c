// One layer of the KV cache as seen by an attention backend (reference
// include/runtherder/attention/kv_view.h:14-19). k, v: OCP E4M3
// [max_seq_len, num_kv_heads, head_dim]; k_scale, v_scale: fp32
// [max_seq_len, num_kv_heads], value = float(k[i]) * k_scale[token, kvh].
#pragma once

#include <hip/hip_fp8.h>

namespace runtherder::attention {

struct KVView {
    const __hip_fp8_e4m3* k;
    const __hip_fp8_e4m3* v;
    const float*          k_scale;
    const float*          v_scale;
    // Paged layout (no reference counterpart; the reference README plans
    // paged attention): when block_table is set, position p lives at row
    // block_table[p / block_size] * block_size + p % block_size of the slabs.
    // Views built as KVView{k, v, k_scale, v_scale} stay contiguous.
    const int* block_table = nullptr;
    int        block_size  = 0;
};

// The writable slabs of one layer, for the fused decode steps that store the
// new token into the cache (no reference counterpart: the reference appends
// through KVCache::append and only ever reads through KVView). Same layout
// and paged fields as KVView; KVCache::slabs / PagedKVCache::slabs build it.
struct KVSlabs {
    __hip_fp8_e4m3* k;
    __hip_fp8_e4m3* v;
    float*          k_scale;
    float*          v_scale;
    const int*      block_table = nullptr;
    int             block_size  = 0;

    // The read-only view of the same slabs (for AttentionBackend::run).
    [[nodiscard]] KVView view() const noexcept {
        return KVView{k, v, k_scale, v_scale, block_table, block_size};
    }
};

}  // namespace runtherder::attention
