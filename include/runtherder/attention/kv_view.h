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
};

}  // namespace runtherder::attention
