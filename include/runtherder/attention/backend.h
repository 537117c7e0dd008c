// Attention backend interface, unchanged from the reference apart from HIP
// types (reference include/runtherder/attention/backend.h:14-53).
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime.h>

#include <runtherder/attention/kv_view.h>

namespace runtherder::attention {

// Head configuration fixed at construction; scale multiplies each score
// before the softmax (normally 1/sqrt(head_dim)).
struct AttnConfig {
    int   num_q_heads;
    int   num_kv_heads;
    int   head_dim;
    float scale;
};

class AttentionBackend {
public:
    virtual ~AttentionBackend() = default;

    AttentionBackend(const AttentionBackend&)            = delete;
    AttentionBackend& operator=(const AttentionBackend&) = delete;

    // Causal attention of n_new queries (q, out: [n_new, Hq, D] bf16) against
    // the layer cache `kv`, whose rows *cache_len .. *cache_len + n_new - 1 hold
    // the new keys already. cache_len is device resident. Every kernel is
    // enqueued on `stream`; nothing synchronizes.
    virtual void run(__hip_bfloat16*       out,
                     const __hip_bfloat16* q,
                     const KVView&         kv,
                     int                   n_new,
                     const int*            cache_len,
                     hipStream_t           stream) = 0;

protected:
    AttentionBackend()                                       = default;
    AttentionBackend(AttentionBackend&&) noexcept            = default;
    AttentionBackend& operator=(AttentionBackend&&) noexcept = default;
};

}  // namespace runtherder::attention
