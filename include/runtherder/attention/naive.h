// The same two-pass causal attention at every shape (reference
// include/runtherder/attention/naive.h).
#pragma once

#include <runtherder/attention/backend.h>

namespace runtherder::attention {

class NaiveAttention final : public AttentionBackend {
public:
    explicit NaiveAttention(const AttnConfig& config) noexcept;

    void run(__hip_bfloat16*       out,
             const __hip_bfloat16* q,
             const KVView&         kv,
             int                   n_new,
             const int*            cache_len,
             hipStream_t           stream) override;

private:
    AttnConfig config_;
};

}  // namespace runtherder::attention
