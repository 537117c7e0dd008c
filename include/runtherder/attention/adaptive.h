// Production backend (reference include/runtherder/attention/adaptive.h):
// n_new == 1 runs the split-K flash decode with backend-owned scratch, n_new > 1
// the MFMA flash prefill. The split count is chosen for the device at
// construction (enough (kv head, split) workgroups to fill every CU) instead of
// the reference's fixed 32.
#pragma once

#include <runtherder/attention/backend.h>
#include <runtherder/device/memory.h>

namespace runtherder::attention {

class AdaptiveAttention final : public AttentionBackend {
public:
    explicit AdaptiveAttention(const AttnConfig& config);
    AdaptiveAttention(const AttnConfig& config, int num_splits);

    void run(__hip_bfloat16*       out,
             const __hip_bfloat16* q,
             const KVView&         kv,
             int                   n_new,
             const int*            cache_len,
             hipStream_t           stream) override;

    [[nodiscard]] int num_splits() const noexcept { return num_splits_; }

private:
    AttnConfig                     config_;
    int                            num_splits_;
    device::DeviceUniquePtr<float> partial_;  // split decode reduction scratch
};

}  // namespace runtherder::attention
