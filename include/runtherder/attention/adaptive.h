// Production backend (reference include/runtherder/attention/adaptive.h):
// n_new == 1 runs the split-K flash decode with backend-owned scratch, n_new > 1
// the MFMA flash prefill. The split count is chosen for the device at
// construction (enough (kv head, split) workgroups to fill every CU) instead of
// the reference's fixed 32. Calls of 2 .. kPrefillSplitTokens tokens on shapes
// the MFMA decode kernel serves run rth_attn_prefill_split over the same
// scratch with num_splits / (2 n_new) splits (no reference counterpart: a few
// tokens after a long cache as split-K decode; 16 / 64 tokens after 8K keys
// 209 / 199 -> 18 / 34 us per call, at an empty cache up to ~2 us slower),
// and at head_dim 128 calls of up to kPrefillRunsTokens tokens run it as the
// flash prefill over key runs (128 / 256 tokens after 32K keys 828 / 830 ->
// 98 / 187 us; at an empty cache 11 / 14 -> 19 / 27 us). For those the
// scratch holds kPrefillRunTokenRuns token-runs (34 MB at 32 q heads).
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

    // The decode step of one layer as one call of two kernels (no reference
    // counterpart): KVCache::append of the token k_new, v_new
    // ([num_kv_heads, head_dim] bf16) at row *cache_len, then
    // run(out, q, kv.view(), 1, cache_len) (reference llama3.cu:232-234). kv
    // holds the layer's writable slabs (KVCache::slabs / PagedKVCache::slabs);
    // paged when kv.block_table is set. Bit-identical to append followed by run.
    void run_decode_append(__hip_bfloat16*       out,
                           const __hip_bfloat16* q,
                           const KVSlabs&        kv,
                           const __hip_bfloat16* k_new,
                           const __hip_bfloat16* v_new,
                           const int*            cache_len,
                           hipStream_t           stream);

    // The same step with rope_bf16(q, k_new) (positions[0], inv_freq;
    // reference rope.cu:14-55) applied in the split kernel's registers
    // (llama3.cu:228-234 in two launches). q and k_new are read only.
    void run_decode_rope_append(__hip_bfloat16*       out,
                                const __hip_bfloat16* q,
                                const KVSlabs&        kv,
                                const __hip_bfloat16* k_new,
                                const __hip_bfloat16* v_new,
                                const int*            positions,
                                const float*          inv_freq,
                                const int*            cache_len,
                                hipStream_t           stream);

    // Qwen3's order (qwen3.cu:189-202): per-head RMSNorm of q and k_new with
    // the q_norm / k_norm gains ([head_dim] bf16), RoPE, append, decode.
    void run_decode_qk_norm_rope_append(__hip_bfloat16*       out,
                                        const __hip_bfloat16* q,
                                        const KVSlabs&        kv,
                                        const __hip_bfloat16* k_new,
                                        const __hip_bfloat16* v_new,
                                        const __hip_bfloat16* q_norm,
                                        const __hip_bfloat16* k_norm,
                                        float                 eps,
                                        const int*            positions,
                                        const float*          inv_freq,
                                        const int*            cache_len,
                                        hipStream_t           stream);

    [[nodiscard]] int num_splits() const noexcept { return num_splits_; }

    static constexpr int kPrefillSplitTokens  = 80;
    static constexpr int kPrefillRunsTokens   = 256;
    static constexpr int kPrefillRunTokenRuns = 2048;

private:
    // Split count of rth_attn_prefill_split for an n_new-token call, 0 when
    // the call takes the flash prefill (or decode) instead.
    [[nodiscard]] int prefill_split_count(int n_new) const noexcept;

    AttnConfig                     config_;
    int                            num_splits_;
    int                            cus_ = 256;
    device::DeviceUniquePtr<float> partial_;  // split decode reduction scratch
};

}  // namespace runtherder::attention
