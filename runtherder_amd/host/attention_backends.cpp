// AdaptiveAttention, NaiveAttention and the backend factory over the C ABI
// (reference src/attention/adaptive.cu, naive.cu, factory.cu).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>

#include <rth_attn.h>
#include <runtherder/attention/adaptive.h>
#include <runtherder/attention/factory.h>
#include <runtherder/attention/naive.h>
#include <runtherder/check.h>
#include <runtherder/device/check.h>

namespace runtherder::attention {

namespace {

int device_num_splits(int num_kv_heads) {
    int dev = 0;
    RUNTHERDER_HIP_CHECK(hipGetDevice(&dev));
    return rth_default_num_splits(num_kv_heads, dev);
}

}  // namespace

AdaptiveAttention::AdaptiveAttention(const AttnConfig& config)
    : AdaptiveAttention(config, device_num_splits(config.num_kv_heads)) {}

AdaptiveAttention::AdaptiveAttention(const AttnConfig& config, int num_splits)
    : config_(config), num_splits_(num_splits) {
    RUNTHERDER_CHECK(num_splits >= 1, "AdaptiveAttention num_splits must be >= 1");
    int dev = 0;
    RUNTHERDER_HIP_CHECK(hipGetDevice(&dev));
    RUNTHERDER_HIP_CHECK(hipDeviceGetAttribute(&cus_, hipDeviceAttributeMultiprocessorCount, dev));
    const std::size_t dec =
        rth_split_scratch_floats(config.num_q_heads, config.head_dim, num_splits);
    const std::size_t runs =
        config.head_dim == 128
            ? rth_split_scratch_floats(config.num_q_heads, config.head_dim, kPrefillRunTokenRuns)
            : 0;
    partial_ = device::make_device_unique<float>(dec > runs ? dec : runs);
}

int AdaptiveAttention::prefill_split_count(int n_new) const noexcept {
    if (n_new >= 2 && n_new <= kPrefillSplitTokens &&
        rth_decode_path(config_.num_q_heads, config_.num_kv_heads, config_.head_dim) ==
            RTH_DECODE_MFMA) {
        return num_splits_ / (2 * n_new) > 1 ? num_splits_ / (2 * n_new) : 1;
    }
    if (n_new > kPrefillSplitTokens && n_new <= kPrefillRunsTokens && config_.head_dim == 128) {
        // About two rounds of 4-wave workgroups, within the scratch.
        const int blocks = (n_new + 127) / 128 * config_.num_q_heads;
        int       runs   = 2 * cus_ / blocks;
        runs             = runs < 16 ? runs : 16;
        runs             = runs < kPrefillRunTokenRuns / n_new ? runs : kPrefillRunTokenRuns / n_new;
        return runs > 1 ? runs : 0;
    }
    return 0;
}

void AdaptiveAttention::run(__hip_bfloat16* out, const __hip_bfloat16* q, const KVView& kv,
                            int n_new, const int* cache_len, hipStream_t stream) {
    auto* o  = reinterpret_cast<std::uint16_t*>(out);
    auto* qq = reinterpret_cast<const std::uint16_t*>(q);
    auto* k  = reinterpret_cast<const std::uint8_t*>(kv.k);
    auto* v  = reinterpret_cast<const std::uint8_t*>(kv.v);
    const bool paged = kv.block_table != nullptr;
    if (const int splits = prefill_split_count(n_new); splits > 0) {
        if (paged) {
            RUNTHERDER_RTH_CHECK(rth_attn_prefill_split_paged(
                o, qq, k, v, kv.k_scale, kv.v_scale, kv.block_table, kv.block_size,
                partial_.get(), splits, n_new, cache_len, config_.num_q_heads,
                config_.num_kv_heads, config_.head_dim, config_.scale, stream));
        } else {
            RUNTHERDER_RTH_CHECK(rth_attn_prefill_split(
                o, qq, k, v, kv.k_scale, kv.v_scale, partial_.get(), splits, n_new, cache_len,
                config_.num_q_heads, config_.num_kv_heads, config_.head_dim, config_.scale,
                stream));
        }
        return;
    }
    if (n_new == 1) {
        if (paged) {
            RUNTHERDER_RTH_CHECK(rth_attn_decode_split_paged(
                o, qq, k, v, kv.k_scale, kv.v_scale, kv.block_table, kv.block_size,
                partial_.get(), num_splits_, cache_len, config_.num_q_heads,
                config_.num_kv_heads, config_.head_dim, config_.scale, stream));
        } else {
            RUNTHERDER_RTH_CHECK(rth_attn_decode_split(o, qq, k, v, kv.k_scale, kv.v_scale,
                                                       partial_.get(), num_splits_, cache_len,
                                                       config_.num_q_heads, config_.num_kv_heads,
                                                       config_.head_dim, config_.scale, stream));
        }
        return;
    }
    if (paged) {
        RUNTHERDER_RTH_CHECK(rth_attn_prefill_paged(
            o, qq, k, v, kv.k_scale, kv.v_scale, kv.block_table, kv.block_size, n_new, cache_len,
            config_.num_q_heads, config_.num_kv_heads, config_.head_dim, config_.scale, stream));
        return;
    }
    RUNTHERDER_RTH_CHECK(rth_attn_prefill(o, qq, k, v, kv.k_scale, kv.v_scale, n_new, cache_len,
                                          config_.num_q_heads, config_.num_kv_heads,
                                          config_.head_dim, config_.scale, stream));
}

namespace {

std::uint8_t* u8(__hip_fp8_e4m3* p) { return reinterpret_cast<std::uint8_t*>(p); }

const std::uint16_t* u16(const __hip_bfloat16* p) {
    return reinterpret_cast<const std::uint16_t*>(p);
}

}  // namespace

void AdaptiveAttention::run_decode_append(__hip_bfloat16* out, const __hip_bfloat16* q,
                                          const KVSlabs& kv, const __hip_bfloat16* k_new,
                                          const __hip_bfloat16* v_new, const int* cache_len,
                                          hipStream_t stream) {
    auto*       o = reinterpret_cast<std::uint16_t*>(out);
    if (kv.block_table != nullptr) {
        RUNTHERDER_RTH_CHECK(rth_attn_decode_append_split_paged(
            o, u16(q), u8(kv.k), u8(kv.v), kv.k_scale, kv.v_scale, kv.block_table, kv.block_size, u16(k_new),
            u16(v_new), partial_.get(), num_splits_, cache_len, config_.num_q_heads,
            config_.num_kv_heads, config_.head_dim, config_.scale, stream));
        return;
    }
    RUNTHERDER_RTH_CHECK(rth_attn_decode_append_split(
        o, u16(q), u8(kv.k), u8(kv.v), kv.k_scale, kv.v_scale, u16(k_new), u16(v_new), partial_.get(), num_splits_,
        cache_len, config_.num_q_heads, config_.num_kv_heads, config_.head_dim, config_.scale,
        stream));
}

void AdaptiveAttention::run_decode_rope_append(__hip_bfloat16* out, const __hip_bfloat16* q,
                                               const KVSlabs& kv, const __hip_bfloat16* k_new,
                                               const __hip_bfloat16* v_new, const int* positions,
                                               const float* inv_freq, const int* cache_len,
                                               hipStream_t stream) {
    auto*       o = reinterpret_cast<std::uint16_t*>(out);
    if (kv.block_table != nullptr) {
        RUNTHERDER_RTH_CHECK(rth_attn_decode_rope_append_split_paged(
            o, u16(q), u8(kv.k), u8(kv.v), kv.k_scale, kv.v_scale, kv.block_table, kv.block_size, u16(k_new),
            u16(v_new), positions, inv_freq, partial_.get(), num_splits_, cache_len,
            config_.num_q_heads, config_.num_kv_heads, config_.head_dim, config_.scale, stream));
        return;
    }
    RUNTHERDER_RTH_CHECK(rth_attn_decode_rope_append_split(
        o, u16(q), u8(kv.k), u8(kv.v), kv.k_scale, kv.v_scale, u16(k_new), u16(v_new), positions, inv_freq,
        partial_.get(), num_splits_, cache_len, config_.num_q_heads, config_.num_kv_heads,
        config_.head_dim, config_.scale, stream));
}

void AdaptiveAttention::run_decode_qk_norm_rope_append(
    __hip_bfloat16* out, const __hip_bfloat16* q, const KVSlabs& kv, const __hip_bfloat16* k_new,
    const __hip_bfloat16* v_new, const __hip_bfloat16* q_norm, const __hip_bfloat16* k_norm,
    float eps, const int* positions, const float* inv_freq, const int* cache_len,
    hipStream_t stream) {
    auto*       o = reinterpret_cast<std::uint16_t*>(out);
    if (kv.block_table != nullptr) {
        RUNTHERDER_RTH_CHECK(rth_attn_decode_qk_norm_rope_append_split_paged(
            o, u16(q), u8(kv.k), u8(kv.v), kv.k_scale, kv.v_scale, kv.block_table, kv.block_size, u16(k_new),
            u16(v_new), u16(q_norm), u16(k_norm), eps, positions, inv_freq, partial_.get(),
            num_splits_, cache_len, config_.num_q_heads, config_.num_kv_heads, config_.head_dim,
            config_.scale, stream));
        return;
    }
    RUNTHERDER_RTH_CHECK(rth_attn_decode_qk_norm_rope_append_split(
        o, u16(q), u8(kv.k), u8(kv.v), kv.k_scale, kv.v_scale, u16(k_new), u16(v_new), u16(q_norm), u16(k_norm), eps,
        positions, inv_freq, partial_.get(), num_splits_, cache_len, config_.num_q_heads,
        config_.num_kv_heads, config_.head_dim, config_.scale, stream));
}

NaiveAttention::NaiveAttention(const AttnConfig& config) noexcept : config_(config) {}

void NaiveAttention::run(__hip_bfloat16* out, const __hip_bfloat16* q, const KVView& kv,
                         int n_new, const int* cache_len, hipStream_t stream) {
    RUNTHERDER_CHECK(kv.block_table == nullptr, "NaiveAttention reads contiguous caches only");
    RUNTHERDER_RTH_CHECK(rth_attn_naive(
        reinterpret_cast<std::uint16_t*>(out), reinterpret_cast<const std::uint16_t*>(q),
        reinterpret_cast<const std::uint8_t*>(kv.k), reinterpret_cast<const std::uint8_t*>(kv.v),
        kv.k_scale, kv.v_scale, n_new, cache_len, config_.num_q_heads, config_.num_kv_heads,
        config_.head_dim, config_.scale, stream));
}

std::unique_ptr<AttentionBackend> make_attention_backend(BackendKind kind,
                                                         const AttnConfig& config) {
    switch (kind) {
        case BackendKind::Naive:
            return std::make_unique<NaiveAttention>(config);
        case BackendKind::Adaptive:
            return std::make_unique<AdaptiveAttention>(config);
    }
    RUNTHERDER_CHECK(false, "unknown attention BackendKind");
}

}  // namespace runtherder::attention
