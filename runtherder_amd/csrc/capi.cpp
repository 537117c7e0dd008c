// extern "C" boundary of libruntherder_attn.so (declared in include/rth_attn.h).
//
// Argument checks mirror the reference's launch-site RUNTHERDER_CHECKs
// (reference src/kernels/flash_decode.cu:286-291, flash_prefill.cu:226-228,
// attention.cu:109-116, quantization.cu:348-352) but report through return
// codes and rth_last_error_string() instead of exiting the process.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/rth_attn.h"
#include "launch.hpp"

namespace rth {
bool decode_mfma_supported(int num_q_heads, int num_kv_heads, int head_dim);

namespace {
constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];   // 0 = not queried yet
}  // namespace

hipError_t device_cu_count(int* cus) {
    int        dev = 0;
    hipError_t e   = hipGetDevice(&dev);
    if (e != hipSuccess) {
        return e;
    }
    if (dev >= 0 && dev < kMaxDevices) {
        const int c = g_cu_count[dev].load(std::memory_order_relaxed);
        if (c > 0) {
            *cus = c;
            return hipSuccess;
        }
    }
    int c = 0;
    e     = hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) {
        return e;
    }
    if (c < 1) {
        return hipErrorInvalidDevice;
    }
    if (dev >= 0 && dev < kMaxDevices) {
        g_cu_count[dev].store(c, std::memory_order_relaxed);
    }
    *cus = c;
    return hipSuccess;
}
}  // namespace rth

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int check_hip(hipError_t e, const char* where) {
    if (e != hipSuccess) {
        return fail(RTH_ERR_HIP, std::string(where) + ": " + hipGetErrorString(e));
    }
    g_last_error.clear();
    return RTH_OK;
}

#define RTH_REQUIRE(cond, msg)                        \
    do {                                              \
        if (!(cond)) {                                \
            return fail(RTH_ERR_INVALID_ARG, (msg));  \
        }                                             \
    } while (0)

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

int check_heads(int num_q_heads, int num_kv_heads) {
    RTH_REQUIRE(num_q_heads >= 1, "num_q_heads must be >= 1");
    RTH_REQUIRE(num_kv_heads >= 1, "num_kv_heads must be >= 1");
    RTH_REQUIRE(num_q_heads % num_kv_heads == 0,
                "num_q_heads must be divisible by num_kv_heads");
    return RTH_OK;
}

int check_quant(const void* q, const void* scale, const void* x, const int* at_pos,
                int rows_per_pos, int num_rows, int head_dim) {
    RTH_REQUIRE(q != nullptr && scale != nullptr && x != nullptr,
                "q, scale and x must not be null");
    RTH_REQUIRE(num_rows >= 1, "num_rows must be >= 1");
    RTH_REQUIRE(at_pos != nullptr, "at_pos must not be null");
    RTH_REQUIRE(rows_per_pos >= 1, "rows_per_pos must be >= 1");
    RTH_REQUIRE(head_dim >= 8, "head_dim must be >= 8");
    RTH_REQUIRE(head_dim % 8 == 0, "head_dim must be divisible by 8");
    RTH_REQUIRE(head_dim <= 16384, "head_dim too large for current dispatch");
    return RTH_OK;
}

int check_attn(const void* out, const void* q, const void* k, const void* v,
               const void* ks, const void* vs, const int* cache_len) {
    RTH_REQUIRE(out != nullptr && q != nullptr, "out and q must not be null");
    RTH_REQUIRE(k != nullptr && v != nullptr && ks != nullptr && vs != nullptr,
                "k, v, k_scale and v_scale must not be null");
    RTH_REQUIRE(cache_len != nullptr, "cache_len must not be null");
    return RTH_OK;
}

// Paged caches: block_size a power of two >= 32 (a decode tile of 32 keys
// never straddles a block); returns the block shift or -1.
int block_shift_of(int block_size) {
    if (block_size < 32 || (block_size & (block_size - 1)) != 0) {
        return -1;
    }
    int sh = 0;
    while ((1 << sh) < block_size) {
        ++sh;
    }
    return sh;
}

// Process-wide decode kernel choice (rth_set_decode_kernel): 0 = the MFMA
// split kernel wherever it supports the shape, RTH_DECODE_VALU = the VALU
// split kernel for every non-paged decode call.
std::atomic<int> g_decode_override{0};

bool use_mfma_decode(int num_q_heads, int num_kv_heads, int head_dim) {
    return g_decode_override.load(std::memory_order_relaxed) != RTH_DECODE_VALU &&
           rth::decode_mfma_supported(num_q_heads, num_kv_heads, head_dim);
}

#define RTH_PAGED_ARGS(bt, bs, shift)                                              \
    RTH_REQUIRE((bt) != nullptr, "block_table must not be null");                  \
    const int shift = block_shift_of(bs);                                          \
    RTH_REQUIRE(shift >= 0, "block_size must be a power of two >= 32")

int prefill_split_common(uint16_t* out, const uint16_t* q, const uint8_t* k, const uint8_t* v,
                         const float* k_scale, const float* v_scale, const int* block_table,
                         int shift, float* partial, int num_splits, int n_new,
                         const int* cache_len, int num_q_heads, int num_kv_heads,
                         int head_dim, float scale, void* stream, const char* what) {
    if (int rc = check_attn(out, q, k, v, k_scale, v_scale, cache_len)) {
        return rc;
    }
    RTH_REQUIRE(partial != nullptr, "partial must not be null");
    RTH_REQUIRE(n_new >= 1 && n_new <= rth::kPrefillSplitMaxTokens,
                "n_new must be in [1, " + std::to_string(rth::kPrefillSplitMaxTokens) + "]");
    RTH_REQUIRE(num_splits >= 1 && num_splits <= 65536, "num_splits must be in [1, 65536]");
    if (int rc = check_heads(num_q_heads, num_kv_heads)) {
        return rc;
    }
    // Up to kPrefillSplitDecodeTokens tokens (or at head_dim != 128, which the
    // flash prefill does not serve): the decode split kernel over (token
    // block, kv head) units; beyond, the flash prefill over key runs.
    if (head_dim == 128 && n_new > rth::kPrefillSplitDecodeTokens) {
        return check_hip(rth::flash_prefill_keysplit_launch(
                             out, q, k, v, k_scale, v_scale, partial, num_splits, n_new, cache_len,
                             num_q_heads, num_kv_heads, head_dim, scale, as_stream(stream),
                             block_table, shift),
                         what);
    }
    RTH_REQUIRE(n_new <= rth::kPrefillSplitDecodeMaxTokens,
                "rth_attn_prefill_split: at head_dim != 128, n_new must be <= " +
                    std::to_string(rth::kPrefillSplitDecodeMaxTokens));
    RTH_REQUIRE(rth::decode_mfma_supported(num_q_heads, num_kv_heads, head_dim),
                "rth_attn_prefill_split: head_dim 64/128/256 with q-head groups the MFMA "
                "decode kernel serves (rth_decode_path == RTH_DECODE_MFMA)");
    return check_hip(rth::flash_prefill_split_launch(out, q, k, v, k_scale, v_scale, partial,
                                                     num_splits, n_new, cache_len, num_q_heads,
                                                     num_kv_heads, head_dim, scale,
                                                     as_stream(stream), block_table, shift),
                     what);
}
}  // namespace

extern "C" {

const char* rth_last_error_string(void) { return g_last_error.c_str(); }

int rth_kv_quantize_fp8(uint8_t* q, float* scale, const uint16_t* x,
                        const int* at_pos, int rows_per_pos, int num_rows,
                        int head_dim, void* stream) {
    if (int rc = check_quant(q, scale, x, at_pos, rows_per_pos, num_rows, head_dim)) {
        return rc;
    }
    return check_hip(rth::quantize_kv_fp8_launch(q, scale, x, at_pos, rows_per_pos,
                                                 num_rows, head_dim, as_stream(stream)),
                     "rth_kv_quantize_fp8");
}

int rth_kv_quantize_fp8_scaled(uint8_t* q, const float* scale,
                               const uint16_t* x, const int* at_pos,
                               int rows_per_pos, int num_rows, int head_dim,
                               void* stream) {
    if (int rc = check_quant(q, scale, x, at_pos, rows_per_pos, num_rows, head_dim)) {
        return rc;
    }
    return check_hip(rth::quantize_kv_fp8_scaled_launch(q, scale, x, at_pos, rows_per_pos,
                                                        num_rows, head_dim,
                                                        as_stream(stream)),
                     "rth_kv_quantize_fp8_scaled");
}

int rth_kv_append_fp8(uint8_t* k_cache, uint8_t* v_cache, float* k_scale,
                      float* v_scale, const uint16_t* k, const uint16_t* v,
                      const int* at_pos, int n_new, int num_kv_heads,
                      int head_dim, void* stream) {
    RTH_REQUIRE(n_new >= 1, "KVCache append n_new must be >= 1");
    RTH_REQUIRE(num_kv_heads >= 1, "num_kv_heads must be >= 1");
    RTH_REQUIRE(k_cache != nullptr && v_cache != nullptr && k_scale != nullptr &&
                    v_scale != nullptr && k != nullptr && v != nullptr,
                "cache slabs, scales and inputs must not be null");
    if (int rc = check_quant(k_cache, k_scale, k, at_pos, num_kv_heads,
                             n_new * num_kv_heads, head_dim)) {
        return rc;
    }
    return check_hip(rth::kv_append_fp8_launch(k_cache, v_cache, k_scale, v_scale, k, v,
                                               at_pos, num_kv_heads, n_new * num_kv_heads,
                                               head_dim, as_stream(stream)),
                     "rth_kv_append_fp8");
}

size_t rth_split_scratch_floats(int num_q_heads, int head_dim, int max_splits) {
    if (num_q_heads < 1 || head_dim < 1 || max_splits < 1) {
        return 0;
    }
    return rth::decode_scratch_floats(num_q_heads, head_dim, max_splits);
}

int rth_default_num_splits(int num_kv_heads, int device) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) !=
            hipSuccess ||
        cus < 1) {
        cus = 256;
    }
    if (num_kv_heads < 1) {
        num_kv_heads = 1;
    }
    // Decode runs one wave per (kv head, split) unit and eight of them per
    // compute unit (two per SIMD), so one full wave of units is 8 * CUs.
    int s = (8 * cus + num_kv_heads - 1) / num_kv_heads;
    return s < 1 ? 1 : (s > 1024 ? 1024 : s);
}

int rth_attn_decode_split(uint16_t* out, const uint16_t* q, const uint8_t* k,
                          const uint8_t* v, const float* k_scale,
                          const float* v_scale, float* partial, int num_splits,
                          const int* cache_len, int num_q_heads,
                          int num_kv_heads, int head_dim, float scale,
                          void* stream) {
    if (int rc = check_attn(out, q, k, v, k_scale, v_scale, cache_len)) {
        return rc;
    }
    RTH_REQUIRE(num_splits >= 1 && num_splits <= 65536, "num_splits must be in [1, 65536]");
    if (int rc = check_heads(num_q_heads, num_kv_heads)) {
        return rc;
    }
    RTH_REQUIRE(head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256 ||
                    head_dim == 512,
                "head_dim must be one of 32, 64, 128, 256, 512");
    if (use_mfma_decode(num_q_heads, num_kv_heads, head_dim)) {
        RTH_REQUIRE(partial != nullptr, "partial must not be null");
        return check_hip(rth::flash_decode_launch(out, q, k, v, k_scale, v_scale, partial,
                                                  num_splits, cache_len, num_q_heads,
                                                  num_kv_heads, head_dim, scale,
                                                  as_stream(stream)),
                         "rth_attn_decode_split");
    }
    RTH_REQUIRE(partial != nullptr, "partial must not be null");
    return check_hip(rth::flash_decode_valu_launch(out, q, k, v, k_scale, v_scale, partial,
                                                   num_splits, cache_len, num_q_heads,
                                                   num_kv_heads, head_dim, scale,
                                                   as_stream(stream)),
                     "rth_attn_decode_split");
}

int rth_decode_path(int num_q_heads, int num_kv_heads, int head_dim) {
    if (num_q_heads < 1 || num_kv_heads < 1 || num_q_heads % num_kv_heads != 0) {
        return 0;
    }
    if (head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256 &&
        head_dim != 512) {
        return 0;
    }
    return use_mfma_decode(num_q_heads, num_kv_heads, head_dim) ? RTH_DECODE_MFMA
                                                                : RTH_DECODE_VALU;
}

int rth_set_decode_kernel(int path) {
    RTH_REQUIRE(path == 0 || path == RTH_DECODE_VALU,
                "rth_set_decode_kernel: path must be 0 (automatic) or RTH_DECODE_VALU");
    g_decode_override.store(path, std::memory_order_relaxed);
    g_last_error.clear();
    return RTH_OK;
}

int rth_attn_decode_split_noalloc(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                  const uint8_t* v, const float* k_scale,
                                  const float* v_scale, int num_splits,
                                  const int* cache_len, int num_q_heads, int num_kv_heads,
                                  int head_dim, float scale, void* stream) {
    if (int rc = check_attn(out, q, k, v, k_scale, v_scale, cache_len)) {
        return rc;
    }
    RTH_REQUIRE(num_splits >= 1 && num_splits <= 65536, "num_splits must be in [1, 65536]");
    if (int rc = check_heads(num_q_heads, num_kv_heads)) {
        return rc;
    }
    RTH_REQUIRE(head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256 ||
                    head_dim == 512,
                "head_dim must be one of 32, 64, 128, 256, 512");
    const std::size_t need = rth::decode_scratch_floats(num_q_heads, head_dim, num_splits);
    RTH_REQUIRE(need <= rth::kNoAllocScratchFloats,
                "rth_attn_decode_split_noalloc: num_q_heads * num_splits * (head_dim + 2) = " +
                    std::to_string(need) + " floats exceeds the fixed scratch of " +
                    std::to_string(rth::kNoAllocScratchFloats) + " floats");
    float* partial = nullptr;
    if (int rc = check_hip(rth::noalloc_scratch(&partial), "rth_attn_decode_split_noalloc")) {
        return rc;
    }
    if (!use_mfma_decode(num_q_heads, num_kv_heads, head_dim)) {
        return check_hip(rth::flash_decode_valu_launch(out, q, k, v, k_scale, v_scale, partial,
                                                       num_splits, cache_len, num_q_heads,
                                                       num_kv_heads, head_dim, scale,
                                                       as_stream(stream)),
                         "rth_attn_decode_split_noalloc");
    }
    return check_hip(rth::flash_decode_launch(out, q, k, v, k_scale, v_scale, partial,
                                              num_splits, cache_len, num_q_heads, num_kv_heads,
                                              head_dim, scale, as_stream(stream)),
                     "rth_attn_decode_split_noalloc");
}

int rth_attn_decode_append_split(uint16_t* out, const uint16_t* q, uint8_t* k_cache,
                                 uint8_t* v_cache, float* k_scale, float* v_scale,
                                 const uint16_t* k_new, const uint16_t* v_new,
                                 float* partial, int num_splits, const int* cache_len,
                                 int num_q_heads, int num_kv_heads, int head_dim,
                                 float scale, void* stream) {
    if (int rc = check_attn(out, q, k_cache, v_cache, k_scale, v_scale, cache_len)) {
        return rc;
    }
    RTH_REQUIRE(k_new != nullptr && v_new != nullptr, "k_new and v_new must not be null");
    RTH_REQUIRE(num_splits >= 1 && num_splits <= 65536, "num_splits must be in [1, 65536]");
    if (int rc = check_heads(num_q_heads, num_kv_heads)) {
        return rc;
    }
    RTH_REQUIRE(head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256 ||
                    head_dim == 512,
                "head_dim must be one of 32, 64, 128, 256, 512");
    if (use_mfma_decode(num_q_heads, num_kv_heads, head_dim)) {
        RTH_REQUIRE(partial != nullptr, "partial must not be null");
        return check_hip(rth::flash_decode_launch(out, q, k_cache, v_cache, k_scale, v_scale,
                                                  partial, num_splits, cache_len, num_q_heads,
                                                  num_kv_heads, head_dim, scale,
                                                  as_stream(stream), k_new, v_new, k_cache,
                                                  v_cache, k_scale, v_scale),
                         "rth_attn_decode_append_split");
    }
    // Shapes without the MFMA decode: the append, then the VALU decode.
    RTH_REQUIRE(partial != nullptr, "partial must not be null");
    if (int rc = check_hip(rth::kv_append_fp8_launch(k_cache, v_cache, k_scale, v_scale, k_new,
                                                     v_new, cache_len, num_kv_heads,
                                                     num_kv_heads, head_dim, as_stream(stream)),
                           "rth_attn_decode_append_split")) {
        return rc;
    }
    return check_hip(rth::flash_decode_valu_launch(out, q, k_cache, v_cache, k_scale, v_scale,
                                                   partial, num_splits, cache_len, num_q_heads,
                                                   num_kv_heads, head_dim, scale,
                                                   as_stream(stream)),
                     "rth_attn_decode_append_split");
}

int rth_attn_decode_rope_append_split(uint16_t* out, const uint16_t* q, uint8_t* k_cache,
                                      uint8_t* v_cache, float* k_scale, float* v_scale,
                                      const uint16_t* k_new, const uint16_t* v_new,
                                      const int* positions, const float* inv_freq,
                                      float* partial, int num_splits, const int* cache_len,
                                      int num_q_heads, int num_kv_heads, int head_dim,
                                      float scale, void* stream) {
    return rth_attn_decode_rope_append_split_paged(
        out, q, k_cache, v_cache, k_scale, v_scale, nullptr, 0, k_new, v_new, positions,
        inv_freq, partial, num_splits, cache_len, num_q_heads, num_kv_heads, head_dim, scale,
        stream);
}

int rth_attn_decode_rope_append_split_paged(uint16_t* out, const uint16_t* q, uint8_t* k_cache,
                                            uint8_t* v_cache, float* k_scale, float* v_scale,
                                            const int* block_table, int block_size,
                                            const uint16_t* k_new, const uint16_t* v_new,
                                            const int* positions, const float* inv_freq,
                                            float* partial, int num_splits,
                                            const int* cache_len, int num_q_heads,
                                            int num_kv_heads, int head_dim, float scale,
                                            void* stream) {
    if (int rc = check_attn(out, q, k_cache, v_cache, k_scale, v_scale, cache_len)) {
        return rc;
    }
    int shift = 0;
    if (block_table != nullptr) {
        RTH_PAGED_ARGS(block_table, block_size, paged_shift);
        shift = paged_shift;
    }
    RTH_REQUIRE(k_new != nullptr && v_new != nullptr, "k_new and v_new must not be null");
    RTH_REQUIRE(positions != nullptr && inv_freq != nullptr,
                "positions and inv_freq must not be null");
    RTH_REQUIRE(num_splits >= 1 && num_splits <= 65536, "num_splits must be in [1, 65536]");
    if (int rc = check_heads(num_q_heads, num_kv_heads)) {
        return rc;
    }
    RTH_REQUIRE(rth::decode_mfma_supported(num_q_heads, num_kv_heads, head_dim),
                "the RoPE decode step supports head_dim 64, 128, 256 with GQA groups of up to "
                "g = min(16, 2048 / head_dim) q heads, or groups in equal blocks of 4 to g "
                "(rth_decode_path)");
    RTH_REQUIRE(partial != nullptr, "partial must not be null");
    return check_hip(rth::flash_decode_launch(out, q, k_cache, v_cache, k_scale, v_scale,
                                              partial, num_splits, cache_len, num_q_heads,
                                              num_kv_heads, head_dim, scale, as_stream(stream),
                                              k_new, v_new, k_cache, v_cache, k_scale, v_scale,
                                              block_table, shift, positions, inv_freq),
                     "rth_attn_decode_rope_append_split");
}

int rth_attn_decode_qk_norm_rope_append_split(
    uint16_t* out, const uint16_t* q, uint8_t* k_cache, uint8_t* v_cache, float* k_scale,
    float* v_scale, const uint16_t* k_new, const uint16_t* v_new, const uint16_t* q_norm,
    const uint16_t* k_norm, float eps, const int* positions, const float* inv_freq,
    float* partial, int num_splits, const int* cache_len, int num_q_heads, int num_kv_heads,
    int head_dim, float scale, void* stream) {
    return rth_attn_decode_qk_norm_rope_append_split_paged(
        out, q, k_cache, v_cache, k_scale, v_scale, nullptr, 0, k_new, v_new, q_norm, k_norm,
        eps, positions, inv_freq, partial, num_splits, cache_len, num_q_heads, num_kv_heads,
        head_dim, scale, stream);
}

int rth_attn_decode_qk_norm_rope_append_split_paged(
    uint16_t* out, const uint16_t* q, uint8_t* k_cache, uint8_t* v_cache, float* k_scale,
    float* v_scale, const int* block_table, int block_size, const uint16_t* k_new,
    const uint16_t* v_new, const uint16_t* q_norm, const uint16_t* k_norm, float eps,
    const int* positions, const float* inv_freq, float* partial, int num_splits,
    const int* cache_len, int num_q_heads, int num_kv_heads, int head_dim, float scale,
    void* stream) {
    if (int rc = check_attn(out, q, k_cache, v_cache, k_scale, v_scale, cache_len)) {
        return rc;
    }
    int shift = 0;
    if (block_table != nullptr) {
        RTH_PAGED_ARGS(block_table, block_size, paged_shift);
        shift = paged_shift;
    }
    RTH_REQUIRE(k_new != nullptr && v_new != nullptr, "k_new and v_new must not be null");
    RTH_REQUIRE(q_norm != nullptr && k_norm != nullptr, "q_norm and k_norm must not be null");
    RTH_REQUIRE(positions != nullptr && inv_freq != nullptr,
                "positions and inv_freq must not be null");
    RTH_REQUIRE(num_splits >= 1 && num_splits <= 65536, "num_splits must be in [1, 65536]");
    if (int rc = check_heads(num_q_heads, num_kv_heads)) {
        return rc;
    }
    RTH_REQUIRE(rth::decode_mfma_supported(num_q_heads, num_kv_heads, head_dim),
                "the q/k-norm RoPE decode step supports head_dim 64, 128, 256 with GQA groups "
                "of up to g = min(16, 2048 / head_dim) q heads, or groups in equal blocks of 4 "
                "to g (rth_decode_path)");
    RTH_REQUIRE(partial != nullptr, "partial must not be null");
    return check_hip(rth::flash_decode_launch(out, q, k_cache, v_cache, k_scale, v_scale,
                                              partial, num_splits, cache_len, num_q_heads,
                                              num_kv_heads, head_dim, scale, as_stream(stream),
                                              k_new, v_new, k_cache, v_cache, k_scale, v_scale,
                                              block_table, shift, positions, inv_freq, q_norm,
                                              k_norm, eps),
                     "rth_attn_decode_qk_norm_rope_append_split");
}

int rth_kv_append_fp8_paged(uint8_t* k_cache, uint8_t* v_cache, float* k_scale,
                            float* v_scale, const uint16_t* k, const uint16_t* v,
                            const int* at_pos, int n_new, int num_kv_heads, int head_dim,
                            const int* block_table, int block_size, void* stream) {
    RTH_REQUIRE(n_new >= 1, "KVCache append n_new must be >= 1");
    RTH_REQUIRE(num_kv_heads >= 1, "num_kv_heads must be >= 1");
    RTH_REQUIRE(k_cache != nullptr && v_cache != nullptr && k_scale != nullptr &&
                    v_scale != nullptr && k != nullptr && v != nullptr,
                "cache slabs, scales and inputs must not be null");
    RTH_PAGED_ARGS(block_table, block_size, shift);
    if (int rc = check_quant(k_cache, k_scale, k, at_pos, num_kv_heads,
                             n_new * num_kv_heads, head_dim)) {
        return rc;
    }
    return check_hip(rth::kv_append_fp8_launch(k_cache, v_cache, k_scale, v_scale, k, v,
                                               at_pos, num_kv_heads, n_new * num_kv_heads,
                                               head_dim, as_stream(stream), block_table, shift),
                     "rth_kv_append_fp8_paged");
}

int rth_attn_decode_split_paged(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                const uint8_t* v, const float* k_scale, const float* v_scale,
                                const int* block_table, int block_size, float* partial,
                                int num_splits, const int* cache_len, int num_q_heads,
                                int num_kv_heads, int head_dim, float scale, void* stream) {
    if (int rc = check_attn(out, q, k, v, k_scale, v_scale, cache_len)) {
        return rc;
    }
    RTH_PAGED_ARGS(block_table, block_size, shift);
    RTH_REQUIRE(num_splits >= 1 && num_splits <= 65536, "num_splits must be in [1, 65536]");
    if (int rc = check_heads(num_q_heads, num_kv_heads)) {
        return rc;
    }
    RTH_REQUIRE(rth::decode_mfma_supported(num_q_heads, num_kv_heads, head_dim),
                "paged decode supports head_dim 64, 128, 256 with GQA groups of up to g = "
                "min(16, 2048 / head_dim) q heads, or groups in equal blocks of 4 to g "
                "(rth_decode_path)");
    RTH_REQUIRE(partial != nullptr, "partial must not be null");
    return check_hip(rth::flash_decode_launch(out, q, k, v, k_scale, v_scale, partial,
                                              num_splits, cache_len, num_q_heads, num_kv_heads,
                                              head_dim, scale, as_stream(stream), nullptr,
                                              nullptr, nullptr, nullptr, nullptr, nullptr,
                                              block_table, shift),
                     "rth_attn_decode_split_paged");
}

int rth_attn_decode_append_split_paged(uint16_t* out, const uint16_t* q, uint8_t* k_cache,
                                       uint8_t* v_cache, float* k_scale, float* v_scale,
                                       const int* block_table, int block_size,
                                       const uint16_t* k_new, const uint16_t* v_new,
                                       float* partial, int num_splits, const int* cache_len,
                                       int num_q_heads, int num_kv_heads, int head_dim,
                                       float scale, void* stream) {
    if (int rc = check_attn(out, q, k_cache, v_cache, k_scale, v_scale, cache_len)) {
        return rc;
    }
    RTH_PAGED_ARGS(block_table, block_size, shift);
    RTH_REQUIRE(k_new != nullptr && v_new != nullptr, "k_new and v_new must not be null");
    RTH_REQUIRE(num_splits >= 1 && num_splits <= 65536, "num_splits must be in [1, 65536]");
    if (int rc = check_heads(num_q_heads, num_kv_heads)) {
        return rc;
    }
    RTH_REQUIRE(rth::decode_mfma_supported(num_q_heads, num_kv_heads, head_dim),
                "paged decode supports head_dim 64, 128, 256 with GQA groups of up to g = "
                "min(16, 2048 / head_dim) q heads, or groups in equal blocks of 4 to g "
                "(rth_decode_path)");
    RTH_REQUIRE(partial != nullptr, "partial must not be null");
    return check_hip(rth::flash_decode_launch(out, q, k_cache, v_cache, k_scale, v_scale,
                                              partial, num_splits, cache_len, num_q_heads,
                                              num_kv_heads, head_dim, scale, as_stream(stream),
                                              k_new, v_new, k_cache, v_cache, k_scale, v_scale,
                                              block_table, shift),
                     "rth_attn_decode_append_split_paged");
}

int rth_attn_prefill_paged(uint16_t* out, const uint16_t* q, const uint8_t* k,
                           const uint8_t* v, const float* k_scale, const float* v_scale,
                           const int* block_table, int block_size, int n_new,
                           const int* cache_len, int num_q_heads, int num_kv_heads,
                           int head_dim, float scale, void* stream) {
    if (int rc = check_attn(out, q, k, v, k_scale, v_scale, cache_len)) {
        return rc;
    }
    RTH_PAGED_ARGS(block_table, block_size, shift);
    RTH_REQUIRE(head_dim == 128, "flash_prefill_bf16 supports head_dim 128 only");
    RTH_REQUIRE(n_new >= 1, "n_new must be >= 1");
    if (int rc = check_heads(num_q_heads, num_kv_heads)) {
        return rc;
    }
    return check_hip(rth::flash_prefill_launch(out, q, k, v, k_scale, v_scale, n_new, cache_len,
                                               num_q_heads, num_kv_heads, head_dim, scale,
                                               as_stream(stream), block_table, shift),
                     "rth_attn_prefill_paged");
}

int rth_attn_prefill(uint16_t* out, const uint16_t* q, const uint8_t* k,
                     const uint8_t* v, const float* k_scale,
                     const float* v_scale, int n_new, const int* cache_len,
                     int num_q_heads, int num_kv_heads, int head_dim,
                     float scale, void* stream) {
    if (int rc = check_attn(out, q, k, v, k_scale, v_scale, cache_len)) {
        return rc;
    }
    RTH_REQUIRE(head_dim == 128, "flash_prefill_bf16 supports head_dim 128 only");
    RTH_REQUIRE(n_new >= 1, "n_new must be >= 1");
    if (int rc = check_heads(num_q_heads, num_kv_heads)) {
        return rc;
    }
    return check_hip(rth::flash_prefill_launch(out, q, k, v, k_scale, v_scale, n_new,
                                               cache_len, num_q_heads, num_kv_heads,
                                               head_dim, scale, as_stream(stream)),
                     "rth_attn_prefill");
}

int rth_attn_prefill_split(uint16_t* out, const uint16_t* q, const uint8_t* k,
                           const uint8_t* v, const float* k_scale, const float* v_scale,
                           float* partial, int num_splits, int n_new, const int* cache_len,
                           int num_q_heads, int num_kv_heads, int head_dim, float scale,
                           void* stream) {
    return prefill_split_common(out, q, k, v, k_scale, v_scale, nullptr, 0, partial,
                                num_splits, n_new, cache_len, num_q_heads, num_kv_heads,
                                head_dim, scale, stream, "rth_attn_prefill_split");
}

int rth_attn_prefill_split_paged(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                 const uint8_t* v, const float* k_scale,
                                 const float* v_scale, const int* block_table,
                                 int block_size, float* partial, int num_splits, int n_new,
                                 const int* cache_len, int num_q_heads, int num_kv_heads,
                                 int head_dim, float scale, void* stream) {
    RTH_PAGED_ARGS(block_table, block_size, shift);
    return prefill_split_common(out, q, k, v, k_scale, v_scale, block_table, shift, partial,
                                num_splits, n_new, cache_len, num_q_heads, num_kv_heads,
                                head_dim, scale, stream, "rth_attn_prefill_split_paged");
}

int rth_attn_naive(uint16_t* out, const uint16_t* q, const uint8_t* k,
                   const uint8_t* v, const float* k_scale, const float* v_scale,
                   int n_new, const int* cache_len, int num_q_heads,
                   int num_kv_heads, int head_dim, float scale, void* stream) {
    if (int rc = check_attn(out, q, k, v, k_scale, v_scale, cache_len)) {
        return rc;
    }
    RTH_REQUIRE(n_new >= 1, "n_new must be >= 1");
    if (int rc = check_heads(num_q_heads, num_kv_heads)) {
        return rc;
    }
    RTH_REQUIRE(head_dim >= 1, "head_dim must be >= 1");
    RTH_REQUIRE(head_dim <= 512, "head_dim exceeds the naive kernel's maximum (512)");
    return check_hip(rth::attention_naive_launch(out, q, k, v, k_scale, v_scale, n_new,
                                                 cache_len, num_q_heads, num_kv_heads,
                                                 head_dim, scale, as_stream(stream)),
                     "rth_attn_naive");
}

int rth_rope_bf16(uint16_t* q, uint16_t* k, const int* positions, const float* inv_freq,
                  int seq_len, int num_q_heads, int num_kv_heads, int head_dim,
                  void* stream) {
    // Checks of rope_bf16 (reference src/kernels/rope.cu:68-73).
    RTH_REQUIRE(q != nullptr && k != nullptr, "q and k must not be null");
    RTH_REQUIRE(positions != nullptr && inv_freq != nullptr,
                "positions and inv_freq must not be null");
    RTH_REQUIRE(seq_len >= 1, "seq_len must be >= 1");
    RTH_REQUIRE(num_q_heads >= 1, "num_q_heads must be >= 1");
    RTH_REQUIRE(num_kv_heads >= 1, "num_kv_heads must be >= 1");
    RTH_REQUIRE(head_dim >= 2, "head_dim must be >= 2");
    RTH_REQUIRE(head_dim % 2 == 0, "head_dim must be even");
    RTH_REQUIRE(head_dim <= 256, "head_dim exceeds kMaxHeadDim (256)");
    return check_hip(rth::rope_bf16_launch(q, k, positions, inv_freq, seq_len, num_q_heads,
                                           num_kv_heads, head_dim, as_stream(stream)),
                     "rth_rope_bf16");
}

int rth_rope_append_fp8(uint16_t* q, uint8_t* k_cache, uint8_t* v_cache, float* k_scale,
                        float* v_scale, const uint16_t* k, const uint16_t* v,
                        const int* positions, const float* inv_freq, const int* at_pos,
                        int n_new, int num_q_heads, int num_kv_heads, int head_dim,
                        void* stream) {
    RTH_REQUIRE(q != nullptr && k != nullptr && v != nullptr, "q, k and v must not be null");
    RTH_REQUIRE(k_cache != nullptr && v_cache != nullptr && k_scale != nullptr &&
                    v_scale != nullptr,
                "cache slabs and scales must not be null");
    RTH_REQUIRE(positions != nullptr && inv_freq != nullptr && at_pos != nullptr,
                "positions, inv_freq and at_pos must not be null");
    RTH_REQUIRE(n_new >= 1, "n_new must be >= 1");
    RTH_REQUIRE(num_q_heads >= 1, "num_q_heads must be >= 1");
    RTH_REQUIRE(num_kv_heads >= 1, "num_kv_heads must be >= 1");
    RTH_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
                "head_dim must be one of 64, 128, 256");
    return check_hip(rth::rope_append_fp8_launch(q, k_cache, v_cache, k_scale, v_scale, k, v,
                                                 nullptr, nullptr, 0.0f, positions, inv_freq,
                                                 at_pos, n_new, num_q_heads, num_kv_heads,
                                                 head_dim, as_stream(stream)),
                     "rth_rope_append_fp8");
}

int rth_qk_norm_rope_append_fp8(uint16_t* q, uint8_t* k_cache, uint8_t* v_cache,
                                float* k_scale, float* v_scale, const uint16_t* k,
                                const uint16_t* v, const uint16_t* q_norm,
                                const uint16_t* k_norm, float eps, const int* positions,
                                const float* inv_freq, const int* at_pos, int n_new,
                                int num_q_heads, int num_kv_heads, int head_dim,
                                void* stream) {
    RTH_REQUIRE(q != nullptr && k != nullptr && v != nullptr, "q, k and v must not be null");
    RTH_REQUIRE(k_cache != nullptr && v_cache != nullptr && k_scale != nullptr &&
                    v_scale != nullptr,
                "cache slabs and scales must not be null");
    RTH_REQUIRE(q_norm != nullptr && k_norm != nullptr, "q_norm and k_norm must not be null");
    RTH_REQUIRE(eps > 0.0f, "eps must be > 0");
    RTH_REQUIRE(positions != nullptr && inv_freq != nullptr && at_pos != nullptr,
                "positions, inv_freq and at_pos must not be null");
    RTH_REQUIRE(n_new >= 1, "n_new must be >= 1");
    RTH_REQUIRE(num_q_heads >= 1, "num_q_heads must be >= 1");
    RTH_REQUIRE(num_kv_heads >= 1, "num_kv_heads must be >= 1");
    RTH_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
                "head_dim must be one of 64, 128, 256");
    return check_hip(rth::rope_append_fp8_launch(q, k_cache, v_cache, k_scale, v_scale, k, v,
                                                 q_norm, k_norm, eps, positions, inv_freq,
                                                 at_pos, n_new, num_q_heads, num_kv_heads,
                                                 head_dim, as_stream(stream)),
                     "rth_qk_norm_rope_append_fp8");
}

int rth_rmsnorm_bf16(uint16_t* y, const uint16_t* x, const uint16_t* g, int num_tokens,
                     int hidden_dim, float eps, void* stream) {
    // Checks of rmsnorm_bf16_forward (reference src/kernels/rmsnorm.cu:172-176).
    RTH_REQUIRE(y != nullptr && x != nullptr && g != nullptr, "y, x and g must not be null");
    RTH_REQUIRE(num_tokens >= 1, "num_tokens must be >= 1");
    RTH_REQUIRE(hidden_dim >= 8, "hidden_dim must be >= 8");
    RTH_REQUIRE(hidden_dim % 8 == 0,
                "hidden_dim must be divisible by 8 for BF16 vectorized load");
    RTH_REQUIRE(hidden_dim <= 16384, "hidden_dim too large for current dispatch");
    RTH_REQUIRE(eps > 0.0f, "eps must be > 0");
    return check_hip(rth::rmsnorm_bf16_launch(y, x, g, num_tokens, hidden_dim, eps,
                                              as_stream(stream)),
                     "rth_rmsnorm_bf16");
}

int rth_rmsnorm_lanes(int hidden_dim) {
    return (hidden_dim >= 8 && hidden_dim % 8 == 0) ? rth::rmsnorm_lanes(hidden_dim) : 0;
}

int rth_advance_position(int* pos, int delta, void* stream) {
    RTH_REQUIRE(pos != nullptr, "pos must not be null");
    return check_hip(rth::advance_position_launch(pos, delta, as_stream(stream)),
                     "rth_advance_position");
}

}  // extern "C"
