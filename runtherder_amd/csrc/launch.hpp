// Internal launch functions behind the C ABI (capi.cpp). Each validates
// nothing: argument checks live in the C ABI layer, these only pick a kernel
// specialisation and enqueue it on `stream`.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace rth {

// Compute units of the current device, queried once per device and cached;
// returns the query's error (and leaves *cus unchanged) if it fails.
hipError_t device_cu_count(int* cus);

hipError_t quantize_kv_fp8_launch(uint8_t* q, float* scale, const uint16_t* x,
                                  const int* at_pos, int rows_per_pos,
                                  int num_rows, int head_dim, hipStream_t stream);

hipError_t quantize_kv_fp8_scaled_launch(uint8_t* q, const float* scale,
                                         const uint16_t* x, const int* at_pos,
                                         int rows_per_pos, int num_rows,
                                         int head_dim, hipStream_t stream);

// block_table != nullptr: paged cache (see flash_prefill_launch).
hipError_t kv_append_fp8_launch(uint8_t* k_q, uint8_t* v_q, float* k_scale,
                                float* v_scale, const uint16_t* k,
                                const uint16_t* v, const int* at_pos,
                                int rows_per_pos, int num_rows, int head_dim,
                                hipStream_t stream, const int* block_table = nullptr,
                                int block_shift = 0);

// Split-K decode scratch in floats: [Hq, S] m, [Hq, S] l, [Hq, S, D] acc.
std::size_t decode_scratch_floats(int num_q_heads, int head_dim, int max_splits);

// Floats of the fixed per-device decode scratch (16 MiB) used by the
// allocation-free decode entry point.
constexpr std::size_t kNoAllocScratchFloats = std::size_t{1} << 22;

// Device address of the current device's fixed decode scratch, looked up
// with hipGetSymbolAddress on the first call per device.
hipError_t noalloc_scratch(float** ptr);

// k_new != nullptr: also append one token (k_new, v_new [Hkv, D] bf16) at row
// *cache_len of the cache (k_w, v_w, ks_w, vs_w: the same slabs as k, v,
// k_scale, v_scale) before attending over *cache_len + 1 keys.
hipError_t flash_decode_launch(uint16_t* out, const uint16_t* q,
                               const uint8_t* k, const uint8_t* v,
                               const float* k_scale, const float* v_scale,
                               float* partial, int num_splits,
                               const int* cache_len, int num_q_heads,
                               int num_kv_heads, int head_dim, float scale,
                               hipStream_t stream, const uint16_t* k_new = nullptr,
                               const uint16_t* v_new = nullptr, uint8_t* k_w = nullptr,
                               uint8_t* v_w = nullptr, float* ks_w = nullptr,
                               float* vs_w = nullptr, const int* block_table = nullptr,
                               int block_shift = 0, const int* positions = nullptr,
                               const float* inv_freq = nullptr,
                               const uint16_t* q_norm = nullptr,
                               const uint16_t* k_norm = nullptr, float eps = 0.0f);

// A causal prefill call of n_new tokens after *cache_len cached keys (their
// K/V already in the cache) as split-K decode over n_new x Hkv virtual kv
// heads: the shapes decode_mfma_supported accepts; partial holds
// decode_scratch_floats(n_new * Hq, D, num_splits) floats.
constexpr int kPrefillSplitMaxTokens       = 4096;   // rth_attn_prefill_split
constexpr int kPrefillSplitDecodeTokens    = 80;     // above: the flash prefill over key runs
constexpr int kPrefillSplitDecodeMaxTokens = 256;    // the decode kernel's route at D != 128
hipError_t flash_prefill_split_launch(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                     const uint8_t* v, const float* k_scale,
                                     const float* v_scale, float* partial, int num_splits,
                                     int n_new, const int* cache_len, int num_q_heads,
                                     int num_kv_heads, int head_dim, float scale,
                                     hipStream_t stream, const int* block_table = nullptr,
                                     int block_shift = 0);

// The decode merge over `rows` rows of num_splits partials each (whole-row
// workgroups): out row r = the merged row r; the live slots follow from
// *cache_len + n_tok keys as in the split kernels, or (run_min > 0) as the
// flash prefill's key runs of max(ceil(tiles / S), run_min) 64-key tiles.
hipError_t split_rows_merge_launch(uint16_t* out, const float* partial, int num_splits,
                                  const int* cache_len, int rows, int n_tok, int head_dim,
                                  hipStream_t stream, int run_min = 0);

// The flash prefill (head_dim 128) with its keys split over num_splits
// workgroups per (128-row block, q head), partials in the split-K decode
// layout (decode_scratch_floats(n_new * Hq, 128, num_splits) floats), then
// split_rows_merge_launch.
hipError_t flash_prefill_keysplit_launch(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                         const uint8_t* v, const float* k_scale,
                                         const float* v_scale, float* partial, int num_splits,
                                         int n_new, const int* cache_len, int num_q_heads,
                                         int num_kv_heads, int head_dim, float scale,
                                         hipStream_t stream, const int* block_table = nullptr,
                                         int block_shift = 0);

// The VALU split kernel + merge: head_dim in {32, 64, 128, 256, 512}, any
// GQA group (no paging, no fused append). The decode entry points use it for
// the shapes decode_mfma_supported rejects.
hipError_t flash_decode_valu_launch(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                   const uint8_t* v, const float* k_scale,
                                   const float* v_scale, float* partial, int num_splits,
                                   const int* cache_len, int num_q_heads, int num_kv_heads,
                                   int head_dim, float scale, hipStream_t stream);

// block_table != nullptr: paged cache, logical block b (2^block_shift keys)
// stored at physical block block_table[b] (same for the decode launch).
hipError_t flash_prefill_launch(uint16_t* out, const uint16_t* q,
                                const uint8_t* k, const uint8_t* v,
                                const float* k_scale, const float* v_scale,
                                int n_new, const int* cache_len,
                                int num_q_heads, int num_kv_heads,
                                int head_dim, float scale, hipStream_t stream,
                                const int* block_table = nullptr, int block_shift = 0);

hipError_t attention_naive_launch(uint16_t* out, const uint16_t* q,
                                  const uint8_t* k, const uint8_t* v,
                                  const float* k_scale, const float* v_scale,
                                  int n_new, const int* cache_len,
                                  int num_q_heads, int num_kv_heads,
                                  int head_dim, float scale, hipStream_t stream);

hipError_t advance_position_launch(int* pos, int delta, hipStream_t stream);

hipError_t rope_bf16_launch(uint16_t* q, uint16_t* k, const int* positions,
                            const float* inv_freq, int seq_len, int num_q_heads,
                            int num_kv_heads, int head_dim, hipStream_t stream);

// q_norm == nullptr: RoPE + append; otherwise per-head RMSNorm of q and k
// (gains q_norm, k_norm [head_dim]) before the RoPE.
hipError_t rope_append_fp8_launch(uint16_t* q, uint8_t* k_cache, uint8_t* v_cache,
                                  float* k_scale, float* v_scale, const uint16_t* k,
                                  const uint16_t* v, const uint16_t* q_norm,
                                  const uint16_t* k_norm, float eps, const int* positions,
                                  const float* inv_freq, const int* at_pos, int n_new,
                                  int num_q_heads, int num_kv_heads, int head_dim,
                                  hipStream_t stream);

int rmsnorm_lanes(int dim);

hipError_t rmsnorm_bf16_launch(uint16_t* y, const uint16_t* x, const uint16_t* g, int rows,
                               int dim, float eps, hipStream_t stream);

}  // namespace rth
