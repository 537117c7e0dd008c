/*
 * C ABI of the MI355X attention hot path (libruntherder_attn.so).
 *
 * Every entry point takes plain device pointers, host int sizes and a HIP
 * stream passed as void* (NULL = the null stream), enqueues its work
 * asynchronously, never synchronizes and never allocates, so calls are
 * HIP-graph capturable. Return value: RTH_OK, or an error code with a message
 * available from rth_last_error_string() (thread-local).
 *
 * Element types at the boundary:
 *   bf16  -> uint16_t (raw bfloat16 bits)
 *   E4M3  -> uint8_t  (OCP FP8 E4M3FN: bias 7, max 448, 0x7F/0xFF NaN)
 *
 * Layouts follow the reference engine (reference paths):
 *   q, out   [n_new, num_q_heads, head_dim] bf16           (backend.h:31-41)
 *   k, v     [max_seq_len, num_kv_heads, head_dim] E4M3   (kv_view.h:7-13)
 *   k_scale, v_scale [max_seq_len, num_kv_heads] fp32, one dequant scale per
 *            (token, kv_head); value = float(code) * scale  (kv_view.h:7-13)
 *   cache_len / at_pos are DEVICE-resident ints, unchecked against the cache
 *   size (the caller owns that bound), as in the reference.
 */
#ifndef RTH_ATTN_H
#define RTH_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    RTH_OK              = 0,
    RTH_ERR_INVALID_ARG = 1, /* argument check failed (message says which) */
    RTH_ERR_HIP         = 2, /* HIP runtime / launch error */
};

/* Message of the last failing call on this thread ("" if none). */
const char* rth_last_error_string(void);

/* Replaces kernels::quantize_kv_fp8 (reference
 * include/runtherder/kernels/quantization.cuh:50-57). Per row of head_dim bf16:
 * scale = amax/448, q = E4M3_satfinite(x * (448/amax)); row r is written at
 * destination row r + (*at_pos) * rows_per_pos. head_dim % 8 == 0,
 * 8 <= head_dim <= 16384. Bit-exact with the reference's arithmetic. */
int rth_kv_quantize_fp8(uint8_t* q, float* scale, const uint16_t* x,
                        const int* at_pos, int rows_per_pos, int num_rows,
                        int head_dim, void* stream);

/* Given-scale variant (no reference counterpart): scale[dst] is an input and
 * q = E4M3_satfinite(x * (1/scale[dst])). Used to fill caches whose scales are
 * set by the caller (e.g. per-head calibration). Same constraints. */
int rth_kv_quantize_fp8_scaled(uint8_t* q, const float* scale,
                               const uint16_t* x, const int* at_pos,
                               int rows_per_pos, int num_rows, int head_dim,
                               void* stream);

/* Replaces the two quantize_kv_fp8 launches of engine::KVCache::append
 * (reference include/runtherder/engine/kv_cache.h:62-78) with one launch:
 * quantizes k and v ([n_new, num_kv_heads, head_dim] bf16) into one layer's
 * slabs at rows *at_pos .. *at_pos + n_new - 1. */
int rth_kv_append_fp8(uint8_t* k_cache, uint8_t* v_cache, float* k_scale,
                      float* v_scale, const uint16_t* k, const uint16_t* v,
                      const int* at_pos, int n_new, int num_kv_heads,
                      int head_dim, void* stream);

/* Replaces kernels::flash_split_scratch_floats (reference
 * include/runtherder/kernels/flash_decode.cuh:16-24): floats of decode
 * scratch for max_splits splits, Hq*S*2 + Hq*S*D, laid out as [Hq*S] m,
 * [Hq*S] l, [Hq*S*D] acc like the reference's. No initialization needed. */
size_t rth_split_scratch_floats(int num_q_heads, int head_dim, int max_splits);

/* Split count AdaptiveAttention uses on `device` for num_kv_heads kv heads:
 * the decode kernel runs one wave per (kv head, split) unit, eight per
 * compute unit, so this is 8 * CUs / num_kv_heads (256 for 8 kv heads on
 * MI355X), capped at 1024. */
int rth_default_num_splits(int num_kv_heads, int device);

/* Replaces kernels::flash_decode_split_bf16 (reference
 * include/runtherder/kernels/flash_decode.cuh:45-59): one query token,
 * attends *cache_len + 1 keys, split-K over num_splits key ranges with a
 * log-sum-exp merge (two kernels: splits, then merge). `partial` is
 * caller-owned scratch of rth_split_scratch_floats(Hq, D, num_splits) floats.
 * head_dim in {32,64,128,256,512}; 64/128/256 run the MFMA split kernel when
 * the group of G = Hq/Hkv q heads splits into equal blocks of 4..16 heads
 * (G itself when G <= 16) with block * head_dim <= 2048, the rest the VALU
 * split kernel (rth_decode_path). */
int rth_attn_decode_split(uint16_t* out, const uint16_t* q, const uint8_t* k,
                          const uint8_t* v, const float* k_scale,
                          const float* v_scale, float* partial, int num_splits,
                          const int* cache_len, int num_q_heads,
                          int num_kv_heads, int head_dim, float scale,
                          void* stream);

enum {
    RTH_DECODE_MFMA = 1, /* bf16 MFMA split kernel */
    RTH_DECODE_VALU = 2, /* VALU split kernel (DPP / shuffle reductions) */
};

/* No counterpart in the reference: which split kernel rth_attn_decode_split,
 * rth_attn_decode_split_noalloc and rth_attn_decode_append_split run for this
 * shape (RTH_DECODE_MFMA or RTH_DECODE_VALU), 0 if the shape is not
 * supported; it follows rth_set_decode_kernel. The paged, RoPE and q/k-norm
 * entries always run the MFMA kernel and accept the shapes this reports as
 * RTH_DECODE_MFMA under the automatic choice (path 0), whatever the switch. */
int rth_decode_path(int num_q_heads, int num_kv_heads, int head_dim);

/* No counterpart in the reference: process-wide choice of the split kernel
 * for rth_attn_decode_split, rth_attn_decode_split_noalloc and
 * rth_attn_decode_append_split, for measurement and tuning (the paged, RoPE
 * and q/k-norm entries ignore it). path 0 (the
 * default) = the MFMA kernel wherever it supports the shape, the VALU kernel
 * elsewhere; RTH_DECODE_VALU = the VALU kernel for every shape. Results of
 * the two kernels agree within the attention tolerance, not bit for bit.
 * Not synchronized with calls in flight on other host threads. */
int rth_set_decode_kernel(int path);

/* No counterpart in the reference: rth_attn_decode_split without the
 * `partial` argument, for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). It calls no
 * hipMalloc/hipFree and no allocating library routine: the split partials
 * live in a fixed 16 MiB device array (2^22 floats) that each GPU holds from
 * the library's load until the process ends. Rejects shapes with
 * num_q_heads * num_splits * (head_dim + 2) > 2^22 floats
 * (RTH_ERR_INVALID_ARG). Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (several streams or host threads) race and
 * must be serialized by the caller. Output is bit-identical to
 * rth_attn_decode_split with the same arguments. */
int rth_attn_decode_split_noalloc(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                  const uint8_t* v, const float* k_scale,
                                  const float* v_scale, int num_splits,
                                  const int* cache_len, int num_q_heads, int num_kv_heads,
                                  int head_dim, float scale, void* stream);

/* No counterpart in the reference: KVCache::append(layer, k_new, v_new, 1,
 * cache_len) followed by the decode call (reference
 * src/model/supported/llama/llama3.cu:232-234 with n_new == 1) in one call
 * of two kernels instead of three. The new token ([Hkv, D] bf16) is
 * quantized into row *cache_len of the layer's cache slabs (bytes identical
 * to rth_kv_append_fp8) and attended with the *cache_len earlier keys;
 * output equals rth_kv_append_fp8 + rth_attn_decode_split. Same shapes and
 * scratch as rth_attn_decode_split. */
int rth_attn_decode_append_split(uint16_t* out, const uint16_t* q, uint8_t* k_cache,
                                 uint8_t* v_cache, float* k_scale, float* v_scale,
                                 const uint16_t* k_new, const uint16_t* v_new,
                                 float* partial, int num_splits, const int* cache_len,
                                 int num_q_heads, int num_kv_heads, int head_dim,
                                 float scale, void* stream);

/* Replaces kernels::flash_prefill_bf16 (reference
 * include/runtherder/kernels/flash_prefill.cuh:26-39): causal attention of
 * n_new queries at positions *cache_len .. *cache_len + n_new - 1 over keys
 * 0 .. *cache_len + n_new - 1. head_dim == 128. */
int rth_attn_prefill(uint16_t* out, const uint16_t* q, const uint8_t* k,
                     const uint8_t* v, const float* k_scale,
                     const float* v_scale, int n_new, const int* cache_len,
                     int num_q_heads, int num_kv_heads, int head_dim,
                     float scale, void* stream);

/* No counterpart in the reference: the causal attention of rth_attn_prefill
 * split over the keys, for calls after a long cache (speculative-decoding
 * verification, prefill chunks), instead of one workgroup per q tile
 * streaming every key (reference flash_prefill.cu:34-241 walks all keys
 * serially per tile: n_new = 4 at 32K keys costs ~50x a decode step).
 * n_new <= 80, or head_dim != 128: the decode split kernel over (block of
 * tokens, kv head) units, token t over the first *cache_len + t + 1 keys
 * (shapes of the MFMA decode kernel, rth_decode_path == RTH_DECODE_MFMA:
 * head_dim 64 / 128 / 256; n_new <= 256). n_new > 80 at head_dim 128: the
 * flash prefill with each (row block, q head) split over num_splits runs of
 * key tiles. Both end in the decode merge. n_new's K/V must already be in the
 * cache (as for rth_attn_prefill). partial: rth_split_scratch_floats(n_new *
 * num_q_heads, head_dim, num_splits) floats, no initialization needed;
 * 1 <= n_new <= 4096. Results match rth_attn_prefill within the attention
 * tolerance (a different summation order). */
int rth_attn_prefill_split(uint16_t* out, const uint16_t* q, const uint8_t* k,
                           const uint8_t* v, const float* k_scale, const float* v_scale,
                           float* partial, int num_splits, int n_new, const int* cache_len,
                           int num_q_heads, int num_kv_heads, int head_dim, float scale,
                           void* stream);
int rth_attn_prefill_split_paged(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                 const uint8_t* v, const float* k_scale,
                                 const float* v_scale, const int* block_table,
                                 int block_size, float* partial, int num_splits, int n_new,
                                 const int* cache_len, int num_q_heads, int num_kv_heads,
                                 int head_dim, float scale, void* stream);

/* Replaces kernels::attention_causal_bf16 (reference
 * include/runtherder/kernels/attention.cuh:21-34): the same causal attention
 * as rth_attn_prefill at any n_new, by the plain two-pass algorithm.
 * head_dim <= 512. */
int rth_attn_naive(uint16_t* out, const uint16_t* q, const uint8_t* k,
                   const uint8_t* v, const float* k_scale, const float* v_scale,
                   int n_new, const int* cache_len, int num_q_heads,
                   int num_kv_heads, int head_dim, float scale, void* stream);

/* *pos += delta on device. No counterpart in the reference (which advances
 * the decode position with a host copy, reference
 * include/runtherder/engine/context.h:41-45); lets one captured graph hold
 * several decode steps. */
int rth_advance_position(int* pos, int delta, void* stream);

/* Replaces kernels::rope_bf16 (reference include/runtherder/kernels/
 * rope.cuh:16-25): in-place rotate-half RoPE on q [seq_len, Hq, D] and
 * k [seq_len, Hkv, D] bf16; token t rotates by positions[t] (device array)
 * with inv_freq [D/2] (device). head_dim even, <= 256. sin/cos are taken in
 * double precision of the fp32 angle, rounded to fp32. */
int rth_rope_bf16(uint16_t* q, uint16_t* k, const int* positions,
                  const float* inv_freq, int seq_len, int num_q_heads,
                  int num_kv_heads, int head_dim, void* stream);

/* No counterpart in the reference: fuses the caller sequence
 * rope_bf16(q, k) then KVCache::append(layer, k, v, n_new, at_pos)
 * (reference src/model/supported/llama/llama3.cu:228-232) into one launch.
 * q is rotated in place exactly as rth_rope_bf16 does; rotated K and V rows
 * are quantized into the layer's cache slabs at rows *at_pos .. *at_pos +
 * n_new - 1, byte-identical to rth_rope_bf16 followed by rth_kv_append_fp8.
 * The k input is read only (left unrotated, unlike the two-step sequence).
 * head_dim in {64, 128, 256}. */
int rth_rope_append_fp8(uint16_t* q, uint8_t* k_cache, uint8_t* v_cache,
                        float* k_scale, float* v_scale, const uint16_t* k,
                        const uint16_t* v, const int* positions,
                        const float* inv_freq, const int* at_pos, int n_new,
                        int num_q_heads, int num_kv_heads, int head_dim,
                        void* stream);

/* Paged KV cache (no counterpart in the reference, whose README plans paged
 * attention, README.md:142-143): the cache slabs hold physical blocks of
 * block_size positions ([num_blocks * block_size, Hkv, D] E4M3 and
 * [num_blocks * block_size, Hkv] fp32 scales); logical position p of the
 * sequence lives at physical position block_table[p / block_size] *
 * block_size + p % block_size. block_table is a device int array covering
 * every block up to the last position used; block_size is a power of two
 * >= 32. Each entry below equals its contiguous counterpart on the gathered
 * cache, bit for bit. */
int rth_kv_append_fp8_paged(uint8_t* k_cache, uint8_t* v_cache, float* k_scale,
                            float* v_scale, const uint16_t* k, const uint16_t* v,
                            const int* at_pos, int n_new, int num_kv_heads, int head_dim,
                            const int* block_table, int block_size, void* stream);
int rth_attn_decode_split_paged(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                const uint8_t* v, const float* k_scale, const float* v_scale,
                                const int* block_table, int block_size, float* partial,
                                int num_splits, const int* cache_len, int num_q_heads,
                                int num_kv_heads, int head_dim, float scale, void* stream);
int rth_attn_decode_append_split_paged(uint16_t* out, const uint16_t* q, uint8_t* k_cache,
                                       uint8_t* v_cache, float* k_scale, float* v_scale,
                                       const int* block_table, int block_size,
                                       const uint16_t* k_new, const uint16_t* v_new,
                                       float* partial, int num_splits, const int* cache_len,
                                       int num_q_heads, int num_kv_heads, int head_dim,
                                       float scale, void* stream);
/* No counterpart in the reference: fuses the per-layer decode step
 * rope_bf16(q, k, positions, inv_freq) -> KVCache::append(layer, k, v, 1,
 * cache_len) -> AttentionBackend::run(out, q, view, 1, cache_len) (reference
 * src/model/supported/llama/llama3.cu:228-234) into the two launches of
 * rth_attn_decode_append_split. q and k_new ([Hq, D] and [Hkv, D] bf16,
 * unrotated) are read only: both are rotated in registers by the angles of
 * positions[0] with rth_rope_bf16's arithmetic, so the cache row written at
 * *cache_len is byte-identical to rth_rope_bf16 + rth_kv_append_fp8 and the
 * output is bit-identical to rth_attn_decode_append_split on the rotated q
 * and k. Shapes
 * rth_decode_path reports as RTH_DECODE_MFMA under the automatic choice
 * (head_dim 64, 128, 256); others fail with an error. block_table == NULL (or the first entry point): the
 * contiguous layout. */
int rth_attn_decode_rope_append_split(uint16_t* out, const uint16_t* q, uint8_t* k_cache,
                                      uint8_t* v_cache, float* k_scale, float* v_scale,
                                      const uint16_t* k_new, const uint16_t* v_new,
                                      const int* positions, const float* inv_freq,
                                      float* partial, int num_splits, const int* cache_len,
                                      int num_q_heads, int num_kv_heads, int head_dim,
                                      float scale, void* stream);
int rth_attn_decode_rope_append_split_paged(uint16_t* out, const uint16_t* q, uint8_t* k_cache,
                                            uint8_t* v_cache, float* k_scale, float* v_scale,
                                            const int* block_table, int block_size,
                                            const uint16_t* k_new, const uint16_t* v_new,
                                            const int* positions, const float* inv_freq,
                                            float* partial, int num_splits,
                                            const int* cache_len, int num_q_heads,
                                            int num_kv_heads, int head_dim, float scale,
                                            void* stream);
/* No counterpart in the reference: the Qwen3 decode step,
 * rmsnorm_bf16_forward(q, q_norm) and (k, k_norm) per head -> rope_bf16 ->
 * KVCache::append -> run (reference src/model/supported/llama/
 * qwen3.cu:189-202), in the two launches of rth_attn_decode_append_split.
 * q and k_new are read only; the cache row equals rth_qk_norm_rope_append_fp8's
 * byte for byte, and the output is bit-identical to
 * rth_attn_decode_append_split on q and
 * k_new after rth_rmsnorm_bf16 (per head) and rth_rope_bf16. Shapes as
 * rth_attn_decode_rope_append_split. */
int rth_attn_decode_qk_norm_rope_append_split(
    uint16_t* out, const uint16_t* q, uint8_t* k_cache, uint8_t* v_cache, float* k_scale,
    float* v_scale, const uint16_t* k_new, const uint16_t* v_new, const uint16_t* q_norm,
    const uint16_t* k_norm, float eps, const int* positions, const float* inv_freq,
    float* partial, int num_splits, const int* cache_len, int num_q_heads, int num_kv_heads,
    int head_dim, float scale, void* stream);
int rth_attn_decode_qk_norm_rope_append_split_paged(
    uint16_t* out, const uint16_t* q, uint8_t* k_cache, uint8_t* v_cache, float* k_scale,
    float* v_scale, const int* block_table, int block_size, const uint16_t* k_new,
    const uint16_t* v_new, const uint16_t* q_norm, const uint16_t* k_norm, float eps,
    const int* positions, const float* inv_freq, float* partial, int num_splits,
    const int* cache_len, int num_q_heads, int num_kv_heads, int head_dim, float scale,
    void* stream);
int rth_attn_prefill_paged(uint16_t* out, const uint16_t* q, const uint8_t* k,
                           const uint8_t* v, const float* k_scale, const float* v_scale,
                           const int* block_table, int block_size, int n_new,
                           const int* cache_len, int num_q_heads, int num_kv_heads,
                           int head_dim, float scale, void* stream);

/* No counterpart in the reference: fuses the Qwen3 caller sequence
 * rmsnorm_bf16_forward(q, q_norm) [per q head], rmsnorm_bf16_forward(k,
 * k_norm) [per kv head], rope_bf16(q, k), KVCache::append(k, v) (reference
 * src/model/supported/llama/qwen3.cu:189-200) into one launch. q is
 * normalized and rotated in place; the cache receives exactly the bytes of
 * rth_rmsnorm_bf16 + rth_rope_bf16 + rth_kv_append_fp8; k is read only.
 * q_norm, k_norm: [head_dim] bf16 gains. head_dim in {64, 128, 256}. */
int rth_qk_norm_rope_append_fp8(uint16_t* q, uint8_t* k_cache, uint8_t* v_cache,
                                float* k_scale, float* v_scale, const uint16_t* k,
                                const uint16_t* v, const uint16_t* q_norm,
                                const uint16_t* k_norm, float eps, const int* positions,
                                const float* inv_freq, const int* at_pos, int n_new,
                                int num_q_heads, int num_kv_heads, int head_dim,
                                void* stream);

/* Replaces kernels::rmsnorm_bf16_forward (reference include/runtherder/
 * kernels/rmsnorm.cuh:14-22): y = bf16((x * rrms) * g) per row of
 * x [num_tokens, hidden_dim] bf16, rrms = 1 / sqrt(sum(x^2) / hidden_dim +
 * eps) with a correctly rounded sqrt and division; y may alias x.
 * hidden_dim a multiple of 8, <= 16384. The sum of squares runs over
 * rth_rmsnorm_lanes(hidden_dim) lane partials in a fixed order. */
int rth_rmsnorm_bf16(uint16_t* y, const uint16_t* x, const uint16_t* g, int num_tokens,
                     int hidden_dim, float eps, void* stream);

/* Lanes per row of rth_rmsnorm_bf16's reduction (the next power of two of
 * hidden_dim / 8, at most 64); 0 for an invalid hidden_dim. No reference
 * counterpart: lets a checker restate the summation order. */
int rth_rmsnorm_lanes(int hidden_dim);

#ifdef __cplusplus
}
#endif

#endif /* RTH_ATTN_H */
