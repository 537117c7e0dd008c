/*
 * CPU oracle for the attention hot path (TEST INFRASTRUCTURE ONLY).
 *
 * This library restates, in plain C, the arithmetic of the reference engine's
 * attention hot path so the HIP kernels can be checked against it. Only the
 * tests, the smoke check and the CPU-baseline leg of the benchmark may load it;
 * the product library never links or calls it.
 *
 * Every function cites the reference file:line it follows (paths relative to
 * the reference repository root). Parity status of each function is stated in
 * rth_oracle.c next to its definition.
 */
#ifndef RTH_ORACLE_H
#define RTH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar formats ---------------------------------------------------- */
uint16_t rth_ref_f32_to_bf16(float x);
float    rth_ref_bf16_to_f32(uint16_t b);
uint8_t  rth_ref_e4m3_encode(float x);
float    rth_ref_e4m3_decode(uint8_t b);
void     rth_ref_e4m3_encode_array(const float* x, uint8_t* out, int64_t n);
void     rth_ref_e4m3_encode_bits_range(uint32_t first_bits, uint64_t count,
                                        uint8_t* out);
int64_t  rth_ref_e4m3_sweep_check(uint32_t stride, int nthreads);

/* ---- seeded inputs ----------------------------------------------------- */
void rth_ref_fill_normal_bf16(uint16_t* out, int64_t n, uint64_t seed);
void rth_ref_fill_normal_f32(float* out, int64_t n, uint64_t seed);
void rth_ref_fill_uniform_f32(float* out, int64_t n, float lo, float hi,
                              uint64_t seed);
void rth_ref_mt19937_raw(uint32_t seed, int64_t n, uint32_t* out);
void rth_ref_fill_mt19937_uniform_bf16(uint16_t* out, int64_t n, float scale,
                                       uint32_t seed);

/* ---- KV quantization --------------------------------------------------- */
void rth_ref_quantize_kv_fp8(uint8_t* q, float* scale, const uint16_t* x,
                             int at_pos, int rows_per_pos, int num_rows,
                             int head_dim);
void rth_ref_quantize_kv_fp8_scaled(uint8_t* q, const float* scale,
                                    const uint16_t* x, int at_pos,
                                    int rows_per_pos, int num_rows,
                                    int head_dim);

/* ---- attention --------------------------------------------------------- */
void rth_ref_attention_f32(uint16_t* out, const uint16_t* q, const uint8_t* k,
                           const uint8_t* v, const float* k_scale,
                           const float* v_scale, int n_new, int cache_len,
                           int num_q_heads, int num_kv_heads, int head_dim,
                           float scale, int nthreads);
void rth_ref_attention_f64(double* out, const uint16_t* q, const uint8_t* k,
                           const uint8_t* v, const float* k_scale,
                           const float* v_scale, int n_new, int cache_len,
                           int num_q_heads, int num_kv_heads, int head_dim,
                           double scale);
void rth_ref_decode_split_f32(uint16_t* out, const uint16_t* q,
                              const uint8_t* k, const uint8_t* v,
                              const float* k_scale, const float* v_scale,
                              int num_splits, int cache_len, int num_q_heads,
                              int num_kv_heads, int head_dim, float scale);

/* ---- RoPE input preparation ------------------------------------------- */
void rth_ref_rope_inv_freq_plain(float* inv_freq, int head_dim,
                                 float theta_base);
void rth_ref_rope_inv_freq_llama3(float* inv_freq, int head_dim,
                                  float theta_base, float factor,
                                  float low_freq_factor,
                                  float high_freq_factor,
                                  int original_max_position_embeddings);
void rth_ref_rmsnorm_bf16(uint16_t* y, const uint16_t* x, const uint16_t* g,
                          int rows, int dim, float eps, int lanes);
void rth_ref_rope_apply_bf16(uint16_t* x, const int* positions,
                             const float* inv_freq, int n_tokens,
                             int num_heads, int head_dim);

#ifdef __cplusplus
}
#endif

#endif /* RTH_ORACLE_H */
