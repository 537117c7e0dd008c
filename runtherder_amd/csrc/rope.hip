// Rotate-half RoPE on bf16 Q/K, standalone and fused with the FP8 KV append,
// gfx950.
//
// Math follows rope_bf16 (reference src/kernels/rope.cu:14-55): token t
// rotates the pair (i, i + D/2) of every q and k head by theta =
// float(positions[t]) * inv_freq[i]:
//     a' = bf16(a*cos - b*sin),  b' = bf16(a*sin + b*cos).
// This build evaluates each output as one fma over a rounded product,
// fma(a, c, -(b*s)) and fma(a, s, b*c), and takes sin/cos of the fp32 angle
// in double precision, rounded to fp32 (the reference uses the __sincosf
// approximation; its own test bound is max-abs 5e-2 against double,
// include/runtherder/kernels/rope.cuh:14).
//
// One workgroup per token: the D/2 (cos, sin) pairs of the token are
// computed once into LDS and shared by all Hq + Hkv heads.
//
// The fused entry (no reference counterpart) replaces the caller sequence
// rope_bf16(q, k) -> KVCache::append(k, v) (reference
// src/model/supported/llama/llama3.cu:228-232): q is rotated in place, each
// K row is rotated in registers, rounded to bf16 exactly as the standalone
// kernel writes it, and quantized straight into the cache with the append's
// arithmetic (amax / 448, 448 / amax, E4M3 satfinite), V rows are
// quantized; the k input is left unrotated. Cache bytes and scales equal
// those of rope_bf16 followed by the append, bit for bit.
#include "device_common.hpp"
#include "launch.hpp"
#include "rmsnorm_row.hpp"

namespace rth {
namespace {

constexpr int kRopeBlock   = 256;
constexpr int kRopeMaxHalf = 128;   // head_dim <= 256

__device__ __forceinline__ void rope_table(float* sm_c, float* sm_s, int pos,
                                           const float* __restrict__ inv_freq, int half) {
    for (int i = static_cast<int>(threadIdx.x); i < half; i += kRopeBlock) {
        const float th = static_cast<float>(pos) * inv_freq[i];
        double      s, c;
        sincos(static_cast<double>(th), &s, &c);
        sm_c[i] = static_cast<float>(c);
        sm_s[i] = static_cast<float>(s);
    }
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Rotates 8 consecutive pairs (i0 .. i0+7) given as bf16 words of a (first
// half) and b (second half); results are bf16 words.
__device__ __forceinline__ void rotate8(u32x4& a, u32x4& b, const float* sm_c,
                                        const float* sm_s, int i0) {
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(sm_c + i0);
    const f32x4 c1 = *reinterpret_cast<const f32x4*>(sm_c + i0 + 4);
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(sm_s + i0);
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(sm_s + i0 + 4);
    const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
    const float s[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
    u32x4 ra, rb;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float a0 = bf16_lo(a[w]), a1 = bf16_hi(a[w]);
        const float b0 = bf16_lo(b[w]), b1 = bf16_hi(b[w]);
        const int   j  = 2 * w;
        ra[w] = pack_bf16x2(fmaf(a0, c[j], -(b0 * s[j])), fmaf(a1, c[j + 1], -(b1 * s[j + 1])));
        rb[w] = pack_bf16x2(fmaf(a0, s[j], b0 * c[j]), fmaf(a1, s[j + 1], b1 * c[j + 1]));
    }
    a = ra;
    b = rb;
}

// Rotates `rows` contiguous head rows of one token in place. kVec: the
// half-width is a multiple of 8 (16-byte accesses), else one pair per item.
template <bool kVec>
__device__ __forceinline__ void rope_rows(uint16_t* __restrict__ x, int rows, int head_dim,
                                          const float* sm_c, const float* sm_s) {
    const int half = head_dim / 2;
    if constexpr (kVec) {
        const int per_row = half / 8;
        for (int it = static_cast<int>(threadIdx.x); it < rows * per_row; it += kRopeBlock) {
            const int r  = it / per_row;
            const int i0 = 8 * (it - r * per_row);
            uint16_t* xr = x + static_cast<int64_t>(r) * head_dim;
            u32x4     a  = *reinterpret_cast<const u32x4*>(xr + i0);
            u32x4     b  = *reinterpret_cast<const u32x4*>(xr + half + i0);
            rotate8(a, b, sm_c, sm_s, i0);
            *reinterpret_cast<u32x4*>(xr + i0)        = a;
            *reinterpret_cast<u32x4*>(xr + half + i0) = b;
        }
    } else {
        for (int it = static_cast<int>(threadIdx.x); it < rows * half; it += kRopeBlock) {
            const int   r  = it / half;
            const int   i  = it - r * half;
            uint16_t*   xr = x + static_cast<int64_t>(r) * head_dim;
            const float a  = bf16_to_f32(xr[i]);
            const float b  = bf16_to_f32(xr[i + half]);
            const float c  = sm_c[i];
            const float s  = sm_s[i];
            xr[i]          = f32_to_bf16_bits(fmaf(a, c, -(b * s)));
            xr[i + half]   = f32_to_bf16_bits(fmaf(a, s, b * c));
        }
    }
}

template <bool kVec>
__global__ __launch_bounds__(kRopeBlock) void rope_bf16_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k, const int* __restrict__ positions,
    const float* __restrict__ inv_freq, int hq, int hkv, int head_dim) {
    __shared__ __attribute__((aligned(16))) float sm_c[kRopeMaxHalf];
    __shared__ __attribute__((aligned(16))) float sm_s[kRopeMaxHalf];
    const int t = static_cast<int>(blockIdx.x);
    rope_table(sm_c, sm_s, positions[t], inv_freq, head_dim / 2);
    __syncthreads();
    rope_rows<kVec>(q + static_cast<int64_t>(t) * hq * head_dim, hq, head_dim, sm_c, sm_s);
    rope_rows<kVec>(k + static_cast<int64_t>(t) * hkv * head_dim, hkv, head_dim, sm_c, sm_s);
}

// Quantizes one cache row held by kLpr lanes (8 bf16 per lane, as words)
// with the append's arithmetic and stores codes and scale.
template <int kLpr>
__device__ __forceinline__ void quantize_row_regs(const u32x4 w4, int sub, uint8_t* qrow,
                                                  float* scale_slot) {
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        amax = fmaxf(amax, fabsf(bf16_lo(w4[e])));
        amax = fmaxf(amax, fabsf(bf16_hi(w4[e])));
    }
#pragma unroll
    for (int m = 1; m < kLpr; m <<= 1) {
        amax = wave_xor_max(amax, m);
    }
    const float sc  = amax / kE4M3Max;
    const float inv = (amax > 0.0f) ? (kE4M3Max / amax) : 0.0f;
    if (sub == 0) {
        *scale_slot = sc;
    }
    uint32_t lo = 0, hi = 0;
    lo = e4m3x2_pack<false>(bf16_lo(w4.x) * inv, bf16_hi(w4.x) * inv, lo);
    lo = e4m3x2_pack<true>(bf16_lo(w4.y) * inv, bf16_hi(w4.y) * inv, lo);
    hi = e4m3x2_pack<false>(bf16_lo(w4.z) * inv, bf16_hi(w4.z) * inv, hi);
    hi = e4m3x2_pack<true>(bf16_lo(w4.w) * inv, bf16_hi(w4.w) * inv, hi);
    u32x2 out;
    out.x = lo;
    out.y = hi;
    *reinterpret_cast<u32x2*>(qrow + 8 * sub) = out;
}

// Rotates one row held as one vector per lane (kLpr lanes, head_dim =
// 8 * kLpr): the RoPE partner of lane l's elements sits in lane l ^ (kLpr/2).
template <int kLpr>
__device__ __forceinline__ u32x4 rope_vec(const u32x4 w4, int sub, const float* sm_c,
                                          const float* sm_s) {
    u32x4 other;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        other[e] = static_cast<uint32_t>(__shfl_xor(static_cast<int>(w4[e]), kLpr / 2, kWave));
    }
    const bool first = sub < kLpr / 2;
    u32x4      a     = first ? w4 : other;
    u32x4      b     = first ? other : w4;
    rotate8(a, b, sm_c, sm_s, 8 * (first ? sub : sub - kLpr / 2));
    return first ? a : b;
}

// Per token: q rows [optional RMSNorm] -> RoPE -> stored in place; K rows
// [optional RMSNorm] -> RoPE -> quantized into the cache; V rows quantized.
// A row is one group of kLpr lanes; every lane of a group takes the same
// branch and trip count, so the shuffles stay within converged groups.
template <int kLpr, bool kNorm>
__global__ __launch_bounds__(kRopeBlock) void rope_append_kernel(
    uint16_t* __restrict__ q, uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache,
    float* __restrict__ k_scale, float* __restrict__ v_scale, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ q_norm,
    const uint16_t* __restrict__ k_norm, float eps, const int* __restrict__ positions,
    const float* __restrict__ inv_freq, const int* __restrict__ at_pos, int hq, int hkv) {
    constexpr int kHeadDim = 8 * kLpr;
    constexpr int kRowsPB  = kRopeBlock / kLpr;
    __shared__ __attribute__((aligned(16))) float sm_c[kRopeMaxHalf];
    __shared__ __attribute__((aligned(16))) float sm_s[kRopeMaxHalf];

    const int t = static_cast<int>(blockIdx.x);
    rope_table(sm_c, sm_s, positions[t], inv_freq, kHeadDim / 2);
    __syncthreads();

    const int     sub  = static_cast<int>(threadIdx.x) % kLpr;
    const int64_t row0 = static_cast<int64_t>(*at_pos + t) * hkv;
    for (int r = static_cast<int>(threadIdx.x) / kLpr; r < hq + 2 * hkv; r += kRowsPB) {
        if (r < hq) {
            uint16_t* xr = q + (static_cast<int64_t>(t) * hq + r) * kHeadDim + 8 * sub;
            u32x4     w4 = *reinterpret_cast<const u32x4*>(xr);
            if constexpr (kNorm) {
                w4 = rmsnorm_vec<kLpr>(w4, q_norm, sub, eps);
            }
            *reinterpret_cast<u32x4*>(xr) = rope_vec<kLpr>(w4, sub, sm_c, sm_s);
            continue;
        }
        const bool      is_k = r < hq + hkv;
        const int       h    = is_k ? r - hq : r - hq - hkv;
        const uint16_t* xr   = (is_k ? k : v) + (static_cast<int64_t>(t) * hkv + h) * kHeadDim;
        u32x4           w4   = *reinterpret_cast<const u32x4*>(xr + 8 * sub);
        if (is_k) {
            if constexpr (kNorm) {
                w4 = rmsnorm_vec<kLpr>(w4, k_norm, sub, eps);
            }
            w4 = rope_vec<kLpr>(w4, sub, sm_c, sm_s);
        }
        const int64_t dst = row0 + h;
        quantize_row_regs<kLpr>(w4, sub, (is_k ? k_cache : v_cache) + dst * kHeadDim,
                                (is_k ? k_scale : v_scale) + dst);
    }
}

}  // namespace

hipError_t rope_bf16_launch(uint16_t* q, uint16_t* k, const int* positions,
                            const float* inv_freq, int seq_len, int num_q_heads,
                            int num_kv_heads, int head_dim, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(seq_len));
    if ((head_dim / 2) % 8 == 0) {
        hipLaunchKernelGGL(rope_bf16_kernel<true>, grid, dim3(kRopeBlock), 0, stream, q, k,
                           positions, inv_freq, num_q_heads, num_kv_heads, head_dim);
    } else {
        hipLaunchKernelGGL(rope_bf16_kernel<false>, grid, dim3(kRopeBlock), 0, stream, q, k,
                           positions, inv_freq, num_q_heads, num_kv_heads, head_dim);
    }
    return hipGetLastError();
}

hipError_t rope_append_fp8_launch(uint16_t* q, uint8_t* k_cache, uint8_t* v_cache,
                                  float* k_scale, float* v_scale, const uint16_t* k,
                                  const uint16_t* v, const uint16_t* q_norm,
                                  const uint16_t* k_norm, float eps, const int* positions,
                                  const float* inv_freq, const int* at_pos, int n_new,
                                  int num_q_heads, int num_kv_heads, int head_dim,
                                  hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(n_new));
    const bool norm = q_norm != nullptr;
    switch (head_dim) {
#define RTH_RA_CASE(D)                                                                      \
    case D:                                                                                 \
        if (norm) {                                                                         \
            hipLaunchKernelGGL((rope_append_kernel<D / 8, true>), grid, dim3(kRopeBlock), 0, \
                               stream, q, k_cache, v_cache, k_scale, v_scale, k, v, q_norm, \
                               k_norm, eps, positions, inv_freq, at_pos, num_q_heads,       \
                               num_kv_heads);                                              \
        } else {                                                                            \
            hipLaunchKernelGGL((rope_append_kernel<D / 8, false>), grid, dim3(kRopeBlock), 0, \
                               stream, q, k_cache, v_cache, k_scale, v_scale, k, v, q_norm, \
                               k_norm, eps, positions, inv_freq, at_pos, num_q_heads,       \
                               num_kv_heads);                                              \
        }                                                                                   \
        break;
        RTH_RA_CASE(64)
        RTH_RA_CASE(128)
        RTH_RA_CASE(256)
#undef RTH_RA_CASE
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rth
