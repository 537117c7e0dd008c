// Device-side helpers shared by the attention kernels (gfx950 / CDNA4 only).
//
// Vector types for the bf16 MFMA operands, OCP E4M3 conversion through the
// gfx950 hardware converters, bf16 rounding, and wave64 lane utilities.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rth {

typedef __bf16   bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16   bf16x2 __attribute__((ext_vector_type(2)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));
typedef float    f32x16 __attribute__((ext_vector_type(16)));
typedef float    f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int   kWave     = 64;
constexpr float kE4M3Max  = 448.0f;
constexpr float kLog2e    = 1.4426950408889634f;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (finite inputs; NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return static_cast<uint16_t>((u >> 16) | 0x40u);
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// Two fp32 -> two OCP E4M3 bytes (RNE, saturate to +-448, NaN -> 0x7F),
// merged into bits [16*hi, 16*hi+16) of `old`. The hardware converter rounds
// to nearest even; inputs are clamped first so it never sees an out-of-range
// value, and NaN lanes are patched to the canonical 0x7F afterwards.
template <bool kHi>
__device__ __forceinline__ uint32_t e4m3x2_pack(float a, float b, uint32_t old) {
    const float ca = fminf(fmaxf(a, -kE4M3Max), kE4M3Max);
    const float cb = fminf(fmaxf(b, -kE4M3Max), kE4M3Max);
    uint32_t    r  = static_cast<uint32_t>(
        __builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, static_cast<int>(old), kHi));
    constexpr int sh = kHi ? 16 : 0;
    if (a != a) {
        r = (r & ~(0xffu << sh)) | (0x7fu << sh);
    }
    if (b != b) {
        r = (r & ~(0xffu << (sh + 8))) | (0x7fu << (sh + 8));
    }
    return r;
}

// Four E4M3 bytes of one dword -> four exact bf16 values (E4M3 is a subset of
// bf16). Returns dwords {b0|b1<<16, b2|b3<<16} in bf16 bits.
__device__ __forceinline__ u32x2 e4m3x4_to_bf16x4(uint32_t w) {
    const bf16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
    const bf16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
    u32x2        r;
    r.x = __builtin_bit_cast(uint32_t, lo);
    r.y = __builtin_bit_cast(uint32_t, hi);
    return r;
}

// 16 E4M3 bytes -> two bf16x8 operands (bytes 0..7, bytes 8..15).
__device__ __forceinline__ void e4m3x16_to_bf16x8x2(const u32x4 w, bf16x8& a,
                                                    bf16x8& b) {
    const u32x2 p0 = e4m3x4_to_bf16x4(w.x);
    const u32x2 p1 = e4m3x4_to_bf16x4(w.y);
    const u32x2 p2 = e4m3x4_to_bf16x4(w.z);
    const u32x2 p3 = e4m3x4_to_bf16x4(w.w);
    u32x4       ua = {p0.x, p0.y, p1.x, p1.y};
    u32x4       ub = {p2.x, p2.y, p3.x, p3.y};
    a              = __builtin_bit_cast(bf16x8, ua);
    b              = __builtin_bit_cast(bf16x8, ub);
}

// 8 E4M3 bytes -> one bf16x8 operand.
__device__ __forceinline__ bf16x8 e4m3x8_to_bf16x8(const u32x2 w) {
    const u32x2 p0 = e4m3x4_to_bf16x4(w.x);
    const u32x2 p1 = e4m3x4_to_bf16x4(w.y);
    u32x4       u  = {p0.x, p0.y, p1.x, p1.y};
    return __builtin_bit_cast(bf16x8, u);
}

// Pack two fp32 into one dword of two bf16 (RNE, hardware converter).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 v;
    v.x = static_cast<__bf16>(lo);
    v.y = static_cast<__bf16>(hi);
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

// This lane's value and that of lane ^ mask, as a pair in some order. For
// masks 16 and 32 a gfx950 row swap of v with itself (one VALU instruction:
// v_permlane16_swap exchanges the odd 16-lane rows of its first operand with
// the even rows of its second, v_permlane32_swap the upper 32 lanes of the
// first with the lower 32 of the second) leaves every lane holding both;
// other masks take a lane shuffle (an LDS crossbar round trip). Wave-wide
// callers only: every lane of the wave must be active.
struct LanePair {
    float a, b;
};
__device__ __forceinline__ LanePair wave_xor_pair(float v, int mask) {
    const uint32_t x = __float_as_uint(v);
    if (mask == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return {__uint_as_float(r[0]), __uint_as_float(r[1])};
    }
    if (mask == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        return {__uint_as_float(r[0]), __uint_as_float(r[1])};
    }
    return {v, __shfl_xor(v, mask, kWave)};
}

// The value of lane ^ mask. After v_permlane32_swap the first result holds
// the lower 32 lanes' values and the second the upper's; after
// v_permlane16_swap the first holds the even rows' and the second the odd
// rows'.
__device__ __forceinline__ float wave_xor_partner(float v, int mask) {
    const uint32_t x = __float_as_uint(v);
    const int      l = static_cast<int>(threadIdx.x) & (kWave - 1);
    if (mask == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return __uint_as_float((l & 32) ? r[0] : r[1]);
    }
    if (mask == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        return __uint_as_float((l & 16) ? r[0] : r[1]);
    }
    return __shfl_xor(v, mask, kWave);
}

// max / sum of this lane's value and lane ^ mask's (both lanes get the same
// result, bit for bit).
__device__ __forceinline__ float wave_xor_max(float v, int mask) {
    const LanePair p = wave_xor_pair(v, mask);
    return fmaxf(p.a, p.b);
}

__device__ __forceinline__ float wave_xor_sum(float v, int mask) {
    const LanePair p = wave_xor_pair(v, mask);
    return p.a + p.b;
}

}  // namespace rth
