// Row RMSNorm routines shared by the standalone kernel (rmsnorm.hip) and the
// fused q/k-norm -> RoPE -> append kernel (rope.hip). The reduction order is
// fixed: each lane accumulates fma(x, x, s) over its 16-byte vectors in
// order, then an xor butterfly over the kLanes lanes of the row.
#pragma once

#include "device_common.hpp"

namespace rth {

template <int kLanes>
__device__ __forceinline__ float rms_butterfly(float s) {
#pragma unroll
    for (int m = 1; m < kLanes; m <<= 1) {
        s += __shfl_xor(s, m, kWave);
    }
    return s;
}

__device__ __forceinline__ float sumsq8(const u32x4 w, float s) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float lo = __uint_as_float(w[e] << 16);
        const float hi = __uint_as_float(w[e] & 0xffff0000u);
        s              = fmaf(lo, lo, s);
        s              = fmaf(hi, hi, s);
    }
    return s;
}

// Plain `/` and sqrtf: with this compiler's defaults they lower to the
// correctly rounded sequences (div_scale/div_fmas/div_fixup, and v_sqrt with
// a one-ulp residual correction), unlike the __fdiv_rn / __fsqrt_rn
// intrinsics, which lower to the approximate hardware instructions.
__device__ __forceinline__ float rms_inverse(float ss, int dim, float eps) {
    return 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
}

// y = bf16((x * rrms) * g) for the 8 elements of one vector.
__device__ __forceinline__ u32x4 scale8(const u32x4 w, const u32x4 gw, float rrms) {
    u32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float lo = __uint_as_float(w[e] << 16);
        const float hi = __uint_as_float(w[e] & 0xffff0000u);
        const float glo = __uint_as_float(gw[e] << 16);
        const float ghi = __uint_as_float(gw[e] & 0xffff0000u);
        r[e]            = pack_bf16x2((lo * rrms) * glo, (hi * rrms) * ghi);
    }
    return r;
}

// One row held as one vector per lane (dim == 8 * kLanes), normalized in
// registers.
template <int kLanes>
__device__ __forceinline__ u32x4 rmsnorm_vec(const u32x4 w, const uint16_t* __restrict__ g,
                                             int sub, float eps) {
    const float ss   = rms_butterfly<kLanes>(sumsq8(w, 0.0f));
    const float rrms = rms_inverse(ss, 8 * kLanes, eps);
    const u32x4 gw   = *reinterpret_cast<const u32x4*>(g + 8 * sub);
    return scale8(w, gw, rrms);
}

// A row of any dim (multiple of 8) in memory; y may alias x (each vector is
// read and written by the same lane, reads of a vector precede its write).
template <int kLanes>
__device__ __forceinline__ void rmsnorm_row(uint16_t* y, const uint16_t* x,
                                            const uint16_t* __restrict__ g, int dim, float eps,
                                            int sub) {
    constexpr int kCached = 4;
    const int     n_vec   = dim / 8;
    u32x4         cache[kCached];
    float         s = 0.0f;
#pragma unroll
    for (int c = 0; c < kCached; ++c) {
        const int v = sub + c * kLanes;
        if (v < n_vec) {
            cache[c] = *reinterpret_cast<const u32x4*>(x + 8 * v);
            s        = sumsq8(cache[c], s);
        }
    }
    for (int v = sub + kCached * kLanes; v < n_vec; v += kLanes) {
        s = sumsq8(*reinterpret_cast<const u32x4*>(x + 8 * v), s);
    }
    const float rrms = rms_inverse(rms_butterfly<kLanes>(s), dim, eps);
#pragma unroll
    for (int c = 0; c < kCached; ++c) {
        const int v = sub + c * kLanes;
        if (v < n_vec) {
            *reinterpret_cast<u32x4*>(y + 8 * v) =
                scale8(cache[c], *reinterpret_cast<const u32x4*>(g + 8 * v), rrms);
        }
    }
    for (int v = sub + kCached * kLanes; v < n_vec; v += kLanes) {
        *reinterpret_cast<u32x4*>(y + 8 * v) =
            scale8(*reinterpret_cast<const u32x4*>(x + 8 * v),
                   *reinterpret_cast<const u32x4*>(g + 8 * v), rrms);
    }
}

}  // namespace rth
