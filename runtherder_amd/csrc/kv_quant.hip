// FP8 (OCP E4M3) KV-cache append / quantize kernels for gfx950.
//
// Semantics follow quantize_kv_fp8 (reference src/kernels/quantization.cu:
// 200-254): one quant group per row (= one (token, kv_head)), amax = max |x|
// with NaN ignored, scale = amax / 448, inv = amax > 0 ? 448 / amax : 0 (two
// separate IEEE divisions), q = E4M3_satfinite(x * inv), written at
// destination row r + (*at_pos) * rows_per_pos.
//
// Layout on MI355X: a row of head_dim bf16 is read by a group of
// lanes_per_row lanes with 16-byte loads (8 bf16 per lane), reduced with
// in-wave xor shuffles, and written back as 8-byte E4M3 stores plus one fp32
// scale. Several rows share one wave: a 128-wide head uses all 64 lanes for
// 4 rows at once, or, in appends of 32768 rows or more, 8 rows with two
// loads in flight per lane. The K and V append of one layer is one launch
// (blockIdx.y selects the slab).
#include "device_common.hpp"
#include "launch.hpp"

namespace rth {
namespace {

constexpr int kQuantBlock = 256;
constexpr int kMaxCached  = 4;  // 16-byte chunks a lane keeps in registers

struct QuantSlab {
    uint8_t*        q;
    float*          scale;
    const uint16_t* x;
};

// Mode 0: scale from the row amax. Mode 1: scale given at the destination row.
// kPaged: destination position p = *at_pos + row / rows_per_pos is stored at
// physical position (block_table[p >> block_shift] << block_shift) |
// (p & (2^block_shift - 1)).
template <int kLanesPerRow, int kMode, bool kPaged>
__global__ __launch_bounds__(kQuantBlock) void quantize_rows_kernel(
    QuantSlab s0, QuantSlab s1, const int* __restrict__ at_pos,
    int rows_per_pos, int num_rows, int head_dim, const int* __restrict__ block_table,
    int block_shift) {
    const QuantSlab s       = (blockIdx.y == 0) ? s0 : s1;
    constexpr int   kRowsPB = kQuantBlock / kLanesPerRow;
    const int       sub     = static_cast<int>(threadIdx.x) % kLanesPerRow;
    const int       row     = static_cast<int>(blockIdx.x) * kRowsPB +
                    static_cast<int>(threadIdx.x) / kLanesPerRow;
    const bool      live    = row < num_rows;
    const int       n_vec   = head_dim / 8;

    int64_t dst;
    if constexpr (kPaged) {
        const int p    = *at_pos + row / rows_per_pos;
        const int phys = (live ? (block_table[p >> block_shift] << block_shift) : 0) |
                         (p & ((1 << block_shift) - 1));
        dst = static_cast<int64_t>(phys) * rows_per_pos + row % rows_per_pos;
    } else {
        dst = static_cast<int64_t>(row) + static_cast<int64_t>(*at_pos) * rows_per_pos;
    }
    const uint16_t* xr = s.x + static_cast<int64_t>(row) * head_dim;

    u32x4 cache[kMaxCached];
    float amax = 0.0f;
    if (live) {
#pragma unroll
        for (int c = 0; c < kMaxCached; ++c) {
            const int v = sub + c * kLanesPerRow;
            if (v < n_vec) {
                cache[c] = *reinterpret_cast<const u32x4*>(xr + v * 8);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t w = cache[c][e];
                    amax = fmaxf(amax, fabsf(__uint_as_float(w << 16)));
                    amax = fmaxf(amax, fabsf(__uint_as_float(w & 0xffff0000u)));
                }
            }
        }
        for (int v = sub + kMaxCached * kLanesPerRow; v < n_vec; v += kLanesPerRow) {
            const u32x4 w4 = *reinterpret_cast<const u32x4*>(xr + v * 8);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                amax = fmaxf(amax, fabsf(__uint_as_float(w4[e] << 16)));
                amax = fmaxf(amax, fabsf(__uint_as_float(w4[e] & 0xffff0000u)));
            }
        }
    }
#pragma unroll
    for (int m = 1; m < kLanesPerRow; m <<= 1) {
        amax = wave_xor_max(amax, m);
    }
    if (!live) {
        return;
    }

    float inv;
    if constexpr (kMode == 0) {
        const float sc = amax / kE4M3Max;
        inv            = (amax > 0.0f) ? (kE4M3Max / amax) : 0.0f;
        if (sub == 0) {
            s.scale[dst] = sc;
        }
    } else {
        const float sc = s.scale[dst];
        inv            = (sc > 0.0f) ? (1.0f / sc) : 0.0f;
    }

    uint8_t* qr = s.q + dst * head_dim;
    auto emit = [&](int v, const u32x4 w4) {
        u32x2 out;
        uint32_t lo = 0, hi = 0;
        lo = e4m3x2_pack<false>(__uint_as_float(w4.x << 16) * inv,
                         __uint_as_float(w4.x & 0xffff0000u) * inv, lo);
        lo = e4m3x2_pack<true>(__uint_as_float(w4.y << 16) * inv,
                         __uint_as_float(w4.y & 0xffff0000u) * inv, lo);
        hi = e4m3x2_pack<false>(__uint_as_float(w4.z << 16) * inv,
                         __uint_as_float(w4.z & 0xffff0000u) * inv, hi);
        hi = e4m3x2_pack<true>(__uint_as_float(w4.w << 16) * inv,
                         __uint_as_float(w4.w & 0xffff0000u) * inv, hi);
        out.x = lo;
        out.y = hi;
        *reinterpret_cast<u32x2*>(qr + v * 8) = out;
    };
#pragma unroll
    for (int c = 0; c < kMaxCached; ++c) {
        const int v = sub + c * kLanesPerRow;
        if (v < n_vec) {
            emit(v, cache[c]);
        }
    }
    for (int v = sub + kMaxCached * kLanesPerRow; v < n_vec; v += kLanesPerRow) {
        emit(v, *reinterpret_cast<const u32x4*>(xr + v * 8));
    }
}

template <int kMode, bool kPaged>
hipError_t launch_quant(QuantSlab s0, QuantSlab s1, int n_slabs,
                        const int* at_pos, int rows_per_pos, int num_rows,
                        int head_dim, const int* block_table, int block_shift,
                        hipStream_t stream) {
    const int n_vec = head_dim / 8;
    int       lpr   = 1;
    while (lpr < n_vec && lpr < kWave) {
        lpr <<= 1;
    }
    // Large appends: half the lanes per row, so every lane keeps two 16-byte
    // loads in flight (n = 4096 at 8 kv heads: 7.1 -> 6.0 us; 16384: 22.4 ->
    // 18.9 us). Small ones keep the wider groups, which finish sooner.
    if (num_rows * n_slabs >= 32768 && lpr >= 16) {
        lpr /= 2;
    }
    const int rows_pb = kQuantBlock / lpr;
    const dim3 grid(static_cast<unsigned>((num_rows + rows_pb - 1) / rows_pb),
                    static_cast<unsigned>(n_slabs));
    switch (lpr) {
#define RTH_Q_CASE(L)                                                                    \
    case L:                                                                              \
        hipLaunchKernelGGL((quantize_rows_kernel<L, kMode, kPaged>), grid,               \
                           dim3(kQuantBlock), 0, stream, s0, s1, at_pos, rows_per_pos,   \
                           num_rows, head_dim, block_table, block_shift);                \
        break;
        RTH_Q_CASE(1)
        RTH_Q_CASE(2)
        RTH_Q_CASE(4)
        RTH_Q_CASE(8)
        RTH_Q_CASE(16)
        RTH_Q_CASE(32)
        RTH_Q_CASE(64)
#undef RTH_Q_CASE
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t quantize_kv_fp8_launch(uint8_t* q, float* scale, const uint16_t* x,
                                  const int* at_pos, int rows_per_pos,
                                  int num_rows, int head_dim, hipStream_t stream) {
    const QuantSlab s{q, scale, x};
    return launch_quant<0, false>(s, s, 1, at_pos, rows_per_pos, num_rows, head_dim, nullptr, 0,
                                  stream);
}

hipError_t quantize_kv_fp8_scaled_launch(uint8_t* q, const float* scale,
                                         const uint16_t* x, const int* at_pos,
                                         int rows_per_pos, int num_rows,
                                         int head_dim, hipStream_t stream) {
    const QuantSlab s{q, const_cast<float*>(scale), x};
    return launch_quant<1, false>(s, s, 1, at_pos, rows_per_pos, num_rows, head_dim, nullptr, 0,
                                  stream);
}

hipError_t kv_append_fp8_launch(uint8_t* k_q, uint8_t* v_q, float* k_scale,
                                float* v_scale, const uint16_t* k,
                                const uint16_t* v, const int* at_pos,
                                int rows_per_pos, int num_rows, int head_dim,
                                hipStream_t stream, const int* block_table, int block_shift) {
    const QuantSlab sk{k_q, k_scale, k};
    const QuantSlab sv{v_q, v_scale, v};
    if (block_table != nullptr) {
        return launch_quant<0, true>(sk, sv, 2, at_pos, rows_per_pos, num_rows, head_dim,
                                     block_table, block_shift, stream);
    }
    return launch_quant<0, false>(sk, sv, 2, at_pos, rows_per_pos, num_rows, head_dim, nullptr,
                                  0, stream);
}

}  // namespace rth
