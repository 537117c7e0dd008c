// Naive causal GQA attention over an E4M3 KV cache (the NaiveAttention
// backend). Same math as attention_causal_bf16_kernel (reference
// src/kernels/attention.cu:34-91): per output row (token, q head) a max pass
// over the scaled scores, then an exp-weighted sum of dequantized values,
// fp32 throughout, bf16 RNE output. It is kept for debugging and as the
// drop-in for BackendKind::Naive, not for speed.
//
// One wave64 owns one output row; lane i holds head_dim elements
// i, i+64, ..., so a q.k dot is a wave reduction. head_dim <= 512.
#include "device_common.hpp"
#include "launch.hpp"

namespace rth {
namespace {

constexpr int kNaiveWaves = 4;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        v += __shfl_xor(v, m, kWave);
    }
    return v;
}

template <int kPer>
__global__ __launch_bounds__(kNaiveWaves * kWave) void attention_naive_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ q,
    const uint8_t* __restrict__ k, const uint8_t* __restrict__ v,
    const float* __restrict__ ks, const float* __restrict__ vs, int n_new,
    const int* __restrict__ cache_len, int hq, int hkv, int head_dim, float scale) {
    const int row = static_cast<int>(blockIdx.x) * kNaiveWaves +
                    static_cast<int>(threadIdx.x) / kWave;
    if (row >= n_new * hq) {
        return;
    }
    const int lane   = lane_id();
    const int qt     = row / hq;
    const int qh     = row % hq;
    const int kvh    = qh / (hq / hkv);
    const int n_keys = *cache_len + qt + 1;

    const uint16_t* qr = q + static_cast<int64_t>(row) * head_dim;
    float           qv[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int d = lane + kWave * i;
        qv[i]       = (d < head_dim) ? bf16_to_f32(qr[d]) : 0.0f;
    }

    auto score = [&](int j) {
        const int64_t  krow = static_cast<int64_t>(j) * hkv + kvh;
        const uint8_t* kr   = k + krow * head_dim;
        const float    sc   = ks[krow];
        float          s    = 0.0f;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int d = lane + kWave * i;
            if (d < head_dim) {
                const float kd = __builtin_amdgcn_cvt_f32_fp8(kr[d], 0) * sc;
                s              = fmaf(qv[i], kd, s);
            }
        }
        return wave_sum(s) * scale;
    };

    float m = -INFINITY;
    for (int j = 0; j < n_keys; ++j) {
        m = fmaxf(m, score(j));
    }

    float acc[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        acc[i] = 0.0f;
    }
    float denom = 0.0f;
    for (int j = 0; j < n_keys; ++j) {
        const float    w    = expf(score(j) - m);
        const int64_t  vrow = static_cast<int64_t>(j) * hkv + kvh;
        const uint8_t* vr   = v + vrow * head_dim;
        const float    sc   = vs[vrow];
        denom += w;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int d = lane + kWave * i;
            if (d < head_dim) {
                acc[i] = fmaf(w, __builtin_amdgcn_cvt_f32_fp8(vr[d], 0) * sc, acc[i]);
            }
        }
    }

    uint16_t* orow = out + static_cast<int64_t>(row) * head_dim;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int d = lane + kWave * i;
        if (d < head_dim) {
            orow[d] = f32_to_bf16_bits(acc[i] / denom);
        }
    }
}

}  // namespace

hipError_t attention_naive_launch(uint16_t* out, const uint16_t* q,
                                  const uint8_t* k, const uint8_t* v,
                                  const float* k_scale, const float* v_scale,
                                  int n_new, const int* cache_len,
                                  int num_q_heads, int num_kv_heads,
                                  int head_dim, float scale, hipStream_t stream) {
    const int  rows = n_new * num_q_heads;
    const dim3 grid(static_cast<unsigned>((rows + kNaiveWaves - 1) / kNaiveWaves));
    const dim3 block(kNaiveWaves * kWave);
    const int  per = (head_dim + kWave - 1) / kWave;
    switch (per) {
#define RTH_N_CASE(P)                                                                  \
    case P:                                                                            \
        hipLaunchKernelGGL(attention_naive_kernel<P>, grid, block, 0, stream, out, q, k, \
                           v, k_scale, v_scale, n_new, cache_len, num_q_heads,        \
                           num_kv_heads, head_dim, scale);                             \
        break;
        RTH_N_CASE(1)
        RTH_N_CASE(2)
        RTH_N_CASE(4)
        RTH_N_CASE(8)
#undef RTH_N_CASE
        case 3:
            hipLaunchKernelGGL(attention_naive_kernel<4>, grid, block, 0, stream, out, q, k,
                               v, k_scale, v_scale, n_new, cache_len, num_q_heads,
                               num_kv_heads, head_dim, scale);
            break;
        case 5:
        case 6:
        case 7:
            hipLaunchKernelGGL(attention_naive_kernel<8>, grid, block, 0, stream, out, q, k,
                               v, k_scale, v_scale, n_new, cache_len, num_q_heads,
                               num_kv_heads, head_dim, scale);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rth
