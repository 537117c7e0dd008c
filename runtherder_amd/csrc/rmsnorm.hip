// RMSNorm over bf16 rows, gfx950.
//
// Math follows rmsnorm_bf16_forward (reference src/kernels/rmsnorm.cu:45-136):
// y = bf16((x * rrms) * g) with rrms = 1 / sqrt(ss / dim + eps), ss the row
// sum of squares in fp32 (the reference forms rrms with rsqrtf; this build
// uses a correctly rounded square root and division, the form of the
// reference test's CPU oracle, tests/kernels/test_rmsnorm.cpp:39-60).
//
// A row is handled by a group of `lanes` lanes (a power of two, up to one
// wave): lane l accumulates fma(x, x, s) over the 16-byte vectors l,
// l + lanes, ... and the group reduces with an xor butterfly, so every lane
// holds the same sum and the order is fixed (the oracle restates it). Small
// rows (a head_dim of 64..256) share a wave: several rows per wave, no LDS.
// The same row routine serves the fused q/k-norm -> RoPE -> append entry.
#include "device_common.hpp"
#include "launch.hpp"
#include "rmsnorm_row.hpp"

namespace rth {
namespace {

constexpr int kNormBlock = 256;

template <int kLanes>
__global__ __launch_bounds__(kNormBlock) void rmsnorm_kernel(
    uint16_t* __restrict__ y, const uint16_t* __restrict__ x, const uint16_t* __restrict__ g,
    int rows, int dim, float eps) {
    constexpr int kRowsPB = kNormBlock / kLanes;
    const int     sub     = static_cast<int>(threadIdx.x) % kLanes;
    const int     row     = static_cast<int>(blockIdx.x) * kRowsPB +
                    static_cast<int>(threadIdx.x) / kLanes;
    if (row >= rows) {   // whole lane groups leave together
        return;
    }
    rmsnorm_row<kLanes>(y + static_cast<int64_t>(row) * dim, x + static_cast<int64_t>(row) * dim,
                        g, dim, eps, sub);
}

}  // namespace

int rmsnorm_lanes(int dim) {
    const int n_vec = dim / 8;
    int       lanes = 1;
    while (lanes < n_vec && lanes < kWave) {
        lanes <<= 1;
    }
    return lanes;
}

hipError_t rmsnorm_bf16_launch(uint16_t* y, const uint16_t* x, const uint16_t* g, int rows,
                               int dim, float eps, hipStream_t stream) {
    const int  lanes   = rmsnorm_lanes(dim);
    const int  rows_pb = kNormBlock / lanes;
    const dim3 grid(static_cast<unsigned>((rows + rows_pb - 1) / rows_pb));
    switch (lanes) {
#define RTH_N_CASE(L)                                                                    \
    case L:                                                                              \
        hipLaunchKernelGGL(rmsnorm_kernel<L>, grid, dim3(kNormBlock), 0, stream, y, x, g, \
                           rows, dim, eps);                                              \
        break;
        RTH_N_CASE(1)
        RTH_N_CASE(2)
        RTH_N_CASE(4)
        RTH_N_CASE(8)
        RTH_N_CASE(16)
        RTH_N_CASE(32)
        RTH_N_CASE(64)
#undef RTH_N_CASE
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace rth
