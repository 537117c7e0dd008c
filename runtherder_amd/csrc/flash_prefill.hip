// Causal flash prefill over an OCP E4M3 KV cache on bf16 MFMA, gfx950.
//
// Math follows flash_prefill_bf16 (reference src/kernels/flash_prefill.cu:
// 34-241): causal rule "query t at position cache_len + t sees keys
// 0 .. cache_len + t" (:127-139), online softmax in fp32, bf16 RNE output of
// O / l. head_dim is 128, as in the reference (:226).
//
// MI355X design:
//  * Workgroup = one q head x 128 query rows, 4 waves of 32 rows. Grid order
//    puts the longest (last) row blocks first (a grid resident in one round
//    pairs them with the lightest instead) and keeps the q heads of one kv
//    head on one XCD so their K/V tiles share an L2.
//  * Each 64-key tile is staged in LDS as bf16 converted exactly from the E4M3
//    codes: K row-major [key][d], V transposed [d][key] (the transpose is done
//    in registers with v_perm before the LDS write). Row pitches are padded by
//    16 bytes so the 128-bit MFMA operand reads are bank-conflict free. The next
//    tile's global loads are issued before the current tile's MFMAs.
//  * Scores are computed transposed, S^T = K Q^T with
//    v_mfma_f32_32x32x16_bf16 (A = K from LDS, B = Q^T held in registers), so
//    each lane owns one query row: the softmax max/sum need one cross-lane
//    step and the O^T rescale is a per-lane scalar. P^T feeds O^T += V^T P^T
//    straight from the score registers (the V^T LDS columns are stored in the
//    matching key order).
//  * The per-(token, kv_head) scales stay in fp32: k_scale * softmax_scale *
//    log2(e) multiplies each score column, v_scale multiplies P before its
//    bf16 rounding. The softmax runs in base 2.
//  * Tiles beyond a wave's last query position are skipped per wave; masking
//    is evaluated only on tiles that cross the diagonal or the key end.
#include "device_common.hpp"
#include "launch.hpp"

namespace rth {
namespace {

constexpr int kPfWaves   = 4;
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kBM        = 128;          // query rows per workgroup
constexpr int kBN        = 64;           // keys per tile
constexpr int kHD        = 128;          // head_dim
constexpr int kKPitch    = kHD + 8;      // bf16 per K row in LDS   (272 B)
constexpr int kVPitch    = kBN + 8;      // bf16 per V^T row in LDS (144 B)

// LDS column of key o (0..63) in the V^T tile: within each group of 16 keys,
// offset 8a + 4h + b is stored at 8h + 4a + b, so the 8 keys one MFMA lane
// feeds are contiguous.
__device__ __forceinline__ int vt_pos(int o) {
    const int grp = o & ~15;
    const int a   = (o >> 3) & 1;
    const int h   = (o >> 2) & 1;
    return grp + 8 * h + 4 * a + (o & 3);
}

struct PfRaw {
    u32x4 k[2];   // 32 E4M3 bytes of one K row
    u32x2 v[4];   // 8 E4M3 bytes (d0..d0+7) of 4 consecutive V rows
    float sc;     // k_scale or v_scale of one key
};

// Physical cache row of logical key `key` (identity unless paged: blocks of
// 2^block_shift keys, logical block b at physical block block_table[b]).
template <bool kPaged>
__device__ __forceinline__ int pf_row(int key, const int* __restrict__ block_table,
                                      int block_shift) {
    if constexpr (kPaged) {
        return (block_table[key >> block_shift] << block_shift) |
               (key & ((1 << block_shift) - 1));
    } else {
        return key;
    }
}

template <bool kPaged>
__device__ __forceinline__ void pf_load(PfRaw& r, const uint8_t* __restrict__ k,
                                        const uint8_t* __restrict__ v,
                                        const float* __restrict__ ks,
                                        const float* __restrict__ vs, int key0,
                                        int total, int kvh, int hkv, int tid,
                                        const int* __restrict__ bt, int bshift) {
    // Paged: the tile's two 32-key halves each lie inside one block (blocks
    // hold a power of two >= 32 keys), so two uniform lookups give the
    // physical offsets; clamped keys stay inside the tile.
    int d_lo = 0, d_hi = 0;
    if constexpr (kPaged) {
        d_lo = pf_row<true>(key0, bt, bshift) - key0;
        d_hi = (key0 + 32 < total) ? pf_row<true>(key0 + 32, bt, bshift) - (key0 + 32) : d_lo;
    }
    auto phys = [&](int key) { return key + ((key - key0 < 32) ? d_lo : d_hi); };
    {
        const int      key = phys(min(key0 + (tid >> 2), total - 1));
        const uint8_t* kr  = k + (static_cast<int64_t>(key) * hkv + kvh) * kHD + 32 * (tid & 3);
        r.k[0] = *reinterpret_cast<const u32x4*>(kr);
        r.k[1] = *reinterpret_cast<const u32x4*>(kr + 16);
    }
    {
        const int kq = tid & 15;           // key quad 0..15
        const int d0 = 8 * (tid >> 4);     // 8 d of those 4 keys
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int key = phys(min(key0 + 4 * kq + j, total - 1));
            r.v[j] = *reinterpret_cast<const u32x2*>(
                v + (static_cast<int64_t>(key) * hkv + kvh) * kHD + d0);
        }
    }
    if (tid < 2 * kBN) {
        const int     key = phys(min(key0 + (tid & (kBN - 1)), total - 1));
        const int64_t row = static_cast<int64_t>(key) * hkv + kvh;
        r.sc = (tid < kBN) ? ks[row] : vs[row];
    }
}

__device__ __forceinline__ void pf_stage(const PfRaw& r, uint16_t* sK, uint16_t* sVt,
                                         float* sKf, float* sVf, int tid,
                                         float scale_log2) {
    {
        const int row = tid >> 2;
        const int c0  = 32 * (tid & 3);
        bf16x8    a, b, c, d;
        e4m3x16_to_bf16x8x2(r.k[0], a, b);
        e4m3x16_to_bf16x8x2(r.k[1], c, d);
        uint16_t* dst = sK + row * kKPitch + c0;
        *reinterpret_cast<bf16x8*>(dst)      = a;
        *reinterpret_cast<bf16x8*>(dst + 8)  = b;
        *reinterpret_cast<bf16x8*>(dst + 16) = c;
        *reinterpret_cast<bf16x8*>(dst + 24) = d;
    }
    {
        // Lanes 16i..16i+15 share d0 and cover the 16 key quads, so each
        // 16-lane pass of the 8-byte LDS writes fills one whole V^T row
        // (bank-conflict free).
        const int kq = tid & 15;
        const int d0 = 8 * (tid >> 4);
        // 4 keys x 8 bytes -> 8 dwords, each holding one d for the 4 keys.
        uint32_t x[8];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const uint32_t a0 = half ? r.v[0].y : r.v[0].x;
            const uint32_t a1 = half ? r.v[1].y : r.v[1].x;
            const uint32_t a2 = half ? r.v[2].y : r.v[2].x;
            const uint32_t a3 = half ? r.v[3].y : r.v[3].x;
            const uint32_t t01l = __builtin_amdgcn_perm(a1, a0, 0x05010400u);
            const uint32_t t01h = __builtin_amdgcn_perm(a1, a0, 0x07030602u);
            const uint32_t t23l = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
            const uint32_t t23h = __builtin_amdgcn_perm(a3, a2, 0x07030602u);
            x[4 * half + 0] = __builtin_amdgcn_perm(t23l, t01l, 0x05040100u);
            x[4 * half + 1] = __builtin_amdgcn_perm(t23l, t01l, 0x07060302u);
            x[4 * half + 2] = __builtin_amdgcn_perm(t23h, t01h, 0x05040100u);
            x[4 * half + 3] = __builtin_amdgcn_perm(t23h, t01h, 0x07060302u);
        }
        const int col = vt_pos(4 * kq);
#pragma unroll
        for (int dd = 0; dd < 8; ++dd) {
            *reinterpret_cast<u32x2*>(sVt + (d0 + dd) * kVPitch + col) = e4m3x4_to_bf16x4(x[dd]);
        }
    }
    if (tid < kBN) {
        sKf[tid] = r.sc * scale_log2;
    } else if (tid < 2 * kBN) {
        sVf[tid - kBN] = r.sc;
    }
}

template <bool kPaged>
__global__ __launch_bounds__(kPfThreads, 2) void flash_prefill_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ q,
    const uint8_t* __restrict__ k, const uint8_t* __restrict__ v,
    const float* __restrict__ ks, const float* __restrict__ vs, int n_new,
    const int* __restrict__ cache_len, int hq, int hkv, float scale_log2,
    const int* __restrict__ block_table, int block_shift, bool one_round) {
    __shared__ __attribute__((aligned(16))) uint16_t sK[kBN * kKPitch];
    __shared__ __attribute__((aligned(16))) uint16_t sVt[kHD * kVPitch];
    __shared__ __attribute__((aligned(16))) float    sKf[kBN];
    __shared__ __attribute__((aligned(16))) float    sVf[kBN];

    const int tid  = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid & (kWave - 1);
    const int qn   = lane & 31;   // query row of this lane within the wave
    const int h    = lane >> 5;   // k-group

    // Block mapping: heavy row blocks first; q heads of one kv head on one XCD.
    // When the whole grid is resident at once (one_round), the second half of
    // the grid runs the light blocks in ascending order, so the two
    // workgroups sharing a compute unit pair a heavy block with a light one.
    const int n_blk    = (n_new + kBM - 1) / kBM;
    const int bid      = static_cast<int>(blockIdx.x);
    const int half_wgs = (n_blk / 2) * hq;
    const int blk      = (one_round && bid >= half_wgs) ? (bid - half_wgs) / hq
                                                        : n_blk - 1 - bid / hq;
    const int hb    = bid % hq;
    const int qh    = ((hq & 7) == 0) ? ((hb & 7) * (hq >> 3) + (hb >> 3)) : hb;
    const int G     = hq / hkv;
    const int kvh   = qh / G;

    const int clen  = *cache_len;
    const int total = clen + n_new;
    const int q0    = blk * kBM;
    const int last  = min(q0 + kBM, n_new) - 1;
    const int n_tiles = min((total + kBN - 1) / kBN, (clen + last) / kBN + 1);

    const int wq0        = q0 + wave * 32;                 // first row of this wave
    const int wlast      = min(wq0 + 31, n_new - 1);       // may be < wq0 (idle wave)
    const int w_tiles    = (wlast < wq0) ? 0 : (clen + wlast) / kBN + 1;
    const int my_q       = wq0 + qn;
    const int my_pos     = clen + my_q;

    // Q^T (B operand): lane holds row my_q, d = 8h + 16s .. +8 for s = 0..7.
    bf16x8 qop[8];
    {
        const bool      has = my_q < n_new;
        const uint16_t* qr  = q + (static_cast<int64_t>(has ? my_q : 0) * hq + qh) * kHD;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            u32x4 w = *reinterpret_cast<const u32x4*>(qr + 8 * h + 16 * s);
            if (!has) {
                w = u32x4{0u, 0u, 0u, 0u};
            }
            qop[s] = __builtin_bit_cast(bf16x8, w);
        }
    }

    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o[i] = f32x16{};
    }
    float m_ref = 0.0f;   // lazy reference maximum of this lane's row (log2 units)
    float l_run = 0.0f;

    PfRaw raw;
    pf_load<kPaged>(raw, k, v, ks, vs, 0, total, kvh, hkv, tid, block_table, block_shift);

    for (int kt = 0; kt < n_tiles; ++kt) {
        __syncthreads();
        pf_stage(raw, sK, sVt, sKf, sVf, tid, scale_log2);
        __syncthreads();
        if (kt + 1 < n_tiles) {
            pf_load<kPaged>(raw, k, v, ks, vs, (kt + 1) * kBN, total, kvh, hkv, tid, block_table,
                            block_shift);
        }
        if (kt >= w_tiles) {
            continue;
        }
        const int key0 = kt * kBN;

        // S^T = K Q^T for two 32-key blocks. The LDS operand reads run four
        // MFMAs ahead (scheduling groups), so their latency is hidden.
        f32x16 s[2];
        {
            bf16x8 ka[2][8];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const uint16_t* arow = sK + (32 * kb + qn) * kKPitch + 8 * h;
#pragma unroll
                for (int st = 0; st < 8; ++st) {
                    ka[kb][st] = *reinterpret_cast<const bf16x8*>(arow + 16 * st);
                }
            }
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                s[kb] = f32x16{};
#pragma unroll
                for (int st = 0; st < 8; ++st) {
                    s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[kb][st], qop[st], s[kb], 0, 0, 0);
                }
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
            for (int i = 0; i < 12; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        }

        // t = s * (k_scale * scale * log2 e) - m_ref, one fma per score, in
        // place. Register r of block kb is key 32kb + 8(r/4) + 4h + r%4 of the
        // tile.
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const f32x4 kf = *reinterpret_cast<const f32x4*>(sKf + 32 * kb + 8 * rg + 4 * h);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    s[kb][4 * rg + e] = fmaf(s[kb][4 * rg + e], kf[e], -m_ref);
                }
            }
        }
        // Causal / key-end mask, only on tiles that cross the diagonal or the
        // end of the keys (a wave-uniform branch).
        if ((key0 + kBN - 1 > clen + wq0) || (key0 + kBN > total)) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int kp = key0 + 32 * kb + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (kp > my_pos || kp >= total) {
                        s[kb][r] = -INFINITY;
                    }
                }
            }
        }

        // p = 2^t against the lazy reference maximum m_ref, the row sum of p
        // and the P^T operands (p * v_scale rounded to bf16).
        bf16x8 pop[4];
        float  psum  = 0.0f;
        auto   exp_p = [&]() {
            psum = 0.0f;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    u32x4 pw;
#pragma unroll
                    for (int rr = 0; rr < 2; ++rr) {
                        const int   rg = 2 * half + rr;
                        const f32x4 vf = *reinterpret_cast<const f32x4*>(sVf + 32 * kb + 8 * rg + 4 * h);
                        const float p0 = __builtin_amdgcn_exp2f(s[kb][4 * rg + 0]);
                        const float p1 = __builtin_amdgcn_exp2f(s[kb][4 * rg + 1]);
                        const float p2 = __builtin_amdgcn_exp2f(s[kb][4 * rg + 2]);
                        const float p3 = __builtin_amdgcn_exp2f(s[kb][4 * rg + 3]);
                        psum += (p0 + p1) + (p2 + p3);
                        pw[2 * rr]     = pack_bf16x2(p0 * vf[0], p1 * vf[1]);
                        pw[2 * rr + 1] = pack_bf16x2(p2 * vf[2], p3 * vf[3]);
                    }
                    pop[2 * kb + half] = __builtin_bit_cast(bf16x8, pw);
                }
            }
        };
        exp_p();
        // Lazy reference maximum (exact): m_ref moves to the row maximum only
        // on the first tile or when a row sum exceeds 2^64 (some score more
        // than 64 above m_ref); otherwise the tile needs no max reduction, no
        // cross-lane step and no accumulator rescale. Every p and l use the
        // same m_ref, and p <= 2^64 keeps l and O finite in fp32.
        if (__any((kt == 0) || !(psum <= 0x1p64f))) {
            float tmax = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    tmax = fmaxf(tmax, s[kb][r]);
                }
            }
            tmax              = wave_xor_max(tmax, 32);
            const float delta = (tmax == -INFINITY) ? 0.0f : tmax;
            // On the first tile l and O are still zero (and 2^-delta may be inf).
            const float alpha = (kt == 0) ? 1.0f : __builtin_amdgcn_exp2f(-delta);
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                s[kb] -= delta;
            }
            m_ref += delta;
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                o[db] *= alpha;
            }
            exp_p();
        }
        l_run += psum;

        // O^T += V^T P^T, operand reads four MFMAs ahead as above.
        {
            bf16x8 va[4][4];
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const uint16_t* arow = sVt + (32 * db + qn) * kVPitch + 8 * h;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    va[db][t] = *reinterpret_cast<const bf16x8*>(arow + 16 * t);
                }
            }
#pragma unroll
            for (int db = 0; db < 4; ++db) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[db][t], pop[t], o[db], 0, 0, 0);
                }
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
#pragma unroll
            for (int i = 0; i < 12; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
        }
    }

    const float l_tot = wave_xor_sum(l_run, 32);
    if (my_q < n_new) {
        const float inv_l = 1.0f / l_tot;
        uint16_t*   orow  = out + (static_cast<int64_t>(my_q) * hq + qh) * kHD;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                u32x2 w;
                w.x = pack_bf16x2(o[db][4 * rg + 0] * inv_l, o[db][4 * rg + 1] * inv_l);
                w.y = pack_bf16x2(o[db][4 * rg + 2] * inv_l, o[db][4 * rg + 3] * inv_l);
                *reinterpret_cast<u32x2*>(orow + 32 * db + 8 * rg + 4 * h) = w;
            }
        }
    }
}

}  // namespace

hipError_t flash_prefill_launch(uint16_t* out, const uint16_t* q,
                                const uint8_t* k, const uint8_t* v,
                                const float* k_scale, const float* v_scale,
                                int n_new, const int* cache_len,
                                int num_q_heads, int num_kv_heads,
                                int head_dim, float scale, hipStream_t stream,
                                const int* block_table, int block_shift) {
    if (head_dim != kHD) {
        return hipErrorInvalidValue;
    }
    const int  n_blk = (n_new + kBM - 1) / kBM;
    const dim3 grid(static_cast<unsigned>(n_blk * num_q_heads));
    // Two workgroups fit per compute unit (LDS and registers).
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
        cus = 0;
    }
    const bool one_round = n_blk * num_q_heads <= 2 * cus;
    if (block_table != nullptr) {
        hipLaunchKernelGGL(flash_prefill_kernel<true>, grid, dim3(kPfThreads), 0, stream, out, q,
                           k, v, k_scale, v_scale, n_new, cache_len, num_q_heads, num_kv_heads,
                           scale * kLog2e, block_table, block_shift, one_round);
    } else {
        hipLaunchKernelGGL(flash_prefill_kernel<false>, grid, dim3(kPfThreads), 0, stream, out,
                           q, k, v, k_scale, v_scale, n_new, cache_len, num_q_heads,
                           num_kv_heads, scale * kLog2e, nullptr, 0, one_round);
    }
    return hipGetLastError();
}

}  // namespace rth
