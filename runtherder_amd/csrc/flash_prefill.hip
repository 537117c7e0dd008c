// Causal flash prefill over an OCP E4M3 KV cache, gfx950.
//
// Math follows flash_prefill_bf16 (reference src/kernels/flash_prefill.cu:
// 34-241): causal rule "query t at position cache_len + t sees keys
// 0 .. cache_len + t" (:127-139), online softmax in fp32, bf16 RNE output of
// O / l. head_dim is 128, as in the reference (:226).
//
// MI355X design:
//  * Workgroup = one q head x (32 x waves) query rows, 32 rows per wave:
//    8 waves (256 rows, one workgroup per compute unit) when the grid takes
//    at least two rounds of those, else 128 rows: as two 4-wave halves that
//    split the block's key tiles (even / odd) and merge in LDS, for grids of
//    4+ blocks per head up to ~1.5 rounds, or as 4 waves (two per compute
//    unit, heavy and light row blocks paired when the grid is resident in
//    one round). Longest (last) row blocks first; the q heads of one kv head
//    on one XCD so their K/V tiles share an L2.
//  * Keys go in 64-key tiles. The K tile's E4M3 codes are copied unchanged
//    into LDS by the LDS-DMA loads (global_load_lds_dwordx4, 16-byte chunks
//    XOR-swizzled by row so the operand reads are bank-conflict free), ahead
//    of use, with no registers or VALU work.
//  * Scores S^T = K Q^T run on the fp8 MFMA v_mfma_scale_f32_32x32x64_f8f6f4
//    with A = the raw K codes from LDS and B = Q split into two E4M3
//    parts: q * 2^a = hi + lo / 16 (a per row, so the row maximum lands in
//    [128, 256)), the MFMA's per-lane E8M0 scales undoing 2^a and 16. A bf16
//    q has 8 significant bits and hi takes the top 4, so for scaled elements
//    |y| >= 2^-6 the split is exact and every product is the exact code * q
//    product, accumulated in fp32. Below 2^-6 (elements more than ~13
//    binades under their row maximum) lo falls into E4M3 subnormals and the
//    split errs by at most 2^-14 in scaled units, 2^-21 of the row maximum
//    (tests/test_prefill_q_split.py checks both over every bf16 value).
//  * Each lane owns one query row (the S^T column), so the softmax needs no
//    cross-lane step except on a rebase. t = s * (k_scale * scale * log2 e)
//    - m_ref against a lazy reference maximum; p = 2^t rounded to f16, the
//    row sum taken from the fp32 2^t.
//  * V is dequantized into LDS as f16(code * v_scale), transposed to V^T in
//    registers (v_perm) before the LDS write, and O^T += V^T P^T runs on
//    v_mfma_f32_32x32x16_f16 with P^T straight from the score registers.
//  * Buffers are separate LDS arrays indexed statically (the tile loop is
//    unrolled), so the compiler sees the LDS-DMA into one buffer and the reads
//    of another as independent. One barrier per tile, which waits only for
//    the K copy the next tile needs.
//  * 8-wave workgroups run two phase-shifted groups so that the softmax
//    (VALU) of one wave meets the MFMAs of the other wave on its SIMD, and a
//    wave in its softmax or P V runs at a higher issue priority than one in
//    its score MFMAs; the 4-wave workgroups weave the next tile's copies and
//    V staging between their own MFMAs.
//  * Key runs (flash_prefill_keysplit_launch, kPart): for chunks after a long
//    cache, each (row block, q head) of the 4-wave kernel is split over
//    gridDim.y workgroups, each walking one run of key tiles and storing
//    partials in the split-K decode layout for the decode merge.
#include "device_common.hpp"
#include "launch.hpp"

namespace rth {
namespace {

typedef int      i32x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kBN     = 64;          // keys per tile
constexpr int kHD     = 128;         // head_dim
constexpr int kKTile  = kBN * kHD;   // bytes of E4M3 K codes per tile
constexpr int kVPitch = kBN + 8;     // f16 per V^T row in LDS (144 B)
constexpr int kE8M0One = 127;        // E8M0 encoding of 1.0

// LDS column of key o (0..63) in the V^T tile: within each group of 16 keys,
// offset 8a + 4h + b is stored at 8h + 4a + b, so the 8 keys one MFMA lane
// feeds are contiguous.
__device__ __forceinline__ int vt_pos(int o) {
    const int grp = o & ~15;
    const int a   = (o >> 3) & 1;
    const int h   = (o >> 2) & 1;
    return grp + 8 * h + 4 * a + (o & 3);
}

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

// Physical row of key `key` of the tile starting at key0, clamped to the last
// key (a tile past the end maps to the last tile). Paged: the tile's two
// 32-key halves each lie inside one block (blocks hold a power of two >= 32
// keys), so two uniform lookups per tile suffice.
template <bool kPaged>
struct TileRows {
    int key0, total, d_lo, d_hi;
    __device__ __forceinline__ TileRows(int key0_, int total_, const int* __restrict__ bt,
                                        int bshift)
        : key0(min(key0_, (total_ - 1) & ~(kBN - 1))), total(total_), d_lo(0), d_hi(0) {
        if constexpr (kPaged) {
            d_lo = pf_row<true>(key0, bt, bshift) - key0;
            d_hi = (key0 + 32 < total) ? pf_row<true>(key0 + 32, bt, bshift) - (key0 + 32) : d_lo;
        }
    }
    __device__ __forceinline__ int operator()(int i) const {   // i = key offset in the tile
        const int key = min(key0 + i, total - 1);
        return key + ((key - key0 < 32) ? d_lo : d_hi);
    }
};

// Byte offset of 16-byte chunk c (0..7) of K row r (0..63) in an LDS K tile.
__device__ __forceinline__ int k_chunk(int r, int c) {
    return r * kHD + 16 * (c ^ (r & 7));
}

// Issues the LDS-DMA copy of one K tile: slot s (16 bytes) holds chunk
// (s & 7) ^ (row & 7) of row s >> 3, so that k_chunk() finds it.
template <int kThreads, bool kPaged>
__device__ __forceinline__ void k_tile_dma(uint8_t* dst, const uint8_t* __restrict__ k,
                                           const TileRows<kPaged>& rows, int kvh, int hkv,
                                           int tid) {
#pragma unroll
    for (int rep = 0; rep < kKTile / 16 / kThreads; ++rep) {
        const int      s   = tid + rep * kThreads;
        const int      r   = s >> 3;
        const int      c   = (s & 7) ^ (r & 7);
        const uint8_t* src = k + (static_cast<int64_t>(rows(r)) * hkv + kvh) * kHD + 16 * c;
        // The destination base is wave-uniform; lane l lands at base + 16 l.
        __builtin_amdgcn_global_load_lds(src, dst + 16 * (s & ~(kWave - 1)), 16, 0, 0);
    }
}

// Registers of the next tile's V staging: per unit, 8 E4M3 bytes (d0..d0+7)
// of two consecutive keys and their v_scale; plus one k_scale.
template <int kReps>
struct VRaw {
    u32x2 a[kReps], b[kReps];
    float sa[kReps], sb[kReps];
    float ks;
};

// V staging units: unit u = (key pair kp = u & 31, d group u >> 5 of 8 d).
template <int kThreads, bool kPaged>
__device__ __forceinline__ void v_tile_load(VRaw<4096 / 8 / kThreads>& r,
                                            const uint8_t* __restrict__ v,
                                            const float* __restrict__ ks,
                                            const float* __restrict__ vs,
                                            const TileRows<kPaged>& rows, int kvh, int hkv,
                                            int tid) {
    constexpr int kReps = 4096 / 8 / kThreads;
#pragma unroll
    for (int rep = 0; rep < kReps; ++rep) {
        const int     u  = tid + rep * kThreads;
        const int     kp = u & 31;
        const int     d0 = 8 * (u >> 5);
        const int64_t r0 = static_cast<int64_t>(rows(2 * kp)) * hkv + kvh;
        const int64_t r1 = static_cast<int64_t>(rows(2 * kp + 1)) * hkv + kvh;
        r.a[rep]  = *reinterpret_cast<const u32x2*>(v + r0 * kHD + d0);
        r.b[rep]  = *reinterpret_cast<const u32x2*>(v + r1 * kHD + d0);
        r.sa[rep] = vs[r0];
        r.sb[rep] = vs[r1];
    }
    r.ks = ks[static_cast<int64_t>(rows(tid & (kBN - 1))) * hkv + kvh];
}

// Exponent field of x alone: 2^floor(log2 x) for normal x > 0, 0 for 0.
__device__ __forceinline__ uint32_t pow2_bits(float x) {
    return __float_as_uint(x) & 0x7f800000u;
}

// Writes V'^T = f16(code * v_scale) for the staged units and the k_scale
// factors of the tile. The two keys of a unit share the larger power of two
// 2^e of their scales, applied exactly by the converter; the f16 factors
// v_scale / 2^e (rounded once per key, a relative error below 2^-11 that
// enters O linearly) are applied with one packed f16 multiply.
template <int kThreads>
__device__ __forceinline__ void v_tile_stage(const VRaw<4096 / 8 / kThreads>& r, uint16_t* vt,
                                             float* kf, int tid, float scale_log2) {
    constexpr int kReps = 4096 / 8 / kThreads;
#pragma unroll
    for (int rep = 0; rep < kReps; ++rep) {
        const int      u   = tid + rep * kThreads;
        const int      kp  = u & 31;
        const int      d0  = 8 * (u >> 5);
        const uint32_t e   = max(pow2_bits(r.sa[rep]), pow2_bits(r.sb[rep]));
        const float    p   = __uint_as_float(e);
        const float    inv = __uint_as_float(0x7f000000u - e);   // 2^-e
        const f16x2    m   = {static_cast<_Float16>(r.sa[rep] * inv),
                              static_cast<_Float16>(r.sb[rep] * inv)};
        uint32_t*      col = reinterpret_cast<uint32_t*>(vt + vt_pos(2 * kp));
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const uint32_t wa = half ? r.a[rep].y : r.a[rep].x;
            const uint32_t wb = half ? r.b[rep].y : r.b[rep].x;
            // [a0 b0 a1 b1] and [a2 b2 a3 b3]: the two keys of one d per word.
            const uint32_t lo = __builtin_amdgcn_perm(wb, wa, 0x05010400u);
            const uint32_t hi = __builtin_amdgcn_perm(wb, wa, 0x07030602u);
            const int      d  = d0 + 4 * half;
            const f16x2 x0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, p, false) * m;
            const f16x2 x1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, p, true) * m;
            const f16x2 x2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, p, false) * m;
            const f16x2 x3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, p, true) * m;
            col[(d + 0) * (kVPitch / 2)] = __builtin_bit_cast(uint32_t, x0);
            col[(d + 1) * (kVPitch / 2)] = __builtin_bit_cast(uint32_t, x1);
            col[(d + 2) * (kVPitch / 2)] = __builtin_bit_cast(uint32_t, x2);
            col[(d + 3) * (kVPitch / 2)] = __builtin_bit_cast(uint32_t, x3);
        }
    }
    if (tid < kBN) {
        kf[tid] = r.ks * scale_log2;
    }
}

// Four fp32 -> four E4M3 bytes (RNE; inputs within range).
__device__ __forceinline__ uint32_t pack_e4m3x4(float a, float b, float c, float d) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
}

// Workgroup barrier that orders LDS accesses only: waits for this wave's LDS
// operations, not for its outstanding global loads.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// s_waitcnt immediate (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt
// 6:4, lgkmcnt 11:8) waiting until at most n vector-memory operations are
// outstanding, and for nothing else.
constexpr int waitcnt_vm(int n) {
    return (n & 0xf) | (0x7 << 4) | (0xf << 8) | ((n >> 4) << 14);
}

// kEarly (4-wave workgroups, four or more row blocks per head): the first two
// tiles' K copies and V loads go out before the q load, and q's eight loads
// go out together, so the prologue waits for one memory round trip instead of
// three. Smaller grids, the key split and the 8-wave kernel keep the order
// below (measured slower there, or spilling).
// kPart (4-wave workgroups): the keys are split over gridDim.y workgroups per
// (row block, q head); workgroup y takes the y-th run of
// max(ceil(tiles / S), kPartMinTiles) key tiles and stores its rows'
// partials (m in log2 units, l, unnormalized O) in the split-K decode layout
// ([rows, S] m, [rows, S] l, [rows, S, D] O, rows t * Hq + h) for the decode
// merge; a row with no key in the run stores m = -inf, l = 0 and, in a
// workgroup that has keys, O = 0 (a workgroup without keys leaves O unwritten;
// the merge drops slots with m = -inf). When run 0 holds every key (at most
// kPartMinTiles tiles in all), it stores the normalized output instead and
// the merge returns at once.
constexpr int kPartMinTiles = 8;   // a run's minimum: short caches use few runs
template <int kWaves, bool kPaged, bool kSplit = false, bool kEarly = false, bool kPart = false>
__global__ __launch_bounds__(kWaves * kWave, kSplit ? 1 : 2) void flash_prefill_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ q,
    const uint8_t* __restrict__ k, const uint8_t* __restrict__ v,
    const float* __restrict__ ks, const float* __restrict__ vs, int n_new,
    const int* __restrict__ cache_len, int hq, int hkv, float scale_log2,
    const int* __restrict__ block_table, int block_shift, bool one_round,
    float* __restrict__ partial, int num_splits) {
    static_assert(!kSplit || kWaves == 8, "the key split pairs two 4-wave halves");
    static_assert(!kEarly || (kWaves == 4 && !kSplit), "early issue: 4-wave workgroups only");
    static_assert(!kPart || (kWaves == 4 && !kSplit && !kEarly), "key runs: 4-wave workgroups");
    constexpr int kThreads = kWaves * kWave;
    constexpr int kRowWaves = kSplit ? 4 : kWaves;  // waves with distinct rows
    constexpr int kBM      = 32 * kRowWaves;        // query rows per workgroup
    // Threads of one tile pipeline (the whole workgroup, or one split half).
    constexpr int kPThreads = kSplit ? kThreads / 2 : kThreads;
    constexpr int kReps    = 4096 / 8 / kPThreads;  // V staging units per thread
    // Vector-memory operations of one v_tile_load (4 per unit, 1 k_scale).
    constexpr int kWaitAllButVLoads = waitcnt_vm(4 * kReps + 1);

    // Separate arrays per buffer (not one indexed array), so that the
    // compiler sees the LDS-DMA into one K buffer and the operand reads from
    // the other as independent and does not wait for the DMA before them.
    __shared__ __attribute__((aligned(16))) uint8_t  sK0[kKTile];
    __shared__ __attribute__((aligned(16))) uint8_t  sK1[kKTile];
    __shared__ __attribute__((aligned(16))) uint8_t  sK2[kKTile];   // 8-wave path only
    __shared__ __attribute__((aligned(16))) uint8_t  sK3[kKTile];   // 8-wave path only
    __shared__ __attribute__((aligned(16))) uint16_t sVt0[kHD * kVPitch];
    __shared__ __attribute__((aligned(16))) uint16_t sVt1[kHD * kVPitch];
    __shared__ __attribute__((aligned(16))) float    sKf0[kBN];
    __shared__ __attribute__((aligned(16))) float    sKf1[kBN];
    __shared__ __attribute__((aligned(16))) uint16_t sVt2[kHD * kVPitch];   // not 4-wave
    __shared__ __attribute__((aligned(16))) uint16_t sVt3[kHD * kVPitch];   // not 4-wave
    __shared__ __attribute__((aligned(16))) float    sKf2[kBN];             // key split only
    __shared__ __attribute__((aligned(16))) float    sKf3[kBN];             // key split only

    const int tid  = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid & (kWave - 1);
    const int qn   = lane & 31;   // query row of this lane within the wave
    const int h    = lane >> 5;   // k-group

    // Heavy (last) row blocks first; q heads of one kv head on one XCD. When
    // the whole grid is resident at once (one_round, two workgroups per
    // compute unit), the second half of the grid runs the light blocks in
    // ascending order, so the two workgroups sharing a compute unit pair a
    // heavy block with a light one.
    const int n_blk    = (n_new + kBM - 1) / kBM;
    const int bid      = static_cast<int>(blockIdx.x);
    const int half_wgs = (n_blk / 2) * hq;
    const int blk      = (one_round && bid >= half_wgs) ? (bid - half_wgs) / hq
                                                        : n_blk - 1 - bid / hq;
    const int hb    = bid % hq;
    const int qh    = ((hq & 7) == 0) ? ((hb & 7) * (hq >> 3) + (hb >> 3)) : hb;
    const int kvh   = qh / (hq / hkv);

    const int clen    = *cache_len;
    const int total   = clen + n_new;
    const int q0      = blk * kBM;
    const int last    = min(q0 + kBM, n_new) - 1;
    const int n_tiles = min((total + kBN - 1) / kBN, (clen + last) / kBN + 1);
    // kPart: this workgroup's run of key tiles [kt_lo, kt_hi).
    [[maybe_unused]] int  kt_lo   = 0;
    [[maybe_unused]] int  kt_hi   = 0;
    [[maybe_unused]] bool one_run = false;   // kPart: run 0 holds every key
    if constexpr (kPart) {
        const int tiles_all = (total + kBN - 1) / kBN;
        const int per       = max((tiles_all + num_splits - 1) / num_splits, kPartMinTiles);
        one_run             = tiles_all <= per;
        kt_lo               = static_cast<int>(blockIdx.y) * per;
        kt_hi               = min(kt_lo + per, n_tiles);
        if (kt_hi <= kt_lo) {   // no key of this run for any row of the block: m, l only
            const int r = q0 + tid;
            if (!one_run && tid < kBM && r < n_new) {
                const int64_t rows = static_cast<int64_t>(n_new) * hq;
                const int64_t slot = (static_cast<int64_t>(r) * hq + qh) * num_splits +
                                     static_cast<int64_t>(blockIdx.y);
                partial[slot]                     = -INFINITY;
                partial[rows * num_splits + slot] = 0.0f;
            }
            return;
        }
    }

    // Key split: waves w and w + 4 hold the same rows; half g = w / 4 runs
    // the key tiles kt = g, g + 2, g + 4, ... and the halves merge at the end.
    const int split_g = kSplit ? (wave >> 2) : 0;
    const int first_kt = kPart ? kt_lo : split_g;   // a wave's first tile
    const int wq0     = q0 + (kSplit ? (wave & 3) : wave) * 32;   // first row of this wave
    const int wlast   = min(wq0 + 31, n_new - 1);    // may be < wq0 (idle wave)
    const int w_tiles = (wlast < wq0) ? 0 : (clen + wlast) / kBN + 1;
    const int my_q    = wq0 + qn;
    const int my_pos  = clen + my_q;

    [[maybe_unused]] VRaw<kReps> pre_raw0, pre_raw1;
    if constexpr (kEarly) {
        const TileRows<kPaged> r0(0, total, block_table, block_shift);
        const TileRows<kPaged> r1(kBN, total, block_table, block_shift);
        k_tile_dma<kPThreads>(sK0, k, r0, kvh, hkv, tid);
        v_tile_load<kPThreads>(pre_raw0, v, ks, vs, r0, kvh, hkv, tid);
        k_tile_dma<kPThreads>(sK1, k, r1, kvh, hkv, tid);
        v_tile_load<kPThreads>(pre_raw1, v, ks, vs, r1, kvh, hkv, tid);
    }
    // Q^T (B operand) as hi + lo E4M3 parts. Lane (row my_q, group h) holds,
    // for k-step j, d = 64j + 32h .. +32 (the same d the K operand lanes of
    // group h hold, so the MFMA pairs matching d).
    i32x8 qhi[2], qlo[2];
    int   sc_hi, sc_lo;
    {
        const bool      has = my_q < n_new;
        const uint16_t* qr  = q + (static_cast<int64_t>(has ? my_q : 0) * hq + qh) * kHD;
        float           x[2][32];
        float           amax = 0.0f;
        [[maybe_unused]] u32x4 qraw[2][4];
        if constexpr (kEarly) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    qraw[j][c] = *reinterpret_cast<const u32x4*>(qr + 64 * j + 32 * h + 8 * c);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                u32x4 w;
                if constexpr (kEarly) {
                    w = qraw[j][c];
                } else {
                    w = *reinterpret_cast<const u32x4*>(qr + 64 * j + 32 * h + 8 * c);
                }
                if (!has) {
                    w = u32x4{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[j][8 * c + 2 * i]     = __uint_as_float(w[i] << 16);
                    x[j][8 * c + 2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
                    amax = fmaxf(amax, fmaxf(fabsf(x[j][8 * c + 2 * i]),
                                             fabsf(x[j][8 * c + 2 * i + 1])));
                }
            }
        }
        amax = wave_xor_max(amax, 32);
        // 2^a with amax * 2^a in [128, 256); a zero row keeps a = 0.
        // (a is clamped so that 2^a, 2^-a and 2^(-a-4) stay normal: only rows
        // with max |q| below 2^-116 land under 128.)
        const int a = (amax > 0.0f)
                          ? min(max(7 - (static_cast<int>(pow2_bits(amax) >> 23) - 127), -120), 123)
                          : 0;
        const float s2a = __uint_as_float(static_cast<uint32_t>(127 + a) << 23);
        sc_hi = kE8M0One - a;
        sc_lo = kE8M0One - a - 4;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                float y[4], r[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    y[i] = x[j][4 * w + i] * s2a;
                }
                const uint32_t hw = pack_e4m3x4(y[0], y[1], y[2], y[3]);
                const f32x2    h0 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(hw), false);
                const f32x2    h1 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(hw), true);
                r[0] = (y[0] - h0.x) * 16.0f;
                r[1] = (y[1] - h0.y) * 16.0f;
                r[2] = (y[2] - h1.x) * 16.0f;
                r[3] = (y[3] - h1.y) * 16.0f;
                qhi[j][w] = static_cast<int>(hw);
                qlo[j][w] = static_cast<int>(pack_e4m3x4(r[0], r[1], r[2], r[3]));
            }
        }
    }

    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o[i] = f32x16{};
    }
    float m_ref = 0.0f;   // lazy reference maximum of this lane's row (log2 units)
    float l_run = 0.0f;

    // S^T = K Q^T for one tile: per 32-key block, two k-steps of 64 d, each
    // as hi and lo MFMAs sharing the K operand; all eight K operand reads are
    // issued before the first MFMA.
    auto qk = [&](const uint8_t* kbuf, f32x16 (&sc)[2]) {
        i32x8 ka[2][2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int r = 32 * kb + qn;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int   c0 = 4 * j + 2 * h;
                const u32x4 lo = *reinterpret_cast<const u32x4*>(kbuf + k_chunk(r, c0));
                const u32x4 hi = *reinterpret_cast<const u32x4*>(kbuf + k_chunk(r, c0 + 1));
                ka[kb][j] = i32x8{static_cast<int>(lo.x), static_cast<int>(lo.y),
                                  static_cast<int>(lo.z), static_cast<int>(lo.w),
                                  static_cast<int>(hi.x), static_cast<int>(hi.y),
                                  static_cast<int>(hi.z), static_cast<int>(hi.w)};
            }
        }
        sc[0] = f32x16{};
        sc[1] = f32x16{};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                sc[kb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    ka[kb][j], qhi[j], sc[kb], 0, 0, 0, kE8M0One, 0, sc_hi);
            }
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                sc[kb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    ka[kb][j], qlo[j], sc[kb], 0, 0, 0, kE8M0One, 0, sc_lo);
            }
        }
    };
    // Softmax of tile kt's scores (in place) into the P^T operands:
    // t = s * (k_scale * scale * log2 e) - m_ref (register r of block kb is key
    // 32kb + 8(r/4) + 4h + r%4 of the tile), the causal / key-end mask only on
    // tiles that cross the diagonal or the end of the keys (a wave-uniform
    // branch), e = 2^t in fp32, p = e rounded to f16 for the P V MFMAs, and
    // the row sum of the fp32 e (four partial sums of VALU adds, as the
    // reference sums its fp32 exponentials; a v_dot2c sum of the f16 p runs on
    // the MFMA pipe and measured ~1 % slower; the key-split kernel keeps that
    // form for its register budget). Lazy reference maximum (exact): m_ref moves to the row
    // maximum only on a wave's first tile or when a row sum exceeds 2^15 (some
    // score more than 15 above m_ref); otherwise the tile needs no max
    // reduction, no cross-lane step and no rescale of l and O. Every p and l
    // use the same m_ref, and p <= 2^15 keeps every p inside the f16 range.
    // The k-factors of the 32 keys a lane holds, read before the score MFMAs
    // so that the LDS latency hides behind them.
    auto load_kf = [&](const float* kfb, f32x4 (&kfv)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            kfv[i] = *reinterpret_cast<const f32x4*>(kfb + 32 * (i >> 2) + 8 * (i & 3) + 4 * h);
        }
    };
    auto softmax = [&](f32x16 (&sx)[2], const f32x4 (&kfv)[8], int kt, f16x8 (&pop)[4]) {
        __builtin_amdgcn_s_setprio(1);
        const int key0 = kt * kBN;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const f32x4 f = kfv[4 * kb + rg];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sx[kb][4 * rg + e] = fmaf(sx[kb][4 * rg + e], f[e], -m_ref);
                }
            }
        }
        if ((key0 + kBN - 1 > clen + wq0) || (key0 + kBN > total)) {
            // Key kp is visible iff kp <= min(my_pos, total - 1): one compare
            // of the tile offset (a constant per register) against a per-lane
            // threshold.
            const int lim = min(my_pos, total - 1) - key0 - 4 * h;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    if (32 * kb + 8 * (r >> 2) + (r & 3) > lim) {
                        sx[kb][r] = -INFINITY;
                    }
                }
            }
        }
        float psum  = 0.0f;
        auto  exp_p = [&]() {
            float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    f16x8 pw;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int   r  = 8 * half + 2 * i;
                        const float e0 = __builtin_amdgcn_exp2f(sx[kb][r]);
                        const float e1 = __builtin_amdgcn_exp2f(sx[kb][r + 1]);
                        const f16x2 pp = {static_cast<_Float16>(e0), static_cast<_Float16>(e1)};
                        if constexpr (kSplit) {
                            // The key-split kernel sits at 256 VGPRs; the fp32
                            // sum would spill there.
                            part[i] = __builtin_amdgcn_fdot2(pp, f16x2{1.0f16, 1.0f16},
                                                             part[i], false);
                        } else {
                            part[i] += e0 + e1;
                        }
                        pw[2 * i]     = pp.x;
                        pw[2 * i + 1] = pp.y;
                    }
                    pop[2 * kb + half] = pw;
                }
            }
            psum = (part[0] + part[1]) + (part[2] + part[3]);
        };
        exp_p();
        if (__any((kt == first_kt) || !(psum <= 0x1p15f))) {
            float tmax = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    tmax = fmaxf(tmax, sx[kb][r]);
                }
            }
            tmax = wave_xor_max(tmax, 32);
            // The first tile sets the reference; later tiles only raise it. A
            // row that is here because another row of the wave overflowed may
            // sit far below its reference: lowering it would scale O and l by
            // 2^-tmax, which overflows.
            const float delta = (kt == first_kt) ? ((tmax == -INFINITY) ? 0.0f : tmax)
                                          : fmaxf(tmax, 0.0f);
            const float alpha = (kt == first_kt) ? 1.0f : __builtin_amdgcn_exp2f(-delta);
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                sx[kb] -= delta;
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
        __builtin_amdgcn_s_setprio(0);
    };
    // O^T += V^T P^T, the operand reads running four MFMAs ahead.
    // The softmax and the P V run at wave priority 1, the score MFMAs and
    // the copies at 0: when both waves of a SIMD can issue, the one past its
    // scores goes first (measured +3 % at 4K-16K; priority on the scores
    // instead: -7 %).
    auto pv = [&](const uint16_t* vtb, const f16x8 (&pop)[4]) {
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const uint16_t* arow = vtb + (32 * db + qn) * kVPitch + 8 * h;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const f16x8 va = *reinterpret_cast<const f16x8*>(arow + 16 * t);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pop[t], o[db], 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 2);
#pragma unroll
        for (int i = 0; i < 12; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 2);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 2);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 2);
        __builtin_amdgcn_s_setprio(0);
    };

    if constexpr (kWaves == 8 && !kSplit) {
        // The two waves sharing a SIMD (w and w + 4) run each tile in
        // different phase orders so that one's softmax (VALU) meets the
        // other's MFMAs: the early group (waves 0-3) copies the next K tile
        // and does scores, softmax, P V of tile kt; the late group (waves
        // 4-7) does P V of tile kt - 1 (its P kept in registers across the
        // barrier), scores and softmax of tile kt, then stages V(kt + 1) into
        // the fourth V^T buffer of a ring of four.
        const bool late = wave >= kWaves / 2;
        const int  gtid = tid & (kThreads / 2 - 1);   // thread index within the group

        constexpr int kGThreads = kThreads / 2;
        constexpr int kGReps    = 4096 / 8 / kGThreads;
        // K codes go through a ring of four buffers, copied two tiles ahead.
        // Prologue: tile 0 staged by everyone, K(1) copied; V(1) into the
        // late group's registers.
        VRaw<kGReps> raw0, raw1;
        {
            const TileRows<kPaged> r0(0, total, block_table, block_shift);
            const TileRows<kPaged> r1(kBN, total, block_table, block_shift);
            k_tile_dma<kThreads>(sK0, k, r0, kvh, hkv, tid);
            k_tile_dma<kThreads>(sK1, k, r1, kvh, hkv, tid);
            VRaw<kReps> rz;
            v_tile_load<kThreads>(rz, v, ks, vs, r0, kvh, hkv, tid);
            v_tile_stage<kThreads>(rz, sVt0, sKf0, tid, scale_log2);
            if (late) {
                const TileRows<kPaged> r1(kBN, total, block_table, block_shift);
                v_tile_load<kGThreads>(raw1, v, ks, vs, r1, kvh, hkv, gtid);
            }
        }
        __syncthreads();

        auto kbuf4 = [&]<int R>() -> uint8_t* {
            if constexpr (R == 0) return sK0;
            else if constexpr (R == 1) return sK1;
            else if constexpr (R == 2) return sK2;
            else return sK3;
        };
        // V^T(kt) lives in buffer kt % 4: during tile kt the early group reads
        // V^T(kt), the late group reads V^T(kt - 1) and then stages
        // V^T(kt + 1), so the staging never writes a buffer that another
        // wave of its group may still be reading.
        auto vbuf4 = [&]<int R>() -> uint16_t* {
            if constexpr (R == 0) return sVt0;
            else if constexpr (R == 1) return sVt1;
            else if constexpr (R == 2) return sVt2;
            else return sVt3;
        };
        if (!late) {
            constexpr int kDmaOps = kKTile / 16 / kGThreads;   // copies issued per tile
            // Rows of the tile two ahead, looked up (paged) one tile before use.
            TileRows<kPaged> rn(2 * kBN, total, block_table, block_shift);
            auto tile = [&]<int R>(int kt) {
                constexpr int  B    = R & 1;
                const uint8_t* kcur = kbuf4.template operator()<R>();
                uint8_t*       nk   = kbuf4.template operator()<(R + 2) & 3>();
                const float*   kfb  = B ? sKf1 : sKf0;
                const uint16_t* vtb = vbuf4.template operator()<R>();
                const TileRows<kPaged> r2 = rn;
                rn = TileRows<kPaged>((kt + 3) * kBN, total, block_table, block_shift);
                k_tile_dma<kGThreads>(nk, k, r2, kvh, hkv, gtid);
                if (kt < w_tiles) {
                    f32x16 sx[2];
                    f16x8  pop[4];
                    f32x4  kfv[8];
                    load_kf(kfb, kfv);
                    qk(kcur, sx);
                    softmax(sx, kfv, kt, pop);
                    pv(vtb, pop);
                }
                // K(kt + 1), copied during the previous tile, must have landed;
                // this tile's copy of K(kt + 2) stays in flight.
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(kDmaOps));
                lds_barrier();
            };
            for (int kt = 0; kt < n_tiles; kt += 4) {
                tile.template operator()<0>(kt);
                if (kt + 1 < n_tiles) tile.template operator()<1>(kt + 1);
                if (kt + 2 < n_tiles) tile.template operator()<2>(kt + 2);
                if (kt + 3 < n_tiles) tile.template operator()<3>(kt + 3);
            }
        } else {
            f16x8 pop_keep[4];
            TileRows<kPaged> rn(2 * kBN, total, block_table, block_shift);
            auto  tile = [&]<int R>(int kt) {
                constexpr int  B     = R & 1;
                const uint8_t* kcur  = kbuf4.template operator()<R>();
                const float*   kfb   = B ? sKf1 : sKf0;
                uint16_t*      vprev = vbuf4.template operator()<(R + 3) & 3>();   // V^T(kt - 1)
                uint16_t*      vnext = vbuf4.template operator()<(R + 1) & 3>();   // V^T(kt + 1)
                float*         nkf   = B ? sKf0 : sKf1;
                VRaw<kGReps>&  rawc  = B ? raw1 : raw0;
                VRaw<kGReps>&  rawn  = B ? raw0 : raw1;
                const TileRows<kPaged> r2 = rn;
                rn = TileRows<kPaged>((kt + 3) * kBN, total, block_table, block_shift);
                if (kt >= 1 && kt - 1 < w_tiles) {
                    pv(vprev, pop_keep);
                }
                v_tile_load<kGThreads>(rawc, v, ks, vs, r2, kvh, hkv, gtid);
                if (kt < w_tiles) {
                    f32x16 sx[2];
                    f32x4  kfv[8];
                    load_kf(kfb, kfv);
                    qk(kcur, sx);
                    softmax(sx, kfv, kt, pop_keep);
                }
                v_tile_stage<kGThreads>(rawn, vnext, nkf, gtid, scale_log2);
                lds_barrier();
            };
            for (int kt = 0; kt < n_tiles; kt += 4) {
                tile.template operator()<0>(kt);
                if (kt + 1 < n_tiles) tile.template operator()<1>(kt + 1);
                if (kt + 2 < n_tiles) tile.template operator()<2>(kt + 2);
                if (kt + 3 < n_tiles) tile.template operator()<3>(kt + 3);
            }
            // P V of the last tile.
            if (n_tiles - 1 < w_tiles) {
                switch ((n_tiles - 1) & 3) {
                    case 0: pv(sVt0, pop_keep); break;
                    case 1: pv(sVt1, pop_keep); break;
                    case 2: pv(sVt2, pop_keep); break;
                    default: pv(sVt3, pop_keep); break;
                }
            }
        }
    } else {
    // One tile pipeline per half G (the whole workgroup unless key split):
    // the stream of tiles G, G + kStride, G + 2 kStride, ... Each half has its
    // own LDS buffers; both halves take the same number of barriers.
    constexpr int kStride = kSplit ? 2 : 1;
    const int     ptid    = tid & (kPThreads - 1);   // thread index within the pipeline
    auto pipeline = [&]<int G>() {
    // V staging registers, two sets: raw0 holds the even tiles, raw1 the odd
        // ones, so the loads of tile kt + 2 go out a whole tile before the
        // staging of tile kt + 1 needs its registers.
        // Prologue: the stream's first tile staged, the second's K copied
        // and V in raw1. (Tile "kt + 1" below is the stream's next tile,
        // kt + kStride.)
        VRaw<kReps> raw0, raw1;
        const int t0 = kPart ? kt_lo : G;   // the stream's first tile
        {
            const TileRows<kPaged> r0(t0 * kBN, total, block_table, block_shift);
            const TileRows<kPaged> r1((t0 + kStride) * kBN, total, block_table, block_shift);
            if constexpr (kEarly) {
                raw0 = pre_raw0;
                raw1 = pre_raw1;
                v_tile_stage<kPThreads>(raw0, sVt0, sKf0, ptid, scale_log2);
            } else {
                k_tile_dma<kPThreads>(G ? sK2 : sK0, k, r0, kvh, hkv, ptid);
                v_tile_load<kPThreads>(raw0, v, ks, vs, r0, kvh, hkv, ptid);
                v_tile_stage<kPThreads>(raw0, G ? sVt2 : sVt0, G ? sKf2 : sKf0, ptid, scale_log2);
                k_tile_dma<kPThreads>(G ? sK3 : sK1, k, r1, kvh, hkv, ptid);
                v_tile_load<kPThreads>(raw1, v, ks, vs, r1, kvh, hkv, ptid);
            }
        }
        __syncthreads();

        // Rows of the tiles one and two ahead, looked up (paged) a tile
        // before use.
        TileRows<kPaged> rn1((t0 + kStride) * kBN, total, block_table, block_shift);
        TileRows<kPaged> rn2((t0 + 2 * kStride) * kBN, total, block_table, block_shift);
        // One tile from buffer B (static, so each buffer is a distinct array).
        auto tile = [&]<int B>(int kt) {
            uint8_t*  kb0 = G ? sK2 : sK0;
            uint8_t*  kb1 = G ? sK3 : sK1;
            uint16_t* vb0 = G ? sVt2 : sVt0;
            uint16_t* vb1 = G ? sVt3 : sVt1;
            float*    fb0 = G ? sKf2 : sKf0;
            float*    fb1 = G ? sKf3 : sKf1;
            uint8_t*  kt_s = B ? kb1 : kb0;
            uint16_t* vt   = B ? vb1 : vb0;
            float*    kf   = B ? fb1 : fb0;
            uint8_t*  nk   = B ? kb0 : kb1;
            uint16_t* nvt  = B ? vb0 : vb1;
            float*    nkf  = B ? fb0 : fb1;
            // On entry V(kt + 1) is in registers rawn (loaded during tile
            // kt - 1). This tile copies K(kt + 1) into K buffer 1 - B, loads
            // V(kt + 2) into rawc (issued after the copy, so that waiting for
            // all but the V loads at the barrier covers the copy) and stages
            // V(kt + 1) into V^T buffer 1 - B. Past the end the copies repeat
            // the last tile into idle buffers, which nobody reads; doing them
            // unconditionally keeps the copies and the staging in the same
            // scheduling regions as the MFMAs, whose execution hides their VALU
            // work.
            VRaw<kReps>& rawc = B ? raw1 : raw0;
            VRaw<kReps>& rawn = B ? raw0 : raw1;
            const TileRows<kPaged> r1 = rn1;
            const TileRows<kPaged> r2 = rn2;
            rn1 = rn2;
            rn2 = TileRows<kPaged>((kt + 3 * kStride) * kBN, total, block_table, block_shift);
            if (kt < w_tiles) {
                k_tile_dma<kPThreads>(nk, k, r1, kvh, hkv, ptid);
                v_tile_load<kPThreads>(rawc, v, ks, vs, r2, kvh, hkv, ptid);

                // S^T = K Q^T: per 32-key block, two k-steps of 64 d, each as
                // hi and lo MFMAs sharing the K operand.
                f32x16 s[2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    s[kb] = f32x16{};
                    const int r = 32 * kb + qn;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int c0 = 4 * j + 2 * h;
                        const u32x4 lo = *reinterpret_cast<const u32x4*>(kt_s + k_chunk(r, c0));
                        const u32x4 hi = *reinterpret_cast<const u32x4*>(kt_s + k_chunk(r, c0 + 1));
                        const i32x8 ka = {static_cast<int>(lo.x), static_cast<int>(lo.y),
                                          static_cast<int>(lo.z), static_cast<int>(lo.w),
                                          static_cast<int>(hi.x), static_cast<int>(hi.y),
                                          static_cast<int>(hi.z), static_cast<int>(hi.w)};
                        s[kb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            ka, qhi[j], s[kb], 0, 0, 0, kE8M0One, 0, sc_hi);
                        s[kb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            ka, qlo[j], s[kb], 0, 0, 0, kE8M0One, 0, sc_lo);
                    }
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // global load
                }

                f16x8 pop[4];
                f32x4 kfv[8];
                load_kf(kf, kfv);
                softmax(s, kfv, kt, pop);

                // O^T += V^T P^T.
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const uint16_t* arow = vt + (32 * db + qn) * kVPitch + 8 * h;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const f16x8 va = *reinterpret_cast<const f16x8*>(arow + 16 * t);
                        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pop[t], o[db], 0, 0, 0);
                    }
                }
                v_tile_stage<kPThreads>(rawn, nvt, nkf, ptid, scale_log2);
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);   // LDS read
                    __builtin_amdgcn_sched_group_barrier(0x002, 2, 1);   // VALU
                    __builtin_amdgcn_sched_group_barrier(0x200, 1, 1);   // LDS write
                }
            } else {
                k_tile_dma<kPThreads>(nk, k, r1, kvh, hkv, ptid);
                v_tile_load<kPThreads>(rawc, v, ks, vs, r2, kvh, hkv, ptid);
                v_tile_stage<kPThreads>(rawn, nvt, nkf, ptid, scale_log2);
            }
            // K(kt + 1) must have landed and the staged LDS writes be visible
            // before the next tile; the V loads of tile kt + 2 stay in flight.
            __builtin_amdgcn_s_waitcnt(kWaitAllButVLoads);
            lds_barrier();
        };

        const int n_steps = kPart ? kt_hi - kt_lo : (n_tiles + kStride - 1) / kStride;
        for (int i = 0; i < n_steps; i += 2) {
            tile.template operator()<0>(t0 + kStride * i);
            if (i + 1 < n_steps) {
                tile.template operator()<1>(t0 + kStride * (i + 1));
            }
        }
    };
    if constexpr (kSplit) {
        if (split_g == 0) {
            pipeline.template operator()<0>();
        } else {
            pipeline.template operator()<1>();
        }
        // Merge of the halves: half 1 leaves O, m_ref and its lane's l in LDS
        // (the tile buffers, free after the barrier), half 0 rescales both to
        // the larger reference and stores. A half that saw no key of a row
        // (row sum 0) has weight 0.
        __syncthreads();
        // The merge reuses the tile buffers: each V^T buffer holds one d block
        // of O (16 floats per thread), sK0 holds m_ref and l of every thread.
        static_assert(kHD * kVPitch * sizeof(uint16_t) >= 16 * kPThreads * sizeof(float),
                      "a V^T buffer must hold a d block of O for every thread");
        static_assert(kKTile >= 2 * kPThreads * sizeof(float),
                      "a K buffer must hold m_ref and l for every thread");
        float* mo[4] = {reinterpret_cast<float*>(sVt0), reinterpret_cast<float*>(sVt1),
                        reinterpret_cast<float*>(sVt2), reinterpret_cast<float*>(sVt3)};
        float* ml    = reinterpret_cast<float*>(sK0);   // [256] m_ref, [256] l
        if (split_g == 1) {
#pragma unroll
            for (int db = 0; db < 4; ++db) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    mo[db][r * kPThreads + ptid] = o[db][r];
                }
            }
            ml[ptid]             = m_ref;
            ml[kPThreads + ptid] = l_run;
        }
        __syncthreads();
        if (split_g == 1) {
            return;
        }
        const float m1   = ml[ptid];
        const float l1   = ml[kPThreads + ptid];
        const bool  use1 = wave_xor_sum(l1, 32) > 0.0f;
        const float mm   = use1 ? fmaxf(m_ref, m1) : m_ref;
        const float f0   = __builtin_amdgcn_exp2f(m_ref - mm);
        const float f1   = use1 ? __builtin_amdgcn_exp2f(m1 - mm) : 0.0f;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                o[db][r] = o[db][r] * f0 + mo[db][r * kPThreads + ptid] * f1;
            }
        }
        l_run = l_run * f0 + l1 * f1;
    } else {
        pipeline.template operator()<0>();
    }
    }

    const float l_tot = wave_xor_sum(l_run, 32);
    // kPart with a single live run (short caches): run 0 stores the output
    // itself, as the plain kernel does, and the merge skips the call.
    if (kPart && !one_run) {
        if (my_q < n_new) {
            const int64_t rows   = static_cast<int64_t>(n_new) * hq;
            const int64_t slot   = (static_cast<int64_t>(my_q) * hq + qh) * num_splits +
                                 static_cast<int64_t>(blockIdx.y);
            const bool    any    = l_tot > 0.0f;
            float*        part_o = partial + 2 * rows * num_splits + slot * kHD;
            if (h == 0) {
                partial[slot]                     = any ? m_ref : -INFINITY;
                partial[rows * num_splits + slot] = l_tot;
            }
#pragma unroll
            for (int db = 0; db < 4; ++db) {
#pragma unroll
                for (int rg = 0; rg < 4; ++rg) {
                    *reinterpret_cast<f32x4*>(part_o + 32 * db + 8 * rg + 4 * h) =
                        any ? f32x4{o[db][4 * rg], o[db][4 * rg + 1], o[db][4 * rg + 2],
                                    o[db][4 * rg + 3]}
                            : f32x4{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
        return;
    }
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

template <int kWaves, bool kSplit = false>
void launch_prefill(uint16_t* out, const uint16_t* q, const uint8_t* k, const uint8_t* v,
                    const float* k_scale, const float* v_scale, int n_new, const int* cache_len,
                    int hq, int hkv, float scale_log2, hipStream_t stream,
                    const int* block_table, int block_shift, bool one_round) {
    constexpr int kBM   = 32 * (kSplit ? 4 : kWaves);
    const int     n_blk = (n_new + kBM - 1) / kBM;
    const dim3    grid(static_cast<unsigned>(n_blk * hq));
    // 4-wave grids of four or more row blocks per head: the early-issue
    // prologue (+4-6 % at n = 2048-3072, 32 heads); grids of one to three
    // blocks (n <= 384) keep the plain prologue (4-6 % faster there).
    constexpr bool kEarlyOk = (kWaves == 4 && !kSplit);
    const bool     early    = kEarlyOk && n_blk >= 4;
    if (block_table != nullptr) {
        if (early) {
            hipLaunchKernelGGL((flash_prefill_kernel<kWaves, true, kSplit, kEarlyOk>), grid,
                               dim3(kWaves * kWave), 0, stream, out, q, k, v, k_scale, v_scale,
                               n_new, cache_len, hq, hkv, scale_log2, block_table, block_shift,
                               one_round, nullptr, 1);
        } else {
            hipLaunchKernelGGL((flash_prefill_kernel<kWaves, true, kSplit>), grid,
                               dim3(kWaves * kWave), 0, stream, out, q, k, v, k_scale, v_scale,
                               n_new, cache_len, hq, hkv, scale_log2, block_table, block_shift,
                               one_round, nullptr, 1);
        }
    } else {
        if (early) {
            hipLaunchKernelGGL((flash_prefill_kernel<kWaves, false, kSplit, kEarlyOk>), grid,
                               dim3(kWaves * kWave), 0, stream, out, q, k, v, k_scale, v_scale,
                               n_new, cache_len, hq, hkv, scale_log2, nullptr, 0, one_round,
                               nullptr, 1);
        } else {
            hipLaunchKernelGGL((flash_prefill_kernel<kWaves, false, kSplit>), grid,
                               dim3(kWaves * kWave), 0, stream, out, q, k, v, k_scale, v_scale,
                               n_new, cache_len, hq, hkv, scale_log2, nullptr, 0, one_round,
                               nullptr, 1);
        }
    }
}

// The flash prefill with its keys split over num_splits workgroups per (row
// block, q head), then the decode merge over the n_new * Hq rows.
template <bool kPaged>
hipError_t launch_prefill_part(uint16_t* out, const uint16_t* q, const uint8_t* k,
                               const uint8_t* v, const float* k_scale, const float* v_scale,
                               float* partial, int num_splits, int n_new, const int* cache_len,
                               int hq, int hkv, float scale_log2, hipStream_t stream,
                               const int* block_table, int block_shift) {
    constexpr int kBM   = 32 * 4;
    const int     n_blk = (n_new + kBM - 1) / kBM;
    const dim3    grid(static_cast<unsigned>(n_blk * hq), static_cast<unsigned>(num_splits));
    hipLaunchKernelGGL((flash_prefill_kernel<4, kPaged, false, false, true>), grid,
                       dim3(4 * kWave), 0, stream, out, q, k, v, k_scale, v_scale, n_new,
                       cache_len, hq, hkv, scale_log2, block_table, block_shift, false, partial,
                       num_splits);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return e;
    }
    return split_rows_merge_launch(out, partial, num_splits, cache_len, n_new * hq, n_new, kHD,
                                   stream, kPartMinTiles);
}

}  // namespace

hipError_t flash_prefill_keysplit_launch(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                         const uint8_t* v, const float* k_scale,
                                         const float* v_scale, float* partial, int num_splits,
                                         int n_new, const int* cache_len, int num_q_heads,
                                         int num_kv_heads, int head_dim, float scale,
                                         hipStream_t stream, const int* block_table,
                                         int block_shift) {
    if (head_dim != kHD) {
        return hipErrorInvalidValue;
    }
    const float sl = scale * kLog2e;
    return block_table != nullptr
               ? launch_prefill_part<true>(out, q, k, v, k_scale, v_scale, partial, num_splits,
                                           n_new, cache_len, num_q_heads, num_kv_heads, sl,
                                           stream, block_table, block_shift)
               : launch_prefill_part<false>(out, q, k, v, k_scale, v_scale, partial, num_splits,
                                            n_new, cache_len, num_q_heads, num_kv_heads, sl,
                                            stream, nullptr, 0);
}

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
    // 8-wave workgroups (256 rows, one per compute unit: half the staging
    // per wave) when the grid takes at least two rounds of them. Below that,
    // a compute unit holds too few waves to hide one tile's dependency chain
    // (~1.4 us per 64-key tile for a lone wave): grids of up to 1.5 rounds of
    // 128-row blocks, 4 blocks or more per head, split each block's keys over
    // two 4-wave halves of one workgroup (heaviest block: half the serial
    // tiles; 1500 x 24 heads 49 -> 36 us, 2048 x 24 50 us from 60); the rest
    // take 4-wave workgroups (128 rows, two per compute unit) with heavy/light
    // pairing, which balance the causal work of a single round better.
    int        cus = 0;
    hipError_t ce  = device_cu_count(&cus);
    if (ce != hipSuccess) {
        return ce;
    }
    const float sl       = scale * kLog2e;
    const int   n_blk128 = (n_new + 127) / 128;
    if (((n_new + 255) / 256) * num_q_heads >= 2 * cus) {
        launch_prefill<8>(out, q, k, v, k_scale, v_scale, n_new, cache_len, num_q_heads,
                          num_kv_heads, sl, stream, block_table, block_shift, false);
    } else if (n_blk128 >= 4 && 2 * n_blk128 * num_q_heads <= 3 * cus) {
        launch_prefill<8, true>(out, q, k, v, k_scale, v_scale, n_new, cache_len, num_q_heads,
                                num_kv_heads, sl, stream, block_table, block_shift, false);
    } else {
        const bool one_round = n_blk128 * num_q_heads <= 2 * cus;
        launch_prefill<4>(out, q, k, v, k_scale, v_scale, n_new, cache_len, num_q_heads,
                          num_kv_heads, sl, stream, block_table, block_shift, one_round);
    }
    return hipGetLastError();
}

}  // namespace rth
