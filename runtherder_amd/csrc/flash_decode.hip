// Split-K GQA flash decode over an OCP E4M3 KV cache, gfx950.
//
// Math follows flash_decode_split_bf16 (reference src/kernels/
// flash_decode.cu:118-325): per split an online softmax over its key range,
// then a log-sum-exp merge of the splits, bf16 RNE output. The MI355X design
// differs from the reference's one-block-per-q-head layout:
//
//  * One (kv head, split) unit serves the whole GQA group, so every K/V byte
//    is read from HBM once, not Hq/Hkv times.
//  * Scores and the value product run on bf16 MFMA (v_mfma_f32_16x16x32_bf16)
//    with the GQA group as the 16-wide N dimension: S^T = K Q^T, then
//    O^T += V^T P^T. Groups wider than 16 q heads run as equal blocks of
//    4-16 q heads, each block a unit of its own over the same K/V rows. E4M3 codes convert exactly to bf16 in registers
//    (v_cvt_scalef32_pk_bf16_fp8); the per-(token, kv_head) scales are folded
//    in fp32 into the score column (k_scale) and into P (v_scale).
//  * K is loaded as whole rows (16 bytes per lane) and moved into the MFMA
//    layout through the wave's LDS; V is loaded 8 bytes per (key, lane) and
//    transposed in registers with v_perm so P^T needs no cross-lane
//    movement. Each wave keeps a ring of two register tiles in
//    flight.
//  * Softmax runs in base 2 (scores pre-multiplied by scale*log2(e)); the
//    running-max rescale of the accumulator is skipped when no lane's max
//    moved.
//  * Partitions (see DecPartition):
//      - num_splits * Hkv >= 8 * CUs units: one WAVE per (kv head, split)
//        unit. A workgroup holds the kv heads of one split (its waves share
//        the interleaved scale lines in L1), or, when no split holds more
//        than two tiles, 8 splits of one kv head S/8 apart on one XCD (so the merge
//        reads that XCD's L2); waves never wait for each other and each
//        writes its own partial.
//      - fewer units (e.g. 64 splits x 8 kv heads): one workgroup per
//        (group of kv heads, split), sized so the grid fills the chip; the
//        waves of one kv head take every (8 / kvg)-th tile of the split
//        and merge in LDS (at most two tiles per split: the first wave of
//        each kv head streams the split alone and the others leave).
//        Workgroups of one split land on one XCD.
//  * A second small kernel merges the splits of every (q head, 16-wide d
//    slice): the head maximum from the m row, then weighted sums over a
//    strided subset of splits per thread, lane exchanges, one LDS step. The scratch layout is the reference's ([Hq,S] m, [Hq,S]
//    l, [Hq,S,D] acc); it needs no initialization. A whole-row variant
//    (one workgroup per row) merges calls of many rows and few splits.
//  * The same split kernel serves a causal prefill of a few tokens after
//    the cache (flash_decode_multi_kernel): blocks of tokens share a virtual
//    kv head's MFMA columns, each column with its own key limit.
//
// Split si holds an even share of the kTileKeys-key tiles over the keys; the
// merge folds the first n_eff = min(splits, tiles) slots. n_keys =
// *cache_len + 1 is read on device, so one launch configuration serves every
// decode step (graph capturable).
#include <algorithm>
#include <mutex>

#include "device_common.hpp"
#include "launch.hpp"
#include "rmsnorm_row.hpp"

namespace rth {
namespace {

constexpr int kDecWaves   = 8;
constexpr int kDecThreads = kDecWaves * kWave;
constexpr int kTileKeys   = 32;     // keys per wave iteration (two 16-key MFMAs)
constexpr int kMaxGroupD  = 2048;   // G * head_dim bound of a wave's LDS partial staging
constexpr int kMaxD       = 256;    // largest head_dim of the MFMA decode kernel
constexpr int kCombineThreads = 128;
constexpr int kCombineSlice   = 16;    // head_dim slice per merge workgroup
constexpr int kNtMinTiles     = 2;     // tiles past the first a wave streams with nontemporal loads
constexpr int kValuNtMinSteps = 32;    // VALU kernel: steps above which its loads are nontemporal

template <int D>
struct DecTraits {
    static_assert(D == 64 || D == 128 || D == 256, "decode MFMA path: D in {64,128,256}");
    static constexpr int kKChunks = D / 64;   // 16-byte K loads per lane per key
    static constexpr int kKSteps  = D / 32;   // MFMA k-steps of S^T
    static constexpr int kVBytes  = D / 16;   // V bytes per lane per key
    static constexpr int kVWords  = kVBytes / 4;
    static constexpr int kOMfma   = D / 16;   // PV MFMAs, one per d offset c
    // Register tiles in the ring (deeper measured slower); D 256 tiles are
    // 65 registers each, so that width keeps one (two spill).
    static constexpr int kRing    = (D == 256) ? 1 : 2;
};

// Physical cache row of logical key `key` when the cache is paged: blocks of
// 2^block_shift keys, logical block b stored at physical block
// block_table[b]. A 32-key tile never straddles a block (blocks hold a
// multiple of 32 keys and tiles start at multiples of 32), so one lookup per
// tile gives the tile's offset `delta` (physical - logical key).
__device__ __forceinline__ int paged_row(int key, const int* __restrict__ block_table,
                                         int block_shift) {
    const int mask = (1 << block_shift) - 1;
    return (block_table[key >> block_shift] << block_shift) | (key & mask);
}

// One tile's raw global data held by a lane.
template <int D>
struct TileRaw {
    u32x4    kraw[2][DecTraits<D>::kKChunks];
    uint32_t vraw[8][DecTraits<D>::kVWords];
    float    sc;       // lane l < 32: k_scale of key l, else v_scale of key l - 32
};

__device__ __forceinline__ int key_of(int g, int j) {  // P^T k-index -> key in tile
    return (j < 4) ? (4 * g + j) : (16 + 4 * g + (j - 4));
}

template <bool kNT, typename T>
__device__ __forceinline__ T ld(const T* p) {
    if constexpr (kNT) {
        return __builtin_nontemporal_load(p);
    } else {
        return *p;
    }
}

// Chunk swizzle of a wave's LDS K tile (32 rows of D bytes): row r keeps
// its 16-byte chunk c at position c ^ k_swz(r), so that the MFMA-layout reads
// (16 lanes = 16 rows x one chunk) hit 16 distinct 4-bank groups.
template <int D>
__device__ __forceinline__ int k_swz(int r) {
    return (r / (256 / D)) & (D / 16 - 1);
}

// Loads one tile's codes and scales. The K codes are read as whole rows:
// each load instruction covers 1024 / D complete D-byte rows (D / 16 lanes
// per row), which streams faster than loading the MFMA layout directly (16
// half rows per instruction; a read probe of the two access patterns at 128K
// keys x 8 kv heads: 6.3 vs 5.7 TB/s). The lane of row r, position c loads
// chunk c ^ k_swz(r); k_rows_to_mfma moves the tile into the MFMA layout
// through LDS. V rows are read 16 lanes x kVBytes per key (whole rows
// already), the scales one per lane. kNT: the K/V codes (read exactly once
// per call) use nontemporal loads, which stream faster once a wave has
// several tiles to read but have a longer latency than plain loads.
template <int D, bool kNT>
__device__ __forceinline__ void load_tile(TileRaw<D>& t, const uint8_t* __restrict__ k,
                                               const uint8_t* __restrict__ v,
                                               const float* __restrict__ ks,
                                               const float* __restrict__ vs, int kb, int k1,
                                               int kvh, int hkv, int lane, int delta) {
    using T             = DecTraits<D>;
    constexpr int kCpr  = D / 16;          // 16-byte chunks per row
    constexpr int kRpi  = kWave / kCpr;    // rows per load instruction
    const int     rr    = lane / kCpr;
    const int     ch    = lane % kCpr;
    if (!kNT && D <= 128 && kb + kTileKeys <= k1) {
        // A full tile of a short (latency-bound) stream: wave-uniform row
        // bases (scalar) plus per-lane 32-bit offsets that do not change from
        // tile to tile, so the addresses cost no per-tile vector arithmetic
        // (8K: 12.38 -> 12.12 us per call; the nontemporal streams of longer
        // contexts measured 0.3-0.4 us slower with it at 128K, and at head_dim
        // 256 the fixed offsets spill; both keep the clamped per-row
        // addresses below).
        const int64_t  rs = static_cast<int64_t>(hkv) * D;   // bytes per token row
        const uint8_t* kt = k + (static_cast<int64_t>(kb + delta) * hkv + kvh) * D;
        const uint8_t* vt = v + (static_cast<int64_t>(kb + delta) * hkv + kvh) * D;
#pragma unroll
        for (int i = 0; i < kTileKeys / kRpi; ++i) {
            const int      r   = i * kRpi + rr;
            const uint32_t off = static_cast<uint32_t>(r * rs) + 16u * (ch ^ k_swz<D>(r));
            t.kraw[i / T::kKChunks][i % T::kKChunks] =
                ld<kNT>(reinterpret_cast<const u32x4*>(kt + off));
        }
        const int n = lane & 15;
        const int g = lane >> 4;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t off = static_cast<uint32_t>(key_of(g, j) * rs) + T::kVBytes * n;
            if constexpr (T::kVWords == 1) {
                t.vraw[j][0] = ld<kNT>(reinterpret_cast<const uint32_t*>(vt + off));
            } else if constexpr (T::kVWords == 2) {
                const u32x2 w = ld<kNT>(reinterpret_cast<const u32x2*>(vt + off));
                t.vraw[j][0]  = w.x;
                t.vraw[j][1]  = w.y;
            } else {
                const u32x4 w = ld<kNT>(reinterpret_cast<const u32x4*>(vt + off));
                t.vraw[j][0]  = w.x;
                t.vraw[j][1]  = w.y;
                t.vraw[j][2]  = w.z;
                t.vraw[j][3]  = w.w;
            }
        }
        const int64_t srow = static_cast<int64_t>(kb + delta) * hkv + kvh;
        const float*  sp   = (lane < 32) ? ks + srow : vs + srow;
        t.sc               = sp[(lane & 31) * hkv];
        return;
    }
#pragma unroll
    for (int i = 0; i < kTileKeys / kRpi; ++i) {
        const int      r   = i * kRpi + rr;
        const int      key = min(kb + r, k1 - 1);
        const uint8_t* kr  = k + (static_cast<int64_t>(key + delta) * hkv + kvh) * D;
        t.kraw[i / T::kKChunks][i % T::kKChunks] =
            ld<kNT>(reinterpret_cast<const u32x4*>(kr + 16 * (ch ^ k_swz<D>(r))));
    }
    const int n = lane & 15;
    const int g = lane >> 4;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int      key = min(kb + key_of(g, j), k1 - 1);
        const uint8_t* vr  = v + (static_cast<int64_t>(key + delta) * hkv + kvh) * D + T::kVBytes * n;
        if constexpr (T::kVWords == 1) {
            t.vraw[j][0] = ld<kNT>(reinterpret_cast<const uint32_t*>(vr));
        } else if constexpr (T::kVWords == 2) {
            const u32x2 w = ld<kNT>(reinterpret_cast<const u32x2*>(vr));
            t.vraw[j][0]  = w.x;
            t.vraw[j][1]  = w.y;
        } else {
            const u32x4 w = ld<kNT>(reinterpret_cast<const u32x4*>(vr));
            t.vraw[j][0]  = w.x;
            t.vraw[j][1]  = w.y;
            t.vraw[j][2]  = w.z;
            t.vraw[j][3]  = w.w;
        }
    }
    {
        const int     key = min(kb + (lane & 31), k1 - 1);
        const int64_t row = static_cast<int64_t>(key + delta) * hkv + kvh;
        t.sc              = (lane < 32) ? ks[row] : vs[row];
    }
}

// Rewrites the K registers of a load_tile tile into the MFMA layout
// (lane (n, g) holds bytes 16g + 64c of row 16u + n in kraw[u][c])
// through buf, D * 32 bytes of this wave's LDS: the tile is stored as loaded
// (slot lane + 64i) and read back by rows. LDS operations of one wave run in
// order, so no wait separates the stores from the loads.
template <int D>
__device__ __forceinline__ void k_rows_to_mfma(TileRaw<D>& t, uint8_t* buf, int lane) {
    using T = DecTraits<D>;
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
        *reinterpret_cast<u32x4*>(buf + 16 * (lane + kWave * i)) =
            t.kraw[i / T::kKChunks][i % T::kKChunks];
    }
    const int n = lane & 15;
    const int g = lane >> 4;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int c = 0; c < T::kKChunks; ++c) {
            const int r  = 16 * u + n;
            t.kraw[u][c] = *reinterpret_cast<const u32x4*>(buf + r * D +
                                                           16 * ((4 * c + g) ^ k_swz<D>(r)));
        }
    }
}

// Partition of the decode work for one call. With fewer units than one
// round of wave slots (num_splits * hkv < 8 * CUs) the host launches one
// workgroup per (group of kvg kv heads, split): the workgroup's waves are kvg kv heads x
// 8 / kvg waves per kv head, the waves of one kv head take interleaved shares
// of the split's tiles (every (8 / kvg)-th tile; contiguous shares measured
// 128K at 64 splits 53.4 vs 52.0 us) and merge in LDS ("coop"); kvg is chosen so the grid still fills
// the chip (more kv heads per workgroup read longer runs of each interleaved
// [token, kv_head] row). Otherwise (kvg = 0, and always in the VALU kernel)
// it launches one wave per (kv head, split) unit, eight per workgroup, with
// no merge inside a workgroup. (Cooperative workgroups over 8x fewer splits
// at short contexts, which leave 8x fewer partials for the merge kernel,
// measured 1.1-1.5 us per call slower than one wave per unit from 35 to
// 16384 keys.) Both kernels derive the same split bounds from *cache_len and
// kvg, so they are decided on device per call.
//
// The key range is cut into kTileKeys-key tiles dealt out evenly: split si
// holds tiles [split_tile(si), split_tile(si + 1)), floor or ceil of
// tiles / n_eff of them, and n_eff = min(splits, tiles) splits are live, the
// first n_eff slots of the partials (at ctx 8196 and 256 splits: one split
// of two tiles and 255 of one, where equal 64-key ranges would leave 127
// splits empty and their workgroups idle).
struct DecPartition {
    bool coop;
    int  splits;   // partial slots per q head
    int  n_eff;    // live splits: min(splits, tiles)
    int  base;     // tiles / n_eff
    int  rem;      // tiles % n_eff: the first rem splits hold one more tile
    int  gkv;      // coop: kv heads per workgroup
};

__device__ __forceinline__ int split_tile(const DecPartition& pt, int si) {
    return si * pt.base + min(si, pt.rem);
}

__device__ __forceinline__ DecPartition dec_partition(int n_keys, int num_splits, int kvg) {
    DecPartition pt;
    pt.coop   = kvg > 0;
    pt.splits = num_splits;
    pt.gkv    = pt.coop ? kvg : 1;
    const int tiles = (n_keys + kTileKeys - 1) / kTileKeys;
    pt.n_eff        = min(pt.splits, tiles);
    pt.base         = tiles / pt.n_eff;
    pt.rem          = tiles - pt.base * pt.n_eff;
    return pt;
}

// kv heads per workgroup of a coop launch (0: one wave per unit, solo): of 1, 2,
// 4, 8 dividing hkv, the one whose grid takes the fewest rounds of one
// workgroup per compute unit, and among those the smallest (the most
// workgroups). (Preferring the fewest workgroups that still fill the chip
// put 192 or 224 splits x 8 kv heads in two rounds: 15 us per call at 8K
// against 11 in one.)
__host__ __device__ constexpr int dec_group_kv(int num_splits, int hkv, int cus) {
    if (num_splits * hkv >= kDecWaves * cus) {
        return 0;
    }
    int best = 1;
    int best_rounds = (num_splits * hkv + cus - 1) / cus;
    for (int g = 2; g <= kDecWaves; g *= 2) {
        if (hkv % g == 0) {
            const int rounds = (num_splits * (hkv / g) + cus - 1) / cus;
            if (rounds < best_rounds) {
                best        = g;
                best_rounds = rounds;
            }
        }
    }
    // Eight kv heads per workgroup is one wave per kv head: the solo layout,
    // without the in-workgroup merge and with its XCD placement and the
    // appended key's own split (2041 keys at 160-224 splits 11.1 -> 7.4 us).
    return best == kDecWaves ? 0 : best;
}

// q blocks per cache kv head for the MFMA kernel (0: the shape goes to the
// VALU kernel): the fewest blocks nqb dividing G with G / nqb <= 16 (the
// MFMA's columns) and G / nqb * D within a wave's LDS staging row; blocks of
// fewer than 4 q heads are left to the VALU kernel, whose units take 4.
__host__ __device__ constexpr int dec_q_blocks(int hq, int hkv, int head_dim) {
    if ((head_dim != 64 && head_dim != 128 && head_dim != 256) || hkv <= 0 || hq % hkv != 0) {
        return 0;
    }
    const int G = hq / hkv;
    for (int nqb = 1; nqb <= G; ++nqb) {
        const int gb = G / nqb;
        if (G % nqb == 0 && gb <= 16 && gb * head_dim <= kMaxGroupD) {
            return (gb >= 4 || nqb == 1) ? nqb : 0;
        }
    }
    return 0;
}

// Whether a solo launch may put all units of each kv head on one XCD
// (workgroup bid runs on XCD bid % 8) and the merge workgroups of its q heads
// on the same XCD: a kernel reads what the previous kernel wrote on its own
// XCD from L2, from another XCD only after a much longer trip (measured: a
// 3 MB exchange 0.9 us same-XCD against 3.0 us cross-XCD). The split kernel
// takes this mapping only when every live split holds one tile (tiles < 2 *
// splits, decided on device from *cache_len): with more tiles the kernel
// streams, and every XCD fetching all the interleaved [token, kv_head] scale
// lines for the 4 bytes of its kv head costs more than the merge saves
// (131072 keys: 48 -> 61 us per call). The merge takes it on every call of
// such a shape.
__host__ __device__ constexpr bool dec_xcd_local(int hkv, int num_splits) {
    return (hkv & 7) == 0 && (num_splits & 7) == 0;
}

__host__ __device__ constexpr int dec_workgroups(int num_splits, int hkv, int kvg) {
    return (kvg > 0) ? num_splits * (hkv / kvg)
                     : (num_splits * hkv + kDecWaves - 1) / kDecWaves;
}

// Sum over aligned groups of N lanes (N a power of two <= 64); every lane of
// a group ends with the group's sum. Each level adds the partner group's
// partial to the lane's own, as the xor butterfly does (rms_butterfly), so
// the sums are bit-identical to it.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (N >= 2) {   // lanes xor 1
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    }
    if constexpr (N >= 4) {   // lanes xor 2
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    }
    if constexpr (N >= 8) {   // the other quad of the 8 (row_half_mirror)
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    }
    if constexpr (N >= 16) {  // the other 8 of the row (row_mirror)
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
    }
    if constexpr (N >= 32) {
        v = wave_xor_sum(v, 16);
    }
    if constexpr (N >= 64) {
        v = wave_xor_sum(v, 32);
    }
    return v;
}

// Rotate-half RoPE of the bf16 words a lane holds of one head row (the q
// load and new-token layout: chunk c, half h, word i = elements
// 16g + 64c + 8h + 2i, +1), as rope_bf16 computes it (rope.hip): element d
// pairs with d + D/2 by angle theta_f, f = d mod D/2, with
// a' = bf16(fma(a, cos, -(b sin))), b' = bf16(fma(a, sin, b cos)); rc/rs hold
// cos/sin of the D/2 angles. The partner words sit in the same lane (chunk
// c ^ (kKChunks/2)) for D 128 and 256, in lane l ^ 32 for D 64.
template <int D>
__device__ __forceinline__ void rope_row_words(u32x4 (&w)[DecTraits<D>::kKChunks][2],
                                               const float* rc, const float* rs, int lane) {
    using T     = DecTraits<D>;
    const int g = lane >> 4;
    // Rotates word i of a and b (8 angles from f0) as pairs of bf16.
    auto rot = [&](uint32_t a, uint32_t b, int f, uint32_t& ra, uint32_t& rb) {
        float oa[2], ob[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float x  = __uint_as_float(e ? (a & 0xffff0000u) : (a << 16));
            const float y  = __uint_as_float(e ? (b & 0xffff0000u) : (b << 16));
            const float co = rc[f + e];
            const float si = rs[f + e];
            oa[e]          = fmaf(x, co, -(y * si));
            ob[e]          = fmaf(x, si, y * co);
        }
        ra = pack_bf16x2(oa[0], oa[1]);
        rb = pack_bf16x2(ob[0], ob[1]);
    };
    if constexpr (D == 64) {
        // Lanes 0-31 hold elements 0-31 (a), lanes 32-63 their partners (b).
        const bool first = g < 2;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t own  = w[0][h][i];
                const uint32_t part = __float_as_uint(wave_xor_partner(__uint_as_float(own), 32));
                uint32_t       ra, rb;
                rot(first ? own : part, first ? part : own, 16 * (g & 1) + 8 * h + 2 * i, ra, rb);
                w[0][h][i] = first ? ra : rb;
            }
        }
    } else {
        constexpr int kHalf = T::kKChunks / 2;
#pragma unroll
        for (int c = 0; c < kHalf; ++c) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t ra, rb;
                    rot(w[c][h][i], w[c + kHalf][h][i], 16 * g + 64 * c + 8 * h + 2 * i, ra, rb);
                    w[c][h][i]         = ra;
                    w[c + kHalf][h][i] = rb;
                }
            }
        }
    }
}

// cos / sin of the D/2 RoPE angles float(pos) * inv_freq[f] into rc / rs,
// taken in double precision and rounded to fp32 as rope_bf16 does; one wave.
// inv[j] = inv_freq[lane + 64 j], loaded ahead (see decode_body).
constexpr int kRopeIter = kMaxD / 2 / kWave;   // angles per lane at the largest head_dim
template <int D>
__device__ __forceinline__ void rope_table_wave(float* rc, float* rs, int pos,
                                                const float (&inv)[kRopeIter], int lane) {
#pragma unroll 1
    for (int j = 0; j * kWave < D / 2; ++j) {   // one double sincos live at a time
        const int f = lane + j * kWave;
        if (f >= D / 2) {
            break;
        }
        const float th = static_cast<float>(pos) * inv[j];
        double      sn, cs;
        sincos(static_cast<double>(th), &sn, &cs);
        rc[f] = static_cast<float>(cs);
        rs[f] = static_cast<float>(sn);
    }
    __builtin_amdgcn_wave_barrier();
}

// The appended token's quantized K/V codes for one (kv head) unit, laid out
// as the tile registers of key 0 of a tile after k_rows_to_mfma, plus the
// scales. rc != nullptr: K is rotated first (RoPE, see rope_row_words).
// pk / pv != nullptr: the row's words were loaded at kernel start (every lane
// loads its would-be words unconditionally; the n / g ownership selects stay
// here), so the wave does not wait on them after the key stream.
template <int D>
__device__ __forceinline__ void quantize_new_token(TileRaw<D>& vt, const uint16_t* __restrict__ kx,
                                                   const uint16_t* __restrict__ vx,
                                                   uint8_t* kc_row, uint8_t* vc_row,
                                                   float* ks_slot, float* vs_slot, int lane,
                                                   bool write, const float* rc = nullptr,
                                                   const float* rs = nullptr,
                                                   const uint16_t* k_norm = nullptr,
                                                   float eps = 0.0f, const u32x4* pk = nullptr,
                                                   const uint32_t* pv = nullptr,
                                                   const u32x4* pr = nullptr) {
    using T     = DecTraits<D>;
    const int n = lane & 15;
    const int g = lane >> 4;
    // K: lane (n = 0, g) owns bytes 16g + 64c .. +15 of the row (kraw[0][c]).
    u32x4 kw[T::kKChunks][2];
    float kmax = 0.0f;
#pragma unroll
    for (int c = 0; c < T::kKChunks; ++c) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (pr != nullptr) {
                // Element 16g + 64c + 8h of the row sits in lane 2g + 8c + h
                // of the preloaded rmsnorm_vec layout.
                const int src = 4 * (2 * g + 8 * c + h);
                u32x4     w;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    w[e] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>((*pr)[e])));
                }
                kw[c][h] = (n == 0) ? w : u32x4{0u, 0u, 0u, 0u};
            } else {
                kw[c][h] = (n == 0) ? (pk != nullptr ? pk[2 * c + h]
                                                     : *reinterpret_cast<const u32x4*>(kx + 16 * g + 64 * c + 8 * h))
                                    : u32x4{0u, 0u, 0u, 0u};
            }
        }
    }
    if (k_norm != nullptr) {
        // RMSNorm of the row in rmsnorm_vec's order: lanes 0 .. D/8-1 hold
        // one 16-byte vector each for the sum of squares.
        constexpr int kL = D / 8;
        u32x4 rv = {0u, 0u, 0u, 0u};
        if (lane < kL) {
            rv = (pr != nullptr) ? *pr : *reinterpret_cast<const u32x4*>(kx + 8 * lane);
        }
        const float rrms = __builtin_bit_cast(
            float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(
                       int, rms_inverse(group_sum<kL>(sumsq8(rv, 0.0f)), D, eps))));
#pragma unroll
        for (int c = 0; c < T::kKChunks; ++c) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const u32x4 gw =
                    *reinterpret_cast<const u32x4*>(k_norm + 16 * g + 64 * c + 8 * h);
                kw[c][h] = scale8(kw[c][h], gw, rrms);
            }
        }
    }
    if (rc != nullptr) {
        rope_row_words<D>(kw, rc, rs, lane);
    }
#pragma unroll
    for (int c = 0; c < T::kKChunks; ++c) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kmax = fmaxf(kmax, fabsf(__uint_as_float(kw[c][h][e] << 16)));
                kmax = fmaxf(kmax, fabsf(__uint_as_float(kw[c][h][e] & 0xffff0000u)));
            }
        }
    }
    // V: lane (n, g = 0) owns bytes kVBytes * n .. + kVBytes - 1 (vraw[0][*]).
    constexpr int kVW = T::kVBytes / 2;   // bf16 words
    uint32_t      vw[kVW];
    float         vmax = 0.0f;
#pragma unroll
    for (int i = 0; i < kVW; ++i) {
        vw[i] = (g == 0) ? (pv != nullptr ? pv[i] : *reinterpret_cast<const uint32_t*>(vx + T::kVBytes * n + 2 * i)) : 0u;
        vmax  = fmaxf(vmax, fabsf(__uint_as_float(vw[i] << 16)));
        vmax  = fmaxf(vmax, fabsf(__uint_as_float(vw[i] & 0xffff0000u)));
    }
    // Lanes without data hold 0, so a full-wave max leaves every lane with
    // the row maxima (lane 32 passes the V scale to the tile registers).
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) {
        kmax = wave_xor_max(kmax, m);
        vmax = wave_xor_max(vmax, m);
    }
    // The append's arithmetic (quantize_rows_kernel): two separate divisions.
    const float ksc  = kmax / kE4M3Max;
    const float kinv = (kmax > 0.0f) ? (kE4M3Max / kmax) : 0.0f;
    const float vsc  = vmax / kE4M3Max;
    const float vinv = (vmax > 0.0f) ? (kE4M3Max / vmax) : 0.0f;
    auto code4 = [](uint32_t w0, uint32_t w1, float inv) {
        uint32_t r = 0;
        r = e4m3x2_pack<false>(__uint_as_float(w0 << 16) * inv,
                               __uint_as_float(w0 & 0xffff0000u) * inv, r);
        r = e4m3x2_pack<true>(__uint_as_float(w1 << 16) * inv,
                              __uint_as_float(w1 & 0xffff0000u) * inv, r);
        return r;
    };
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int c = 0; c < T::kKChunks; ++c) {
            vt.kraw[u][c] = u32x4{0u, 0u, 0u, 0u};
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int w = 0; w < T::kVWords; ++w) {
            vt.vraw[j][w] = 0u;
        }
    }
#pragma unroll
    for (int c = 0; c < T::kKChunks; ++c) {
        u32x4 cw;
        cw.x = code4(kw[c][0].x, kw[c][0].y, kinv);
        cw.y = code4(kw[c][0].z, kw[c][0].w, kinv);
        cw.z = code4(kw[c][1].x, kw[c][1].y, kinv);
        cw.w = code4(kw[c][1].z, kw[c][1].w, kinv);
        if (n == 0) {
            vt.kraw[0][c] = cw;
            if (write) {
                *reinterpret_cast<u32x4*>(kc_row + 16 * g + 64 * c) = cw;
            }
        }
    }
#pragma unroll
    for (int w = 0; w < T::kVWords; ++w) {
        const uint32_t cw = code4(vw[2 * w], vw[2 * w + 1], vinv);
        if (g == 0) {
            vt.vraw[0][w] = cw;
            if (write) {
                *reinterpret_cast<uint32_t*>(vc_row + T::kVBytes * n + 4 * w) = cw;
            }
        }
    }
    vt.sc = (lane == 0) ? ksc : ((lane == 32) ? vsc : 0.0f);
    if (write && lane == 0) {
        *ks_slot = ksc;
        *vs_slot = vsc;
    }
}

// kAppend: the call also appends one token (k_new, v_new [Hkv, D] bf16) at
// row *cache_len of the cache; the owner unit (a split of its own when the
// cache keys leave one, else the last split) quantizes it, stores codes and
// scales, and attends to it from registers, so no wave reads the row being
// written.
// kPaged: K/V/scale rows are addressed through block_table (see paged_row).
// nqb: q blocks per cache kv head. A group of more than 16 q heads (the
// MFMA's 16 columns) is served as nqb virtual kv heads of G / nqb q heads
// each: `hkv` counts virtual heads (cache heads x nqb), virtual head kvh reads
// the K/V rows of cache head kvh / nqb, and q heads, partial slots and the
// merge keep their global q-head index (kvh * G + n). Only the first virtual
// head of a cache head stores the appended token.
// kRope (with kAppend): q and the appended k row are rotated in registers by
// the angles of positions[0] (rope_bf16's arithmetic, see rope_row_words);
// each wave builds its own cos/sin table after issuing its first tile loads.
// kNorm (with kRope): before the rotation, q rows and the appended k row
// are RMS-normalized per head with the q_norm / k_norm gains (Qwen3's order,
// rmsnorm_vec's arithmetic and reduction order).
// kMulti (not with kAppend): n_tok query tokens of one causal prefill call
// whose keys are all in the cache (*cache_len keys before them). A virtual
// kv head is (block of tb tokens, cache head, q block), in that order of
// significance (`hkv` counts them); its G = hq / hkv MFMA columns are the
// block's tokens x gb = G / tb q heads (column n: token n / gb, head n % gb),
// so one pass over a key tile serves tb tokens. q and out are
// [n_tok, hq_real, D]; the partials use the rows t * hq_real + h (the merge
// runs over n_tok * hq_real rows). Token t attends to the first
// *cache_len + t + 1 keys: a per-column limit in the tile mask; columns past
// the block's tokens or G mirror column 0 and are never stored.
template <int D, bool kAppend, bool kPaged, bool kRope, bool kNorm = false, bool kMulti = false>
__device__ __forceinline__ void decode_body(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ k,
    const uint8_t* __restrict__ v, const float* __restrict__ ks,
    const float* __restrict__ vs, float* __restrict__ partial, int num_splits,
    const int* __restrict__ cache_len, int hq, int hkv, float scale_log2,
    const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
    uint8_t* k_w, uint8_t* v_w, float* ks_w, float* vs_w,
    const int* __restrict__ block_table, int block_shift, int kvg, int nqb,
    const int* __restrict__ positions, const float* __restrict__ inv_freq,
    const uint16_t* __restrict__ q_norm = nullptr, const uint16_t* __restrict__ k_norm = nullptr,
    float eps = 0.0f, int n_tok = 1, int hq_real = 0, int tb = 1) {
    using T = DecTraits<D>;
    static_assert(!kRope || kAppend, "the RoPE variant is the fused decode step");
    static_assert(!kMulti || !kAppend, "the multi-token kernel attends to cached keys only");
    static_assert(!kNorm || kRope, "the q/k norm runs before the RoPE");

    __shared__ __attribute__((aligned(16))) float sm_sc[kDecWaves][64];
    __shared__ __attribute__((aligned(16))) float sm_o[kDecWaves][kMaxGroupD];
    __shared__ float sm_m[kDecWaves][16];
    __shared__ float sm_l[kDecWaves][16];
    // kRope: cos (first D/2) and sin (next D/2) of the RoPE angles, built by
    // every wave for itself (no workgroup barrier).
    __shared__ __attribute__((aligned(16))) float sm_rope_w[kRope ? kDecWaves : 1][kRope ? D : 1];
    // kNorm: the q_norm (first D) and k_norm gains, staged by every wave.
    __shared__ __attribute__((aligned(16))) uint16_t sm_gain_w[kNorm ? kDecWaves : 1][kNorm ? 2 * D : 1];

    const int G    = hq / hkv;
    const int tid  = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid & (kWave - 1);
    const int n    = lane & 15;
    const int g    = lane >> 4;
    const int bid  = static_cast<int>(blockIdx.x);

    const int          n_keys = *cache_len + (kMulti ? n_tok : 1);
    DecPartition pt = dec_partition(n_keys, num_splits, kvg);
    // Append calls with at most two cache tiles per split
    // when one split is kept back: the appended key gets that split of its
    // own (slot owner_si), so its wave attends to it alone instead of behind
    // a cache tile (that wave finished last: 2041 keys 8.8 -> 7.4 us per
    // call, 8196 keys 10.97 -> 10.71); the cache tiles go one or two per
    // split over the others. The merge derives the same slot count. (Kept out
    // of dec_partition: otherwise the prologue of every kernel is scheduled
    // around it, 0.1-0.2 us per call at 8K.)
    int owner_si = pt.n_eff - 1;
    int n_live   = pt.n_eff;
    int key_end  = n_keys;   // cache keys a non-owner split may read
    if constexpr (kAppend) {
        const int cache_tiles = (n_keys - 1 + kTileKeys - 1) / kTileKeys;
        // Grouped launches take it too (every split then holds at most two
        // tiles, so their waves run alone: 64 splits at 480 keys 8.0 -> 6.7
        // us per call). Written as two terms, the solo one marked likely:
        // the plain condition scheduled the solo prologue worse (8196 keys
        // at 256 splits 10.40 -> 10.73 us).
        const bool own_ok = cache_tiles <= 2 * (num_splits - 1);
        if (__builtin_expect(!pt.coop && own_ok, 1) || (pt.coop && own_ok)) {
            const int n = min(num_splits - 1, cache_tiles);
            pt.n_eff = n;
            pt.base  = 1;                 // at most two cache tiles per split
            pt.rem   = cache_tiles - n;
            owner_si = n;
            n_live   = n + 1;
            key_end  = n_keys - 1;
        }
    }
    // coop: workgroup = (group of gkv kv heads, split); wave w serves kv head
    //       w % gkv of the group and share j = w / gkv of its tiles
    // solo: wave = (kv head, split) unit; adjacent units are the kv heads of
    //       one split, so a workgroup's waves share the scale lines in L1,
    //       except with one tile per split on XCD-local shapes (below).
    int       kvh, si;
    const int wpk = kDecWaves / pt.gkv;   // coop: waves per kv head
    if (!pt.coop && pt.base <= 1 && dec_xcd_local(hkv, num_splits)) {
        // Workgroup = 8 splits of one kv head, on XCD kvh % 8
        // (dec_xcd_local): splits sg, sg + S/8, ..., so that the live
        // splits of a short context (the first ones) spread over the kv
        // head's S/8 workgroups, one wave per compute unit, instead of
        // filling the first workgroups (8 waves sharing one CU's load path:
        // 200 keys 7.32 -> 6.48 us per call, 2041 keys 7.42 -> 6.91, 8196
        // keys 10.63 -> 10.47).
        const int r  = bid >> 3;
        const int hh = hkv >> 3;   // kv heads per XCD
        int       kh, sg;
        if ((hh & (hh - 1)) == 0) {
            kh = r & (hh - 1);
            sg = r >> __builtin_ctz(hh);
        } else {
            kh = r % hh;
            sg = r / hh;
        }
        kvh = kh * 8 + (bid & 7);
        si  = wave * (num_splits >> 3) + sg;
    } else if (!pt.coop) {
        const int unit = bid * kDecWaves + wave;
        // hkv is a power of two in every common shape: shifts, not divisions.
        if ((hkv & (hkv - 1)) == 0) {
            kvh = unit & (hkv - 1);
            si  = unit >> __builtin_ctz(hkv);
        } else {
            kvh = unit % hkv;
            si  = unit / hkv;
        }
    } else {
        const int groups = hkv / pt.gkv;
        int       grp;
        if ((pt.splits & 7) == 0) {
            // All kv heads of one split on one XCD (bid % 8), so the
            // interleaved [token, kv_head] K/V rows and scale lines are
            // fetched into one L2.
            const int r = bid >> 3;
            si          = (r / groups) * 8 + (bid & 7);
            grp         = r % groups;
        } else {
            si  = bid / groups;
            grp = bid % groups;
        }
        kvh = grp * pt.gkv + wave % pt.gkv;
    }
    // kRope: the angle inputs are loaded here, ahead of every tile load, so
    // building the table later waits for nothing else in flight. Each wave
    // builds its own table behind its first tile loads, where the double
    // sincos hides under their latency (one table per workgroup behind a
    // workgroup barrier measured 0.4-1.2 us slower per call).
    [[maybe_unused]] float    rope_inv[kRopeIter] = {};
    [[maybe_unused]] int      rope_pos            = 0;
    [[maybe_unused]] uint32_t gain_q[kRopeIter]   = {};   // 2 bf16 per lane and step
    [[maybe_unused]] uint32_t gain_k[kRopeIter]   = {};
    if constexpr (kRope) {
        rope_pos = *positions;
#pragma unroll
        for (int j = 0; j < kRopeIter; ++j) {
            if (lane + j * kWave < D / 2) {
                rope_inv[j] = inv_freq[lane + j * kWave];
                if constexpr (kNorm) {
                    gain_q[j] = reinterpret_cast<const uint32_t*>(q_norm)[lane + j * kWave];
                    gain_k[j] = reinterpret_cast<const uint32_t*>(k_norm)[lane + j * kWave];
                }
            }
        }
    }
    float*    sm_rope = sm_rope_w[kRope ? wave : 0];
    uint16_t* sm_gain = sm_gain_w[kNorm ? wave : 0];
    auto rope_sync = [&]() {
        if constexpr (kRope) {
            if constexpr (kNorm) {
#pragma unroll
                for (int j = 0; j < kRopeIter; ++j) {
                    if (lane + j * kWave < D / 2) {
                        reinterpret_cast<uint32_t*>(sm_gain)[lane + j * kWave] = gain_q[j];
                        reinterpret_cast<uint32_t*>(sm_gain + D)[lane + j * kWave] = gain_k[j];
                    }
                }
            }
            rope_table_wave<D>(sm_rope, sm_rope + D / 2, rope_pos, rope_inv, lane);
        }
    };
    if (si >= n_live) {   // uniform per workgroup in coop mode
        return;
    }
    // Coop workgroups whose splits hold at most two tiles (short contexts,
    // uniform over the grid): the first wave of each kv head streams its
    // split alone and stores its partial as a solo wave does; the others
    // leave (no LDS merge, no barrier).
    const bool lone = pt.coop && pt.base + (pt.rem > 0 ? 1 : 0) <= 2;
    if (lone && wave >= pt.gkv) {
        return;
    }
    // Wave-uniform by construction; kept in scalar registers so that tile
    // addresses are a scalar base plus fixed per-lane offsets.
    int kvc_v = nqb == 1 ? kvh : kvh / nqb;   // cache kv head (kMulti: token-block major)
    int hkc_v = nqb == 1 ? hkv : hkv / nqb;   // cache kv heads (kMulti: x token blocks)
    [[maybe_unused]] int lim_lo = 0;          // kMulti: the block's first token's key limit
    [[maybe_unused]] int gbm    = G;          // kMulti: q heads per token of a column block
    if constexpr (kMulti) {
        hkc_v /= (n_tok + tb - 1) / tb;
        const int tblk = kvc_v / hkc_v;
        kvc_v -= tblk * hkc_v;
        const int tok0 = tblk * tb;
        key_end = n_keys - n_tok + min(tok0 + tb, n_tok);   // the block's last token's limit
        lim_lo  = n_keys - n_tok + tok0 + 1;
        gbm     = G / tb;
    }
    const int kvc = __builtin_amdgcn_readfirstlane(kvc_v);
    const int hkc = __builtin_amdgcn_readfirstlane(hkc_v);
    // kMulti: output row of column col of virtual kv head vk (-1: padding).
    [[maybe_unused]] auto mrow = [&](int vk, int col) -> int {
        const int qbv = nqb == 1 ? 0 : vk % nqb;
        const int vh  = nqb == 1 ? vk : vk / nqb;
        const int tbk = vh / hkc;
        const int t   = tbk * tb + col / gbm;
        if (col >= G || t >= n_tok) {
            return -1;
        }
        return t * hq_real + (vh - tbk * hkc) * (gbm * nqb) + qbv * gbm + col % gbm;
    };
    [[maybe_unused]] int row_n = 0;   // kMulti: this lane's column's row (-1: padding)
    [[maybe_unused]] int lim_n = 0;   // kMulti: its key limit
    if constexpr (kMulti) {
        row_n = mrow(kvh, n);
        lim_n = row_n < 0 ? lim_lo : lim_lo + (n / gbm);
    }
    // The appended row's bf16 words, issued before the stream (D <= 128: the
    // 40 VGPRs they hold through the stream spill the D = 256 kernels). Plain
    // loads, not loads inside the owner branch: a branch-merged load makes the
    // compiler wait for every outstanding load at the merge. The q/k-norm
    // kernels hold the K row once, in rmsnorm_vec's layout (16 bytes on each
    // of lanes 0 .. D/8-1), and gather the tile layout from it with lane
    // permutes (both layouts held through the stream spill there; per call
    // at 8K the preload saves ~1 us of the owner wave's round trip).
    [[maybe_unused]] u32x4    pre_k[DecTraits<D>::kKChunks * 2];
    [[maybe_unused]] uint32_t pre_v[DecTraits<D>::kVBytes / 2];
    [[maybe_unused]] u32x4    pre_r = {0u, 0u, 0u, 0u};   // kNorm: the row in rmsnorm_vec's layout
    if constexpr (kAppend && D <= 128) {
        const uint16_t* kx = k_new + static_cast<int64_t>(kvc) * D;
        const uint16_t* vx = v_new + static_cast<int64_t>(kvc) * D;
        if constexpr (kNorm) {
            pre_r = *reinterpret_cast<const u32x4*>(kx + 8 * (lane & (D / 8 - 1)));
        } else {
#pragma unroll
            for (int c = 0; c < DecTraits<D>::kKChunks; ++c) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    pre_k[2 * c + h] = *reinterpret_cast<const u32x4*>(kx + 16 * ((lane >> 4) & 3) + 64 * c + 8 * h);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < DecTraits<D>::kVBytes / 2; ++i) {
            pre_v[i] = *reinterpret_cast<const uint32_t*>(vx + DecTraits<D>::kVBytes * (lane & 15) + 2 * i);
        }
    }
    const int k0 = split_tile(pt, si) * kTileKeys;
    // With an append, no split reads key p_new from the cache (it is being
    // written); one wave of the owner split adds it from registers.
    const int  p_new   = n_keys - 1;
    const bool owner   = kAppend && (si == owner_si);
    const bool virt    = owner && (!pt.coop || lone || wave >= kDecWaves - pt.gkv);
    const int  k1      = owner ? p_new : min(split_tile(pt, si + 1) * kTileKeys, key_end);
    const int  n_tiles = (k1 - k0 + kTileKeys - 1) / kTileKeys;
    // The wave's cnt tiles of the split, tile_at(0 .. cnt - 1): all of them
    // for a solo wave; in coop mode wave j of its kv head's wpk waves takes
    // tiles j, j + wpk, j + 2 wpk, ..., so the waves of a kv head read
    // neighbouring tiles at the same time.
    const int  wj        = pt.coop ? wave / pt.gkv : 0;
    const int  wn        = (pt.coop && !lone) ? wpk : 1;
    const int  cnt       = (pt.coop && !lone) ? (n_tiles - wj + wn - 1) / wn : n_tiles;
    auto       tile_at   = [&](int i) { return (pt.coop && !lone) ? wj + i * wn : i; };

    // Q^T as the B operand: column n = q head n of the group. Columns past
    // G repeat head 0: their scores only ever mirror head 0's (so they never
    // change the wave-wide lazy-max vote) and their m, l and O are never
    // stored. Zeroing them instead made the wave wait for q before issuing
    // its first K/V tile loads (measured 0.3-0.7 us per call at 8K).
    bf16x8 qop[T::kKSteps];
    {
        const int64_t   qrow = kMulti ? static_cast<int64_t>(row_n >= 0 ? row_n : mrow(kvh, 0))
                                          : static_cast<int64_t>(kvh * G + (n < G ? n : 0));
        const uint16_t* qr   = q + qrow * D;
#pragma unroll
        for (int c = 0; c < T::kKChunks; ++c) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(qr + 16 * g + 64 * c + 8 * h);
                qop[2 * c + h] = __builtin_bit_cast(bf16x8, w);
            }
        }
    }
    // kNorm: the q rows again in rmsnorm_vec's layout (D/8 lanes per row, one
    // 16-byte vector each), for the per-row sums of squares; loaded here, with
    // q, and used behind the first tile loads.
    constexpr int kQnL    = D / 8;
    constexpr int kQnRpp  = kWave / kQnL;                            // rows per load
    constexpr int kQnRows = (kMaxGroupD / D < 16) ? kMaxGroupD / D : 16;
    constexpr int kQnPass = (kQnRows + kQnRpp - 1) / kQnRpp;
    [[maybe_unused]] u32x4 qn_raw[kQnPass];
    if constexpr (kNorm) {
#pragma unroll
        for (int p = 0; p < kQnPass; ++p) {
            const int r = min(p * kQnRpp + lane / kQnL, G - 1);
            qn_raw[p]   = *reinterpret_cast<const u32x4*>(
                q + static_cast<int64_t>(kvh * G + r) * D + 8 * (lane % kQnL));
        }
    }

    f32x4 oacc[T::kOMfma];
#pragma unroll
    for (int c = 0; c < T::kOMfma; ++c) {
        oacc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float m_run = -INFINITY;
    float l_run = 0.0f;

    // kRope: the table barrier, then q rotated in registers. The barrier
    // goes behind the first tile loads, except at head_dim 256 (a one-tile
    // ring), where the table is built before any tile registers are live
    // (behind them its double-precision sincos spilled).
    constexpr bool kTableFirst = kRope && D == 256;
    auto rope_xform = [&]() {
        if constexpr (kRope) {
            u32x4 qw[T::kKChunks][2];
#pragma unroll
            for (int c = 0; c < T::kKChunks; ++c) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    qw[c][h] = __builtin_bit_cast(u32x4, qop[2 * c + h]);
                }
            }
            if constexpr (kNorm) {
                // Per-row 1/rms through this wave's sm_m row (free until the
                // cooperative merge); padding columns (n >= G) hold head 0's
                // q, so they take head 0's factor.
#pragma unroll
                for (int p = 0; p < kQnPass; ++p) {
                    if (p * kQnRpp < G) {   // passes holding real rows only
                        const float rr =
                            rms_inverse(group_sum<kQnL>(sumsq8(qn_raw[p], 0.0f)), D, eps);
                        const int r = p * kQnRpp + lane / kQnL;
                        if (lane % kQnL == 0 && r < kQnRows) {
                            sm_m[wave][r] = rr;
                        }
                    }
                }
                __builtin_amdgcn_wave_barrier();
                const float rrms = sm_m[wave][n < G ? n : 0];
#pragma unroll
                for (int c = 0; c < T::kKChunks; ++c) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const u32x4 gw = *reinterpret_cast<const u32x4*>(sm_gain + 16 * g +
                                                                         64 * c + 8 * h);
                        qw[c][h] = scale8(qw[c][h], gw, rrms);
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
            rope_row_words<D>(qw, sm_rope, sm_rope + D / 2, lane);
#pragma unroll
            for (int c = 0; c < T::kKChunks; ++c) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    qop[2 * c + h] = __builtin_bit_cast(bf16x8, qw[c][h]);
                }
            }
        }
    };

    // Softmax state: m_ref is this lane's head reference maximum (shared by the
    // four lanes of a head); scores are exponentiated against it. It is raised
    // only when some score exceeds it by more than 2^kLazy, so the usual tile
    // needs no cross-lane step and no accumulator rescale. Exact: every p and
    // l use the same reference, and p <= 2^kLazy keeps them in range.
    // q transform point: here for head_dim 256, else behind the first tile
    // loads (rope_q, called once per wave).
    if constexpr (kTableFirst) {
        rope_sync();
        rope_xform();
    }
    auto rope_q = [&]() {
        if constexpr (kRope && !kTableFirst) {
            rope_sync();
            rope_xform();
        }
    };

    constexpr float kLazy = 8.0f;
    auto process = [&](const TileRaw<D>& cur, const int kb, const int klim) {
        sm_sc[wave][lane] = (lane < 32) ? cur.sc * scale_log2 : cur.sc;   // k-factors pre-scaled
        __builtin_amdgcn_wave_barrier();
        // S^T = K Q^T, two 16-key halves.
        f32x4 s[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            s[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < T::kKChunks; ++c) {
                bf16x8 a0, a1;
                e4m3x16_to_bf16x8x2(cur.kraw[u][c], a0, a1);
                s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, qop[2 * c], s[u], 0, 0, 0);
                s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, qop[2 * c + 1], s[u], 0, 0, 0);
            }
        }

        // Register j of this lane is key key_of(g, j) of the tile; its scales
        // come from the lanes that loaded them, through this wave's LDS row.
        const f32x4 kf0 = *reinterpret_cast<const f32x4*>(&sm_sc[wave][4 * g]);
        const f32x4 kf1 = *reinterpret_cast<const f32x4*>(&sm_sc[wave][16 + 4 * g]);
        const f32x4 vf0 = *reinterpret_cast<const f32x4*>(&sm_sc[wave][32 + 4 * g]);
        const f32x4 vf1 = *reinterpret_cast<const f32x4*>(&sm_sc[wave][48 + 4 * g]);
        float x[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            x[r]     = s[0][r] * kf0[r];
            x[4 + r] = s[1][r] * kf1[r];
        }
        if constexpr (kMulti) {
            if (kb + kTileKeys > min(klim, lim_lo)) {  // a column's limit or the split's end
                const int lim = min(klim, lim_n);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (kb + key_of(g, j) >= lim) {
                        x[j] = -INFINITY;
                    }
                }
            }
        } else if (kb + kTileKeys > klim) {  // ragged last tile of the split
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (kb + key_of(g, j) >= klim) {
                    x[j] = -INFINITY;
                }
            }
        }
        float lmax = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])),
                           fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
        if (!__all(lmax <= m_run + kLazy)) {
            lmax              = wave_xor_max(lmax, 16);
            lmax              = wave_xor_max(lmax, 32);
            const float m_new = fmaxf(m_run, lmax);
            // A wave's first tile (nothing accumulated yet) needs no rescale.
            if (!__all(m_run == -INFINITY)) {
                // kMulti: a column whose keys all lie past its limit keeps
                // m = -inf (and l = 0) while others move.
                const float alpha = (kMulti && m_new == -INFINITY)
                                        ? 1.0f
                                        : __builtin_amdgcn_exp2f(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int c = 0; c < T::kOMfma; ++c) {
                    oacc[c] *= alpha;
                }
            }
            m_run = m_new;
        }
        float p[8];
        const float m_sub = (kMulti && m_run == -INFINITY) ? 0.0f : m_run;   // p = 0, not NaN
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            p[j] = __builtin_amdgcn_exp2f(x[j] - m_sub);
        }
        l_run += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));

        u32x4 pw;
        pw.x = pack_bf16x2(p[0] * vf0[0], p[1] * vf0[1]);
        pw.y = pack_bf16x2(p[2] * vf0[2], p[3] * vf0[3]);
        pw.z = pack_bf16x2(p[4] * vf1[0], p[5] * vf1[1]);
        pw.w = pack_bf16x2(p[6] * vf1[2], p[7] * vf1[3]);
        const bf16x8 pop = __builtin_bit_cast(bf16x8, pw);

        // V^T operands: dword pj[j][w] holds bf16 of d = 2w, 2w+1 of key j.
        uint32_t pj[8][T::kVBytes / 2];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
#pragma unroll
            for (int w = 0; w < T::kVWords; ++w) {
                const u32x2 b = e4m3x4_to_bf16x4(cur.vraw[j][w]);
                pj[j][2 * w]     = b.x;
                pj[j][2 * w + 1] = b.y;
            }
        }
#pragma unroll
        for (int c = 0; c < T::kOMfma; ++c) {
            const int      pi  = c >> 1;
            const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
            u32x4          aw;
            aw.x = __builtin_amdgcn_perm(pj[1][pi], pj[0][pi], sel);
            aw.y = __builtin_amdgcn_perm(pj[3][pi], pj[2][pi], sel);
            aw.z = __builtin_amdgcn_perm(pj[5][pi], pj[4][pi], sel);
            aw.w = __builtin_amdgcn_perm(pj[7][pi], pj[6][pi], sel);
            oacc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, aw), pop, oacc[c], 0, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();
    };

    // Ring of kRing register tiles: the load of the tile kRing - 1 steps ahead
    // is issued before the current tile is consumed, with compile-time
    // buffer indices, so kRing - 1 tiles stay in flight per wave while it
    // computes. Past this wave's last tile no load is issued on a contiguous
    // cache (a wave-uniform branch; reloading the clamped last tile instead
    // cost 0.5 us per call at 2K), while the paged kernels keep issuing the
    // clamped reload (measured per call with a shuffled block table: 8K
    // 13.2 us with it vs 15.1 without, 128K 50.4 vs 51.3, 2K 9.6 vs 9.3).
    // The appended key (owner waves): quantized, stored and attended to.
    // kEarlyKey: right behind the first tile's loads, so that the work
    // overlaps their latency instead of trailing the stream (in the RoPE /
    // q-k-norm kernels after the rotation table's barrier; head_dim 256 does
    // it after the stream: earlier, it spills).
    constexpr bool kEarlyKey = kAppend && D <= 128;
    auto new_key = [&]() __attribute__((always_inline)) {
    if (kAppend && virt) {
        TileRaw<D>    vt;
        const int     prow = kPaged ? paged_row(p_new, block_table, block_shift) : p_new;
        const int64_t row  = static_cast<int64_t>(prow) * hkc + kvc;
        quantize_new_token<D>(vt, k_new + static_cast<int64_t>(kvc) * D,
                              v_new + static_cast<int64_t>(kvc) * D, k_w + row * D,
                              v_w + row * D, ks_w + row, vs_w + row, lane, kvh == kvc * nqb,
                              kRope ? sm_rope : nullptr, kRope ? sm_rope + D / 2 : nullptr,
                              kNorm ? sm_gain + D : nullptr, eps,
                              (kAppend && !kNorm && D <= 128) ? pre_k : nullptr,
                              (kAppend && D <= 128) ? pre_v : nullptr,
                              (kAppend && kNorm && D <= 128) ? &pre_r : nullptr);
        process(vt, p_new, p_new + 1);
    }
    };
    constexpr int kRing     = DecTraits<D>::kRing;
    if (cnt > 0) {
        auto tile_delta = [&](int kb) {
            if constexpr (kPaged) {
                return paged_row(kb, block_table, block_shift) - kb;
            } else {
                return 0;
            }
        };
        // The wave's own sm_o row is free until the partial is written.
        static_assert(kMaxGroupD * sizeof(float) >= kTileKeys * D, "K tile fits in an sm_o row");
        uint8_t* kbuf = reinterpret_cast<uint8_t*>(sm_o[wave]);
        auto stream = [&]<bool kNT>() {
            auto load = [&](TileRaw<D>& t, int kb) {
                load_tile<D, kNT>(t, k, v, ks, vs, kb, k1, kvc, hkc, lane, tile_delta(kb));
            };
            TileRaw<D> ring[kRing];
#pragma unroll
            for (int r = 0; r + 1 < kRing; ++r) {
                load(ring[r], k0 + tile_at(min(r, cnt - 1)) * kTileKeys);
            }
            rope_q();   // behind the first tile loads
            if constexpr (kEarlyKey) {
                new_key();
            }
            for (int t = 0;; t += kRing) {
                bool done = false;
#pragma unroll
                for (int r = 0; r < kRing; ++r) {
                    if (!done) {
                        const int tr  = t + r;
                        const int kbn = k0 + tile_at(min(tr + kRing - 1, cnt - 1)) * kTileKeys;
                        if (kPaged || tr + kRing - 1 <= cnt - 1) {
                            load(ring[(r + kRing - 1) % kRing], kbn);
                        }
                        k_rows_to_mfma<D>(ring[r], kbuf, lane);
                        process(ring[r], k0 + tile_at(tr) * kTileKeys, k1);
                        done = tr + 1 > cnt - 1;
                    }
                }
                if (done) {
                    break;
                }
            }
        };
        // A wave that streams three or more tiles is bandwidth-bound:
        // nontemporal loads. One- and two-tile runs (8K at 256 splits) and
        // the one-kv-head cooperative workgroups are latency-bound: plain
        // loads (measured: 128K at 256 splits 56.3 -> 51.8 us with
        // nontemporal loads, 32K at 256 splits (4 tiles per wave) 20.5 ->
        // 19.5 us; 8K at 256 splits and 128K at 64 one-kv-head cooperative
        // splits 6-8 % slower with them).
        if ((!pt.coop || pt.gkv > 1) && cnt - 1 >= kNtMinTiles) {
            stream.template operator()<true>();
        } else {
            stream.template operator()<false>();
        }
    } else {
        rope_q();
        if constexpr (kEarlyKey) {
            new_key();
        }
    }

    if constexpr (!kEarlyKey) {
        new_key();
    }

    // ---- partial of this split, reference layout: m at [h*S + si] (log2
    // units), l at [Hq*S + h*S + si], acc at [2*Hq*S + (h*S + si)*D + d]
    // with S = num_splits.
    l_run = wave_xor_sum(l_run, 16);
    l_run = wave_xor_sum(l_run, 32);
    const int64_t hs     = static_cast<int64_t>(kMulti ? n_tok * hq_real : hq) * num_splits;
    float*        part_m = partial;
    float*        part_l = partial + hs;
    float*        part_o = partial + 2 * hs;
    if (pt.coop && !lone) {
        // Merge the waves of each kv head (waves kl, kl + gkv, ...): each
        // puts its m, l and unscaled O^T rows in LDS; after one barrier the
        // threads sum the rows along d with the weights 2^(m_w - M), which
        // each derives from the waves' m (a second barrier, with the waves
        // scaling their own rows first, cost ~0.3 us per call).
        if (g == 0) {
            sm_m[wave][n] = m_run;
            sm_l[wave][n] = l_run;
        }
        if (n < G) {
#pragma unroll
            for (int c = 0; c < T::kOMfma; ++c) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    sm_o[wave][n * D + T::kVBytes * (4 * g + r) + c] = oacc[c][r];
                }
            }
        }
        __syncthreads();
        // Loops over the waves of one kv head run over all kDecWaves slots
        // with a predicate, unrolled, so their LDS reads issue together.
        const int kl   = wave % pt.gkv;
        const int kvh0 = kvh - kl;   // first kv head of the workgroup's group
        for (int e = tid; e < pt.gkv * G * (D / 4); e += kDecThreads) {
            const int hg = e / (D / 4);   // (kv head of the group, q head) pair
            const int el = hg % pt.gkv;
            const int h  = hg / pt.gkv;
            const int d0 = 4 * (e - hg * (D / 4));
            float     M  = -INFINITY;
#pragma unroll
            for (int j = 0; j < kDecWaves; ++j) {
                if (j < wpk) {
                    M = fmaxf(M, sm_m[el + j * pt.gkv][h]);
                }
            }
            f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < kDecWaves; ++j) {
                if (j < wpk) {
                    const float mw = sm_m[el + j * pt.gkv][h];
                    const float w  = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
                    a += *reinterpret_cast<const f32x4*>(&sm_o[el + j * pt.gkv][h * D + d0]) * w;
                }
            }
            const int64_t row  = kMulti ? mrow(kvh0 + el, h) : (kvh0 + el) * G + h;
            const int64_t slot = row * num_splits + si;
            if (!kMulti || row >= 0) {
                *reinterpret_cast<f32x4*>(&part_o[slot * D + d0]) = a;
            }
        }
        if (tid < pt.gkv * G) {
            const int el = tid % pt.gkv;
            const int h  = tid / pt.gkv;
            float     M  = -INFINITY;
#pragma unroll
            for (int j = 0; j < kDecWaves; ++j) {
                if (j < wpk) {
                    M = fmaxf(M, sm_m[el + j * pt.gkv][h]);
                }
            }
            float L = 0.0f;
#pragma unroll
            for (int j = 0; j < kDecWaves; ++j) {
                if (j < wpk) {
                    const float mw = sm_m[el + j * pt.gkv][h];
                    L += (mw == -INFINITY) ? 0.0f : sm_l[el + j * pt.gkv][h] * __builtin_amdgcn_exp2f(mw - M);
                }
            }
            const int64_t row  = kMulti ? mrow(kvh0 + el, h) : (kvh0 + el) * G + h;
            const int64_t slot = row * num_splits + si;
            if (!kMulti || row >= 0) {
                part_m[slot] = M;
                part_l[slot] = L;
            }
        }
    } else {
        // Straight from the MFMA layout: lane (n, g) holds, for each r, the
        // kOMfma consecutive values d = kVBytes * (4g + r) + c of q head n
        // (oacc[c][r]), so it stores them as 16-byte runs with no LDS pass.
        if (kMulti ? row_n >= 0 : n < G) {
            const int64_t row  = kMulti ? row_n : kvh * G + n;
            const int64_t slot = row * num_splits + si;
            float*        po   = part_o + slot * D;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
#pragma unroll
                for (int c = 0; c < T::kOMfma; c += 4) {
                    *reinterpret_cast<f32x4*>(po + T::kVBytes * (4 * g + r) + c) =
                        f32x4{oacc[c][r], oacc[c + 1][r], oacc[c + 2][r], oacc[c + 3][r]};
                }
            }
        }
        if (g == 0 && (kMulti ? row_n >= 0 : n < G)) {
            const int64_t row  = kMulti ? row_n : kvh * G + n;
            const int64_t slot = row * num_splits + si;
            part_m[slot]       = m_run;
            part_l[slot]       = l_run;
        }
    }
}

template <int D, bool kAppend, bool kPaged>
__global__ __launch_bounds__(kDecThreads) void flash_decode_kernel(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ k,
    const uint8_t* __restrict__ v, const float* __restrict__ ks,
    const float* __restrict__ vs, float* __restrict__ partial, int num_splits,
    const int* __restrict__ cache_len, int hq, int hkv, float scale_log2,
    const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
    uint8_t* k_w, uint8_t* v_w, float* ks_w, float* vs_w,
    const int* __restrict__ block_table, int block_shift, int kvg, int nqb) {
    decode_body<D, kAppend, kPaged, false>(q, k, v, ks, vs, partial, num_splits, cache_len, hq,
                                           hkv, scale_log2, k_new, v_new, k_w, v_w, ks_w, vs_w,
                                           block_table, block_shift, kvg, nqb, nullptr,
                                           nullptr);
}

// A causal prefill call of a few tokens over a long cache as split-K decode:
// every (token, kv head) a virtual kv head (see decode_body's kMulti).
template <int D, bool kPaged>
__global__ __launch_bounds__(kDecThreads) void flash_decode_multi_kernel(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ k,
    const uint8_t* __restrict__ v, const float* __restrict__ ks,
    const float* __restrict__ vs, float* __restrict__ partial, int num_splits,
    const int* __restrict__ cache_len, int hq, int hkv, float scale_log2,
    const int* __restrict__ block_table, int block_shift, int kvg, int nqb, int n_tok,
    int hq_real, int tb) {
    decode_body<D, false, kPaged, false, false, true>(
        q, k, v, ks, vs, partial, num_splits, cache_len, hq, hkv, scale_log2, nullptr, nullptr,
        nullptr, nullptr, nullptr, nullptr, block_table, block_shift, kvg, nqb, nullptr, nullptr,
        nullptr, nullptr, 0.0f, n_tok, hq_real, tb);
}

// The decode step with RoPE fused: rope of q and of the appended k row, the
// append, and the split partials (the merge kernel follows as usual).
template <int D, bool kPaged>
__global__ __launch_bounds__(kDecThreads) void flash_decode_rope_kernel(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ k,
    const uint8_t* __restrict__ v, const float* __restrict__ ks,
    const float* __restrict__ vs, float* __restrict__ partial, int num_splits,
    const int* __restrict__ cache_len, int hq, int hkv, float scale_log2,
    const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
    uint8_t* k_w, uint8_t* v_w, float* ks_w, float* vs_w,
    const int* __restrict__ block_table, int block_shift, int kvg, int nqb,
    const int* __restrict__ positions, const float* __restrict__ inv_freq) {
    decode_body<D, true, kPaged, true>(q, k, v, ks, vs, partial, num_splits, cache_len, hq, hkv,
                                       scale_log2, k_new, v_new, k_w, v_w, ks_w, vs_w,
                                       block_table, block_shift, kvg, nqb, positions, inv_freq);
}

// The Qwen3 decode step: per-head RMSNorm of q and of the appended k row,
// then RoPE, the append and the split partials.
template <int D, bool kPaged>
__global__ __launch_bounds__(kDecThreads) void flash_decode_qk_norm_rope_kernel(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ k,
    const uint8_t* __restrict__ v, const float* __restrict__ ks,
    const float* __restrict__ vs, float* __restrict__ partial, int num_splits,
    const int* __restrict__ cache_len, int hq, int hkv, float scale_log2,
    const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
    uint8_t* k_w, uint8_t* v_w, float* ks_w, float* vs_w,
    const int* __restrict__ block_table, int block_shift, int kvg, int nqb,
    const int* __restrict__ positions, const float* __restrict__ inv_freq,
    const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm, float eps) {
    decode_body<D, true, kPaged, true, true>(q, k, v, ks, vs, partial, num_splits, cache_len, hq,
                                             hkv, scale_log2, k_new, v_new, k_w, v_w, ks_w, vs_w,
                                             block_table, block_shift, kvg, nqb, positions,
                                             inv_freq, q_norm, k_norm, eps);
}

// Maximum over the whole wave, every lane ending with it: DPP exchanges
// inside each 16-lane row (quad xor 1, xor 2, half-row and row mirrors),
// then the two cross-row swaps; no LDS traffic.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float wave_max_all(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));    // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f<0x4E>(v));    // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f<0x141>(v));   // row_half_mirror
    v = fmaxf(v, dpp_f<0x140>(v));   // row_mirror
    v = fmaxf(v, wave_xor_partner(v, 16));
    return fmaxf(v, wave_xor_partner(v, 32));
}

// Sum over the lanes of a wave that share lane % kQuads (the merge's
// groups of kQuads lanes): rotations inside each 16-lane row, then the two
// cross-row swaps.
template <int kQuads>
__device__ __forceinline__ float quad_group_sum(float v) {
    static_assert(kQuads >= 2 && kQuads <= 64 && (kQuads & (kQuads - 1)) == 0,
                  "groups of 2 .. 64 lanes");
    if constexpr (kQuads == 2) {
        v += dpp_f<0x122>(v);   // row_ror:2
    }
    if constexpr (kQuads <= 4) {
        v += dpp_f<0x124>(v);   // row_ror:4
    }
    if constexpr (kQuads <= 8) {
        v += dpp_f<0x128>(v);   // row_ror:8
    }
    if constexpr (kQuads <= 16) {
        v += wave_xor_partner(v, 16);
    }
    if constexpr (kQuads <= 32) {
        v += wave_xor_partner(v, 32);
    }
    return v;
}

// One workgroup per (q head, 16-wide slice of head_dim): merges the n_eff
// split partials, out = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s
// (reference src/kernels/flash_decode.cu:222-247), in two passes so that no
// exponential sits in a reduction tree: every wave first takes M, the
// maximum of the head's live m_s, from the m row itself (four coalesced
// loads per lane for up to 256 splits, a wave reduction); then thread (group grp,
// quad qd) sums 2^(m_s - M) l_s and 2^(m_s - M) acc_s for splits grp,
// grp + kGroups, ... and d = 4qd .. 4qd+3 of the slice (weights <= 1, eight
// loads in flight), and the sums add up by lane exchanges and one LDS step.
// The first loads are issued before the split count is known (slot indices
// clamped into the scratch), so they share one round trip with the read of
// *cache_len; slots no split wrote in this call are dropped by a select.
// kSlice: the head_dim slice of a workgroup (the multi-token launches take
// whole rows: many rows, few splits).
template <int D, int kSlice = kCombineSlice>
__global__ __launch_bounds__(kCombineThreads) void flash_decode_combine_kernel(
    uint16_t* __restrict__ out, const float* __restrict__ partial, int num_splits,
    const int* __restrict__ cache_len, int hq, int kvg, int xl_g, int append, int n_tok,
    int run_min = 0) {
    static_assert(D % kSlice == 0, "slices tile the row");
    constexpr int kQuads  = kSlice / 4;
    constexpr int kGroups = kCombineThreads / kQuads;
    constexpr int kCWaves = kCombineThreads / kWave;
    static_assert((kQuads & (kQuads - 1)) == 0 && kQuads <= kWave, "lane = kQuads * group + quad");
    __shared__ __attribute__((aligned(16))) f32x4 sm_acc[kCWaves][kQuads];
    __shared__ float sm_ll[kCWaves];

    // xl_g > 0 (an XCD-local shape, xl_g q heads per kv head): workgroup L
    // (on XCD L % 8) takes a (q head, slice) of a kv head on that XCD. With
    // one tile per split the split kernel wrote that kv head's partials on
    // the same XCD (dec_xcd_local); otherwise they are spread over all XCDs
    // whichever head a workgroup takes, so the assignment needs no
    // *cache_len and the first loads go out before that read.
    int qh, dsl;
    if (xl_g > 0) {
        constexpr int kSlices = D / kSlice;
        const int     L       = static_cast<int>(blockIdx.x + blockIdx.y * gridDim.x);
        const int     m       = L >> 3;
        const int     t       = m / kSlices;
        qh  = ((t / xl_g) * 8 + (L & 7)) * xl_g + t % xl_g;
        dsl = (m % kSlices) * kSlice;
    } else {
        qh  = static_cast<int>(blockIdx.x);
        dsl = static_cast<int>(blockIdx.y) * kSlice;
    }
    const int tid  = static_cast<int>(threadIdx.x);
    const int grp  = tid / kQuads;
    const int qd   = tid - grp * kQuads;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);

    const int64_t hs     = static_cast<int64_t>(hq) * num_splits;
    const float*  part_m = partial + static_cast<int64_t>(qh) * num_splits;
    const float*  part_l = partial + hs + static_cast<int64_t>(qh) * num_splits;
    const float*  part_o = partial + 2 * hs + static_cast<int64_t>(qh) * num_splits * D + dsl;

    float ms[8], ls[8];
    f32x4 os[8];
    // Unconditional loads of slots s0 + u * kGroups, clamped to slot `cap`.
    auto load8 = [&](int s0, int cap) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int s = min(s0 + u * kGroups, cap);
            ms[u]       = part_m[s];
            ls[u]       = part_l[s];
            os[u]       = *reinterpret_cast<const f32x4*>(&part_o[static_cast<int64_t>(s) * D + 4 * qd]);
        }
    };
    load8(grp, num_splits - 1);
    // The m row for M: slots lane + 64 e, e < 4 (then the next 256, ...).
    float mr[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        mr[e] = part_m[min(lane + kWave * e, num_splits - 1)];
    }
    const int n_keys = *cache_len + n_tok;   // the last (or only) token's keys
    // Live slots: as the split kernel derives them (an append call's key may
    // hold a slot of its own).
    const int cache_t = (n_keys + kTileKeys - 2) / kTileKeys;
    int       n_eff   = (append != 0 && cache_t <= 2 * (num_splits - 1))
                            ? min(num_splits - 1, cache_t) + 1
                            : dec_partition(n_keys, num_splits, kvg).n_eff;
    if (kSlice == D && run_min > 0) {   // the flash prefill's key runs (64-key tiles)
        const int tiles = (n_keys + 63) / 64;
        const int per   = max((tiles + num_splits - 1) / num_splits, run_min);
        n_eff           = (tiles + per - 1) / per;
        if (n_eff == 1) {   // run 0 stored the output itself
            return;
        }
    }
    float     M       = -INFINITY;
    for (int s0 = 0;; s0 += 4 * kWave) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (s0 + lane + kWave * e < n_eff) {
                M = fmaxf(M, mr[e]);
            }
        }
        if (s0 + 4 * kWave >= n_eff) {
            break;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            mr[e] = part_m[min(s0 + 4 * kWave + lane + kWave * e, num_splits - 1)];
        }
    }
    M = wave_max_all(M);

    float l   = 0.0f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    // Adds the loaded slots below n_eff; the others may hold anything (NaN
    // included), so they are selected away, never multiplied by zero.
    auto fold = [&](int s0) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const bool  live = s0 + u * kGroups < n_eff;
            const float f    = live ? __builtin_amdgcn_exp2f(ms[u] - M) : 0.0f;
            // Whole-row merges: a slot with m = -inf may hold no O at all.
            const bool  use  = kSlice == D ? (live && ms[u] != -INFINITY) : live;
            const f32x4 o    = use ? os[u] : f32x4{0.f, 0.f, 0.f, 0.f};
            acc += o * f;
            l += (live ? ls[u] : 0.0f) * f;
        }
    };
    fold(grp);
    for (int s0 = grp + 8 * kGroups; s0 < n_eff; s0 += 8 * kGroups) {
        load8(s0, n_eff - 1);
        fold(s0);
    }
    // The groups of a wave differ in the lane bits above the quad index.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        acc[e] = quad_group_sum<kQuads>(acc[e]);
    }
    l = quad_group_sum<kQuads>(l);
    if (lane < kQuads) {
        sm_acc[wave][lane] = acc;
        if (lane == 0) {
            sm_ll[wave] = l;
        }
    }
    __syncthreads();
    if (wave == 0 && lane < kQuads) {
#pragma unroll
        for (int w = 1; w < kCWaves; ++w) {
            acc += sm_acc[w][lane];
            l += sm_ll[w];
        }
        const float inv = __builtin_amdgcn_rcpf(l);   // 1 ulp; the output is bf16
        u32x2       w2;
        w2.x = pack_bf16x2(acc[0] * inv, acc[1] * inv);
        w2.y = pack_bf16x2(acc[2] * inv, acc[3] * inv);
        *reinterpret_cast<u32x2*>(out + static_cast<int64_t>(qh) * D + dsl + 4 * lane) = w2;
    }
}

// Serves the shapes the MFMA kernel does not (head_dim 32 and 512, GQA groups
// that do not split into blocks of 4-16 q heads) with the same partition (one
// wave per (kv head, split, block of kVGroup q heads) unit at every context;
// kvg = 0 for the merge), the same scratch and the same merge kernel. No
// MFMA: a key row of D E4M3 bytes is spread over D / 16 lanes, 16 bytes per
// lane (one coalesced 128-bit load of K and one of V), so a wave takes
// 64 / (D / 16) keys per step. Each lane
// converts its 16 codes exactly to bf16 (K) and fp32 (V) in registers, takes
// its share of q . k with v_dot2c_f32_bf16, and the partial dots of a key
// are summed by DPP row exchanges (quad_perm, row_half_mirror, row_mirror:
// after each level every lane of the group holds the group sum) plus one
// lane shuffle per level above 16 lanes. Every lane group
// keeps its own online softmax over its keys (base 2, lazy reference as in
// the MFMA kernel) and its 16 output columns of each q head; the lane groups
// merge by lane shuffles at the end, and lane group 0 writes the partial.
constexpr int kVGroup = 4;   // q heads per VALU unit

template <int D>
struct ValuTraits {
    static_assert(D == 32 || D == 64 || D == 128 || D == 256 || D == 512,
                  "VALU decode: D in {32, 64, 128, 256, 512}");
    static constexpr int kLPK  = D / 16;         // lanes per key row
    static constexpr int kKPS  = kWave / kLPK;   // keys per wave step
    static constexpr int kRing = 4;              // steps in flight per wave
};


template <int D>
struct ValuStep {
    u32x4 kraw;
    u32x4 vraw;
    float ksc;
    float vsc;
};

template <int D, bool kNT>
__device__ __forceinline__ void valu_load(ValuStep<D>& st, const uint8_t* __restrict__ k,
                                          const uint8_t* __restrict__ v,
                                          const float* __restrict__ ks,
                                          const float* __restrict__ vs, int key, int kvh,
                                          int hkv, int j) {
    const int64_t row = static_cast<int64_t>(key) * hkv + kvh;
    st.kraw           = ld<kNT>(reinterpret_cast<const u32x4*>(k + row * D + 16 * j));
    st.vraw           = ld<kNT>(reinterpret_cast<const u32x4*>(v + row * D + 16 * j));
    st.ksc            = ks[row];
    st.vsc            = vs[row];
}

template <int D>
__global__ __launch_bounds__(kDecThreads) void flash_decode_valu_kernel(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ k,
    const uint8_t* __restrict__ v, const float* __restrict__ ks,
    const float* __restrict__ vs, float* __restrict__ partial, int num_splits,
    const int* __restrict__ cache_len, int hq, int hkv, float scale_log2) {
    using T = ValuTraits<D>;
    const int G    = hq / hkv;
    const int nb   = (G + kVGroup - 1) / kVGroup;
    const int tid  = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid & (kWave - 1);
    const int kl   = lane / T::kLPK;   // key of the step this lane works on
    const int j    = lane % T::kLPK;   // 16-byte chunk of the row
    const int          n_keys = *cache_len + 1;
    const DecPartition pt     = dec_partition(n_keys, num_splits, 0);
    // unit = ((split * hkv) + kv head) * nb + head block. Splits of up to
    // three tiles: wave w of workgroup b takes unit w * grid + b, so that a
    // short context's live units (the first ones) sit one per workgroup and
    // no compute unit holds more than one loading wave, and with 8 kv heads
    // of one head block a workgroup's waves are splits of kv head b % 8 (the
    // XCD of workgroup b). Longer splits: unit b * 8 + w, the head blocks of
    // one (kv head, split) in adjacent waves reading the same rows, the kv
    // heads of one split sharing the interleaved scale lines in L1.
    // (24Q/8KV, D 128, per call: 35 keys 15.0 -> 12.2 us, 2041 keys 16.4 ->
    // 14.2, 8196 keys 21.9 -> 19.8, 20000 keys 25.6 -> 23.5; at 32768 keys,
    // four tiles per split, the strided form is 0.5 us slower.)
    const int bid   = static_cast<int>(blockIdx.x);
    const int n_wg  = static_cast<int>(gridDim.x);
    const int unit  = (pt.base <= 2) ? wave * n_wg + bid : bid * kDecWaves + wave;
    const int hb    = unit % nb;
    const int kvh   = (unit / nb) % hkv;
    const int si    = unit / nb / hkv;
    if (si >= pt.n_eff) {
        return;
    }
    const int k0 = split_tile(pt, si) * kTileKeys;
    const int k1 = min(split_tile(pt, si + 1) * kTileKeys, n_keys);
    const int h0 = hb * kVGroup;
    const int gh = min(kVGroup, G - h0);

    // q of the block's heads, this lane's 16 columns, as bf16 pairs.
    bf16x2 qv[kVGroup][8];
#pragma unroll
    for (int h = 0; h < kVGroup; ++h) {
        const uint16_t* qr = q + static_cast<int64_t>(kvh * G + h0 + min(h, gh - 1)) * D + 16 * j;
        u32x4           w0 = *reinterpret_cast<const u32x4*>(qr);
        u32x4           w1 = *reinterpret_cast<const u32x4*>(qr + 8);
        if (h >= gh) {
            w0 = u32x4{0u, 0u, 0u, 0u};
            w1 = w0;
        }
        // Elements go through a scalar first: hipcc (ROCm 7.2) miscompiles
        // __builtin_bit_cast of a vector subscript (it reads element 0).
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t a = w0[e];
            const uint32_t b = w1[e];
            qv[h][e]         = __builtin_bit_cast(bf16x2, a);
            qv[h][4 + e]     = __builtin_bit_cast(bf16x2, b);
        }
    }
    float acc[kVGroup][16];
    float m_run[kVGroup], l_run[kVGroup];
#pragma unroll
    for (int h = 0; h < kVGroup; ++h) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            acc[h][e] = 0.0f;
        }
    }

    constexpr float kLazy  = 8.0f;
    auto            process = [&](const ValuStep<D>& st, int key) {
        const bool valid = key < k1;
        // K codes -> 8 bf16 pairs (exact).
        bf16x2 kb[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            kb[2 * e]     = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(st.kraw[e], 1.0f, false);
            kb[2 * e + 1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(st.kraw[e], 1.0f, true);
        }
        // V codes -> 16 fp32 (exact).
        float vf[16];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const f32x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(st.vraw[e], 1.0f, false);
            const f32x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(st.vraw[e], 1.0f, true);
            vf[4 * e]      = lo.x;
            vf[4 * e + 1]  = lo.y;
            vf[4 * e + 2]  = hi.x;
            vf[4 * e + 3]  = hi.y;
        }
        const float kf = st.ksc * scale_log2;
#pragma unroll
        for (int h = 0; h < kVGroup; ++h) {
            float sd = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                sd = __builtin_amdgcn_fdot2_f32_bf16(qv[h][e], kb[e], sd, false);
            }
            const float x = group_sum<T::kLPK>(sd) * kf;
            if (valid && x > m_run[h] + kLazy) {
                const float alpha = __builtin_amdgcn_exp2f(m_run[h] - x);
                l_run[h] *= alpha;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    acc[h][e] *= alpha;
                }
                m_run[h] = x;
            }
            const float p = valid ? __builtin_amdgcn_exp2f(x - m_run[h]) : 0.0f;
            l_run[h] += p;
            const float pv = p * st.vsc;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                acc[h][e] = fmaf(pv, vf[e], acc[h][e]);
            }
        }
    };

    const int n_steps = (k1 - k0 + T::kKPS - 1) / T::kKPS;
    if (n_steps > 0) {
        auto key_of_step = [&](int st) { return k0 + st * T::kKPS + kl; };
        auto stream      = [&]<bool kNT>() {
            constexpr int  R = T::kRing;
            ValuStep<D>    ring[R];
            const int      last = n_steps - 1;
#pragma unroll
            for (int r = 0; r + 1 < R; ++r) {
                const int key = min(key_of_step(min(r, last)), k1 - 1);
                valu_load<D, kNT>(ring[r], k, v, ks, vs, key, kvh, hkv, j);
            }
            for (int t = 0;; t += R) {
                bool done = false;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    if (!done) {
                        const int tr  = t + r;
                        const int key = min(key_of_step(min(tr + R - 1, last)), k1 - 1);
                        valu_load<D, kNT>(ring[(r + R - 1) % R], k, v, ks, vs, key, kvh, hkv,
                                          j);
                        process(ring[r], key_of_step(tr));
                        done = tr >= last;
                    }
                }
                if (done) {
                    break;
                }
            }
        };
        if (n_steps > kValuNtMinSteps) {
            stream.template operator()<true>();
        } else {
            stream.template operator()<false>();
        }
    }

    // Merge the lane groups (lanes j, j + kLPK, ... hold the same columns).
#pragma unroll
    for (int mask = T::kLPK; mask < kWave; mask <<= 1) {
#pragma unroll
        for (int h = 0; h < kVGroup; ++h) {
            const float m2 = wave_xor_partner(m_run[h], mask);
            const float l2 = wave_xor_partner(l_run[h], mask);
            const float M  = fmaxf(m_run[h], m2);
            const float f1 = (m_run[h] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run[h] - M);
            const float f2 = (m2 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m2 - M);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float a2 = wave_xor_partner(acc[h][e], mask);
                acc[h][e]      = acc[h][e] * f1 + a2 * f2;
            }
            l_run[h] = l_run[h] * f1 + l2 * f2;
            m_run[h] = M;
        }
    }
    if (kl == 0) {
        const int64_t hs     = static_cast<int64_t>(hq) * num_splits;
        float*        part_m = partial;
        float*        part_l = partial + hs;
        float*        part_o = partial + 2 * hs;
#pragma unroll
        for (int h = 0; h < kVGroup; ++h) {
            if (h < gh) {
                const int64_t slot = static_cast<int64_t>(kvh * G + h0 + h) * num_splits + si;
                float*        o    = part_o + slot * D + 16 * j;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    *reinterpret_cast<f32x4*>(o + 4 * e) =
                        f32x4{acc[h][4 * e], acc[h][4 * e + 1], acc[h][4 * e + 2], acc[h][4 * e + 3]};
                }
                if (j == 0) {
                    part_m[slot] = m_run[h];
                    part_l[slot] = l_run[h];
                }
            }
        }
    }
}

template <int D>
hipError_t launch_decode_valu(uint16_t* out, const uint16_t* q, const uint8_t* k,
                              const uint8_t* v, const float* ks, const float* vs,
                              float* partial, int num_splits, const int* cache_len, int hq,
                              int hkv, float scale, hipStream_t stream) {
    const int     nb    = (hq / hkv + kVGroup - 1) / kVGroup;
    const int64_t units = static_cast<int64_t>(num_splits) * hkv * nb;
    const int     n_wgs = static_cast<int>((units + kDecWaves - 1) / kDecWaves);
    hipLaunchKernelGGL(flash_decode_valu_kernel<D>, dim3(static_cast<unsigned>(n_wgs)),
                       dim3(kDecThreads), 0, stream, q, k, v, ks, vs, partial, num_splits,
                       cache_len, hq, hkv, scale * kLog2e);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return e;
    }
    hipLaunchKernelGGL(flash_decode_combine_kernel<D>,
                       dim3(static_cast<unsigned>(hq), static_cast<unsigned>(D / kCombineSlice)),
                       dim3(kCombineThreads), 0, stream, out, partial, num_splits, cache_len,
                       hq, 0, 0, 0, 1);
    return hipGetLastError();
}

__global__ void advance_position_kernel(int* pos, int delta) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        *pos += delta;
    }
}

template <int D, bool kPaged>
hipError_t launch_decode(uint16_t* out, const uint16_t* q, const uint8_t* k,
                         const uint8_t* v, const float* ks, const float* vs,
                         float* partial, int num_splits, const int* cache_len,
                         int hq, int hkv, float scale, const uint16_t* k_new,
                         const uint16_t* v_new, uint8_t* k_w, uint8_t* v_w, float* ks_w,
                         float* vs_w, const int* block_table, int block_shift,
                         hipStream_t stream, const int* positions, const float* inv_freq,
                         const uint16_t* q_norm, const uint16_t* k_norm, float eps) {
    int        cus = 0;
    hipError_t ce  = device_cu_count(&cus);
    if (ce != hipSuccess) {
        return ce;
    }
    const int nqb = dec_q_blocks(hq, hkv, D);
    if (nqb == 0) {
        return hipErrorInvalidValue;
    }
    const int  hkv_v = hkv * nqb;   // virtual kv heads of at most 16 q heads each
    const int  kvg   = dec_group_kv(num_splits, hkv_v, cus);
    const int  n_wgs = dec_workgroups(num_splits, hkv_v, kvg);
    const dim3 grid(static_cast<unsigned>(n_wgs));
    if (q_norm != nullptr) {
        if (k_new == nullptr || inv_freq == nullptr || positions == nullptr ||
            k_norm == nullptr) {
            return hipErrorInvalidValue;
        }
        hipLaunchKernelGGL((flash_decode_qk_norm_rope_kernel<D, kPaged>), grid,
                           dim3(kDecThreads), 0, stream, q, k, v, ks, vs, partial, num_splits,
                           cache_len, hq, hkv_v, scale * kLog2e, k_new, v_new, k_w, v_w, ks_w,
                           vs_w, block_table, block_shift, kvg, nqb, positions, inv_freq,
                           q_norm, k_norm, eps);
    } else if (positions != nullptr) {
        if (k_new == nullptr || inv_freq == nullptr) {
            return hipErrorInvalidValue;
        }
        hipLaunchKernelGGL((flash_decode_rope_kernel<D, kPaged>), grid, dim3(kDecThreads), 0,
                           stream, q, k, v, ks, vs, partial, num_splits, cache_len, hq, hkv_v,
                           scale * kLog2e, k_new, v_new, k_w, v_w, ks_w, vs_w, block_table,
                           block_shift, kvg, nqb, positions, inv_freq);
    } else if (k_new != nullptr) {
        hipLaunchKernelGGL((flash_decode_kernel<D, true, kPaged>), grid, dim3(kDecThreads), 0,
                           stream, q, k, v, ks, vs, partial, num_splits, cache_len, hq, hkv_v,
                           scale * kLog2e, k_new, v_new, k_w, v_w, ks_w, vs_w, block_table,
                           block_shift, kvg, nqb);
    } else {
        hipLaunchKernelGGL((flash_decode_kernel<D, false, kPaged>), grid, dim3(kDecThreads), 0,
                           stream, q, k, v, ks, vs, partial, num_splits, cache_len, hq, hkv_v,
                           scale * kLog2e, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                           block_table, block_shift, kvg, nqb);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return e;
    }
    hipLaunchKernelGGL(flash_decode_combine_kernel<D>,
                       dim3(static_cast<unsigned>(hq), static_cast<unsigned>(D / kCombineSlice)),
                       dim3(kCombineThreads), 0, stream, out, partial, num_splits,
                       cache_len, hq, kvg,
                       (kvg == 0 && dec_xcd_local(hkv_v, num_splits)) ? hq / hkv_v : 0,
                       k_new != nullptr ? 1 : 0, 1);
    return hipGetLastError();
}

// A causal prefill call of n_tok tokens over the cache as split-K decode:
// the split kernel over n_tok x Hkv (x q blocks) virtual kv heads, then the
// merge over the n_tok x Hq rows of out. Scratch: the decode layout for
// n_tok * Hq q heads.
template <int D, bool kPaged>
hipError_t launch_prefill_split(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                const uint8_t* v, const float* ks, const float* vs,
                                float* partial, int num_splits, int n_tok,
                                const int* cache_len, int hq, int hkv, float scale,
                                const int* block_table, int block_shift, hipStream_t stream) {
    int        cus = 0;
    hipError_t ce  = device_cu_count(&cus);
    if (ce != hipSuccess) {
        return ce;
    }
    const int nqb = dec_q_blocks(hq, hkv, D);
    if (nqb == 0) {
        return hipErrorInvalidValue;
    }
    // Tokens per virtual kv head: as many as fill the MFMA's 16 columns (and
    // a wave's LDS staging row) with the block's q heads.
    const int gb  = hq / hkv / nqb;
    const int tb  = std::max(1, std::min({16 / gb, kMaxGroupD / (gb * D), n_tok}));
    const int ntb = (n_tok + tb - 1) / tb;
    const int  hq_v  = hq * n_tok;                 // rows of out and of the partials
    const int  hkv_v = hkv * nqb * ntb;
    const int  kvg   = dec_group_kv(num_splits, hkv_v, cus);
    const int  n_wgs = dec_workgroups(num_splits, hkv_v, kvg);
    hipLaunchKernelGGL((flash_decode_multi_kernel<D, kPaged>), dim3(static_cast<unsigned>(n_wgs)),
                       dim3(kDecThreads), 0, stream, q, k, v, ks, vs, partial, num_splits,
                       cache_len, hkv_v * tb * gb, hkv_v, scale * kLog2e, block_table,
                       block_shift, kvg, nqb, n_tok, hq, tb);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return e;
    }
    const int xl_g = (tb == 1 && kvg == 0 && dec_xcd_local(hkv_v, num_splits)) ? hq_v / hkv_v : 0;
    if (n_tok == 1) {   // the decode call's merge: results identical to it
        hipLaunchKernelGGL(flash_decode_combine_kernel<D>,
                           dim3(static_cast<unsigned>(hq_v), static_cast<unsigned>(D / kCombineSlice)),
                           dim3(kCombineThreads), 0, stream, out, partial, num_splits, cache_len,
                           hq_v, kvg, xl_g, 0, n_tok);
    } else {
        // Whole-row merge workgroups: n_tok * Hq rows of few splits each
        // (16-wide slices launch 8x the workgroups for the same loads: 32 tokens
        // after 8K keys 30.3 -> 23.9 us per call, at an empty cache 14.2 -> 7.8).
        hipLaunchKernelGGL((flash_decode_combine_kernel<D, D>), dim3(static_cast<unsigned>(hq_v)),
                           dim3(kCombineThreads), 0, stream, out, partial, num_splits, cache_len,
                           hq_v, kvg, xl_g, 0, n_tok);
    }
    return hipGetLastError();
}

// Decode scratch of the allocation-free entry point: one fixed array per
// device, shared by every call on that device (the reference layout, the
// first Hq*S*(D+2) floats in use). The kernels need it uninitialized, and
// calls that overlap on one device race on it. In host code `scratch` is a
// host-side stand-in: its device address comes from hipGetSymbolAddress.
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

constexpr int      kMaxScratchDevices = 64;
std::mutex         g_scratch_mu;
float*             g_scratch_ptr[kMaxScratchDevices];   // nullptr: not looked up yet

}  // namespace

hipError_t noalloc_scratch(float** ptr) {
    int        dev = 0;
    hipError_t e   = hipGetDevice(&dev);
    if (e != hipSuccess) {
        return e;
    }
    if (dev < 0 || dev >= kMaxScratchDevices) {
        return hipErrorInvalidDevice;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e       = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) {
            return e;
        }
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *ptr = g_scratch_ptr[dev];
    return hipSuccess;
}

std::size_t decode_scratch_floats(int num_q_heads, int head_dim, int max_splits) {
    const std::size_t hs = static_cast<std::size_t>(num_q_heads) *
                           static_cast<std::size_t>(max_splits);
    return hs * 2 + hs * static_cast<std::size_t>(head_dim);
}

bool decode_mfma_supported(int num_q_heads, int num_kv_heads, int head_dim) {
    return dec_q_blocks(num_q_heads, num_kv_heads, head_dim) > 0;
}

hipError_t flash_decode_launch(uint16_t* out, const uint16_t* q,
                               const uint8_t* k, const uint8_t* v,
                               const float* k_scale, const float* v_scale,
                               float* partial, int num_splits,
                               const int* cache_len, int num_q_heads,
                               int num_kv_heads, int head_dim, float scale,
                               hipStream_t stream, const uint16_t* k_new,
                               const uint16_t* v_new, uint8_t* k_w, uint8_t* v_w,
                               float* ks_w, float* vs_w, const int* block_table,
                               int block_shift, const int* positions, const float* inv_freq,
                               const uint16_t* q_norm, const uint16_t* k_norm, float eps) {
    const bool paged = block_table != nullptr;
    switch (head_dim) {
#define RTH_DEC_CASE(DD)                                                                      \
    case DD:                                                                                  \
        return paged ? launch_decode<DD, true>(out, q, k, v, k_scale, v_scale, partial,       \
                                               num_splits, cache_len, num_q_heads,            \
                                               num_kv_heads, scale, k_new, v_new, k_w, v_w,   \
                                               ks_w, vs_w, block_table, block_shift, stream,  \
                                               positions, inv_freq, q_norm, k_norm, eps)      \
                     : launch_decode<DD, false>(out, q, k, v, k_scale, v_scale, partial,      \
                                                num_splits, cache_len, num_q_heads,           \
                                                num_kv_heads, scale, k_new, v_new, k_w, v_w,  \
                                                ks_w, vs_w, nullptr, 0, stream, positions,    \
                                                inv_freq, q_norm, k_norm, eps);
        RTH_DEC_CASE(64)
        RTH_DEC_CASE(128)
        RTH_DEC_CASE(256)
#undef RTH_DEC_CASE
        default:
            return hipErrorInvalidValue;
    }
}

hipError_t flash_prefill_split_launch(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                     const uint8_t* v, const float* k_scale,
                                     const float* v_scale, float* partial, int num_splits,
                                     int n_new, const int* cache_len, int num_q_heads,
                                     int num_kv_heads, int head_dim, float scale,
                                     hipStream_t stream, const int* block_table,
                                     int block_shift) {
    const bool paged = block_table != nullptr;
    switch (head_dim) {
#define RTH_PFS_CASE(DD)                                                                      \
    case DD:                                                                                  \
        return paged ? launch_prefill_split<DD, true>(out, q, k, v, k_scale, v_scale, partial, \
                                                      num_splits, n_new, cache_len,           \
                                                      num_q_heads, num_kv_heads, scale,       \
                                                      block_table, block_shift, stream)       \
                     : launch_prefill_split<DD, false>(out, q, k, v, k_scale, v_scale,        \
                                                       partial, num_splits, n_new, cache_len, \
                                                       num_q_heads, num_kv_heads, scale,      \
                                                       nullptr, 0, stream);
        RTH_PFS_CASE(64)
        RTH_PFS_CASE(128)
        RTH_PFS_CASE(256)
#undef RTH_PFS_CASE
        default:
            return hipErrorInvalidValue;
    }
}

hipError_t split_rows_merge_launch(uint16_t* out, const float* partial, int num_splits,
                                  const int* cache_len, int rows, int n_tok, int head_dim,
                                  hipStream_t stream, int run_min) {
    switch (head_dim) {
#define RTH_MERGE_CASE(DD)                                                                    \
    case DD:                                                                                  \
        hipLaunchKernelGGL((flash_decode_combine_kernel<DD, DD>),                            \
                           dim3(static_cast<unsigned>(rows)), dim3(kCombineThreads), 0,      \
                           stream, out, partial, num_splits, cache_len, rows, 0, 0, 0, n_tok,  \
                           run_min);                                                           \
        return hipGetLastError();
        RTH_MERGE_CASE(64)
        RTH_MERGE_CASE(128)
        RTH_MERGE_CASE(256)
#undef RTH_MERGE_CASE
        default:
            return hipErrorInvalidValue;
    }
}

hipError_t flash_decode_valu_launch(uint16_t* out, const uint16_t* q, const uint8_t* k,
                                   const uint8_t* v, const float* k_scale,
                                   const float* v_scale, float* partial, int num_splits,
                                   const int* cache_len, int num_q_heads, int num_kv_heads,
                                   int head_dim, float scale, hipStream_t stream) {
    switch (head_dim) {
#define RTH_VALU_CASE(DD)                                                                     \
    case DD:                                                                                  \
        return launch_decode_valu<DD>(out, q, k, v, k_scale, v_scale, partial, num_splits,   \
                                      cache_len, num_q_heads, num_kv_heads, scale, stream);
        RTH_VALU_CASE(32)
        RTH_VALU_CASE(64)
        RTH_VALU_CASE(128)
        RTH_VALU_CASE(256)
        RTH_VALU_CASE(512)
#undef RTH_VALU_CASE
        default:
            return hipErrorInvalidValue;
    }
}

hipError_t advance_position_launch(int* pos, int delta, hipStream_t stream) {
    hipLaunchKernelGGL(advance_position_kernel, dim3(1), dim3(64), 0, stream, pos, delta);
    return hipGetLastError();
}

}  // namespace rth
