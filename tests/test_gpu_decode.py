"""Split-K flash decode on the GPU against the oracle (reference
src/kernels/flash_decode.cu; cases of tests/kernels/test_flash_decode.cpp:
148-170 plus the BASELINE configurations). Tolerance: max-abs 2e-2,
mean-abs 2e-3 on bf16 outputs."""
import numpy as np
import pytest
import torch

import oracle_lib as O
import runtherder_amd as R
from gpu_util import (DEV, NTHREADS, bf16_dev, bf16_host, f32_dev, int_dev, step, sync,
                      u8_dev)

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def make_cache(total, hkv, d, kind="mt", seed=0, per_head_scale=None):
    if kind == "mt":
        kx = O.mt19937_uniform_bf16((total * hkv, d), 1.0, 0xB0B)
        vx = O.mt19937_uniform_bf16((total * hkv, d), 1.0, 0xCAFE)
    else:
        kx = O.normal_bf16((total * hkv, d), 1000 + seed)
        vx = O.normal_bf16((total * hkv, d), 2000 + seed)
    if per_head_scale is None:
        k8, ks = O.quantize_kv_fp8(kx, d)
        v8, vs = O.quantize_kv_fp8(vx, d)
    else:
        ks = np.tile(per_head_scale[0], total).astype(np.float32)
        vs = np.tile(per_head_scale[1], total).astype(np.float32)
        k8 = O.quantize_kv_fp8_scaled(kx, ks, d)
        v8 = O.quantize_kv_fp8_scaled(vx, vs, d)
    return kx, vx, k8, v8, ks, vs


def gpu_decode(q, k8, v8, ks, vs, cache_len, hq, hkv, d, splits, scale):
    step(f"decode ctx={cache_len + 1} hq={hq} hkv={hkv} d={d} splits={splits}")
    out = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    partial = R.new_flash_split_scratch(hq, d, splits)
    R.flash_decode_split_bf16(out, bf16_dev(q), u8_dev(k8), u8_dev(v8), f32_dev(ks),
                              f32_dev(vs), partial, splits, int_dev(cache_len), hq, hkv, d,
                              scale)
    sync()
    return bf16_host(out)


def check(got, q, k8, v8, ks, vs, cache_len, hq, hkv, d, scale):
    want = O.attention_f32(q, k8, v8, ks, vs, 1, cache_len, hq, hkv, d, scale, NTHREADS)
    mx, mean = O.bf16_err(got, want[0])
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)
    return mx, mean


@pytest.mark.parametrize("cache_len,hq,hkv,d,splits", [
    (300, 32, 8, 128, 4), (0, 32, 8, 128, 1), (2, 8, 2, 64, 8), (1000, 32, 8, 128, 8),
    (1000, 32, 8, 256, 8), (777, 16, 16, 64, 16), (99, 8, 1, 128, 3),
    (40, 32, 8, 32, 4), (40, 8, 2, 512, 4), (130, 64, 4, 128, 8),
])
def test_reference_cases(cache_len, hq, hkv, d, splits):
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.mt19937_uniform_bf16((hq, d), 1.0, 0xA11CE)
    _, _, k8, v8, ks, vs = make_cache(cache_len + 1, hkv, d)
    got = gpu_decode(q, k8, v8, ks, vs, cache_len, hq, hkv, d, splits, scale)
    check(got, q, k8, v8, ks, vs, cache_len, hq, hkv, d, scale)


@pytest.mark.parametrize("splits", [1, 2, 3, 8, 31, 32, 64, 100, 256])
def test_split_count_sweep(splits):
    hq, hkv, d, cache_len = 24, 8, 128, 2040
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((hq, d), 5)
    _, _, k8, v8, ks, vs = make_cache(cache_len + 1, hkv, d, kind="normal", seed=1)
    got = gpu_decode(q, k8, v8, ks, vs, cache_len, hq, hkv, d, splits, scale)
    check(got, q, k8, v8, ks, vs, cache_len, hq, hkv, d, scale)


@pytest.mark.parametrize("hq,hkv,d,splits", [
    (24, 8, 128, 32), (24, 8, 128, 64), (24, 8, 128, 96), (32, 4, 64, 64), (16, 2, 256, 128),
])
@pytest.mark.parametrize("where", ["short", "edge", "past"])
def test_grouped_workgroups_at_two_tiles_per_split(hq, hkv, d, splits, where):
    """Grouped (cooperative) launches of 1, 2 and 4 kv heads per workgroup
    on both sides of two 32-key tiles per split: up to two, the first wave
    of each kv head streams its split alone; one key more and the waves of
    a kv head share the tiles and merge in LDS."""
    n_keys = {"short": 33, "edge": 64 * splits, "past": 64 * splits + 1}[where]
    cache_len = n_keys - 1
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((hq, d), 17 + splits)
    _, _, k8, v8, ks, vs = make_cache(n_keys, hkv, d, kind="normal", seed=n_keys)
    step(f"grouped decode ctx={n_keys} splits={splits} hq={hq} hkv={hkv} d={d}")
    got = gpu_decode(q, k8, v8, ks, vs, cache_len, hq, hkv, d, splits, scale)
    check(got, q, k8, v8, ks, vs, cache_len, hq, hkv, d, scale)


@pytest.mark.parametrize("splits", [1, 16, 64])
def test_q_heads_of_extreme_magnitude(splits):
    """q heads scaled from zero and bf16 subnormals up to 2^6: scores several
    hundred apart across tiles and splits must raise the running maximum
    without overflow, and near-zero heads give the mean of V."""
    hq, hkv, d, cache_len = 32, 8, 128, 4999
    scale = np.float32(1.0 / np.sqrt(d))
    f = np.tile(np.array([0.0, 2.0**-130, 2.0**-121, 2.0**-60, 1.0, 2.0**3, 2.0**5, 2.0**6],
                         dtype=np.float32), hq // 8)
    q = O.f32_to_bf16(O.bf16_to_f32(O.normal_bf16((hq, d), 77)) * f[:, None])
    _, _, k8, v8, ks, vs = make_cache(cache_len + 1, hkv, d, kind="normal", seed=7)
    got = gpu_decode(q, k8, v8, ks, vs, cache_len, hq, hkv, d, splits, scale)
    assert np.isfinite(O.bf16_to_f32(got)).all()
    check(got, q, k8, v8, ks, vs, cache_len, hq, hkv, d, scale)


def test_config1_per_tensor_scale():
    """24Q/8KV, D 128, ctx 511; K/V N(0,1) quantized with one per-tensor
    scale amax/448 broadcast into the per-(token, kv_head) slab."""
    hq, hkv, d, ctx = 24, 8, 128, 511
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((hq, d), 11)
    kx = O.normal_bf16((ctx * hkv, d), 12)
    vx = O.normal_bf16((ctx * hkv, d), 13)
    kt = np.float32(np.max(np.abs(O.bf16_to_f32(kx)))) / np.float32(448)
    vt = np.float32(np.max(np.abs(O.bf16_to_f32(vx)))) / np.float32(448)
    ks = np.full(ctx * hkv, kt, np.float32)
    vs = np.full(ctx * hkv, vt, np.float32)
    # the GPU given-scale quantizer must reproduce the oracle's bytes
    step("config1 quantize_scaled")
    k8d = torch.empty((ctx * hkv, d), dtype=torch.uint8, device=DEV)
    v8d = torch.empty((ctx * hkv, d), dtype=torch.uint8, device=DEV)
    R.quantize_kv_fp8_scaled(k8d, f32_dev(ks), bf16_dev(kx), int_dev(0), 1, ctx * hkv, d)
    R.quantize_kv_fp8_scaled(v8d, f32_dev(vs), bf16_dev(vx), int_dev(0), 1, ctx * hkv, d)
    sync()
    k8 = O.quantize_kv_fp8_scaled(kx, ks, d)
    v8 = O.quantize_kv_fp8_scaled(vx, vs, d)
    assert np.array_equal(k8d.cpu().numpy(), k8) and np.array_equal(v8d.cpu().numpy(), v8)
    got = gpu_decode(q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, 32, scale)
    check(got, q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, scale)


@pytest.mark.parametrize("ctx", [35, 2041, 8196, 32768])
def test_config3_depths_single_layer(ctx):
    hq, hkv, d = 24, 8, 128
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((hq, d), 21)
    _, _, k8, v8, ks, vs = make_cache(ctx, hkv, d, kind="normal", seed=ctx)
    got = gpu_decode(q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, R.default_num_splits(hkv), scale)
    check(got, q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, scale)


@pytest.mark.parametrize("splits", [64, None])
def test_config5_long_context_per_head_scales(splits):
    """32Q/8KV, ctx 131072, per-head scales ~U(0.01, 0.1); the config's 64
    splits (cooperative workgroups) and the default split count (one wave per
    512-key split: the nontemporal streaming loads)."""
    hq, hkv, d, ctx = 32, 8, 128, 131072
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((hq, d), 51)
    ph = (O.uniform_f32(hkv, 0.01, 0.1, 52), O.uniform_f32(hkv, 0.01, 0.1, 53))
    _, _, k8, v8, ks, vs = make_cache(ctx, hkv, d, kind="normal", seed=5, per_head_scale=ph)
    s = splits if splits is not None else R.default_num_splits(hkv)
    got = gpu_decode(q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, s, scale)
    check(got, q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, scale)


def test_long_splits_ragged_tail():
    """One wave per 320-key split (the nontemporal loads) with a partial
    last split: ctx 40000, 128 splits, 24Q/8KV."""
    hq, hkv, d, ctx = 24, 8, 128, 40000
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((hq, d), 55)
    _, _, k8, v8, ks, vs = make_cache(ctx, hkv, d, kind="normal", seed=7)
    got = gpu_decode(q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, 128, scale)
    check(got, q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, scale)


@pytest.mark.parametrize("ctx,hq,hkv,splits,d", [
    (20000, 32, 8, 64, 128), (20001, 32, 8, 128, 128), (7000, 32, 8, 16, 128),
    (12345, 16, 4, 128, 128), (3000, 32, 8, 128, 128), (33, 32, 8, 64, 128),
    (20000, 32, 8, 64, 64), (9001, 16, 4, 128, 64), (20000, 32, 8, 64, 256),
    (9001, 16, 4, 128, 256),
    # split counts whose grid is laid out for the fewest rounds (96 -> 4 kv
    # heads per workgroup; 160 / 192 / 224 -> one wave per kv head, i.e. the
    # solo layout)
    (9000, 24, 8, 96, 128), (5000, 24, 8, 192, 128), (20000, 32, 8, 160, 128),
    (7001, 24, 8, 224, 64),
])
def test_grouped_workgroups(ctx, hq, hkv, splits, d):
    """Launches with fewer (kv head, split) units than one round of wave
    slots run one workgroup per (group of kv heads, split), the waves of a kv
    head on contiguous shares of the split's tiles, merged in LDS. On 256
    compute units: 64 splits x 8 kv heads -> 2 kv heads per workgroup,
    128 x 8 -> 4, 16 x 8 -> 1, 128 x 4 -> 2; short contexts leave most splits
    empty. head_dim 64 and 256 cover the other whole-row K layouts (16 and 4
    rows per load instruction; 256 with its one-tile register ring)."""
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((hq, d), 81)
    _, _, k8, v8, ks, vs = make_cache(ctx, hkv, d, kind="normal", seed=ctx)
    got = gpu_decode(q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, splits, scale)
    check(got, q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, scale)


@pytest.mark.parametrize("cache_len,hq,hkv,d,splits", [
    (8191, 8, 2, 32, None), (131071, 32, 8, 32, 64), (9000, 16, 4, 512, 64),
    (65535, 8, 2, 512, None), (10000, 36, 4, 256, None), (5000, 34, 2, 64, 100),
    (40, 32, 8, 32, 4), (3, 8, 2, 512, 8), (2999, 68, 4, 256, 32),
])
def test_valu_split_kernel(cache_len, hq, hkv, d, splits):
    """Shapes the MFMA split kernel does not take (head_dim 32 and 512, GQA
    groups that do not split into blocks of 4-16 q heads) run the VALU split
    kernel (reference src/kernels/flash_decode.cu:296-319 serves all five head
    sizes with one split kernel): contexts up to 128K, ragged head blocks (17
    and 9 q heads per kv head), more splits than tiles."""
    assert R.decode_path(hq, hkv, d) == R.DECODE_VALU
    scale = np.float32(1.0 / np.sqrt(d))
    splits = splits or R.default_num_splits(hkv)
    q = O.normal_bf16((hq, d), 91 + d)
    _, _, k8, v8, ks, vs = make_cache(cache_len + 1, hkv, d, kind="normal", seed=cache_len)
    got = gpu_decode(q, k8, v8, ks, vs, cache_len, hq, hkv, d, splits, scale)
    check(got, q, k8, v8, ks, vs, cache_len, hq, hkv, d, scale)


@pytest.mark.parametrize("cache_len,hq,hkv,d,splits", [
    (10000, 64, 2, 128, None), (5000, 40, 2, 64, 100), (8195, 32, 1, 128, None),
    (3000, 96, 2, 128, 64), (4000, 16, 1, 256, 32), (20000, 24, 1, 128, None),
    (30000, 64, 2, 128, 16), (2040, 48, 2, 256, 8), (100, 128, 4, 64, 3),
])
def test_mfma_q_blocks(cache_len, hq, hkv, d, splits):
    """GQA groups wider than the MFMA's 16 columns (or than a wave's 2048-value
    staging row) run the MFMA kernel as blocks of 4-16 q heads per kv head
    (two blocks of 16, of 10, of 12, three of 16, two of 8 at head_dim 256),
    one-kv-head (MQA) caches, grouped workgroups at 16 splits; oracle parity."""
    assert R.decode_path(hq, hkv, d) == R.DECODE_MFMA
    scale = np.float32(1.0 / np.sqrt(d))
    splits = splits or R.default_num_splits(hkv)
    q = O.normal_bf16((hq, d), 71 + hq)
    _, _, k8, v8, ks, vs = make_cache(cache_len + 1, hkv, d, kind="normal", seed=cache_len + hq)
    got = gpu_decode(q, k8, v8, ks, vs, cache_len, hq, hkv, d, splits, scale)
    check(got, q, k8, v8, ks, vs, cache_len, hq, hkv, d, scale)


def test_decode_path_selection():
    """The reference test shapes with head_dim 32 / 512 take the VALU kernel;
    head_dim 64 / 128 / 256 with groups up to 16 the MFMA kernel."""
    assert R.decode_path(32, 8, 32) == R.DECODE_VALU
    assert R.decode_path(8, 2, 512) == R.DECODE_VALU
    assert R.decode_path(68, 4, 256) == R.DECODE_VALU    # 17 q heads: no blocks of 4-16
    assert R.decode_path(36, 4, 256) == R.DECODE_VALU    # 9 x 256 > 2048, blocks of 3
    assert R.decode_path(64, 2, 128) == R.DECODE_MFMA    # two blocks of 16
    assert R.decode_path(16, 1, 256) == R.DECODE_MFMA    # two blocks of 8
    assert R.decode_path(96, 2, 64) == R.DECODE_MFMA     # three blocks of 16
    for d in (64, 128, 256):
        assert R.decode_path(32, 8, d) == R.DECODE_MFMA
    assert R.decode_path(64, 4, 128) == R.DECODE_MFMA
    assert R.decode_path(30, 8, 128) == 0 and R.decode_path(32, 8, 96) == 0


def test_repeated_calls_share_scratch():
    """Back-to-back calls with different depths on one scratch stay correct
    (the scratch carries no state between calls)."""
    hq, hkv, d = 32, 8, 128
    scale = np.float32(1.0 / np.sqrt(d))
    total = 3000
    q = O.normal_bf16((hq, d), 61)
    _, _, k8, v8, ks, vs = make_cache(total, hkv, d, kind="normal", seed=6)
    partial = R.new_flash_split_scratch(hq, d, 32)
    k8d, v8d, ksd, vsd, qd = u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs), bf16_dev(q)
    for cl in (2999, 5, 1500, 0, 2999):
        step(f"decode repeated cache_len={cl}")
        out = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
        R.flash_decode_split_bf16(out, qd, k8d, v8d, ksd, vsd, partial, 32, int_dev(cl),
                                  hq, hkv, d, scale)
        sync()
        check(bf16_host(out), q, k8, v8, ks, vs, cl, hq, hkv, d, scale)


@pytest.mark.parametrize("splits", [1, 4, 32])
def test_score_dynamic_range(splits):
    """Deep negative scores on the first keys and a far jump above the running
    maximum at keys 400..404 (the split softmax must rescale exactly)."""
    total, hq, hkv, d = 700, 8, 2, 128
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((hq, d), 41) & np.uint16(0x7FFF)
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((total * hkv, d), 42), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16((total * hkv, d), 43), d)
    k8[: 64 * hkv] |= np.uint8(0x80)
    ks[: 64 * hkv] = 0.5
    k8[400 * hkv: 405 * hkv] &= np.uint8(0x7F)
    ks[400 * hkv: 405 * hkv] = 0.05
    got = gpu_decode(q, k8, v8, ks, vs, total - 1, hq, hkv, d, splits, scale)
    assert np.isfinite(O.bf16_to_f32(got)).all()
    check(got, q, k8, v8, ks, vs, total - 1, hq, hkv, d, scale)


@pytest.mark.parametrize("hq,hkv,splits", [(24, 8, 32), (32, 16, 32), (64, 2, 16), (16, 4, 32)])
def test_xcd_local_mapping_switch(hq, hkv, splits):
    """With 8k (virtual) kv heads and 8k splits, the split and merge kernels
    put each kv head's units on one XCD while every live split holds one
    32-key tile (tiles < 2 * splits) and use the split-major mapping beyond;
    both kernels decide from *cache_len. Depths on either side of the switch,
    in both orders on one scratch, match the oracle (64Q/2KV runs as 8
    virtual kv heads; 16Q/4KV never switches)."""
    d = 128
    scale = np.float32(1.0 / np.sqrt(d))
    edge = 2 * splits * 32
    total = edge + 40
    q = O.normal_bf16((hq, d), 71)
    _, _, k8, v8, ks, vs = make_cache(total, hkv, d, kind="normal", seed=hq + hkv)
    partial = R.new_flash_split_scratch(hq, d, splits)
    k8d, v8d, ksd, vsd, qd = u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs), bf16_dev(q)
    for ctx in (edge + 33, edge - 32, edge, edge - 31, edge + 1, splits * 32 - 5):
        step(f"decode xcd switch hq={hq} hkv={hkv} splits={splits} ctx={ctx}")
        out = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
        R.flash_decode_split_bf16(out, qd, k8d, v8d, ksd, vsd, partial, splits,
                                  int_dev(ctx - 1), hq, hkv, d, scale)
        sync()
        check(bf16_host(out), q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, scale)


@pytest.mark.parametrize("cache_len,hq,hkv,d,splits", [
    (0, 24, 8, 128, None), (1, 24, 8, 128, None), (31, 24, 8, 128, None), (32, 24, 8, 128, None),
    (2040, 24, 8, 128, None), (8195, 24, 8, 128, None), (9000, 32, 8, 128, 64),
    (130, 8, 2, 64, 8), (700, 8, 4, 256, 16), (77, 64, 4, 128, 4), (40, 8, 2, 32, 4),
    (5000, 32, 8, 128, 128), (6000, 16, 4, 128, 128),
    # q blocks: several units per cache head attend the new token, one stores it
    (700, 64, 2, 128, 16), (3000, 32, 1, 128, None), (130, 16, 1, 256, 8),
    # 256 splits: the appended key has a split of its own while the cache
    # keys fill at most 2 x 255 tiles (cache_len <= 16320), one or two per
    # split, then shares the last split's tile
    (8159, 24, 8, 128, None), (8160, 24, 8, 128, None), (8161, 24, 8, 128, None),
    (8192, 24, 8, 128, None), (16319, 24, 8, 128, None), (16320, 24, 8, 128, None),
    (16321, 24, 8, 128, None), (16352, 24, 8, 128, None),
    # 64 kv heads x 32 splits (solo): the key's own split while the cache keys
    # fit 2 x 31 tiles (cache_len <= 1984), one per split up to 31 tiles
    (0, 64, 64, 128, 32), (31, 64, 64, 128, 32), (992, 64, 64, 128, 32),
    (993, 64, 64, 128, 32), (1983, 64, 64, 128, 32), (1984, 64, 64, 128, 32),
    (1985, 64, 64, 128, 32), (2100, 64, 64, 128, 32),
])
def test_decode_append_fused(cache_len, hq, hkv, d, splits):
    """Fused append + decode: the cache row equals the append kernel's bytes
    and the output matches the oracle (and the two-call sequence) within the
    attention tolerance."""
    scale = np.float32(1.0 / np.sqrt(d))
    total = cache_len + 1
    splits = splits or R.default_num_splits(hkv)
    _, _, k8, v8, ks, vs = make_cache(total, hkv, d, kind="normal", seed=cache_len)
    kn = O.normal_bf16((hkv, d), 3000 + cache_len)
    vn = O.normal_bf16((hkv, d), 4000 + cache_len)
    q = O.normal_bf16((hq, d), 5000 + cache_len)
    rows = slice(cache_len * hkv, total * hkv)
    k8[rows] = 0
    v8[rows] = 0
    kc, vc, ksd, vsd = u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs)
    out = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    partial = R.new_flash_split_scratch(hq, d, splits)
    step(f"decode+append ctx={total} hq={hq} hkv={hkv} d={d} splits={splits}")
    R.flash_decode_append_split_bf16(out, bf16_dev(q), kc, vc, ksd, vsd, bf16_dev(kn),
                                     bf16_dev(vn), partial, splits, int_dev(cache_len), hq, hkv,
                                     d, scale)
    sync()
    wk, wks = O.quantize_kv_fp8(kn, d)
    wv, wvs = O.quantize_kv_fp8(vn, d)
    gk, gv = kc.cpu().numpy(), vc.cpu().numpy()
    gks, gvs = ksd.cpu().numpy(), vsd.cpu().numpy()
    assert np.array_equal(gk[rows], wk) and np.array_equal(gv[rows], wv)
    assert np.array_equal(gks[rows].view(np.uint32), wks.view(np.uint32))
    assert np.array_equal(gvs[rows].view(np.uint32), wvs.view(np.uint32))
    others = np.ones(total * hkv, bool)
    others[rows] = False
    assert np.array_equal(gk[others], k8[others]) and np.array_equal(gks[others], ks[others])
    got = bf16_host(out)
    check(got, q, gk, gv, gks, gvs, cache_len, hq, hkv, d, scale)
    two = gpu_decode(q, gk, gv, gks, gvs, cache_len, hq, hkv, d, splits, scale)
    mx, mean = O.bf16_err(got, two)
    assert mx <= MAX_ABS and mean <= 1e-3, (mx, mean)


@pytest.mark.parametrize("splits", [1, 3, 32, 96, 160, 256, 300])
@pytest.mark.parametrize("cache_len", [0, 33, 1000, 5000])
def test_decode_append_partition_sweep(splits, cache_len):
    """Fused append + decode over the launch layouts a split count selects
    (cooperative groups of 1/2/4 kv heads, the solo layout, the appended
    key's own split, XCD-local placement) at depths on either side of one
    tile per split: the cache row is the append kernel's and the output
    matches the oracle."""
    hq, hkv, d = 24, 8, 128
    scale = np.float32(1.0 / np.sqrt(d))
    total = cache_len + 1
    _, _, k8, v8, ks, vs = make_cache(total, hkv, d, kind="normal", seed=splits + cache_len)
    kn = O.normal_bf16((hkv, d), 6000 + splits)
    vn = O.normal_bf16((hkv, d), 7000 + splits)
    q = O.normal_bf16((hq, d), 8000 + cache_len)
    kc, vc, ksd, vsd = u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs)
    out = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    partial = R.new_flash_split_scratch(hq, d, splits)
    step(f"decode+append sweep ctx={total} splits={splits}")
    R.flash_decode_append_split_bf16(out, bf16_dev(q), kc, vc, ksd, vsd, bf16_dev(kn),
                                     bf16_dev(vn), partial, splits, int_dev(cache_len), hq, hkv,
                                     d, scale)
    sync()
    rows = slice(cache_len * hkv, total * hkv)
    wk, wks = O.quantize_kv_fp8(kn, d)
    gk, gv = kc.cpu().numpy(), vc.cpu().numpy()
    gks, gvs = ksd.cpu().numpy(), vsd.cpu().numpy()
    assert np.array_equal(gk[rows], wk)
    assert np.array_equal(gks[rows].view(np.uint32), wks.view(np.uint32))
    check(bf16_host(out), q, gk, gv, gks, gvs, cache_len, hq, hkv, d, scale)


@pytest.mark.parametrize("splits,d", [(32, 128), (64, 128), (96, 128), (32, 64), (64, 256)])
@pytest.mark.parametrize("extra", [0, 1, 64])
def test_decode_append_grouped_own_split_edge(splits, d, extra):
    """Grouped launches (1, 2 and 4 kv heads per workgroup) of the fused
    append + decode at the edge of the appended key's own split: up to
    64 * (splits - 1) cache keys the key takes a split of its own and every
    other split one or two tiles; one key more and it joins the last split;
    a tile more and the waves of a kv head share the tiles again."""
    cache_len = 64 * (splits - 1) + extra
    hq, hkv = 24, 8
    scale = np.float32(1.0 / np.sqrt(d))
    total = cache_len + 1
    _, _, k8, v8, ks, vs = make_cache(total, hkv, d, kind="normal", seed=splits + extra)
    kn = O.normal_bf16((hkv, d), 6100 + splits)
    vn = O.normal_bf16((hkv, d), 7100 + splits)
    q = O.normal_bf16((hq, d), 8100 + extra)
    kc, vc, ksd, vsd = u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs)
    out = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    partial = R.new_flash_split_scratch(hq, d, splits)
    step(f"decode+append grouped own-split edge ctx={total} splits={splits} d={d}")
    R.flash_decode_append_split_bf16(out, bf16_dev(q), kc, vc, ksd, vsd, bf16_dev(kn),
                                     bf16_dev(vn), partial, splits, int_dev(cache_len), hq, hkv,
                                     d, scale)
    sync()
    rows = slice(cache_len * hkv, total * hkv)
    wk, wks = O.quantize_kv_fp8(kn, d)
    gk, gv = kc.cpu().numpy(), vc.cpu().numpy()
    gks, gvs = ksd.cpu().numpy(), vsd.cpu().numpy()
    assert np.array_equal(gk[rows], wk)
    assert np.array_equal(gks[rows].view(np.uint32), wks.view(np.uint32))
    check(bf16_host(out), q, gk, gv, gks, gvs, cache_len, hq, hkv, d, scale)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_decode_append_fused_special_values(d):
    """The fused entry's quantizer on rows the append kernel's own tests cover
    (quantization.cu:224-250): NaN entries (ignored by the amax), +-inf (scale
    inf, codes from x * 0), an all-zero row (scale 0), bf16 subnormals only,
    the largest finite bf16 values, mixed with ordinary rows. Cache codes and
    scales equal the oracle quantizer's bit for bit (head_dim 64 and 128 take
    the rows loaded at kernel start, 256 the late loads); the output is not
    checked, as a NaN key makes it NaN by design."""
    hq, hkv, cache_len, splits = 32, 8, 1000, 64
    scale = np.float32(1.0 / np.sqrt(d))
    total = cache_len + 1
    _, _, k8, v8, ks, vs = make_cache(total, hkv, d, kind="normal", seed=d)
    kn = O.normal_bf16((hkv, d), 6000 + d)
    vn = O.normal_bf16((hkv, d), 7000 + d)
    for x in (kn, vn):
        x[0, 3], x[0, d - 1] = 0x7FC0, 0xFFC1             # NaNs
        x[1, 5] = 0x7F80                                  # +inf
        x[2, :] = 0                                       # zero row
        x[3, :] = np.arange(1, d + 1, dtype=np.uint16)    # subnormals
        x[4, ::2] = 0x7F7F                                # +-max finite
        x[4, 1::2] = 0xFF7F
        x[5, 7] = 0xFF80                                  # -inf
    q = O.normal_bf16((hq, d), 8000 + d)
    rows = slice(cache_len * hkv, total * hkv)
    kc, vc, ksd, vsd = u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs)
    out = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    partial = R.new_flash_split_scratch(hq, d, splits)
    step(f"decode+append special values d={d}")
    R.flash_decode_append_split_bf16(out, bf16_dev(q), kc, vc, ksd, vsd, bf16_dev(kn),
                                     bf16_dev(vn), partial, splits, int_dev(cache_len), hq, hkv,
                                     d, scale)
    sync()
    wk, wks = O.quantize_kv_fp8(kn, d)
    wv, wvs = O.quantize_kv_fp8(vn, d)
    assert np.array_equal(kc.cpu().numpy()[rows], wk)
    assert np.array_equal(vc.cpu().numpy()[rows], wv)
    assert np.array_equal(ksd.cpu().numpy()[rows].view(np.uint32), wks.view(np.uint32))
    assert np.array_equal(vsd.cpu().numpy()[rows].view(np.uint32), wvs.view(np.uint32))
    # Rows 6 and 7 are ordinary: their kv heads' outputs stay finite.
    got = bf16_host(out).astype(np.uint32) << 16
    finite = np.isfinite(got.view(np.float32))
    assert finite.reshape(hkv, hq // hkv, d)[6:].all()


def test_forced_valu_kernel_matches_oracle():
    """rth_set_decode_kernel(RTH_DECODE_VALU) runs the VALU split kernel for
    a shape the MFMA kernel serves (the A/B switch of the measurements);
    results stay within the attention tolerance, and the default returns."""
    hq, hkv, d, ctx = 24, 8, 128, 8196
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((hq, d), 95)
    _, _, k8, v8, ks, vs = make_cache(ctx, hkv, d, kind="normal", seed=95)
    R.set_decode_kernel(R.DECODE_VALU)
    try:
        assert R.decode_path(hq, hkv, d) == R.DECODE_VALU
        got = gpu_decode(q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, 256, scale)
    finally:
        R.set_decode_kernel(0)
    assert R.decode_path(hq, hkv, d) == R.DECODE_MFMA
    check(got, q, k8, v8, ks, vs, ctx - 1, hq, hkv, d, scale)
