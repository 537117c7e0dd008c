"""Causal flash prefill on the GPU against the oracle (reference
src/kernels/flash_prefill.cu; cases of tests/kernels/test_flash_prefill.cpp:
141-169 plus the BASELINE configurations). Tolerance: max-abs 2e-2,
mean-abs 2e-3 on bf16 outputs."""
import numpy as np
import pytest
import torch

import oracle_lib as O
import runtherder_amd as R
from gpu_util import DEV, NTHREADS, bf16_dev, bf16_host, f32_dev, host, int_dev, step, sync, u8_dev

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def gpu_prefill(q, k8, v8, ks, vs, n_new, clen, hq, hkv, d, scale, naive=False):
    step(f"{'naive' if naive else 'prefill'} n_new={n_new} clen={clen} hq={hq} hkv={hkv}")
    out = torch.empty((n_new, hq, d), dtype=torch.bfloat16, device=DEV)
    fn = R.attention_causal_bf16 if naive else R.flash_prefill_bf16
    fn(out, bf16_dev(q), u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs), n_new,
       int_dev(clen), hq, hkv, d, scale)
    sync()
    return bf16_host(out)


def ref_inputs(n_new, clen, hq, hkv, d):
    total = clen + n_new
    q = O.mt19937_uniform_bf16((n_new, hq, d), 1.0, 0xA11CE)
    k8, ks = O.quantize_kv_fp8(O.mt19937_uniform_bf16((total * hkv, d), 1.0, 0xB0B), d)
    v8, vs = O.quantize_kv_fp8(O.mt19937_uniform_bf16((total * hkv, d), 1.0, 0xCAFE), d)
    return q, k8, v8, ks, vs


@pytest.mark.parametrize("naive", [False, True])
@pytest.mark.parametrize("n_new,clen,hq,hkv", [
    (16, 0, 32, 8), (20, 0, 32, 8), (8, 10, 32, 8), (64, 0, 24, 8), (3, 0, 8, 2),
    (1, 0, 32, 8), (129, 0, 32, 8), (200, 77, 24, 8), (300, 1000, 8, 8), (257, 63, 16, 1),
])
def test_reference_cases(n_new, clen, hq, hkv, naive):
    d = 128
    scale = np.float32(1.0 / np.sqrt(d))
    q, k8, v8, ks, vs = ref_inputs(n_new, clen, hq, hkv, d)
    got = gpu_prefill(q, k8, v8, ks, vs, n_new, clen, hq, hkv, d, scale, naive)
    want = O.attention_f32(q, k8, v8, ks, vs, n_new, clen, hq, hkv, d, scale, NTHREADS)
    mx, mean = O.bf16_err(got, want)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


def dynamic_range_inputs(n, hq, hkv, d):
    """Scores that swing far in both directions: q >= 0; the first 64 keys
    negative with a large scale (every row's first tile scores below -500 in
    natural units); keys 400..404 positive with a large scale (a jump of ~50
    above the running maximum mid-sequence); the rest ordinary."""
    q = O.normal_bf16((n, hq, d), 31) & np.uint16(0x7FFF)
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((n * hkv, d), 32), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16((n * hkv, d), 33), d)
    first = slice(0, 64 * hkv)
    spike = slice(400 * hkv, 405 * hkv)
    k8[first] |= np.uint8(0x80)
    ks[first] = 0.5
    k8[spike] &= np.uint8(0x7F)
    ks[spike] = 0.05
    return q, k8, v8, ks.astype(np.float32), vs


def test_score_dynamic_range_rebases():
    """The lazy reference maximum must rebase on the first tile (deep
    negative scores) and again when a later score jumps far above it."""
    n, hq, hkv, d = 700, 8, 2, 128
    scale = np.float32(1.0 / np.sqrt(d))
    q, k8, v8, ks, vs = dynamic_range_inputs(n, hq, hkv, d)
    got = gpu_prefill(q, k8, v8, ks, vs, n, 0, hq, hkv, d, scale)
    want = O.attention_f32(q, k8, v8, ks, vs, n, 0, hq, hkv, d, scale, NTHREADS)
    assert np.isfinite(O.bf16_to_f32(got)).all()
    mx, mean = O.bf16_err(got, want)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


Q_FACTORS = np.array([0.0, 2.0**-130, 2.0**-121, 2.0**-118, 2.0**-60, 1.0, 2.0**4, 2.0**6],
                     dtype=np.float32)


@pytest.mark.parametrize("n", [300, 700, 4100])
def test_q_rows_of_extreme_magnitude(n):
    """q heads scaled from zero and bf16 subnormals up to 2^6 (scores several
    hundred apart between tiles). Tiny rows must keep a finite q split (their
    weights are near uniform); huge rows overflow P and rebase, and the other
    rows of their wave must not be rebased downwards. n 300 runs the 4-wave
    workgroup and n 700 the key-split one with the full oracle, n 4100 the
    8-wave one on sampled rows."""
    hq, hkv, d = (8, 2, 128) if n < 1000 else (32, 8, 128)
    scale = np.float32(1.0 / np.sqrt(d))
    f = np.tile(Q_FACTORS, hq // 8)
    q = O.f32_to_bf16(O.bf16_to_f32(O.normal_bf16((n, hq, d), 41)) * f[None, :, None])
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((n * hkv, d), 42), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16((n * hkv, d), 43), d)
    got = gpu_prefill(q, k8, v8, ks, vs, n, 0, hq, hkv, d, scale)
    assert np.isfinite(O.bf16_to_f32(got)).all()
    if n < 1000:
        want = O.attention_f32(q, k8, v8, ks, vs, n, 0, hq, hkv, d, scale, NTHREADS)
        mx, mean = O.bf16_err(got, want)
        assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)
    else:
        check_rows(got, q, k8, v8, ks, vs, 0, sampled_rows(n, 12, n), hq, hkv, d, scale)


def mixed_magnitude_q(n, hq, d, seed):
    """Rows whose elements span ~22 binades below the row maximum: one element
    at +-2^e (e in [-3, 5]) and the others at +-2^(e - t), t uniform in
    [1, 22]. In the kernel's scaled units (row maximum in [128, 256)) the
    elements below 2^-6, those more than ~13 binades under the maximum, are
    where the two-part E4M3 split of q is not exact (error <= 2^-14 scaled,
    tests/test_prefill_q_split.py); the large ones need the lo part."""
    rng = np.random.default_rng(seed)
    e = rng.integers(-3, 6, size=(n, hq, 1)).astype(np.float64)
    t = rng.uniform(1.0, 22.0, size=(n, hq, d))
    x = np.exp2(e - t) * rng.choice([-1.0, 1.0], size=(n, hq, d))
    top = rng.integers(0, d, size=(n, hq))
    np.put_along_axis(x, top[..., None], np.exp2(e) * rng.choice([-1.0, 1.0], size=(n, hq, 1)),
                      axis=2)
    return O.f32_to_bf16(x.astype(np.float32))


@pytest.mark.parametrize("n", [300, 700, 4100])
def test_q_rows_mixing_max_and_tiny_elements(n):
    """Every row mixes its maximum with elements down to 2^-22 of it: the
    scores come from the exact hi part, the lo part (large elements) and the
    subnormal-limited lo part (tiny elements); the output must still match
    the oracle's scores, which use the bf16 q as is. n 300 / 700 / 4100 run
    the 4-wave, key-split and 8-wave workgroups (the last on sampled rows)."""
    hq, hkv, d = (8, 2, 128) if n < 1000 else (32, 8, 128)
    scale = np.float32(1.0 / np.sqrt(d))
    q = mixed_magnitude_q(n, hq, d, 44)
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((n * hkv, d), 45), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16((n * hkv, d), 46), d)
    got = gpu_prefill(q, k8, v8, ks, vs, n, 0, hq, hkv, d, scale)
    assert np.isfinite(O.bf16_to_f32(got)).all()
    if n < 1000:
        want = O.attention_f32(q, k8, v8, ks, vs, n, 0, hq, hkv, d, scale, NTHREADS)
        mx, mean = O.bf16_err(got, want)
        assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)
    else:
        check_rows(got, q, k8, v8, ks, vs, 0, sampled_rows(n, 12, n), hq, hkv, d, scale)


@pytest.mark.parametrize("n_new,clen,hq,hkv", [
    (513, 0, 8, 2), (513, 129, 16, 4), (640, 64, 8, 8), (777, 1, 24, 8), (1500, 0, 8, 1),
])
def test_key_split_workgroups(n_new, clen, hq, hkv):
    """Grids of at most 1.5 rounds of 128-row blocks (4 or more per head)
    split each block's key tiles over two halves of one workgroup (even and
    odd tiles) and merge their (O, max, sum) at the end. Odd and even tile
    counts, a cache prefix (the odd half's first tile fully masked for the
    block's first rows when clen = 1), GQA groups of 1 to 8."""
    d = 128
    scale = np.float32(1.0 / np.sqrt(d))
    q, k8, v8, ks, vs = ref_inputs(n_new, clen, hq, hkv, d)
    got = gpu_prefill(q, k8, v8, ks, vs, n_new, clen, hq, hkv, d, scale)
    want = O.attention_f32(q, k8, v8, ks, vs, n_new, clen, hq, hkv, d, scale, NTHREADS)
    mx, mean = O.bf16_err(got, want)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


def shape_boundaries(cus, hq):
    """Row counts at the edges of flash_prefill_launch's workgroup-shape choice
    on a device with `cus` compute units (the same formulas as the launcher):
    the last 4-wave / first key-split count (4 blocks of 128 rows), the last
    key-split / first 4-wave count (2 * blocks * hq <= 3 * cus), and the first
    8-wave count (ceil(n / 256) * hq >= 2 * cus)."""
    out = [384, 385]
    nb = (3 * cus) // (2 * hq)            # most 128-row blocks on the key split
    if nb >= 4:
        out += [128 * nb, 128 * nb + 1]
    n8 = 256 * (-(-2 * cus // hq) - 1)     # last row count below the 8-wave path
    out += [n8, n8 + 1]
    return out


@pytest.mark.parametrize("edge", range(6))
def test_workgroup_shape_boundaries(edge):
    """32 q heads at the edges of the launch's shape choice, derived from the
    device's compute-unit count (on 256 CUs: 384 / 385 rows = 3 / 4 blocks of
    128, 4-wave / key split; 1536 / 1537 = 12 / 13 blocks, key split / 4-wave;
    3840 / 3841 = 15 / 16 blocks of 256, 4-wave / 8-wave). Sampled rows of
    every block edge against the oracle."""
    hq, hkv, d, clen = 32, 8, 128, 0
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    edges_n = shape_boundaries(cus, hq)
    if edge >= len(edges_n):
        pytest.skip(f"{cus} compute units leave no key-split range for {hq} heads")
    n_new = edges_n[edge]
    scale = np.float32(1.0 / np.sqrt(d))
    q, k8, v8, ks, vs = ref_inputs(n_new, clen, hq, hkv, d)
    got = gpu_prefill(q, k8, v8, ks, vs, n_new, clen, hq, hkv, d, scale)
    edges = sorted({r for b in range(0, n_new, 128) for r in (b, b + 63, b + 64, b + 127)
                    if r < n_new})
    rows = sorted(set(edges[::3]) | set(sampled_rows(n_new, 6, n_new)))
    check_rows(got, q, k8, v8, ks, vs, clen, rows, hq, hkv, d, scale)


def rope_qkv(n, hq, hkv, d, theta, llama3, seed):
    q = O.normal_bf16((n, hq, d), seed)
    k = O.normal_bf16((n, hkv, d), seed + 1)
    v = O.normal_bf16((n, hkv, d), seed + 2)
    inv = (O.rope_inv_freq_llama3(d, theta, 32.0, 1.0, 4.0, 8192) if llama3
           else O.rope_inv_freq_plain(d, theta))
    pos = np.arange(n, dtype=np.int32)
    return O.rope_apply_bf16(q, pos, inv), O.rope_apply_bf16(k, pos, inv), v


def append_and_check(cache_len, k, v, hkv, d, max_seq):
    """Appends through the fused GPU kernel and checks the bytes bit-exactly."""
    n = k.shape[0]
    cache = R.KVCache(1, max_seq, hkv, d)
    step(f"append n={n} at={cache_len}")
    cache.append(0, bf16_dev(k), bf16_dev(v), n, int_dev(cache_len))
    sync()
    view = cache.view(0)
    rows = slice(cache_len * hkv, (cache_len + n) * hkv)
    wk, wks = O.quantize_kv_fp8(k, d)
    wv, wvs = O.quantize_kv_fp8(v, d)
    assert np.array_equal(host(view.k).reshape(-1, d)[rows], wk)
    assert np.array_equal(host(view.v).reshape(-1, d)[rows], wv)
    assert np.array_equal(host(view.k_scale).reshape(-1)[rows].view(np.uint32), wks.view(np.uint32))
    assert np.array_equal(host(view.v_scale).reshape(-1)[rows].view(np.uint32), wvs.view(np.uint32))
    return cache, view


def test_config2_prefill_1021_rope_llama3():
    """24Q/8KV, 1021 tokens, RoPE theta 5e5 with llama3 scaling (factor 32,
    original context 8192); K/V through the append kernel; full oracle."""
    n, hq, hkv, d = 1021, 24, 8, 128
    scale = np.float32(1.0 / np.sqrt(d))
    q, k, v = rope_qkv(n, hq, hkv, d, 5e5, True, 700)
    cache, view = append_and_check(0, k, v, hkv, d, n)
    out = torch.empty((n, hq, d), dtype=torch.bfloat16, device=DEV)
    backend = R.make_attention_backend(R.BackendKind.Adaptive, R.AttnConfig.for_heads(hq, hkv, d))
    step("config2 prefill")
    backend.run(out, bf16_dev(q), view, n, int_dev(0))
    sync()
    k8, v8 = host(view.k).reshape(-1, d), host(view.v).reshape(-1, d)
    ks, vs = host(view.k_scale).reshape(-1), host(view.v_scale).reshape(-1)
    want = O.attention_f32(q, k8, v8, ks, vs, n, 0, hq, hkv, d, scale, NTHREADS)
    mx, mean = O.bf16_err(bf16_host(out), want)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


def sampled_rows(n, count, seed):
    rng = np.random.default_rng(seed)
    fixed = [0, 1, 63, 64, 127, 128, n // 2, n - 2, n - 1]
    rows = set(r for r in fixed if 0 <= r < n) | set(rng.integers(0, n, count).tolist())
    return sorted(rows)


def check_rows(got, q, k8, v8, ks, vs, clen, rows, hq, hkv, d, scale):
    worst = 0.0
    for t in rows:
        want = O.attention_f32(q[t:t + 1], k8, v8, ks, vs, 1, clen + t, hq, hkv, d, scale,
                               NTHREADS)
        mx, mean = O.bf16_err(got[t], want[0])
        assert mx <= MAX_ABS and mean <= MEAN_ABS, (t, mx, mean)
        worst = max(worst, mx)
    return worst


def check_block(got, q, k8, v8, ks, vs, clen, r0, r1, hq, hkv, d, scale):
    """Rows r0..r1-1 (every head) against the oracle in one call."""
    want = O.attention_f32(q[r0:r1], k8, v8, ks, vs, r1 - r0, clen + r0, hq, hkv, d, scale,
                           NTHREADS)
    mx, mean = O.bf16_err(got[r0:r1], want)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (r0, r1, mx, mean)


@pytest.mark.parametrize("n", [2048, 4096, 8192, 16384])
def test_config4_prefill_sampled_rows(n):
    """32Q/8KV, RoPE theta 1e6, FP8 writeback; oracle on sampled rows."""
    hq, hkv, d = 32, 8, 128
    scale = np.float32(1.0 / np.sqrt(d))
    q, k, v = rope_qkv(n, hq, hkv, d, 1e6, False, 900 + n)
    cache, view = append_and_check(0, k, v, hkv, d, n)
    out = torch.empty((n, hq, d), dtype=torch.bfloat16, device=DEV)
    step(f"config4 prefill n={n}")
    R.flash_prefill_bf16(out, bf16_dev(q), view.k, view.v, view.k_scale, view.v_scale, n,
                         int_dev(0), hq, hkv, d, scale)
    sync()
    k8, v8 = host(view.k).reshape(-1, d), host(view.v).reshape(-1, d)
    ks, vs = host(view.k_scale).reshape(-1), host(view.v_scale).reshape(-1)
    got = bf16_host(out)
    check_rows(got, q, k8, v8, ks, vs, 0, sampled_rows(n, 12, n), hq, hkv, d, scale)
    if n == 16384:
        # The heaviest workgroup's rows (the last 256, every head) in full.
        check_block(got, q, k8, v8, ks, vs, 0, n - 256, n, hq, hkv, d, scale)


@pytest.mark.parametrize("clen", [0, 37, 100, 165])
def test_large_grid_ragged_tile_counts(clen):
    """n_new 4100 takes the 8-wave (two-group) path; with these cache lengths
    the row blocks' tile counts cover every residue mod 4 of the unrolled tile
    loop and the last tile is partial. Oracle on sampled rows."""
    hq, hkv, d, n = 32, 8, 128, 4100
    total = clen + n
    scale = np.float32(1.0 / np.sqrt(d))
    q, k, v = rope_qkv(total, hq, hkv, d, 1e6, False, 4100 + clen)
    cache, view = append_and_check(0, k, v, hkv, d, total)
    out = torch.empty((n, hq, d), dtype=torch.bfloat16, device=DEV)
    step(f"ragged prefill n={n} clen={clen}")
    R.flash_prefill_bf16(out, bf16_dev(q[clen:]), view.k, view.v, view.k_scale, view.v_scale, n,
                         int_dev(clen), hq, hkv, d, scale)
    sync()
    k8, v8 = host(view.k).reshape(-1, d), host(view.v).reshape(-1, d)
    ks, vs = host(view.k_scale).reshape(-1), host(view.v_scale).reshape(-1)
    check_rows(bf16_host(out), q[clen:], k8, v8, ks, vs, clen, sampled_rows(n, 12, n + clen), hq,
               hkv, d, scale)


@pytest.mark.parametrize("hq,hkv", [(64, 64), (64, 4)])
def test_large_grid_group_sizes(hq, hkv):
    """The 8-wave path (ceil(2100 / 256) * 64 heads fills two rounds) with
    GQA groups of 1 and 16 q heads per kv head and a cache offset. Oracle on
    sampled rows."""
    d, n, clen = 128, 2100, 50
    total = clen + n
    scale = np.float32(1.0 / np.sqrt(d))
    q, k, v = rope_qkv(total, hq, hkv, d, 1e6, False, 7000 + hkv)
    cache, view = append_and_check(0, k, v, hkv, d, total)
    out = torch.empty((n, hq, d), dtype=torch.bfloat16, device=DEV)
    step(f"group-size prefill n={n} clen={clen} hq={hq} hkv={hkv}")
    R.flash_prefill_bf16(out, bf16_dev(q[clen:]), view.k, view.v, view.k_scale, view.v_scale, n,
                         int_dev(clen), hq, hkv, d, scale)
    sync()
    k8, v8 = host(view.k).reshape(-1, d), host(view.v).reshape(-1, d)
    ks, vs = host(view.k_scale).reshape(-1), host(view.v_scale).reshape(-1)
    check_rows(bf16_host(out), q[clen:], k8, v8, ks, vs, clen, sampled_rows(n, 10, n + hkv), hq,
               hkv, d, scale)


def test_chunked_prefill_equals_full_tail():
    """Size-independent property: a chunked prefill (cache_len > 0) equals the
    tail rows of one full prefill over the same cache."""
    hq, hkv, d, total, clen = 32, 8, 128, 3000, 2237
    scale = np.float32(1.0 / np.sqrt(d))
    q, k, v = rope_qkv(total, hq, hkv, d, 1e6, False, 1234)
    cache, view = append_and_check(0, k, v, hkv, d, total)
    full = torch.empty((total, hq, d), dtype=torch.bfloat16, device=DEV)
    tail = torch.empty((total - clen, hq, d), dtype=torch.bfloat16, device=DEV)
    qd = bf16_dev(q)
    step("prefill full vs chunk")
    R.flash_prefill_bf16(full, qd, view.k, view.v, view.k_scale, view.v_scale, total,
                         int_dev(0), hq, hkv, d, scale)
    R.flash_prefill_bf16(tail, qd[clen:].contiguous(), view.k, view.v, view.k_scale,
                         view.v_scale, total - clen, int_dev(clen), hq, hkv, d, scale)
    sync()
    mx, mean = O.bf16_err(bf16_host(full)[clen:], bf16_host(tail))
    # The two launches sum in different orders (different tile boundaries), so
    # they may differ by a bf16 ulp; the bar is the attention tolerance.
    assert mx <= MAX_ABS and mean <= 1e-4, (mx, mean)


def test_config5_chunked_prefill_into_128k_cache():
    """4096-token chunk appended at cache_len 126976 of a 131072 cache with
    per-head given scales for the history; oracle on sampled rows."""
    hq, hkv, d, S = 32, 8, 128, 131072
    clen, n = 126976, 4096
    scale = np.float32(1.0 / np.sqrt(d))
    hist_k = O.normal_bf16((clen * hkv, d), 71)
    hist_v = O.normal_bf16((clen * hkv, d), 72)
    pks = np.tile(O.uniform_f32(hkv, 0.01, 0.1, 73), clen)
    pvs = np.tile(O.uniform_f32(hkv, 0.01, 0.1, 74), clen)
    cache = R.KVCache(1, S, hkv, d)
    view = cache.view(0)
    step("config5 history fill")
    R.quantize_kv_fp8_scaled(view.k.view(-1, d)[: clen * hkv], f32_dev(pks), bf16_dev(hist_k),
                             int_dev(0), 1, clen * hkv, d)
    R.quantize_kv_fp8_scaled(view.v.view(-1, d)[: clen * hkv], f32_dev(pvs), bf16_dev(hist_v),
                             int_dev(0), 1, clen * hkv, d)
    view.k_scale.view(-1)[: clen * hkv].copy_(torch.from_numpy(pks))
    view.v_scale.view(-1)[: clen * hkv].copy_(torch.from_numpy(pvs))
    q, k, v = rope_qkv(n, hq, hkv, d, 1e6, False, 75)
    step("config5 append chunk")
    cache.append(0, bf16_dev(k), bf16_dev(v), n, int_dev(clen))
    out = torch.empty((n, hq, d), dtype=torch.bfloat16, device=DEV)
    step("config5 chunked prefill")
    R.flash_prefill_bf16(out, bf16_dev(q), view.k, view.v, view.k_scale, view.v_scale, n,
                         int_dev(clen), hq, hkv, d, scale)
    sync()
    k8, v8 = host(view.k).reshape(-1, d), host(view.v).reshape(-1, d)
    ks, vs = host(view.k_scale).reshape(-1), host(view.v_scale).reshape(-1)
    wk = O.quantize_kv_fp8_scaled(hist_k, pks, d)
    assert np.array_equal(k8[: clen * hkv], wk)
    got = bf16_host(out)
    check_rows(got, q, k8, v8, ks, vs, clen, sampled_rows(n, 4, 5), hq, hkv, d, scale)
    # The heaviest workgroup's rows (the last 256 of the chunk, every head).
    check_block(got, q, k8, v8, ks, vs, clen, n - 256, n, hq, hkv, d, scale)


@pytest.mark.parametrize("mag", [2.0 ** -10, 1.0, 2.0 ** 13])
def test_value_magnitudes_within_f16_staging(mag):
    """V is staged for the P V MFMAs as f16(code * v_scale), as the reference
    stages it (flash_prefill.cuh:21-24): values with |v| inside the f16 normal
    range [2^-14, 65504] keep full precision. Rows of N(0,1) * mag (|v| up to
    ~4.5 * 2^13 = 37k at the top) match the oracle within the tolerance
    relative to mag. Outside that range (|v| > 65504, or far below 2^-14)
    prefill is not supported, like the reference; decode has no such limit
    (bf16 V with the scale folded into P)."""
    n, hq, hkv, d = 600, 8, 2, 128
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((n, hq, d), 81)
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((n * hkv, d), 82), d)
    vx = O.f32_to_bf16(O.bf16_to_f32(O.normal_bf16((n * hkv, d), 83)) * np.float32(mag))
    v8, vs = O.quantize_kv_fp8(vx, d)
    got = gpu_prefill(q, k8, v8, ks, vs, n, 0, hq, hkv, d, scale)
    want = O.attention_f32(q, k8, v8, ks, vs, n, 0, hq, hkv, d, scale, NTHREADS)
    a = O.bf16_to_f32(got).astype(np.float64) / mag
    b = O.bf16_to_f32(want).astype(np.float64) / mag
    assert np.isfinite(a).all()
    err = np.abs(a - b)
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (err.max(), err.mean())


def test_workgroup_shapes_agree_with_each_other():
    """The three prefill workgroup shapes on the same heads: the key-split
    kernel sums each row's exponentials as f16 p (v_dot2c, its register
    budget), the 4- and 8-wave kernels as fp32 e; the P V MFMAs of all three
    use f16 p. The heads are replicated so that one call takes each shape
    (hq 8: key split, hq 128: 4-wave, hq 256: 8-wave); outputs of the same
    head must agree within 2 bf16 ulps where |O| > 1e-2 and within 2e-4
    elsewhere, and each with the oracle."""
    n, hq0, hkv0, d = 700, 8, 2, 128
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((n, hq0, d), 51)
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((n * hkv0, d), 52), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16((n * hkv0, d), 53), d)
    outs = []
    for rep in (1, 16, 32):
        hq, hkv = hq0 * rep, hkv0 * rep
        qr = np.tile(q, (1, rep, 1))
        k_r = np.tile(k8.reshape(n, hkv0, d), (1, rep, 1)).reshape(-1, d)
        v_r = np.tile(v8.reshape(n, hkv0, d), (1, rep, 1)).reshape(-1, d)
        ks_r = np.tile(ks.reshape(n, hkv0), (1, rep)).reshape(-1)
        vs_r = np.tile(vs.reshape(n, hkv0), (1, rep)).reshape(-1)
        got = gpu_prefill(qr, k_r, v_r, ks_r, vs_r, n, 0, hq, hkv, d, scale)
        outs.append(O.bf16_to_f32(got.reshape(n, rep, hq0, d)[:, -1]))
    want = O.attention_f32(q, k8, v8, ks, vs, n, 0, hq0, hkv0, d, scale, NTHREADS)
    for o in outs:
        mx, mean = O.bf16_err(O.f32_to_bf16(o), want)
        assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)
    def ordered(x):   # bf16 bit patterns as integers ordered like the values
        b16 = O.f32_to_bf16(x).astype(np.int32)
        return np.where(b16 & 0x8000, 0x8000 - b16, b16)

    for a in outs[1:]:
        b = outs[0]
        big = np.abs(b) > 1e-2
        ulps = np.abs(ordered(a) - ordered(b))[big]
        assert ulps.max() <= 2, ulps.max()
        assert np.abs(a - b)[~big].max() <= 2e-4, np.abs(a - b)[~big].max()
