"""Causal prefill of a few tokens after a cache as split-K decode
(rth_attn_prefill_split, no reference counterpart): against the oracle's
fp32 attention over the same cache bytes (the reference's math,
attention.cu:34-91) and against the flash prefill kernel on the same inputs;
the paged entry against the contiguous one."""
import numpy as np
import pytest
import torch

import oracle_lib as O
import runtherder_amd as R
from gpu_util import (DEV, NTHREADS, bf16_dev, bf16_host, f32_dev, i32_dev, int_dev, step, sync,
                      u8_dev)
from test_gpu_paged import gather, make_pair

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def split_prefill(q, k8, v8, ks, vs, n_new, clen, hq, hkv, d, splits, scale):
    step(f"prefill split n_new={n_new} clen={clen} hq={hq} hkv={hkv} d={d} splits={splits}")
    out = torch.empty((n_new, hq, d), dtype=torch.bfloat16, device=DEV)
    part = R.new_flash_split_scratch(n_new * hq, d, splits)
    R.flash_prefill_split_bf16(out, bf16_dev(q), u8_dev(k8), u8_dev(v8), f32_dev(ks),
                               f32_dev(vs), part, splits, n_new, int_dev(clen), hq, hkv, d,
                               scale)
    sync()
    return bf16_host(out)


def inputs(n_new, clen, hq, hkv, d, seed):
    total = clen + n_new
    q = O.normal_bf16((n_new, hq, d), seed)
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((total * hkv, d), seed + 1), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16((total * hkv, d), seed + 2), d)
    return q, k8, v8, ks, vs


# (n_new, clen, hq, hkv, d, splits): 2..64 tokens; caches from empty to 8K;
# groups of 1, 2, 3, 4 and 6 q heads, MQA (8), 32 (two q blocks), head_dim
# 64 / 256;
# split counts that are and are not multiples of 8, more splits than tiles,
# grouped (cooperative) and one-wave-per-unit launches.
CASES = [
    (2, 0, 32, 8, 128, 64), (4, 100, 32, 8, 128, 64), (3, 31, 24, 8, 128, 256),
    (16, 1000, 32, 8, 128, 16), (8, 8192, 32, 8, 128, 32), (64, 2000, 24, 8, 128, 4),
    (5, 333, 32, 8, 64, 32), (7, 600, 16, 2, 256, 16), (2, 50, 64, 2, 128, 32),
    (1, 500, 32, 8, 128, 256), (4, 4000, 8, 1, 128, 100), (16, 40, 32, 8, 128, 128),
    (13, 2047, 24, 8, 128, 19), (32, 4096, 32, 8, 128, 8),
    # MHA (16 tokens per virtual head), groups of 2 (8) and 6 (2), head_dim
    # 256 at 8 tokens per virtual head (its LDS staging row), a ragged last
    # token block.
    (37, 1500, 8, 8, 128, 16), (19, 700, 16, 8, 128, 32), (9, 900, 12, 2, 128, 64),
    (20, 1234, 4, 4, 256, 16), (256, 3000, 24, 4, 64, 1), (128, 500, 24, 8, 64, 2),
    # beyond 64 tokens at head_dim 128: the flash prefill over key runs (runs
    # past the cache, more runs than tiles, one run, ragged row blocks).
    (100, 3000, 32, 8, 128, 4), (300, 5000, 24, 8, 128, 8), (1000, 200, 32, 8, 128, 3),
    (129, 0, 8, 1, 128, 16), (517, 7777, 16, 4, 128, 5), (256, 3000, 32, 8, 128, 1),
    # all keys in run 0 (8 tiles: it stores the output itself) and one key
    # tile past it.
    (250, 200, 32, 8, 128, 8), (300, 250, 32, 8, 128, 8),
]


@pytest.mark.parametrize("n_new,clen,hq,hkv,d,splits", CASES)
def test_prefill_split_matches_oracle(n_new, clen, hq, hkv, d, splits):
    scale = np.float32(1.0 / np.sqrt(d))
    q, k8, v8, ks, vs = inputs(n_new, clen, hq, hkv, d, 900 + n_new + clen)
    got = split_prefill(q, k8, v8, ks, vs, n_new, clen, hq, hkv, d, splits, scale)
    want = O.attention_f32(q, k8, v8, ks, vs, n_new, clen, hq, hkv, d, scale, NTHREADS)
    mx, mean = O.bf16_err(got, want)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)
    if d == 128:
        step("prefill kernel on the same inputs")
        ref = torch.empty((n_new, hq, d), dtype=torch.bfloat16, device=DEV)
        R.flash_prefill_bf16(ref, bf16_dev(q), u8_dev(k8), u8_dev(v8), f32_dev(ks),
                             f32_dev(vs), n_new, int_dev(clen), hq, hkv, d, scale)
        sync()
        mx2, mean2 = O.bf16_err(got, bf16_host(ref))
        assert mx2 <= MAX_ABS and mean2 <= 1e-3, (mx2, mean2)


def test_prefill_split_single_token_equals_decode():
    """n_new = 1 is the decode call: same units, same partition, same merge,
    so the outputs are bit-identical."""
    hq, hkv, d, clen, splits = 32, 8, 128, 3000, 64
    scale = np.float32(1.0 / np.sqrt(d))
    q, k8, v8, ks, vs = inputs(1, clen, hq, hkv, d, 77)
    got = split_prefill(q, k8, v8, ks, vs, 1, clen, hq, hkv, d, splits, scale)
    step("decode on the same inputs")
    out = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    part = R.new_flash_split_scratch(hq, d, splits)
    R.flash_decode_split_bf16(out, bf16_dev(q[0]), u8_dev(k8), u8_dev(v8), f32_dev(ks),
                              f32_dev(vs), part, splits, int_dev(clen), hq, hkv, d, scale)
    sync()
    assert np.array_equal(got[0], bf16_host(out))


@pytest.mark.parametrize("total,n_new,block,splits", [(1500, 4, 64, 32), (3000, 16, 32, 16),
                                                      (777, 9, 256, 64), (3000, 200, 64, 4)])
def test_prefill_split_paged_equals_contiguous(total, n_new, block, splits):
    hq, hkv, d = 32, 8, 128
    clen = total - n_new
    cont, paged, bt, table, _, _ = make_pair(total, hq, hkv, d, block, 70 + total)
    qh = O.normal_bf16((n_new, hq, d), 80 + total)
    q = bf16_dev(qh)
    scale = float(1.0 / np.sqrt(d))
    o1 = torch.empty((n_new, hq, d), dtype=torch.bfloat16, device=DEV)
    o2 = torch.empty_like(o1)
    part = R.new_flash_split_scratch(n_new * hq, d, splits)
    step(f"paged prefill split total={total} n_new={n_new} block={block}")
    cv = cont.view(0)
    R.flash_prefill_split_bf16(o1, q, cv.k, cv.v, cv.k_scale, cv.v_scale, part, splits, n_new,
                               int_dev(clen), hq, hkv, d, scale)
    sync()
    got1 = bf16_host(o1)
    from runtherder_amd import _ffi
    from runtherder_amd.ops import _p, _stream
    _ffi.call("rth_attn_prefill_split_paged", _p(o2), _p(q), _p(paged.k[0]), _p(paged.v[0]),
              _p(paged.k_scale[0]), _p(paged.v_scale[0]), _p(bt), block, _p(part), splits,
              n_new, _p(int_dev(clen)), hq, hkv, d, scale, _stream(None))
    sync()
    got2 = bf16_host(o2)
    assert np.array_equal(got1, got2)
    gk, gv, gks, gvs = gather(paged, table, total, block)
    want = O.attention_f32(qh, gk.reshape(total * hkv, d), gv.reshape(total * hkv, d),
                           gks.reshape(-1), gvs.reshape(-1), n_new, clen, hq, hkv, d,
                           np.float32(scale), NTHREADS)
    mx, mean = O.bf16_err(got2, want)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


def test_prefill_split_rejects_bad_arguments():
    hq, hkv, d = 32, 8, 128
    out = torch.empty((4097, hq, d), dtype=torch.bfloat16, device=DEV)
    q = torch.zeros_like(out)
    k = torch.zeros((100, hkv, d), dtype=torch.uint8, device=DEV)
    s = torch.zeros((100, hkv), dtype=torch.float32, device=DEV)
    part = R.new_flash_split_scratch(2 * hq, d, 4)
    with pytest.raises(R._ffi.RthError, match="n_new"):
        R.flash_prefill_split_bf16(out, q, k, k, s, s, part, 4, 4097, int_dev(0), hq, hkv, d, 0.1)
    with pytest.raises(R._ffi.RthError, match="head_dim"):
        R.flash_prefill_split_bf16(out[:2, :, :32].contiguous(), q[:2, :, :32].contiguous(), k,
                                   k, s, s, part, 4, 2, int_dev(0), hq, hkv, 32, 0.1)


@pytest.mark.parametrize("n_new", [2, 80, 81, 256, 257])
def test_adaptive_backend_routes_small_prefill(n_new):
    """AdaptiveAttention.run: 2..80 tokens take the split-K decode route over
    the backend's scratch, 81..256 the flash prefill over key runs, 257 the
    flash prefill; all match the oracle."""
    hq, hkv, d, clen = 32, 8, 128, 3000
    scale = np.float32(1.0 / np.sqrt(d))
    q, k8, v8, ks, vs = inputs(n_new, clen, hq, hkv, d, 500 + n_new)
    be = R.AdaptiveAttention(R.AttnConfig.for_heads(hq, hkv, d))
    assert (be._split_prefill_splits(n_new) > 0) == (n_new <= R.ops.PREFILL_RUNS_TOKENS)
    kv = R.KVView(u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs))
    out = torch.empty((n_new, hq, d), dtype=torch.bfloat16, device=DEV)
    step(f"adaptive run n_new={n_new} clen={clen}")
    be.run(out, bf16_dev(q), kv, n_new, int_dev(clen))
    sync()
    want = O.attention_f32(q, k8, v8, ks, vs, n_new, clen, hq, hkv, d, scale, NTHREADS)
    mx, mean = O.bf16_err(bf16_host(out), want)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


def test_adaptive_backend_small_prefill_paged_equals_contiguous():
    """The backend's few-token route on a paged view gives the contiguous
    view's bytes (the same kernels through the block table)."""
    hq, hkv, d, total, n_new, block = 32, 8, 128, 2100, 8, 64
    clen = total - n_new
    cont, paged, bt, table, _, _ = make_pair(total, hq, hkv, d, block, 90)
    be = R.AdaptiveAttention(R.AttnConfig.for_heads(hq, hkv, d))
    qh = O.normal_bf16((n_new, hq, d), 91)
    q = bf16_dev(qh)
    o1 = torch.empty((n_new, hq, d), dtype=torch.bfloat16, device=DEV)
    o2 = torch.empty_like(o1)
    step(f"adaptive paged few-token prefill total={total} n_new={n_new}")
    be.run(o1, q, cont.view(0), n_new, int_dev(clen))
    be.run(o2, q, paged.view(0, bt), n_new, int_dev(clen))
    sync()
    got = bf16_host(o2)
    assert np.array_equal(bf16_host(o1), got)
    gk, gv, gks, gvs = gather(paged, table, total, block)
    want = O.attention_f32(qh, gk.reshape(total * hkv, d), gv.reshape(total * hkv, d),
                           gks.reshape(-1), gvs.reshape(-1), n_new, clen, hq, hkv, d,
                           np.float32(1.0 / np.sqrt(d)), NTHREADS)
    mx, mean = O.bf16_err(got, want)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)
