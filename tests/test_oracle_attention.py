"""Pins the oracle's attention restatements (reference
src/kernels/attention.cu:34-91, flash_decode.cu:118-247) against an
independent numpy fp64 implementation and against invariants that fix the
math: single key, uniform scores, chunked == tail rows, split invariance."""
import numpy as np
import pytest

import oracle_lib as O


def numpy_attention(q_bits, k8, v8, ks, vs, n_new, cache_len, hq, hkv, d, scale):
    """fp64 causal GQA attention over float(E4M3) * scale, kvh = qh // (hq/hkv)."""
    group = hq // hkv
    q = O.bf16_to_f32(q_bits).astype(np.float64).reshape(n_new, hq, d)
    total = cache_len + n_new
    k = O.e4m3_decode(k8).astype(np.float64).reshape(total, hkv, d) * ks.reshape(total, hkv, 1)
    v = O.e4m3_decode(v8).astype(np.float64).reshape(total, hkv, d) * vs.reshape(total, hkv, 1)
    out = np.empty((n_new, hq, d))
    for t in range(n_new):
        keys = cache_len + t + 1
        for h in range(hq):
            s = (k[:keys, h // group] @ q[t, h]) * scale
            w = np.exp(s - s.max())
            out[t, h] = (w @ v[:keys, h // group]) / w.sum()
    return out


def make_case(n_new, cache_len, hq, hkv, d, uniform=True):
    total = cache_len + n_new
    if uniform:  # the reference tests' inputs
        q = O.mt19937_uniform_bf16((total, hq, d), 1.0, 0xA11CE)[cache_len:]
        kx = O.mt19937_uniform_bf16((total * hkv, d), 1.0, 0xB0B)
        vx = O.mt19937_uniform_bf16((total * hkv, d), 1.0, 0xCAFE)
    else:
        q = O.normal_bf16((n_new, hq, d), 1)
        kx = O.normal_bf16((total * hkv, d), 2)
        vx = O.normal_bf16((total * hkv, d), 3)
    k8, ks = O.quantize_kv_fp8(kx, d)
    v8, vs = O.quantize_kv_fp8(vx, d)
    return np.ascontiguousarray(q), k8, v8, ks, vs


REF_CASES = [  # reference tests/kernels/test_attention.cpp:293-326
    (1, 0, 4, 1, 64), (8, 0, 8, 8, 64), (16, 0, 32, 8, 128), (8, 0, 8, 2, 256),
    (64, 0, 32, 8, 128), (1, 15, 32, 8, 128), (6, 10, 8, 2, 64),
]


@pytest.mark.parametrize("n_new,cache_len,hq,hkv,d", REF_CASES)
def test_f32_oracle_vs_numpy_fp64(n_new, cache_len, hq, hkv, d):
    scale = 1.0 / np.sqrt(d)
    args = make_case(n_new, cache_len, hq, hkv, d)
    got = O.attention_f32(*args, n_new, cache_len, hq, hkv, d, np.float32(scale))
    want = numpy_attention(*args, n_new, cache_len, hq, hkv, d, scale)
    mx, mean = O.bf16_err(got, want)
    assert mx <= 8e-3 and mean <= 1e-3, (mx, mean)
    f64 = O.attention_f64(*args, n_new, cache_len, hq, hkv, d, scale)
    assert np.max(np.abs(f64 - want)) <= 1e-9


def test_single_key_returns_v0_exactly():
    q, k8, v8, ks, vs = make_case(1, 0, 4, 1, 64)
    got = O.attention_f32(q, k8, v8, ks, vs, 1, 0, 4, 1, 64, 0.125)
    v0 = (O.e4m3_decode(v8[0]) * ks.dtype.type(vs[0])).astype(np.float32)
    for h in range(4):
        assert np.array_equal(got[0, h], O.f32_to_bf16(v0))


def test_zero_query_averages_values():
    n, hq, hkv, d = 5, 4, 2, 64
    q, k8, v8, ks, vs = make_case(n, 0, hq, hkv, d, uniform=False)
    q = np.zeros_like(q)
    got = O.attention_f32(q, k8, v8, ks, vs, n, 0, hq, hkv, d, 0.125)
    v = O.e4m3_decode(v8).astype(np.float64).reshape(n, hkv, d) * vs.reshape(n, hkv, 1)
    for t in range(n):
        for h in range(hq):
            want = v[: t + 1, h // 2].mean(axis=0)
            err = np.abs(O.bf16_to_f32(got[t, h]) - want)
            assert np.all(err <= np.abs(want) * 2.0 ** -8 + 1e-6)  # bf16 half-ulp


def test_chunked_equals_tail_rows():
    hq, hkv, d = 8, 2, 64
    total, clen = 16, 10
    q, k8, v8, ks, vs = make_case(total, 0, hq, hkv, d)
    full = O.attention_f32(q, k8, v8, ks, vs, total, 0, hq, hkv, d, 0.125)
    tail = O.attention_f32(q[clen:], k8, v8, ks, vs, total - clen, clen, hq, hkv, d, 0.125)
    assert np.array_equal(full[clen:], tail)


@pytest.mark.parametrize("cache_len,splits", [(300, 4), (0, 1), (2, 8), (1000, 8), (1000, 64),
                                              (511, 3), (37, 32)])
def test_split_decode_matches_attention(cache_len, splits):
    hq, hkv, d = 32, 8, 128
    q, k8, v8, ks, vs = make_case(1, cache_len, hq, hkv, d)
    a = O.attention_f32(q, k8, v8, ks, vs, 1, cache_len, hq, hkv, d, np.float32(d ** -0.5))
    b = O.decode_split_f32(q, k8, v8, ks, vs, splits, cache_len, hq, hkv, d, np.float32(d ** -0.5))
    mx, mean = O.bf16_err(a[0], b)
    assert mx <= 8e-3 and mean <= 5e-4
