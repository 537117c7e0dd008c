"""Pins the oracle's quantize_kv_fp8 restatement (reference
src/kernels/quantization.cu:200-254) with the reference test's checks
(tests/kernels/test_quantization.cpp:64-170) and closed forms."""
import numpy as np
import torch

import oracle_lib as O


def _closed_form(x_bits, head_dim):
    x = O.bf16_to_f32(x_bits).reshape(-1, head_dim)
    amax = np.max(np.abs(x), axis=1).astype(np.float32)
    scale = (amax / np.float32(448.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, np.float32(448.0) / amax, np.float32(0)).astype(np.float32)
    prod = (x * inv[:, None]).astype(np.float32)
    codes = torch.from_numpy(np.clip(prod, -448, 448)).to(torch.float8_e4m3fn)
    return codes.view(torch.uint8).numpy(), scale


def _reference_case(num_rows, head_dim, seed):
    x = O.mt19937_uniform_bf16((num_rows, head_dim), 1.0, seed)
    q, s = O.quantize_kv_fp8(x, head_dim)
    want_q, want_s = _closed_form(x, head_dim)
    assert np.array_equal(s.view(np.uint32), want_s.view(np.uint32))  # scale bit-exact
    assert np.array_equal(q, want_q)
    # round-trip bounds of the reference test
    orig = O.bf16_to_f32(x).astype(np.float64).reshape(num_rows, head_dim)
    deq = (O.e4m3_decode(q).astype(np.float32) * s[:, None]).astype(np.float64)
    cos = (orig * deq).sum() / np.sqrt((orig ** 2).sum() * (deq ** 2).sum())
    assert cos >= 0.998
    big = np.abs(orig) > 0.1 * (s[:, None] * 448.0)
    rel = np.abs(deq - orig)[big] / np.abs(orig)[big]
    assert rel.max() <= 0.08


def test_round_trip_head_dim_128():
    _reference_case(24, 128, 0xC0FFEE)


def test_round_trip_head_dim_256():
    _reference_case(8, 256, 0xBADBEEF)


def test_round_trip_batched():
    _reference_case(512, 128, 0xFEEDFACE)


def test_zero_row_maps_to_zero():
    x = np.zeros((2, 128), np.uint16)
    x[1, :] = 0x8000  # -0.0
    q, s = O.quantize_kv_fp8(x, 128)
    assert np.all(s == 0.0)
    assert np.all(q[0] == 0x00) and np.all(q[1] == 0x80)


def test_nan_ignored_by_amax():
    x = O.normal_bf16((1, 128), 3)
    x[0, 5] = 0x7FC0
    q, s = O.quantize_kv_fp8(x, 128)
    finite = O.bf16_to_f32(np.delete(x[0], 5))
    assert s[0] == np.float32(np.max(np.abs(finite))) / np.float32(448)
    assert q[0, 5] == 0x7F


def test_at_pos_and_rows_per_pos_placement():
    hkv, d = 8, 128
    x = O.normal_bf16((3 * hkv, d), 11)
    q, s = O.quantize_kv_fp8(x, d, at_pos=5, rows_per_pos=hkv, dst_rows=10 * hkv)
    q0, s0 = O.quantize_kv_fp8(x, d)
    assert np.array_equal(q[5 * hkv:8 * hkv], q0) and np.array_equal(s[5 * hkv:8 * hkv], s0)
    assert np.all(q[:5 * hkv] == 0) and np.all(q[8 * hkv:] == 0)


def test_given_scale_variant_saturates():
    x = O.normal_bf16((64, 128), 5)
    scale = O.uniform_f32(64, 0.01, 0.1, 9)
    scale[:8] = np.float32(0.004)  # |x| > 1.8 saturates on these rows
    q = O.quantize_kv_fp8_scaled(x, scale, 128)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    prod = (O.bf16_to_f32(x).reshape(64, 128) * inv[:, None]).astype(np.float32)
    want = torch.from_numpy(np.clip(prod, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8)
    assert np.array_equal(q, want.numpy())
    assert np.any(np.abs(prod) > 448)  # the satfinite path is exercised
