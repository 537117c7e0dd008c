"""FP8 KV append/quantize on the GPU, bit-exact against the oracle
(reference src/kernels/quantization.cu:200-254; test cases of
tests/kernels/test_quantization.cpp:126-170 plus placement, NaN, saturation)."""
import numpy as np
import pytest
import torch

import oracle_lib as O
import runtherder_amd as R
from gpu_util import bf16_dev, f32_dev, host, int_dev, step, sync, u8_dev, DEV

pytestmark = pytest.mark.gpu


def run_quant(x, head_dim, at_pos=0, rows_per_pos=1, dst_rows=None):
    num_rows = x.size // head_dim
    dst_rows = dst_rows or num_rows + at_pos * rows_per_pos
    step(f"quantize rows={num_rows} d={head_dim} at_pos={at_pos} rpp={rows_per_pos}")
    q = torch.zeros((dst_rows, head_dim), dtype=torch.uint8, device=DEV)
    s = torch.zeros(dst_rows, dtype=torch.float32, device=DEV)
    R.quantize_kv_fp8(q, s, bf16_dev(x), int_dev(at_pos), rows_per_pos, num_rows, head_dim)
    sync()
    return host(q), host(s)


@pytest.mark.parametrize("rows,d,seed", [(24, 128, 0xC0FFEE), (8, 256, 0xBADBEEF),
                                         (512, 128, 0xFEEDFACE), (33, 64, 1), (5, 8, 2),
                                         (7, 24, 3), (3, 1024, 4), (2, 4096, 5)])
def test_quantize_bit_exact(rows, d, seed):
    x = O.mt19937_uniform_bf16((rows, d), 1.0, seed)
    q, s = run_quant(x, d)
    wq, ws = O.quantize_kv_fp8(x, d)
    assert np.array_equal(s.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(q, wq)


def test_quantize_normal_wide_range_bit_exact():
    x = O.normal_bf16((4096, 128), 77)
    x[::7] = O.f32_to_bf16(O.bf16_to_f32(x[::7]) * np.float32(1e-3))
    x[3::11] = O.f32_to_bf16(O.bf16_to_f32(x[3::11]) * np.float32(3e4))
    q, s = run_quant(x, 128)
    wq, ws = O.quantize_kv_fp8(x, 128)
    assert np.array_equal(s.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(q, wq)


@pytest.mark.parametrize("rows,d", [(33001, 128), (32770, 256)])
def test_large_append_half_lanes_bit_exact(rows, d):
    """Appends of 32768 rows or more run with half the lanes per row (two
    loads in flight per lane); ragged row counts, wide-range values and
    zero / NaN / inf rows must still match the oracle bit for bit."""
    x = O.normal_bf16((rows, d), 123 + d)
    x[::5] = O.f32_to_bf16(O.bf16_to_f32(x[::5]) * np.float32(1e-3))
    x[2::9] = O.f32_to_bf16(O.bf16_to_f32(x[2::9]) * np.float32(3e4))
    x[rows - 1] = 0
    x[rows - 2] = 0x8000
    x[rows - 3, 17] = 0x7FC0
    x[rows - 4, 5] = 0x7F80
    q, s = run_quant(x, d)
    wq, ws = O.quantize_kv_fp8(x, d)
    assert np.array_equal(s.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(q, wq)


def test_zero_nan_inf_rows():
    x = O.normal_bf16((4, 128), 9)
    x[0] = 0
    x[1] = 0x8000
    x[2, 17] = 0x7FC0  # NaN ignored by amax, encodes to 0x7F
    x[3, 5] = 0x7F80   # +inf: amax = inf, inv = 0, inf * 0 = NaN
    q, s = run_quant(x, 128)
    wq, ws = O.quantize_kv_fp8(x, 128)
    assert np.array_equal(s.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(q, wq)


def test_placement_at_pos_rows_per_pos():
    hkv, d = 8, 128
    x = O.normal_bf16((3 * hkv, d), 10)
    q, s = run_quant(x, d, at_pos=37, rows_per_pos=hkv, dst_rows=64 * hkv)
    wq, ws = O.quantize_kv_fp8(x, d, at_pos=37, rows_per_pos=hkv, dst_rows=64 * hkv)
    assert np.array_equal(q, wq) and np.array_equal(s.view(np.uint32), ws.view(np.uint32))


def test_given_scale_all_bf16_inputs_bit_exact():
    """Every bf16 bit pattern times several scales through the hardware
    E4M3 converter (covers ties, subnormals, saturation, NaN)."""
    x = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(-1, 128)
    scales = [1.0, 0.004, 0.37, 3.1e-3, 1e-6, 250.0, 0.0]
    for sc in scales:
        step(f"quantize_scaled all-bf16 scale={sc}")
        s = np.full(x.shape[0], sc, np.float32)
        q = torch.zeros(x.shape, dtype=torch.uint8, device=DEV)
        R.quantize_kv_fp8_scaled(q, f32_dev(s), bf16_dev(x), int_dev(0), 1, x.shape[0], 128)
        sync()
        want = O.quantize_kv_fp8_scaled(x, s, 128)
        got = host(q)
        bad = np.argwhere(got != want)
        assert bad.size == 0, (sc, [(int(x[i, j]), int(got[i, j]), int(want[i, j]))
                                    for i, j in bad[:8]])


def test_kv_append_fused_matches_two_quantizes():
    hkv, d, n = 8, 128, 21
    cache = R.KVCache(2, 64, hkv, d)
    k = O.normal_bf16((n, hkv, d), 31)
    v = O.normal_bf16((n, hkv, d), 32)
    step("kv append fused")
    cache.append(1, bf16_dev(k), bf16_dev(v), n, int_dev(9))
    sync()
    wk, wks = O.quantize_kv_fp8(k, d, at_pos=9, rows_per_pos=hkv, dst_rows=64 * hkv)
    wv, wvs = O.quantize_kv_fp8(v, d, at_pos=9, rows_per_pos=hkv, dst_rows=64 * hkv)
    view = cache.view(1)
    rows = slice(9 * hkv, (9 + n) * hkv)
    assert np.array_equal(host(view.k).reshape(-1, d)[rows], wk[rows])
    assert np.array_equal(host(view.v).reshape(-1, d)[rows], wv[rows])
    assert np.array_equal(host(view.k_scale).reshape(-1)[rows], wks[rows])
    assert np.array_equal(host(view.v_scale).reshape(-1)[rows], wvs[rows])
