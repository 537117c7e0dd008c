"""RMSNorm oracle (reference src/kernels/rmsnorm.cu:45-136) pinned against
the reference test's own CPU formula (tests/kernels/test_rmsnorm.cpp:39-60:
double sum of squares, rrms = 1.0f / sqrt(float(ss / dim) + eps)) and closed
forms."""
import numpy as np
import pytest

import oracle_lib as O


def reference_test_formula(x_bits, g_bits, eps):
    x = O.bf16_to_f32(x_bits)
    g = O.bf16_to_f32(g_bits)
    ss = (x.astype(np.float64) ** 2).sum(axis=-1, keepdims=True)
    rrms = (np.float32(1.0) / np.sqrt((ss / x.shape[-1]).astype(np.float32) + np.float32(eps)))
    return O.f32_to_bf16((x * rrms.astype(np.float32)) * g)


@pytest.mark.parametrize("dim,lanes", [(128, 16), (64, 8), (256, 32), (4096, 64), (3072, 64),
                                       (24, 4)])
def test_matches_reference_test_formula(dim, lanes):
    x = O.normal_bf16((37, dim), 11 + dim)
    g = O.normal_bf16((dim,), 12 + dim)
    got = O.rmsnorm_bf16(x, g, 1e-6, lanes)
    want = reference_test_formula(x, g, 1e-6)
    diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
    # fp32 vs double sums of squares may move rrms by an ulp, and with it an
    # occasional output by one bf16 ulp.
    assert diff.max() <= 1
    assert np.count_nonzero(diff) <= max(2, got.size // 200)


def test_constant_rows_and_unit_gain():
    dim = 128
    ones = O.f32_to_bf16(np.ones(dim, np.float32))
    for c in (0.5, -3.0, 1024.0):
        x = O.f32_to_bf16(np.full((2, dim), c, np.float32))
        y = O.bf16_to_f32(O.rmsnorm_bf16(x, ones, 0.0, 16))
        assert np.array_equal(y, np.full_like(y, np.sign(c)))


def test_power_of_two_scale_invariance_without_eps():
    x = O.normal_bf16((9, 128), 21)
    g = O.normal_bf16((128,), 22)
    y1 = O.rmsnorm_bf16(x, g, 0.0, 16)
    x8 = O.f32_to_bf16(O.bf16_to_f32(x) * np.float32(8.0))
    assert np.array_equal(O.rmsnorm_bf16(x8, g, 0.0, 16), y1)


def test_zero_row_is_zero():
    x = np.zeros((1, 128), np.uint16)
    g = O.normal_bf16((128,), 23)
    assert np.all(O.bf16_to_f32(O.rmsnorm_bf16(x, g, 1e-6, 16)) == 0.0)
