"""RoPE input preparation (reference src/kernels/rope.cu:32-54,
src/model/supported/llama/llama.cu:128-143, llama3.cu:26-60): closed forms."""
import numpy as np

import oracle_lib as O


def test_plain_table_closed_form():
    f = O.rope_inv_freq_plain(128, 1e6)
    want = (1e6 ** (-2.0 * np.arange(64) / 128)).astype(np.float32)
    assert np.array_equal(f, want)


def test_llama3_bands():
    plain = O.rope_inv_freq_plain(128, 5e5).astype(np.float64)
    f = O.rope_inv_freq_llama3(128, 5e5, 32.0, 1.0, 4.0, 8192).astype(np.float64)
    wl = 2 * np.pi / plain
    hi = wl < 8192 / 4.0
    lo = wl > 8192 / 1.0
    assert np.array_equal(f[hi], plain[hi].astype(np.float32))
    assert np.allclose(f[lo], plain[lo] / 32.0, rtol=1e-7)
    mid = ~(hi | lo)
    assert np.all((f[mid] <= plain[mid]) & (f[mid] >= plain[mid] / 32.0 * (1 - 1e-7)))
    assert np.all(np.diff(f) < 0)


def test_position_zero_is_identity_and_norms_kept():
    x = O.normal_bf16((4, 3, 128), 5)
    inv = O.rope_inv_freq_plain(128, 1e4)
    y0 = O.rope_apply_bf16(x, np.zeros(4, np.int32), inv)
    assert np.array_equal(y0, x)
    y = O.rope_apply_bf16(x, np.array([1, 7, 1024, 5000], np.int32), inv)
    a, b = O.bf16_to_f32(x), O.bf16_to_f32(y)
    na = a[..., :64] ** 2 + a[..., 64:] ** 2
    nb = b[..., :64] ** 2 + b[..., 64:] ** 2
    assert np.allclose(na, nb, rtol=2e-2, atol=1e-3)


def _rope_f64_emulation(x_bits, positions, inv):
    """Independent restatement in numpy: fp32 angle, sin/cos of it in double
    rounded to fp32, then fma(a, c, -(b*s)) / fma(a, s, b*c) evaluated as the
    exact double product plus the fp32-rounded other product, rounded to
    fp32, then to bf16."""
    a_all = O.bf16_to_f32(x_bits)
    d = x_bits.shape[-1]
    half = d // 2
    th = (positions.astype(np.float32)[:, None] * inv[None, :]).astype(np.float32)
    c = np.cos(th.astype(np.float64)).astype(np.float32).astype(np.float64)[:, None, :]
    s = np.sin(th.astype(np.float64)).astype(np.float32).astype(np.float64)[:, None, :]
    a = a_all[..., :half].astype(np.float64)
    b = a_all[..., half:].astype(np.float64)
    bs = (b * s).astype(np.float32).astype(np.float64)
    bc = (b * c).astype(np.float32).astype(np.float64)
    r0 = (a * c - bs).astype(np.float32)
    r1 = (a * s + bc).astype(np.float32)
    return O.f32_to_bf16(np.concatenate([r0, r1], axis=-1))


def test_rope_matches_independent_emulation():
    """Pins the oracle's RoPE (used bit-exactly by the GPU RoPE tests) against
    a separate numpy statement: the pair order, the signs and the angle are
    all checked; only double-rounding corner cases of the emulation may
    differ by one bf16 ulp."""
    x = O.normal_bf16((64, 6, 128), 9)
    pos = np.array(list(range(0, 32)) + [131071, 126976, 8191, 100000] + list(range(5000, 5028)),
                   np.int32)
    for inv in (O.rope_inv_freq_plain(128, 1e6),
                O.rope_inv_freq_llama3(128, 5e5, 32.0, 1.0, 4.0, 8192)):
        got = O.rope_apply_bf16(x, pos, inv)
        want = _rope_f64_emulation(x, pos, inv)
        diff = got.astype(np.int32) - want.astype(np.int32)
        assert np.count_nonzero(diff) <= got.size // 10000, np.count_nonzero(diff)
        assert np.abs(diff).max() <= 1


def test_rope_within_reference_bound_of_double():
    """The reference's own bar for rope_bf16: max-abs 5e-2 against double
    precision (include/runtherder/kernels/rope.cuh:14)."""
    x = O.normal_bf16((16, 4, 128), 10)
    pos = np.arange(16, dtype=np.int32) * 8191
    inv = O.rope_inv_freq_plain(128, 5e5)
    got = O.bf16_to_f32(O.rope_apply_bf16(x, pos, inv)).astype(np.float64)
    a = O.bf16_to_f32(x).astype(np.float64)
    th = pos[:, None].astype(np.float64) * inv[None, :].astype(np.float64)
    c, s = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
    want = np.concatenate([a[..., :64] * c - a[..., 64:] * s, a[..., :64] * s + a[..., 64:] * c],
                          axis=-1)
    assert np.abs(got - want).max() <= 5e-2
