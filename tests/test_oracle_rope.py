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
