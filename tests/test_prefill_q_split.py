"""The prefill kernel scores raw E4M3 K codes against q split into two E4M3
parts (runtherder_amd/csrc/flash_prefill.hip, the q split in
flash_prefill_body): per row, y = q * 2^a with the row maximum in [128, 256),
hi = e4m3(y), lo = e4m3(16 * (y - hi)), and the MFMA computes code * hi +
code * lo / 16. This pins the error of that split over every bf16 value a
scaled element can take, with the E4M3 round-to-nearest-even encoder the GPU
converter matches (pinned against the OCP spec in test_oracle_e4m3.py):

  * |y| >= 2^-6 (every element within 2^-14 of its row maximum, give or take
    a binade): hi + lo / 16 == y exactly;
  * |y| <  2^-6: lo falls into E4M3 subnormals (spacing 2^-9) and loses low
    bits; |y - (hi + lo / 16)| <= 2^-14, i.e. at most 2^-21 of the row
    maximum.
"""
import numpy as np

import oracle_lib as O


def all_scaled_bf16():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    y = O.bf16_to_f32(bits)
    keep = np.isfinite(y) & (np.abs(y) < 256.0)
    return y[keep]


def split(y):
    hi = O.e4m3_decode(O.e4m3_encode(y))
    lo = O.e4m3_decode(O.e4m3_encode((y - hi) * np.float32(16.0)))
    return hi, lo


def test_split_is_exact_above_e4m3_normal_range():
    y = all_scaled_bf16()
    hi, lo = split(y)
    back = hi.astype(np.float64) + lo.astype(np.float64) / 16.0
    big = np.abs(y) >= 2.0 ** -6
    assert big.sum() == 2 * 14 * 128   # 14 binades [2^-6, 2^8) x 128 mantissas x 2 signs
    assert np.array_equal(back[big], y[big].astype(np.float64))


def test_split_error_bound_below_normal_range():
    y = all_scaled_bf16()
    hi, lo = split(y)
    err = np.abs(hi.astype(np.float64) + lo.astype(np.float64) / 16.0 - y.astype(np.float64))
    small = np.abs(y) < 2.0 ** -6
    assert err[small].max() <= 2.0 ** -14
    # the bound is attained (it is the real bound, not a loose one) and the
    # loss really occurs below 2^-6
    assert err[small].max() == 2.0 ** -14
    assert (err[small] > 0).sum() > 1000


def test_dropping_lo_would_be_caught():
    """A split without its lo part (hi only) errs by up to 2^-5 of |y|: the
    GPU mixed-magnitude prefill test (test_gpu_prefill.py) relies on the lo
    term to stay within tolerance."""
    y = all_scaled_bf16()
    hi, _ = split(y)
    rel = np.abs(hi - y)[np.abs(y) >= 1.0] / np.abs(y[np.abs(y) >= 1.0])
    assert rel.max() >= 2.0 ** -5 * 0.99
