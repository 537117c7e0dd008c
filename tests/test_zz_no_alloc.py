"""Allocation-free decode entry point (no reference counterpart; for callers
that cannot call hipMalloc): rth_attn_decode_split_noalloc must return
exactly what rth_attn_decode_split returns with caller scratch (same
kernels, same partition), on consecutive calls that reuse the fixed device
array, the second with a smaller input, and reject shapes beyond the array.
Both entries are also checked against the oracle (max-abs 2e-2, mean-abs
2e-3)."""
import ctypes

import numpy as np
import pytest
import torch

import oracle_lib as O
import runtherder_amd as R
from runtherder_amd import _ffi
from gpu_util import DEV, NTHREADS, bf16_dev, bf16_host, f32_dev, int_dev, step, sync, u8_dev

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def run_both(ctx, hq, hkv, d, splits, seed):
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((hq, d), seed)
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((ctx * hkv, d), seed + 1), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16((ctx * hkv, d), seed + 2), d)
    qd, kd, vd, ksd, vsd = bf16_dev(q), u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs)
    pos = int_dev(ctx - 1)
    o_ref = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    o_na = torch.empty_like(o_ref)
    part = R.new_flash_split_scratch(hq, d, splits)
    step(f"no-alloc decode ctx={ctx} hq={hq} hkv={hkv} d={d} splits={splits}")
    _ffi.call("rth_attn_decode_split", _p(o_ref), _p(qd), _p(kd), _p(vd), _p(ksd), _p(vsd),
              _p(part), splits, _p(pos), hq, hkv, d, ctypes.c_float(scale), _stream())
    _ffi.call("rth_attn_decode_split_noalloc", _p(o_na), _p(qd), _p(kd), _p(vd), _p(ksd),
              _p(vsd), splits, _p(pos), hq, hkv, d, ctypes.c_float(scale), _stream())
    sync()
    got, ref = bf16_host(o_na), bf16_host(o_ref)
    assert np.array_equal(got, ref)
    want = O.attention_f32(q, k8, v8, ks, vs, 1, ctx - 1, hq, hkv, d, scale, NTHREADS)
    mx, mean = O.bf16_err(got, want[0])
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


def test_noalloc_equals_caller_scratch_on_consecutive_calls():
    # first call fills most of the array's used prefix, the second is smaller
    run_both(40000, 32, 8, 128, 256, 900)
    run_both(3000, 24, 8, 128, 64, 910)
    run_both(9000, 16, 8, 256, 100, 920)
    run_both(5000, 16, 4, 32, 64, 930)     # the VALU split kernel


def test_noalloc_rejects_oversized_scratch():
    # 64 q heads x 4096 splits x 130 floats > 2^22: rejected before any launch
    scale = ctypes.c_float(0.088)
    fake = ctypes.c_void_p(0x1000)
    with pytest.raises(_ffi.RthError) as e:
        _ffi.call("rth_attn_decode_split_noalloc", fake, fake, fake, fake, fake, fake, 4096,
                  fake, 64, 8, 128, scale, None)
    assert "exceeds the fixed scratch" in str(e.value)


def test_noalloc_first_then_graph_captured():
    """The allocation-free entry called first in this test (so its own
    per-device set-up runs before any other entry here), then captured in a
    HIP graph in global capture mode (where an allocation would fail the
    capture) and replayed three times with eager work between the replays;
    every replay equals the caller-scratch entry bit for bit."""
    ctx, hq, hkv, d, splits = 6000, 24, 8, 128, 128
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((hq, d), 940)
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((ctx * hkv, d), 941), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16((ctx * hkv, d), 942), d)
    qd, kd, vd, ksd, vsd = bf16_dev(q), u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs)
    pos = int_dev(ctx - 1)
    o_na = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    o_ref = torch.empty_like(o_na)
    args = lambda o, st: (_p(o), _p(qd), _p(kd), _p(vd), _p(ksd), _p(vsd), splits, _p(pos), hq,
                          hkv, d, ctypes.c_float(scale), st)
    step("no-alloc decode first call, then graph capture")
    _ffi.call("rth_attn_decode_split_noalloc", *args(o_na, _stream()))
    sync()
    first = bf16_host(o_na)
    part = R.new_flash_split_scratch(hq, d, splits)
    _ffi.call("rth_attn_decode_split", _p(o_ref), _p(qd), _p(kd), _p(vd), _p(ksd), _p(vsd),
              _p(part), splits, _p(pos), hq, hkv, d, ctypes.c_float(scale), _stream())
    sync()
    ref = bf16_host(o_ref)
    assert np.array_equal(first, ref)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s, capture_error_mode="global"):
            _ffi.call("rth_attn_decode_split_noalloc",
                      *args(o_na, ctypes.c_void_p(s.cuda_stream)))
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        o_na.zero_()
        sync()
        g.replay()
        sync()
        assert np.array_equal(bf16_host(o_na), ref), rep
        # eager work on the same array between replays
        _ffi.call("rth_attn_decode_split_noalloc", *args(o_ref, _stream()))
        sync()
