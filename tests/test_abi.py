"""CPU checks of the boundary: the library loads, exports every symbol that
include/*.h declares, rejects bad arguments before touching the GPU, and the
C++ interface headers compile."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

import runtherder_amd as R
from runtherder_amd import _ffi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "rth_attn.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(rth_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_ffi.LIB_PATH))
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_ffi.exported_symbols())


def _err(name, *args):
    with pytest.raises(_ffi.RthError) as e:
        _ffi.call(name, *args)
    return str(e.value)


FAKE = 0x1000  # never dereferenced: every case fails its argument check first


def test_prefill_rejects_head_dim():
    msg = _err("rth_attn_prefill", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, FAKE, 32, 8, 64,
               ctypes.c_float(0.1), None)
    assert "head_dim 128" in msg


def test_decode_rejects_gqa_ratio_and_null():
    assert "divisible" in _err("rth_attn_decode_split", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                               FAKE, 4, FAKE, 30, 8, 128, ctypes.c_float(0.1), None)
    assert "cache_len" in _err("rth_attn_decode_split", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                               FAKE, 4, None, 32, 8, 128, ctypes.c_float(0.1), None)
    assert "num_splits" in _err("rth_attn_decode_split", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                FAKE, 0, FAKE, 32, 8, 128, ctypes.c_float(0.1), None)
    assert "head_dim" in _err("rth_attn_decode_split", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                              FAKE, 4, FAKE, 32, 8, 96, ctypes.c_float(0.1), None)


def test_decode_rejects_split_count_overflow():
    assert "65536" in _err("rth_attn_decode_split", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                           1 << 20, FAKE, 32, 8, 128, ctypes.c_float(0.1), None)


def test_quantize_rejects_bad_rows():
    assert "divisible by 8" in _err("rth_kv_quantize_fp8", FAKE, FAKE, FAKE, FAKE, 1, 4, 12, None)
    assert "at_pos" in _err("rth_kv_quantize_fp8", FAKE, FAKE, FAKE, None, 1, 4, 128, None)
    assert "num_rows" in _err("rth_kv_quantize_fp8", FAKE, FAKE, FAKE, FAKE, 1, 0, 128, None)
    assert "n_new" in _err("rth_kv_append_fp8", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 8,
                           128, None)


def test_naive_rejects_large_head_dim():
    assert "512" in _err("rth_attn_naive", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1, FAKE, 8, 8,
                         1024, ctypes.c_float(0.1), None)


def test_scratch_size_formula():
    # reference formula Hq*S*2 + Hq*S*D (flash_decode.cuh:16-24)
    assert R.flash_split_scratch_floats(32, 128, 64) == 32 * 64 * 2 + 32 * 64 * 128
    assert R.flash_split_scratch_floats(24, 128, 32) == 24 * 32 * 130
    assert _ffi.load().rth_split_scratch_floats(0, 128, 4) == 0


def test_cpp_headers_compile():
    src = """
#include <runtherder/attention/factory.h>
#include <runtherder/attention/adaptive.h>
#include <runtherder/attention/naive.h>
#include <runtherder/engine/kv_cache.h>
#include <runtherder/engine/paged_kv_cache.h>
#include <runtherder/kernels/quantization.h>
#include <runtherder/kernels/flash_decode.h>
#include <runtherder/kernels/flash_prefill.h>
#include <runtherder/kernels/attention.h>
#include <runtherder/kernels/rope.h>
#include <runtherder/kernels/rmsnorm.h>
static_assert(sizeof(runtherder::attention::KVView) == 6 * sizeof(void*));
// The reference's aggregate form still builds a contiguous view.
static_assert(runtherder::attention::KVView{nullptr, nullptr, nullptr, nullptr}.block_table == nullptr);
// Scratch sizing is a constant expression, as in the reference
// (flash_decode.cuh:16-24).
static_assert(runtherder::kernels::flash_split_scratch_floats(32, 128, 64) == 32 * 64 * 130);
// The fused decode steps take writable slabs: a read-only KVView does not
// convert to them.
#include <type_traits>
static_assert(!std::is_convertible_v<runtherder::attention::KVView,
                                     runtherder::attention::KVSlabs>);
static_assert(std::is_invocable_v<
    decltype(&runtherder::attention::AdaptiveAttention::run_decode_append),
    runtherder::attention::AdaptiveAttention&, __hip_bfloat16*, const __hip_bfloat16*,
    const runtherder::attention::KVSlabs&, const __hip_bfloat16*, const __hip_bfloat16*,
    const int*, hipStream_t>);
static_assert(!std::is_invocable_v<
    decltype(&runtherder::attention::AdaptiveAttention::run_decode_append),
    runtherder::attention::AdaptiveAttention&, __hip_bfloat16*, const __hip_bfloat16*,
    const runtherder::attention::KVView&, const __hip_bfloat16*, const __hip_bfloat16*,
    const int*, hipStream_t>);
int main() { return 0; }
"""
    res = subprocess.run(["/opt/rocm/bin/hipcc", "-std=c++20", "-fsyntax-only", "-x", "hip",
                          f"-I{ROOT / 'include'}", "--offload-arch=gfx950", "-"],
                         input=src, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]


def test_rope_rejects_bad_shapes():
    assert "even" in _err("rth_rope_bf16", FAKE, FAKE, FAKE, FAKE, 4, 32, 8, 127, None)
    assert "256" in _err("rth_rope_bf16", FAKE, FAKE, FAKE, FAKE, 4, 32, 8, 258, None)
    assert "seq_len" in _err("rth_rope_bf16", FAKE, FAKE, FAKE, FAKE, 0, 32, 8, 128, None)
    assert "head_dim" in _err("rth_rope_append_fp8", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                              FAKE, FAKE, FAKE, 4, 32, 8, 96, None)
    assert "at_pos" in _err("rth_rope_append_fp8", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                            FAKE, FAKE, None, 4, 32, 8, 128, None)


def test_rmsnorm_rejects_and_lanes():
    assert "divisible by 8" in _err("rth_rmsnorm_bf16", FAKE, FAKE, FAKE, 4, 12,
                                    ctypes.c_float(1e-6), None)
    assert "eps" in _err("rth_rmsnorm_bf16", FAKE, FAKE, FAKE, 4, 128, ctypes.c_float(0.0), None)
    assert "q_norm" in _err("rth_qk_norm_rope_append_fp8", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                            FAKE, None, FAKE, ctypes.c_float(1e-6), FAKE, FAKE, FAKE, 4, 32, 8,
                            128, None)
    assert [R.rmsnorm_lanes(d) for d in (8, 64, 128, 256, 4096, 12)] == [1, 8, 16, 32, 64, 0]


def test_paged_rejects_block_sizes():
    for bs in (16, 48, 0):
        assert "power of two" in _err("rth_attn_prefill_paged", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                      FAKE, bs, 4, FAKE, 32, 8, 128, ctypes.c_float(0.1), None)
    assert "block_table" in _err("rth_attn_decode_split_paged", FAKE, FAKE, FAKE, FAKE, FAKE,
                                 FAKE, None, 64, FAKE, 4, FAKE, 32, 8, 128, ctypes.c_float(0.1),
                                 None)
    assert "power of two" in _err("rth_kv_append_fp8_paged", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                  FAKE, 4, 8, 128, FAKE, 100, None)


def test_fused_decode_steps_need_writable_slabs():
    import torch
    cache_k = torch.zeros((4, 1, 64), dtype=torch.uint8)
    sc = torch.zeros((4, 1), dtype=torch.float32)
    view = R.KVView(cache_k, cache_k, sc, sc)
    be = R.AdaptiveAttention.__new__(R.AdaptiveAttention)   # no device scratch needed
    be.config = R.AttnConfig.for_heads(4, 1, 64)
    for call in (lambda: be.run_decode_append(None, None, view, None, None, None),
                 lambda: be.run_decode_rope_append(None, None, view, None, None, None, None, None),
                 lambda: be.run_decode_qk_norm_rope_append(None, None, view, None, None, None,
                                                           None, 1e-6, None, None, None)):
        with pytest.raises(TypeError):
            call()
    slabs = R.KVSlabs(cache_k, cache_k, sc, sc)
    v2 = slabs.view()
    assert type(v2) is R.KVView and v2.k is cache_k and v2.block_table is None


def test_prefill_split_rejects_bad_arguments():
    def call(n_new=4, splits=8, hq=32, hkv=8, d=128, partial=FAKE, name="rth_attn_prefill_split"):
        return _err(name, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, partial, splits, n_new, FAKE, hq,
                    hkv, d, ctypes.c_float(0.1), None)
    assert "n_new" in call(n_new=0)
    assert "n_new" in call(n_new=4097)
    assert "<= 256" in call(n_new=300, d=256)
    assert "num_splits" in call(splits=0)
    assert "partial" in call(partial=None)
    assert "divisible" in call(hq=30)
    assert "MFMA" in call(d=32)
    assert "power of two" in _err("rth_attn_prefill_split_paged", FAKE, FAKE, FAKE, FAKE, FAKE,
                                  FAKE, FAKE, 48, FAKE, 8, 4, FAKE, 32, 8, 128,
                                  ctypes.c_float(0.1), None)
