"""numpy front end of the CPU oracle (oracle/librth_oracle.so). Test
infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it, always as the checker."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "oracle" / "librth_oracle.so"

_i, _i64, _u32, _u64, _f, _d = (ctypes.c_int, ctypes.c_int64, ctypes.c_uint32,
                                ctypes.c_uint64, ctypes.c_float, ctypes.c_double)
_vp = ctypes.c_void_p

_SIGS = {
    "rth_ref_f32_to_bf16": (ctypes.c_uint16, [_f]),
    "rth_ref_bf16_to_f32": (_f, [ctypes.c_uint16]),
    "rth_ref_e4m3_encode": (ctypes.c_uint8, [_f]),
    "rth_ref_e4m3_decode": (_f, [ctypes.c_uint8]),
    "rth_ref_e4m3_encode_array": (None, [_vp, _vp, _i64]),
    "rth_ref_e4m3_sweep_check": (_i64, [_u32, _i]),
    "rth_ref_fill_normal_bf16": (None, [_vp, _i64, _u64]),
    "rth_ref_fill_normal_f32": (None, [_vp, _i64, _u64]),
    "rth_ref_fill_uniform_f32": (None, [_vp, _i64, _f, _f, _u64]),
    "rth_ref_mt19937_raw": (None, [_u32, _i64, _vp]),
    "rth_ref_fill_mt19937_uniform_bf16": (None, [_vp, _i64, _f, _u32]),
    "rth_ref_quantize_kv_fp8": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "rth_ref_quantize_kv_fp8_scaled": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "rth_ref_attention_f32": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _i]),
    "rth_ref_attention_f64": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _d]),
    "rth_ref_decode_split_f32": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f]),
    "rth_ref_rope_inv_freq_plain": (None, [_vp, _i, _f]),
    "rth_ref_rope_inv_freq_llama3": (None, [_vp, _i, _f, _f, _f, _f, _i]),
    "rth_ref_rope_apply_bf16": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "rth_ref_rmsnorm_bf16": (None, [_vp, _vp, _vp, _i, _i, _f, _i]),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
        L = ctypes.CDLL(str(LIB))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---- scalar formats --------------------------------------------------------

def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().rth_ref_e4m3_encode_array(_ptr(x), _ptr(out), x.size)
    return out


_E4M3_TABLE = None


def e4m3_decode(b: np.ndarray) -> np.ndarray:
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        _E4M3_TABLE = np.array([lib().rth_ref_e4m3_decode(c) for c in range(256)], np.float32)
    return _E4M3_TABLE[np.asarray(b, dtype=np.uint8)]


# ---- inputs ----------------------------------------------------------------

def normal_bf16(shape, seed: int) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint16)
    lib().rth_ref_fill_normal_bf16(_ptr(out), out.size, seed)
    return out


def uniform_f32(shape, lo: float, hi: float, seed: int) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().rth_ref_fill_uniform_f32(_ptr(out), out.size, lo, hi, seed)
    return out


def mt19937_raw(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    lib().rth_ref_mt19937_raw(seed, n, _ptr(out))
    return out


def mt19937_uniform_bf16(shape, scale: float, seed: int) -> np.ndarray:
    """Inputs of the reference kernel tests (std::mt19937 + U(-scale, scale))."""
    out = np.empty(shape, dtype=np.uint16)
    lib().rth_ref_fill_mt19937_uniform_bf16(_ptr(out), out.size, scale, seed)
    return out


# ---- quantization ----------------------------------------------------------

def quantize_kv_fp8(x: np.ndarray, head_dim: int, at_pos: int = 0, rows_per_pos: int = 1,
                    dst_rows: int | None = None, q=None, scale=None):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    num_rows = x.size // head_dim
    dst_rows = dst_rows or (num_rows + at_pos * rows_per_pos)
    if q is None:
        q = np.zeros((dst_rows, head_dim), dtype=np.uint8)
    if scale is None:
        scale = np.zeros(dst_rows, dtype=np.float32)
    lib().rth_ref_quantize_kv_fp8(_ptr(q), _ptr(scale), _ptr(x), at_pos, rows_per_pos,
                                  num_rows, head_dim)
    return q, scale


def quantize_kv_fp8_scaled(x: np.ndarray, scale: np.ndarray, head_dim: int, at_pos: int = 0,
                           rows_per_pos: int = 1, q=None):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    num_rows = x.size // head_dim
    if q is None:
        q = np.zeros((scale.size, head_dim), dtype=np.uint8)
    lib().rth_ref_quantize_kv_fp8_scaled(_ptr(q), _ptr(scale), _ptr(x), at_pos, rows_per_pos,
                                         num_rows, head_dim)
    return q


# ---- attention -------------------------------------------------------------

def attention_f32(q, k8, v8, ks, vs, n_new, cache_len, hq, hkv, d, scale, nthreads=8):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k8 = np.ascontiguousarray(k8, dtype=np.uint8)
    v8 = np.ascontiguousarray(v8, dtype=np.uint8)
    ks = np.ascontiguousarray(ks, dtype=np.float32)
    vs = np.ascontiguousarray(vs, dtype=np.float32)
    out = np.empty((n_new, hq, d), dtype=np.uint16)
    lib().rth_ref_attention_f32(_ptr(out), _ptr(q), _ptr(k8), _ptr(v8), _ptr(ks), _ptr(vs),
                                n_new, cache_len, hq, hkv, d, scale, nthreads)
    return out


def attention_f64(q, k8, v8, ks, vs, n_new, cache_len, hq, hkv, d, scale):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k8 = np.ascontiguousarray(k8, dtype=np.uint8)
    v8 = np.ascontiguousarray(v8, dtype=np.uint8)
    ks = np.ascontiguousarray(ks, dtype=np.float32)
    vs = np.ascontiguousarray(vs, dtype=np.float32)
    out = np.empty((n_new, hq, d), dtype=np.float64)
    lib().rth_ref_attention_f64(_ptr(out), _ptr(q), _ptr(k8), _ptr(v8), _ptr(ks), _ptr(vs),
                                n_new, cache_len, hq, hkv, d, scale)
    return out


def decode_split_f32(q, k8, v8, ks, vs, num_splits, cache_len, hq, hkv, d, scale):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    out = np.empty((hq, d), dtype=np.uint16)
    lib().rth_ref_decode_split_f32(_ptr(out), _ptr(q), _ptr(np.ascontiguousarray(k8)),
                                   _ptr(np.ascontiguousarray(v8)),
                                   _ptr(np.ascontiguousarray(ks, dtype=np.float32)),
                                   _ptr(np.ascontiguousarray(vs, dtype=np.float32)),
                                   num_splits, cache_len, hq, hkv, d, scale)
    return out


# ---- RoPE ------------------------------------------------------------------

def rope_inv_freq_plain(head_dim, theta):
    out = np.empty(head_dim // 2, dtype=np.float32)
    lib().rth_ref_rope_inv_freq_plain(_ptr(out), head_dim, theta)
    return out


def rope_inv_freq_llama3(head_dim, theta, factor, low, high, orig):
    out = np.empty(head_dim // 2, dtype=np.float32)
    lib().rth_ref_rope_inv_freq_llama3(_ptr(out), head_dim, theta, factor, low, high, orig)
    return out


def rope_apply_bf16(x: np.ndarray, positions: np.ndarray, inv_freq: np.ndarray) -> np.ndarray:
    x = np.array(x, dtype=np.uint16, copy=True, order="C")
    n, h, d = x.shape
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
    lib().rth_ref_rope_apply_bf16(_ptr(x), _ptr(pos), _ptr(inv), n, h, d)
    return x


def rmsnorm_bf16(x: np.ndarray, g: np.ndarray, eps: float, lanes: int) -> np.ndarray:
    """Rows of x (last axis = dim) normalized with gain g, in the GPU's
    summation order over `lanes` lane partials."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    g = np.ascontiguousarray(g, dtype=np.uint16)
    dim = x.shape[-1]
    y = np.empty_like(x)
    lib().rth_ref_rmsnorm_bf16(_ptr(y), _ptr(x), _ptr(g), x.size // dim, dim, eps, lanes)
    return y


# ---- comparisons -----------------------------------------------------------

def bf16_err(a_bits: np.ndarray, b) -> tuple[float, float]:
    """(max-abs, mean-abs) between bf16 bits `a_bits` and bf16 bits or floats `b`."""
    a = bf16_to_f32(a_bits).astype(np.float64)
    bb = np.asarray(b)
    bf = bf16_to_f32(bb).astype(np.float64) if bb.dtype == np.uint16 else bb.astype(np.float64)
    d = np.abs(a - bf)
    return float(d.max()), float(d.mean())
