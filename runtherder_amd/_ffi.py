"""ctypes binding of libruntherder_attn.so (the C ABI in include/rth_attn.h).

The library is loaded from runtherder_amd/lib/. There is no fallback: if the
HIP library is missing, loading raises, so nothing silently computes elsewhere.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libruntherder_attn.so"

_c_int = ctypes.c_int
_vp = ctypes.c_void_p

# name -> (restype, argtypes)
_SIGNATURES = {
    "rth_last_error_string": (ctypes.c_char_p, []),
    "rth_kv_quantize_fp8": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "rth_kv_quantize_fp8_scaled": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "rth_kv_append_fp8": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp]),
    "rth_split_scratch_floats": (ctypes.c_size_t, [_c_int, _c_int, _c_int]),
    "rth_default_num_splits": (_c_int, [_c_int, _c_int]),
    "rth_attn_decode_split": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
                                       _c_int, _c_int, _c_int, ctypes.c_float, _vp]),
    "rth_decode_path": (_c_int, [_c_int, _c_int, _c_int]),
    "rth_set_decode_kernel": (_c_int, [_c_int]),
    "rth_attn_decode_split_noalloc": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
                                               _c_int, _c_int, _c_int, ctypes.c_float, _vp]),
    "rth_attn_decode_append_split": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                              _c_int, _vp, _c_int, _c_int, _c_int,
                                              ctypes.c_float, _vp]),
    "rth_attn_prefill": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
                                  _c_int, _c_int, _c_int, ctypes.c_float, _vp]),
    "rth_attn_naive": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
                                _c_int, _c_int, _c_int, ctypes.c_float, _vp]),
    "rth_advance_position": (_c_int, [_vp, _c_int, _vp]),
    "rth_rope_bf16": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "rth_rope_append_fp8": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _c_int, _c_int, _c_int, _c_int, _vp]),
    "rth_qk_norm_rope_append_fp8": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                             ctypes.c_float, _vp, _vp, _vp, _c_int, _c_int,
                                             _c_int, _c_int, _vp]),
    "rth_rmsnorm_bf16": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, ctypes.c_float, _vp]),
    "rth_rmsnorm_lanes": (_c_int, [_c_int]),
    "rth_kv_append_fp8_paged": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int,
                                         _c_int, _vp, _c_int, _vp]),
    "rth_attn_decode_split_paged": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
                                             _c_int, _vp, _c_int, _c_int, _c_int,
                                             ctypes.c_float, _vp]),
    "rth_attn_decode_append_split_paged": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int,
                                                    _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int,
                                                    _c_int, ctypes.c_float, _vp]),
    "rth_attn_decode_rope_append_split": (_c_int, [_vp] * 11 + [_c_int, _vp, _c_int, _c_int,
                                                                _c_int, ctypes.c_float, _vp]),
    "rth_attn_decode_rope_append_split_paged": (_c_int, [_vp] * 7 + [_c_int] + [_vp] * 5 +
                                                [_c_int, _vp, _c_int, _c_int, _c_int,
                                                 ctypes.c_float, _vp]),
    "rth_attn_decode_qk_norm_rope_append_split": (_c_int, [_vp] * 10 + [ctypes.c_float] +
                                                  [_vp] * 3 + [_c_int, _vp, _c_int, _c_int,
                                                               _c_int, ctypes.c_float, _vp]),
    "rth_attn_decode_qk_norm_rope_append_split_paged": (_c_int, [_vp] * 7 + [_c_int] +
                                                        [_vp] * 4 + [ctypes.c_float] +
                                                        [_vp] * 3 +
                                                        [_c_int, _vp, _c_int, _c_int, _c_int,
                                                         ctypes.c_float, _vp]),
    "rth_attn_prefill_paged": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _vp,
                                        _c_int, _c_int, _c_int, ctypes.c_float, _vp]),
    "rth_attn_prefill_split": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _vp,
                                        _c_int, _c_int, _c_int, ctypes.c_float, _vp]),
    "rth_attn_prefill_split_paged": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
                                              _c_int, _c_int, _vp, _c_int, _c_int, _c_int,
                                              ctypes.c_float, _vp]),
}

_lib: ctypes.CDLL | None = None


class RthError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m runtherder_amd.build`")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.rth_last_error_string().decode()
        raise RthError(f"{name} failed ({rc}): {msg}")
