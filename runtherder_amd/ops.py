"""Torch-tensor front end of the C ABI, mirroring the reference's kernel free
functions and its AttentionBackend / KVCache interface (reference
include/runtherder/kernels/*.cuh, include/runtherder/attention/*.h,
include/runtherder/engine/kv_cache.h). Same names, argument order and
meaning; errors raise RthError instead of exiting the process.

torch only provides device memory and the current stream here: every
computation runs in libruntherder_attn.so.

dtypes: bf16 tensors are torch.bfloat16, E4M3 cache bytes torch.uint8, scales
torch.float32, device-resident positions torch.int32 (one element).
"""
from __future__ import annotations

import enum
import math
from dataclasses import dataclass

import torch

from . import _ffi


def _p(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _need(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise TypeError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise TypeError(f"{name} must be contiguous")


# ---- kernels ---------------------------------------------------------------

def quantize_kv_fp8(q, scale, x, at_pos, rows_per_pos, num_rows, head_dim, stream=None):
    """reference include/runtherder/kernels/quantization.cuh:50-57"""
    _need(q, torch.uint8, "q"); _need(scale, torch.float32, "scale")
    _need(x, torch.bfloat16, "x"); _need(at_pos, torch.int32, "at_pos")
    _ffi.call("rth_kv_quantize_fp8", _p(q), _p(scale), _p(x), _p(at_pos),
              rows_per_pos, num_rows, head_dim, _stream(stream))


def quantize_kv_fp8_scaled(q, scale, x, at_pos, rows_per_pos, num_rows, head_dim, stream=None):
    """Given-scale variant: scale[dst] is an input (no reference counterpart)."""
    _need(q, torch.uint8, "q"); _need(scale, torch.float32, "scale")
    _need(x, torch.bfloat16, "x"); _need(at_pos, torch.int32, "at_pos")
    _ffi.call("rth_kv_quantize_fp8_scaled", _p(q), _p(scale), _p(x), _p(at_pos),
              rows_per_pos, num_rows, head_dim, _stream(stream))


def flash_split_scratch_floats(num_q_heads: int, head_dim: int, max_splits: int) -> int:
    """reference include/runtherder/kernels/flash_decode.cuh:16-24"""
    return int(_ffi.load().rth_split_scratch_floats(num_q_heads, head_dim, max_splits))


def new_flash_split_scratch(num_q_heads, head_dim, max_splits, device="cuda"):
    """Allocates decode scratch (no initialization needed)."""
    n = flash_split_scratch_floats(num_q_heads, head_dim, max_splits)
    return torch.empty(n, dtype=torch.float32, device=device)


def default_num_splits(num_kv_heads: int, device: int = 0) -> int:
    return int(_ffi.load().rth_default_num_splits(num_kv_heads, device))


def flash_decode_split_bf16(out, q, k, v, k_scale, v_scale, partial, num_splits, cache_len,
                            num_q_heads, num_kv_heads, head_dim, scale, stream=None):
    """reference include/runtherder/kernels/flash_decode.cuh:45-59"""
    _need(out, torch.bfloat16, "out"); _need(q, torch.bfloat16, "q")
    _need(k, torch.uint8, "k"); _need(v, torch.uint8, "v")
    _need(k_scale, torch.float32, "k_scale"); _need(v_scale, torch.float32, "v_scale")
    _need(partial, torch.float32, "partial"); _need(cache_len, torch.int32, "cache_len")
    _ffi.call("rth_attn_decode_split", _p(out), _p(q), _p(k), _p(v), _p(k_scale),
              _p(v_scale), _p(partial), num_splits, _p(cache_len), num_q_heads,
              num_kv_heads, head_dim, float(scale), _stream(stream))


DECODE_MFMA, DECODE_VALU = 1, 2


def decode_path(num_q_heads: int, num_kv_heads: int, head_dim: int) -> int:
    """Which split kernel decode runs for the shape: DECODE_MFMA, DECODE_VALU
    or 0 (unsupported). No reference counterpart."""
    return int(_ffi.load().rth_decode_path(num_q_heads, num_kv_heads, head_dim))


def set_decode_kernel(path: int) -> None:
    """Process-wide split-kernel choice for the non-paged decode entries: 0
    (automatic: MFMA where supported) or DECODE_VALU (the VALU kernel for
    every shape), for measurement. No reference counterpart."""
    _ffi.call("rth_set_decode_kernel", int(path))


def flash_decode_split_bf16_noalloc(out, q, k, v, k_scale, v_scale, num_splits, cache_len,
                                    num_q_heads, num_kv_heads, head_dim, scale, stream=None):
    """flash_decode_split_bf16 without caller scratch (no reference
    counterpart): the partials live in the library's fixed per-device array,
    shared by every call on the device (overlapping calls race)."""
    _need(out, torch.bfloat16, "out"); _need(q, torch.bfloat16, "q")
    _need(k, torch.uint8, "k"); _need(v, torch.uint8, "v")
    _need(k_scale, torch.float32, "k_scale"); _need(v_scale, torch.float32, "v_scale")
    _need(cache_len, torch.int32, "cache_len")
    _ffi.call("rth_attn_decode_split_noalloc", _p(out), _p(q), _p(k), _p(v), _p(k_scale),
              _p(v_scale), num_splits, _p(cache_len), num_q_heads, num_kv_heads, head_dim,
              float(scale), _stream(stream))


def flash_decode_append_split_bf16(out, q, k_cache, v_cache, k_scale, v_scale, k_new, v_new,
                                   partial, num_splits, cache_len, num_q_heads, num_kv_heads,
                                   head_dim, scale, stream=None):
    """Append one token at row *cache_len and decode over *cache_len + 1 keys
    in one call (no reference counterpart: KVCache::append then the decode)."""
    _need(out, torch.bfloat16, "out"); _need(q, torch.bfloat16, "q")
    _need(k_cache, torch.uint8, "k_cache"); _need(v_cache, torch.uint8, "v_cache")
    _need(k_scale, torch.float32, "k_scale"); _need(v_scale, torch.float32, "v_scale")
    _need(k_new, torch.bfloat16, "k_new"); _need(v_new, torch.bfloat16, "v_new")
    _need(partial, torch.float32, "partial"); _need(cache_len, torch.int32, "cache_len")
    _ffi.call("rth_attn_decode_append_split", _p(out), _p(q), _p(k_cache), _p(v_cache),
              _p(k_scale), _p(v_scale), _p(k_new), _p(v_new), _p(partial), num_splits,
              _p(cache_len), num_q_heads, num_kv_heads, head_dim, float(scale), _stream(stream))


def flash_decode_rope_append_split_bf16(out, q, k_cache, v_cache, k_scale, v_scale, k_new,
                                        v_new, positions, inv_freq, partial, num_splits,
                                        cache_len, num_q_heads, num_kv_heads, head_dim, scale,
                                        stream=None):
    """The per-layer decode step rope_bf16(q, k) -> KVCache::append -> run in
    one call (no reference counterpart; replaces reference
    src/model/supported/llama/llama3.cu:228-234). q and k_new are read only
    (rotated in registers by positions[0]); cache bytes and output equal
    rope_bf16 + flash_decode_append_split_bf16 on the rotated q and k."""
    _need(out, torch.bfloat16, "out"); _need(q, torch.bfloat16, "q")
    _need(k_cache, torch.uint8, "k_cache"); _need(v_cache, torch.uint8, "v_cache")
    _need(k_scale, torch.float32, "k_scale"); _need(v_scale, torch.float32, "v_scale")
    _need(k_new, torch.bfloat16, "k_new"); _need(v_new, torch.bfloat16, "v_new")
    _need(positions, torch.int32, "positions"); _need(inv_freq, torch.float32, "inv_freq")
    _need(partial, torch.float32, "partial"); _need(cache_len, torch.int32, "cache_len")
    _ffi.call("rth_attn_decode_rope_append_split", _p(out), _p(q), _p(k_cache), _p(v_cache),
              _p(k_scale), _p(v_scale), _p(k_new), _p(v_new), _p(positions), _p(inv_freq),
              _p(partial), num_splits, _p(cache_len), num_q_heads, num_kv_heads, head_dim,
              float(scale), _stream(stream))


def flash_decode_qk_norm_rope_append_split_bf16(out, q, k_cache, v_cache, k_scale, v_scale,
                                                k_new, v_new, q_norm, k_norm, eps, positions,
                                                inv_freq, partial, num_splits, cache_len,
                                                num_q_heads, num_kv_heads, head_dim, scale,
                                                stream=None):
    """The Qwen3 decode step (per-head RMSNorm of q and k, RoPE, append, run)
    in one call (no reference counterpart; replaces reference
    src/model/supported/llama/qwen3.cu:189-202). q and k_new are read only."""
    _need(out, torch.bfloat16, "out"); _need(q, torch.bfloat16, "q")
    _need(k_cache, torch.uint8, "k_cache"); _need(v_cache, torch.uint8, "v_cache")
    _need(k_scale, torch.float32, "k_scale"); _need(v_scale, torch.float32, "v_scale")
    _need(k_new, torch.bfloat16, "k_new"); _need(v_new, torch.bfloat16, "v_new")
    _need(q_norm, torch.bfloat16, "q_norm"); _need(k_norm, torch.bfloat16, "k_norm")
    _need(positions, torch.int32, "positions"); _need(inv_freq, torch.float32, "inv_freq")
    _need(partial, torch.float32, "partial"); _need(cache_len, torch.int32, "cache_len")
    _ffi.call("rth_attn_decode_qk_norm_rope_append_split", _p(out), _p(q), _p(k_cache),
              _p(v_cache), _p(k_scale), _p(v_scale), _p(k_new), _p(v_new), _p(q_norm),
              _p(k_norm), float(eps), _p(positions), _p(inv_freq), _p(partial), num_splits,
              _p(cache_len), num_q_heads, num_kv_heads, head_dim, float(scale),
              _stream(stream))


def flash_prefill_bf16(out, q, k, v, k_scale, v_scale, n_new, cache_len, num_q_heads,
                       num_kv_heads, head_dim, scale, stream=None):
    """reference include/runtherder/kernels/flash_prefill.cuh:26-39"""
    _need(out, torch.bfloat16, "out"); _need(q, torch.bfloat16, "q")
    _need(k, torch.uint8, "k"); _need(v, torch.uint8, "v")
    _need(k_scale, torch.float32, "k_scale"); _need(v_scale, torch.float32, "v_scale")
    _need(cache_len, torch.int32, "cache_len")
    _ffi.call("rth_attn_prefill", _p(out), _p(q), _p(k), _p(v), _p(k_scale), _p(v_scale),
              n_new, _p(cache_len), num_q_heads, num_kv_heads, head_dim, float(scale),
              _stream(stream))


PREFILL_SPLIT_MAX_TOKENS = 4096


def flash_prefill_split_bf16(out, q, k, v, k_scale, v_scale, partial, num_splits, n_new,
                             cache_len, num_q_heads, num_kv_heads, head_dim, scale,
                             stream=None):
    """flash_prefill_bf16 split over the keys, for calls after a long cache
    (no reference counterpart; the reference walks every key serially per q
    tile, flash_prefill.cu:34-241): up to 80 tokens as split-K decode over
    (token block, kv head) units, beyond (head_dim 128) the flash prefill over
    num_splits key runs per (row block, q head), both merged by the decode
    merge. partial: flash_split_scratch_floats(n_new * num_q_heads, head_dim,
    num_splits) floats; 1 <= n_new <= PREFILL_SPLIT_MAX_TOKENS."""
    _need(out, torch.bfloat16, "out"); _need(q, torch.bfloat16, "q")
    _need(k, torch.uint8, "k"); _need(v, torch.uint8, "v")
    _need(k_scale, torch.float32, "k_scale"); _need(v_scale, torch.float32, "v_scale")
    _need(partial, torch.float32, "partial"); _need(cache_len, torch.int32, "cache_len")
    _ffi.call("rth_attn_prefill_split", _p(out), _p(q), _p(k), _p(v), _p(k_scale),
              _p(v_scale), _p(partial), num_splits, n_new, _p(cache_len), num_q_heads,
              num_kv_heads, head_dim, float(scale), _stream(stream))


def attention_causal_bf16(out, q, k, v, k_scale, v_scale, n_new, cache_len, num_q_heads,
                          num_kv_heads, head_dim, scale, stream=None):
    """reference include/runtherder/kernels/attention.cuh:21-34"""
    _need(out, torch.bfloat16, "out"); _need(q, torch.bfloat16, "q")
    _need(k, torch.uint8, "k"); _need(v, torch.uint8, "v")
    _need(k_scale, torch.float32, "k_scale"); _need(v_scale, torch.float32, "v_scale")
    _need(cache_len, torch.int32, "cache_len")
    _ffi.call("rth_attn_naive", _p(out), _p(q), _p(k), _p(v), _p(k_scale), _p(v_scale),
              n_new, _p(cache_len), num_q_heads, num_kv_heads, head_dim, float(scale),
              _stream(stream))


def advance_position(pos, delta=1, stream=None):
    """*pos += delta on device (lets one graph hold several decode steps)."""
    _need(pos, torch.int32, "pos")
    _ffi.call("rth_advance_position", _p(pos), int(delta), _stream(stream))


def rope_bf16(q, k, positions, inv_freq, seq_len, num_q_heads, num_kv_heads, head_dim,
              stream=None):
    """In-place rotate-half RoPE on q and k (reference
    include/runtherder/kernels/rope.cuh:16-25)."""
    _need(q, torch.bfloat16, "q"); _need(k, torch.bfloat16, "k")
    _need(positions, torch.int32, "positions"); _need(inv_freq, torch.float32, "inv_freq")
    _ffi.call("rth_rope_bf16", _p(q), _p(k), _p(positions), _p(inv_freq), seq_len,
              num_q_heads, num_kv_heads, head_dim, _stream(stream))


def rope_append_fp8(q, k_cache, v_cache, k_scale, v_scale, k, v, positions, inv_freq, at_pos,
                    n_new, num_q_heads, num_kv_heads, head_dim, stream=None):
    """rope_bf16(q, k) + KV append in one launch; q rotated in place, k left
    unrotated, cache bytes identical to the two-step sequence (no reference
    counterpart; replaces reference src/model/supported/llama/llama3.cu:228-232)."""
    _need(q, torch.bfloat16, "q"); _need(k, torch.bfloat16, "k"); _need(v, torch.bfloat16, "v")
    _need(k_cache, torch.uint8, "k_cache"); _need(v_cache, torch.uint8, "v_cache")
    _need(k_scale, torch.float32, "k_scale"); _need(v_scale, torch.float32, "v_scale")
    _need(positions, torch.int32, "positions"); _need(inv_freq, torch.float32, "inv_freq")
    _need(at_pos, torch.int32, "at_pos")
    _ffi.call("rth_rope_append_fp8", _p(q), _p(k_cache), _p(v_cache), _p(k_scale), _p(v_scale),
              _p(k), _p(v), _p(positions), _p(inv_freq), _p(at_pos), n_new, num_q_heads,
              num_kv_heads, head_dim, _stream(stream))


def qk_norm_rope_append_fp8(q, k_cache, v_cache, k_scale, v_scale, k, v, q_norm, k_norm, eps,
                            positions, inv_freq, at_pos, n_new, num_q_heads, num_kv_heads,
                            head_dim, stream=None):
    """Per-head RMSNorm of q and k, RoPE, then the KV append, in one launch (no
    reference counterpart; replaces reference
    src/model/supported/llama/qwen3.cu:189-200). q updated in place; k read only."""
    _need(q, torch.bfloat16, "q"); _need(k, torch.bfloat16, "k"); _need(v, torch.bfloat16, "v")
    _need(k_cache, torch.uint8, "k_cache"); _need(v_cache, torch.uint8, "v_cache")
    _need(k_scale, torch.float32, "k_scale"); _need(v_scale, torch.float32, "v_scale")
    _need(q_norm, torch.bfloat16, "q_norm"); _need(k_norm, torch.bfloat16, "k_norm")
    _need(positions, torch.int32, "positions"); _need(inv_freq, torch.float32, "inv_freq")
    _need(at_pos, torch.int32, "at_pos")
    _ffi.call("rth_qk_norm_rope_append_fp8", _p(q), _p(k_cache), _p(v_cache), _p(k_scale),
              _p(v_scale), _p(k), _p(v), _p(q_norm), _p(k_norm), float(eps), _p(positions),
              _p(inv_freq), _p(at_pos), n_new, num_q_heads, num_kv_heads, head_dim,
              _stream(stream))


def rmsnorm_bf16(y, x, g, num_tokens, hidden_dim, eps, stream=None):
    """y = bf16((x * rrms) * g) per row (reference
    include/runtherder/kernels/rmsnorm.cuh:14-22); y may alias x."""
    _need(y, torch.bfloat16, "y"); _need(x, torch.bfloat16, "x"); _need(g, torch.bfloat16, "g")
    _ffi.call("rth_rmsnorm_bf16", _p(y), _p(x), _p(g), num_tokens, hidden_dim, float(eps),
              _stream(stream))


def rmsnorm_lanes(hidden_dim: int) -> int:
    """Lane partials of rmsnorm_bf16's sum of squares (its summation order)."""
    return int(_ffi.load().rth_rmsnorm_lanes(hidden_dim))


# ---- interface -------------------------------------------------------------

@dataclass(frozen=True)
class AttnConfig:
    """reference include/runtherder/attention/backend.h:14-19"""
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    scale: float

    @staticmethod
    def for_heads(num_q_heads, num_kv_heads, head_dim):
        return AttnConfig(num_q_heads, num_kv_heads, head_dim, 1.0 / math.sqrt(head_dim))


@dataclass(frozen=True)
class KVView:
    """reference include/runtherder/attention/kv_view.h:14-19; block_table /
    block_size (no reference counterpart) describe a paged layout."""
    k: torch.Tensor
    v: torch.Tensor
    k_scale: torch.Tensor
    v_scale: torch.Tensor
    block_table: torch.Tensor | None = None
    block_size: int = 0


@dataclass(frozen=True)
class KVSlabs(KVView):
    """The writable slabs of one layer (KVCache.slabs / PagedKVCache.slabs),
    for the fused decode steps that store the new token into the cache. No
    reference counterpart: the reference appends through KVCache::append and
    reads through KVView only."""

    def view(self) -> KVView:
        return KVView(self.k, self.v, self.k_scale, self.v_scale, self.block_table,
                      self.block_size)


def _need_slabs(kv):
    if not isinstance(kv, KVSlabs):
        raise TypeError("the fused decode steps write the cache: pass KVCache.slabs(layer) "
                        "(or PagedKVCache.slabs(layer, block_table)), not a read-only view")


class KVCache:
    """reference include/runtherder/engine/kv_cache.h:23-104"""

    def __init__(self, num_layers, max_seq_len, num_kv_heads, head_dim, device="cuda"):
        for name, val in (("num_layers", num_layers), ("max_seq_len", max_seq_len),
                          ("num_kv_heads", num_kv_heads), ("head_dim", head_dim)):
            if val < 1:
                raise ValueError(f"KVCache {name} must be >= 1")
        self.num_layers, self._max_seq_len = num_layers, max_seq_len
        self.num_kv_heads, self.head_dim = num_kv_heads, head_dim
        shape = (num_layers, max_seq_len, num_kv_heads, head_dim)
        self.k = torch.empty(shape, dtype=torch.uint8, device=device)
        self.v = torch.empty(shape, dtype=torch.uint8, device=device)
        self.k_scale = torch.empty(shape[:3], dtype=torch.float32, device=device)
        self.v_scale = torch.empty(shape[:3], dtype=torch.float32, device=device)

    def append(self, layer, k, v, n_new, at_pos, stream=None):
        if not 0 <= layer < self.num_layers:
            raise ValueError("KVCache append layer out of range")
        if n_new < 1:
            raise ValueError("KVCache append n_new must be >= 1")
        _need(k, torch.bfloat16, "k"); _need(v, torch.bfloat16, "v")
        _need(at_pos, torch.int32, "at_pos")
        _ffi.call("rth_kv_append_fp8", _p(self.k[layer]), _p(self.v[layer]),
                  _p(self.k_scale[layer]), _p(self.v_scale[layer]), _p(k), _p(v),
                  _p(at_pos), n_new, self.num_kv_heads, self.head_dim, _stream(stream))

    def append_rope(self, layer, q, k, v, n_new, positions, inv_freq, at_pos, num_q_heads,
                    stream=None):
        """RoPE on q (in place) and k, then append k, v, in one launch."""
        if not 0 <= layer < self.num_layers:
            raise ValueError("KVCache append layer out of range")
        if n_new < 1:
            raise ValueError("KVCache append n_new must be >= 1")
        rope_append_fp8(q, self.k[layer], self.v[layer], self.k_scale[layer],
                        self.v_scale[layer], k, v, positions, inv_freq, at_pos, n_new,
                        num_q_heads, self.num_kv_heads, self.head_dim, stream)

    def append_qk_norm_rope(self, layer, q, k, v, n_new, q_norm, k_norm, eps, positions,
                            inv_freq, at_pos, num_q_heads, stream=None):
        """Qwen3 order: RMSNorm of q and k per head, RoPE, then the append."""
        if not 0 <= layer < self.num_layers:
            raise ValueError("KVCache append layer out of range")
        if n_new < 1:
            raise ValueError("KVCache append n_new must be >= 1")
        qk_norm_rope_append_fp8(q, self.k[layer], self.v[layer], self.k_scale[layer],
                                self.v_scale[layer], k, v, q_norm, k_norm, eps, positions,
                                inv_freq, at_pos, n_new, num_q_heads, self.num_kv_heads,
                                self.head_dim, stream)

    def view(self, layer) -> KVView:
        if not 0 <= layer < self.num_layers:
            raise ValueError("KVCache view layer out of range")
        return KVView(self.k[layer], self.v[layer], self.k_scale[layer], self.v_scale[layer])

    def slabs(self, layer) -> KVSlabs:
        if not 0 <= layer < self.num_layers:
            raise ValueError("KVCache slabs layer out of range")
        return KVSlabs(self.k[layer], self.v[layer], self.k_scale[layer], self.v_scale[layer])

    def max_seq_len(self) -> int:
        return self._max_seq_len


class PagedKVCache:
    """Paged FP8 KV cache: per layer num_blocks physical blocks of block_size
    positions; the caller's block_table (int32 device tensor, logical block ->
    physical block) goes to append() and view(). No reference counterpart."""

    def __init__(self, num_layers, num_blocks, block_size, num_kv_heads, head_dim,
                 device="cuda"):
        if block_size < 32 or block_size & (block_size - 1):
            raise ValueError("PagedKVCache block_size must be a power of two >= 32")
        self.num_layers, self.num_blocks, self.block_size = num_layers, num_blocks, block_size
        self.num_kv_heads, self.head_dim = num_kv_heads, head_dim
        shape = (num_layers, num_blocks * block_size, num_kv_heads, head_dim)
        self.k = torch.empty(shape, dtype=torch.uint8, device=device)
        self.v = torch.empty(shape, dtype=torch.uint8, device=device)
        self.k_scale = torch.empty(shape[:3], dtype=torch.float32, device=device)
        self.v_scale = torch.empty(shape[:3], dtype=torch.float32, device=device)

    def append(self, layer, k, v, n_new, at_pos, block_table, stream=None):
        if not 0 <= layer < self.num_layers:
            raise ValueError("KVCache append layer out of range")
        if n_new < 1:
            raise ValueError("KVCache append n_new must be >= 1")
        _need(k, torch.bfloat16, "k"); _need(v, torch.bfloat16, "v")
        _need(at_pos, torch.int32, "at_pos"); _need(block_table, torch.int32, "block_table")
        _ffi.call("rth_kv_append_fp8_paged", _p(self.k[layer]), _p(self.v[layer]),
                  _p(self.k_scale[layer]), _p(self.v_scale[layer]), _p(k), _p(v), _p(at_pos),
                  n_new, self.num_kv_heads, self.head_dim, _p(block_table), self.block_size,
                  _stream(stream))

    def view(self, layer, block_table) -> KVView:
        if not 0 <= layer < self.num_layers:
            raise ValueError("KVCache view layer out of range")
        _need(block_table, torch.int32, "block_table")
        return KVView(self.k[layer], self.v[layer], self.k_scale[layer], self.v_scale[layer],
                      block_table, self.block_size)

    def slabs(self, layer, block_table) -> KVSlabs:
        if not 0 <= layer < self.num_layers:
            raise ValueError("KVCache slabs layer out of range")
        _need(block_table, torch.int32, "block_table")
        return KVSlabs(self.k[layer], self.v[layer], self.k_scale[layer], self.v_scale[layer],
                       block_table, self.block_size)


class AttentionBackend:
    """reference include/runtherder/attention/backend.h:24-53"""

    def run(self, out, q, kv: KVView, n_new, cache_len, stream=None):
        raise NotImplementedError


PREFILL_SPLIT_TOKENS = 80
PREFILL_RUNS_TOKENS = 256
PREFILL_RUN_TOKEN_RUNS = 2048


class AdaptiveAttention(AttentionBackend):
    """reference src/attention/adaptive.cu: n_new == 1 -> split decode with
    backend-owned scratch, else flash prefill. Split count defaults to the
    device's (kv head, split) fill count. Calls of 2..PREFILL_SPLIT_TOKENS
    tokens on shapes the MFMA decode kernel serves take the split-K prefill
    (flash_prefill_split_bf16) over the same scratch, with num_splits //
    (2 n_new) splits (no reference counterpart: per call, 16 / 64 tokens
    after 8K keys 209 / 199 -> 18 / 34 us; at an empty cache up to ~2 us
    slower); at head_dim 128, calls of up to PREFILL_RUNS_TOKENS tokens take
    it as the flash prefill over key runs (128 / 256 tokens after 32K keys
    828 / 830 -> 98 / 187 us; at an empty cache 11 / 14 -> 19 / 27 us), for
    which the scratch holds PREFILL_RUN_TOKEN_RUNS token-runs."""

    def __init__(self, config: AttnConfig, num_splits: int | None = None, device="cuda"):
        self.config = config
        self.num_splits = num_splits or default_num_splits(
            config.num_kv_heads, torch.device(device).index or 0)
        dev = torch.device(device)
        self.cus = torch.cuda.get_device_properties(dev).multi_processor_count
        runs = PREFILL_RUN_TOKEN_RUNS if config.head_dim == 128 else 1
        self.partial = new_flash_split_scratch(config.num_q_heads, config.head_dim,
                                               max(self.num_splits, runs), device=device)

    def _split_prefill_splits(self, n_new):
        c = self.config
        if 2 <= n_new <= PREFILL_SPLIT_TOKENS:
            if decode_path(c.num_q_heads, c.num_kv_heads, c.head_dim) != DECODE_MFMA:
                return 0
            return max(1, self.num_splits // (2 * n_new))
        if PREFILL_SPLIT_TOKENS < n_new <= PREFILL_RUNS_TOKENS and c.head_dim == 128:
            blocks = (n_new + 127) // 128 * c.num_q_heads
            runs = min(2 * self.cus // blocks, 16, PREFILL_RUN_TOKEN_RUNS // n_new)
            return runs if runs > 1 else 0
        return 0

    def run(self, out, q, kv, n_new, cache_len, stream=None):
        c = self.config
        ps = self._split_prefill_splits(n_new)
        if kv.block_table is not None:
            if ps:
                _ffi.call("rth_attn_prefill_split_paged", _p(out), _p(q), _p(kv.k), _p(kv.v),
                          _p(kv.k_scale), _p(kv.v_scale), _p(kv.block_table), kv.block_size,
                          _p(self.partial), ps, n_new, _p(cache_len), c.num_q_heads,
                          c.num_kv_heads, c.head_dim, float(c.scale), _stream(stream))
            elif n_new == 1:
                _ffi.call("rth_attn_decode_split_paged", _p(out), _p(q), _p(kv.k), _p(kv.v),
                          _p(kv.k_scale), _p(kv.v_scale), _p(kv.block_table), kv.block_size,
                          _p(self.partial), self.num_splits, _p(cache_len), c.num_q_heads,
                          c.num_kv_heads, c.head_dim, float(c.scale), _stream(stream))
            else:
                _ffi.call("rth_attn_prefill_paged", _p(out), _p(q), _p(kv.k), _p(kv.v),
                          _p(kv.k_scale), _p(kv.v_scale), _p(kv.block_table), kv.block_size,
                          n_new, _p(cache_len), c.num_q_heads, c.num_kv_heads, c.head_dim,
                          float(c.scale), _stream(stream))
            return
        if ps:
            flash_prefill_split_bf16(out, q, kv.k, kv.v, kv.k_scale, kv.v_scale, self.partial,
                                     ps, n_new, cache_len, c.num_q_heads, c.num_kv_heads,
                                     c.head_dim, c.scale, stream)
        elif n_new == 1:
            flash_decode_split_bf16(out, q, kv.k, kv.v, kv.k_scale, kv.v_scale, self.partial,
                                    self.num_splits, cache_len, c.num_q_heads, c.num_kv_heads,
                                    c.head_dim, c.scale, stream)
        else:
            flash_prefill_bf16(out, q, kv.k, kv.v, kv.k_scale, kv.v_scale, n_new, cache_len,
                               c.num_q_heads, c.num_kv_heads, c.head_dim, c.scale, stream)

    def run_decode_append(self, out, q, kv, k_new, v_new, cache_len, stream=None):
        """KVCache.append(layer, k_new, v_new, 1, cache_len) + run(..., n_new=1)
        in one call; kv is the layer's KVSlabs (they receive the new token)."""
        _need_slabs(kv)
        c = self.config
        if kv.block_table is not None:
            _ffi.call("rth_attn_decode_append_split_paged", _p(out), _p(q), _p(kv.k), _p(kv.v),
                      _p(kv.k_scale), _p(kv.v_scale), _p(kv.block_table), kv.block_size,
                      _p(k_new), _p(v_new), _p(self.partial), self.num_splits, _p(cache_len),
                      c.num_q_heads, c.num_kv_heads, c.head_dim, float(c.scale),
                      _stream(stream))
            return
        flash_decode_append_split_bf16(out, q, kv.k, kv.v, kv.k_scale, kv.v_scale, k_new, v_new,
                                       self.partial, self.num_splits, cache_len, c.num_q_heads,
                                       c.num_kv_heads, c.head_dim, c.scale, stream)


    def run_decode_rope_append(self, out, q, kv, k_new, v_new, positions, inv_freq, cache_len,
                               stream=None):
        """rope_bf16(q, k_new, positions, inv_freq) + KVCache.append(layer, k_new,
        v_new, 1, cache_len) + run(..., n_new=1) in one call; q and k_new are
        read only (the rotation happens in registers)."""
        _need_slabs(kv)
        c = self.config
        if kv.block_table is not None:
            _ffi.call("rth_attn_decode_rope_append_split_paged", _p(out), _p(q), _p(kv.k),
                      _p(kv.v), _p(kv.k_scale), _p(kv.v_scale), _p(kv.block_table),
                      kv.block_size, _p(k_new), _p(v_new), _p(positions), _p(inv_freq),
                      _p(self.partial), self.num_splits, _p(cache_len), c.num_q_heads,
                      c.num_kv_heads, c.head_dim, float(c.scale), _stream(stream))
            return
        flash_decode_rope_append_split_bf16(out, q, kv.k, kv.v, kv.k_scale, kv.v_scale, k_new,
                                            v_new, positions, inv_freq, self.partial,
                                            self.num_splits, cache_len, c.num_q_heads,
                                            c.num_kv_heads, c.head_dim, c.scale, stream)


    def run_decode_qk_norm_rope_append(self, out, q, kv, k_new, v_new, q_norm, k_norm, eps,
                                       positions, inv_freq, cache_len, stream=None):
        """Qwen3 order: per-head RMSNorm(q, q_norm) and (k_new, k_norm), RoPE,
        KVCache.append and run(..., n_new=1) in one call; q and k_new read only."""
        _need_slabs(kv)
        c = self.config
        if kv.block_table is not None:
            _ffi.call("rth_attn_decode_qk_norm_rope_append_split_paged", _p(out), _p(q),
                      _p(kv.k), _p(kv.v), _p(kv.k_scale), _p(kv.v_scale), _p(kv.block_table),
                      kv.block_size, _p(k_new), _p(v_new), _p(q_norm), _p(k_norm), float(eps),
                      _p(positions), _p(inv_freq), _p(self.partial), self.num_splits,
                      _p(cache_len), c.num_q_heads, c.num_kv_heads, c.head_dim, float(c.scale),
                      _stream(stream))
            return
        flash_decode_qk_norm_rope_append_split_bf16(
            out, q, kv.k, kv.v, kv.k_scale, kv.v_scale, k_new, v_new, q_norm, k_norm, eps,
            positions, inv_freq, self.partial, self.num_splits, cache_len, c.num_q_heads,
            c.num_kv_heads, c.head_dim, c.scale, stream)


class NaiveAttention(AttentionBackend):
    """reference src/attention/naive.cu"""

    def __init__(self, config: AttnConfig):
        self.config = config

    def run(self, out, q, kv, n_new, cache_len, stream=None):
        if kv.block_table is not None:
            raise ValueError("NaiveAttention reads contiguous caches only")
        c = self.config
        attention_causal_bf16(out, q, kv.k, kv.v, kv.k_scale, kv.v_scale, n_new, cache_len,
                              c.num_q_heads, c.num_kv_heads, c.head_dim, c.scale, stream)


class BackendKind(enum.Enum):
    """reference include/runtherder/attention/factory.h:9-12"""
    Naive = 0
    Adaptive = 1


def make_attention_backend(kind: BackendKind, config: AttnConfig) -> AttentionBackend:
    """reference src/attention/factory.cu:11-21"""
    if kind == BackendKind.Naive:
        return NaiveAttention(config)
    if kind == BackendKind.Adaptive:
        return AdaptiveAttention(config)
    raise ValueError("unknown attention BackendKind")
