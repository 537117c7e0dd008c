"""MI355X-native attention hot path of the Runtherder engine.

Hand-written gfx950 HIP kernels (causal flash prefill on MFMA, split-K
GQA flash decode, FP8 E4M3 KV append/quantize) behind a C ABI
(include/rth_attn.h, libruntherder_attn.so), with the reference engine's
C++20 interface in include/runtherder/ and a torch-tensor front end in
runtherder_amd.ops.
"""
from . import _ffi
from .ops import (  # noqa: F401
    AdaptiveAttention,
    AttentionBackend,
    AttnConfig,
    BackendKind,
    KVCache,
    KVSlabs,
    KVView,
    NaiveAttention,
    PagedKVCache,
    advance_position,
    attention_causal_bf16,
    DECODE_MFMA,
    DECODE_VALU,
    decode_path,
    set_decode_kernel,
    default_num_splits,
    flash_decode_append_split_bf16,
    flash_decode_rope_append_split_bf16,
    flash_decode_qk_norm_rope_append_split_bf16,
    flash_decode_split_bf16,
    flash_decode_split_bf16_noalloc,
    flash_prefill_bf16,
    flash_prefill_split_bf16,
    PREFILL_SPLIT_MAX_TOKENS,
    flash_split_scratch_floats,
    make_attention_backend,
    new_flash_split_scratch,
    quantize_kv_fp8,
    qk_norm_rope_append_fp8,
    quantize_kv_fp8_scaled,
    rmsnorm_bf16,
    rmsnorm_lanes,
    rope_append_fp8,
    rope_bf16,
)

LIB_PATH = _ffi.LIB_PATH
