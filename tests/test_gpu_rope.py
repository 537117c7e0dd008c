"""RoPE (reference src/kernels/rope.cu:14-55) standalone and fused with the
FP8 KV append on the GPU. RoPE outputs are compared bit-exactly with the
oracle (same fp32 angle, double-precision sin/cos rounded to fp32, same fma
grouping); cache codes and scales are compared bit-exactly with the oracle's
rope-then-quantize and with the GPU's own two-step sequence."""
import numpy as np
import pytest
import torch

import oracle_lib as O
import runtherder_amd as R
from gpu_util import DEV, bf16_dev, bf16_host, f32_dev, host, i32_dev, int_dev, step, sync

pytestmark = pytest.mark.gpu


def inv_table(d, kind):
    if kind == "llama3":
        return O.rope_inv_freq_llama3(d, 5e5, 32.0, 1.0, 4.0, 8192)
    return O.rope_inv_freq_plain(d, 1e6)


def positions_for(n, start):
    return np.arange(start, start + n, dtype=np.int32)


@pytest.mark.parametrize("n,hq,hkv,d,start,kind", [
    (1021, 24, 8, 128, 0, "llama3"), (64, 32, 8, 128, 131008, "plain"), (7, 8, 2, 64, 5, "plain"),
    (33, 4, 4, 256, 1000, "llama3"), (5, 6, 3, 96, 77, "plain"), (9, 4, 2, 36, 3, "plain"),
])
def test_rope_matches_oracle_bits(n, hq, hkv, d, start, kind):
    q = O.normal_bf16((n, hq, d), 100 + d)
    k = O.normal_bf16((n, hkv, d), 200 + d)
    pos = positions_for(n, start)
    inv = inv_table(d, kind)
    qd, kd = bf16_dev(q), bf16_dev(k)
    step(f"rope n={n} hq={hq} hkv={hkv} d={d} start={start}")
    R.rope_bf16(qd, kd, i32_dev(pos), f32_dev(inv), n, hq, hkv, d)
    sync()
    assert np.array_equal(bf16_host(qd), O.rope_apply_bf16(q, pos, inv))
    assert np.array_equal(bf16_host(kd), O.rope_apply_bf16(k, pos, inv))


def cache_bytes(cache, layer, rows):
    view = cache.view(layer)
    d = cache.head_dim
    return (host(view.k).reshape(-1, d)[rows], host(view.v).reshape(-1, d)[rows],
            host(view.k_scale).reshape(-1)[rows].view(np.uint32),
            host(view.v_scale).reshape(-1)[rows].view(np.uint32))


@pytest.mark.parametrize("n,hq,hkv,d,at,kind", [
    (1021, 24, 8, 128, 0, "llama3"), (1, 32, 8, 128, 8195, "plain"), (300, 32, 8, 128, 4000, "plain"),
    (17, 8, 2, 64, 3, "plain"), (40, 8, 4, 256, 11, "llama3"),
])
def test_fused_rope_append_equals_two_step_and_oracle(n, hq, hkv, d, at, kind):
    q = O.normal_bf16((n, hq, d), 300 + n)
    k = O.normal_bf16((n, hkv, d), 400 + n)
    v = O.normal_bf16((n, hkv, d), 500 + n)
    pos = positions_for(n, at)
    inv = inv_table(d, kind)
    max_seq = at + n + 2
    rows = slice(at * hkv, (at + n) * hkv)

    # two-step: rope_bf16 then the append kernel
    c2 = R.KVCache(1, max_seq, hkv, d)
    q2, k2, v2 = bf16_dev(q), bf16_dev(k), bf16_dev(v)
    step(f"two-step rope+append n={n} d={d}")
    R.rope_bf16(q2, k2, i32_dev(pos), f32_dev(inv), n, hq, hkv, d)
    c2.append(0, k2, v2, n, int_dev(at))
    # fused
    c1 = R.KVCache(1, max_seq, hkv, d)
    q1, k1, v1 = bf16_dev(q), bf16_dev(k), bf16_dev(v)
    step(f"fused rope+append n={n} d={d}")
    c1.append_rope(0, q1, k1, v1, n, i32_dev(pos), f32_dev(inv), int_dev(at), hq)
    sync()

    assert np.array_equal(bf16_host(q1), bf16_host(q2))
    assert np.array_equal(bf16_host(k1), k)        # k input left unrotated
    for a, b in zip(cache_bytes(c1, 0, rows), cache_bytes(c2, 0, rows)):
        assert np.array_equal(a, b)

    krot = O.rope_apply_bf16(k, pos, inv)
    wk, wks = O.quantize_kv_fp8(krot, d)
    wv, wvs = O.quantize_kv_fp8(v, d)
    gk, gv, gks, gvs = cache_bytes(c1, 0, rows)
    assert np.array_equal(bf16_host(q1), O.rope_apply_bf16(q, pos, inv))
    assert np.array_equal(gk, wk) and np.array_equal(gv, wv)
    assert np.array_equal(gks, wks.view(np.uint32)) and np.array_equal(gvs, wvs.view(np.uint32))


def test_config2_fused_rope_append_then_prefill():
    """Config 2 through the fused entry: 24Q/8KV, 1021 tokens, llama3 RoPE;
    attention against the oracle on the oracle-rotated inputs."""
    n, hq, hkv, d = 1021, 24, 8, 128
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((n, hq, d), 700)
    k = O.normal_bf16((n, hkv, d), 701)
    v = O.normal_bf16((n, hkv, d), 702)
    pos = positions_for(n, 0)
    inv = inv_table(d, "llama3")
    cache = R.KVCache(1, n, hkv, d)
    qd = bf16_dev(q)
    step("config2 fused rope+append")
    cache.append_rope(0, qd, bf16_dev(k), bf16_dev(v), n, i32_dev(pos), f32_dev(inv),
                      int_dev(0), hq)
    out = torch.empty((n, hq, d), dtype=torch.bfloat16, device=DEV)
    view = cache.view(0)
    step("config2 prefill after fused append")
    R.flash_prefill_bf16(out, qd, view.k, view.v, view.k_scale, view.v_scale, n, int_dev(0),
                         hq, hkv, d, scale)
    sync()
    qr = O.rope_apply_bf16(q, pos, inv)
    k8, ks = O.quantize_kv_fp8(O.rope_apply_bf16(k, pos, inv), d)
    v8, vs = O.quantize_kv_fp8(v, d)
    want = O.attention_f32(qr, k8, v8, ks, vs, n, 0, hq, hkv, d, scale, 16)
    got = bf16_host(out)
    mx, mean = O.bf16_err(got, want)
    assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)
