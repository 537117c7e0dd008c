"""RMSNorm (reference src/kernels/rmsnorm.cu:45-136) and the fused Qwen3
q/k-norm -> RoPE -> FP8 append on the GPU, bit-exact against the oracle (which
restates the kernel's summation order) and against the GPU's own unfused
sequence (reference src/model/supported/llama/qwen3.cu:189-200)."""
import numpy as np
import pytest
import torch

import oracle_lib as O
import runtherder_amd as R
from gpu_util import bf16_dev, bf16_host, f32_dev, host, i32_dev, int_dev, step, sync

pytestmark = pytest.mark.gpu

EPS = 1e-6


@pytest.mark.parametrize("rows,dim", [(257, 128), (64, 64), (33, 256), (7, 4096), (5, 3072),
                                      (3, 16384), (11, 24), (32768, 128), (200000, 8)])
def test_rmsnorm_matches_oracle_bits(rows, dim):
    x = O.normal_bf16((rows, dim), 31 + dim)
    g = O.normal_bf16((dim,), 32 + dim)
    y = torch.empty((rows, dim), dtype=torch.bfloat16, device="cuda")
    xd = bf16_dev(x)
    step(f"rmsnorm rows={rows} dim={dim}")
    R.rmsnorm_bf16(y, xd, bf16_dev(g), rows, dim, EPS)
    R.rmsnorm_bf16(xd, xd, bf16_dev(g), rows, dim, EPS)      # in place (y aliases x)
    sync()
    want = O.rmsnorm_bf16(x, g, EPS, R.rmsnorm_lanes(dim))
    assert np.array_equal(bf16_host(y), want)
    assert np.array_equal(bf16_host(xd), want)


@pytest.mark.parametrize("n,hq,hkv,d,at", [(1021, 32, 8, 128, 0), (1, 32, 8, 128, 8195),
                                           (129, 16, 4, 64, 7), (20, 8, 4, 256, 300)])
def test_fused_qk_norm_rope_append(n, hq, hkv, d, at):
    q = O.normal_bf16((n, hq, d), 600 + n)
    k = O.normal_bf16((n, hkv, d), 601 + n)
    v = O.normal_bf16((n, hkv, d), 602 + n)
    qn = O.normal_bf16((d,), 603)
    kn = O.normal_bf16((d,), 604)
    pos = np.arange(at, at + n, dtype=np.int32)
    inv = O.rope_inv_freq_plain(d, 1e6)
    rows = slice(at * hkv, (at + n) * hkv)
    max_seq = at + n + 1

    # unfused GPU sequence
    c2 = R.KVCache(1, max_seq, hkv, d)
    q2, k2, v2 = bf16_dev(q), bf16_dev(k), bf16_dev(v)
    step(f"unfused qk-norm/rope/append n={n} d={d}")
    R.rmsnorm_bf16(q2, q2, bf16_dev(qn), n * hq, d, EPS)
    R.rmsnorm_bf16(k2, k2, bf16_dev(kn), n * hkv, d, EPS)
    R.rope_bf16(q2, k2, i32_dev(pos), f32_dev(inv), n, hq, hkv, d)
    c2.append(0, k2, v2, n, int_dev(at))
    # fused
    c1 = R.KVCache(1, max_seq, hkv, d)
    q1, k1 = bf16_dev(q), bf16_dev(k)
    step(f"fused qk-norm/rope/append n={n} d={d}")
    c1.append_qk_norm_rope(0, q1, k1, bf16_dev(v), n, bf16_dev(qn), bf16_dev(kn), EPS,
                           i32_dev(pos), f32_dev(inv), int_dev(at), hq)
    sync()

    def cache(c):
        view = c.view(0)
        return (host(view.k).reshape(-1, d)[rows], host(view.v).reshape(-1, d)[rows],
                host(view.k_scale).reshape(-1)[rows].view(np.uint32),
                host(view.v_scale).reshape(-1)[rows].view(np.uint32))

    assert np.array_equal(bf16_host(q1), bf16_host(q2))
    assert np.array_equal(bf16_host(k1), k)
    for a, b in zip(cache(c1), cache(c2)):
        assert np.array_equal(a, b)

    lanes = d // 8
    qw = O.rope_apply_bf16(O.rmsnorm_bf16(q, qn, EPS, lanes), pos, inv)
    kw = O.rope_apply_bf16(O.rmsnorm_bf16(k, kn, EPS, lanes), pos, inv)
    wk, wks = O.quantize_kv_fp8(kw, d)
    wv, wvs = O.quantize_kv_fp8(v, d)
    gk, gv, gks, gvs = cache(c1)
    assert np.array_equal(bf16_host(q1), qw)
    assert np.array_equal(gk, wk) and np.array_equal(gv, wv)
    assert np.array_equal(gks, wks.view(np.uint32)) and np.array_equal(gvs, wvs.view(np.uint32))
