"""Paged KV layout (no reference counterpart; the reference README plans paged
attention, README.md:142-143). The oracle is the reference's own math on the
GATHERED cache: the paged slabs, read back through the block table, must hold
the bytes the oracle's quantizer (quantization.cu:200-254) produces, and
decode / fused append+decode / prefill over the paged cache must match the
oracle's attention (attention.cu:34-91) on those gathered bytes within
max-abs 2e-2 / mean-abs 2e-3. Each case also checks that the paged result is
bit-identical to the contiguous cache's (same data, same order of work)."""
import numpy as np
import pytest
import torch

import oracle_lib as O
import runtherder_amd as R
from gpu_util import DEV, NTHREADS, bf16_dev, bf16_host, i32_dev, int_dev, step, sync

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def make_pair(total, hq, hkv, d, block, seed):
    """Contiguous and paged caches holding the same `total` tokens (appended in
    chunks through the respective append kernels)."""
    n_blocks = (total + block - 1) // block + 3
    rng = np.random.default_rng(seed)
    table = rng.permutation(n_blocks).astype(np.int32)
    cont = R.KVCache(1, n_blocks * block, hkv, d)
    paged = R.PagedKVCache(1, n_blocks, block, hkv, d)
    bt = i32_dev(table)
    k = O.normal_bf16((total, hkv, d), seed + 1)
    v = O.normal_bf16((total, hkv, d), seed + 2)
    step(f"paged fill total={total} block={block}")
    s0 = 0
    for n in (min(total, 1000), total):      # two chunks: exercises at_pos > 0
        n = n - s0
        if n <= 0:
            continue
        kd, vd = bf16_dev(k[s0:s0 + n]), bf16_dev(v[s0:s0 + n])
        cont.append(0, kd, vd, n, int_dev(s0))
        paged.append(0, kd, vd, n, int_dev(s0), bt)
        s0 += n
    sync()
    return cont, paged, bt, table, k, v


def gather(paged, table, total, block):
    """Logical rows 0..total-1 of the paged slabs, read through the block table
    on the host (independent of the kernels' address arithmetic)."""
    rows = np.concatenate([np.arange(b * block, (b + 1) * block) for b in table])[:total]
    return (paged.k[0].cpu().numpy()[rows], paged.v[0].cpu().numpy()[rows],
            paged.k_scale[0].cpu().numpy()[rows], paged.v_scale[0].cpu().numpy()[rows])


def assert_bytes_match_oracle(gk, gv, gks, gvs, k, v, d):
    """Gathered cache == the oracle's quantizer on the bf16 rows, bit for bit."""
    total, hkv = k.shape[0], k.shape[1]
    ok, oks = O.quantize_kv_fp8(k, d)
    ov, ovs = O.quantize_kv_fp8(v, d)
    assert np.array_equal(gk.reshape(total * hkv, d), ok)
    assert np.array_equal(gv.reshape(total * hkv, d), ov)
    assert np.array_equal(gks.reshape(-1).view(np.uint32), oks.view(np.uint32))
    assert np.array_equal(gvs.reshape(-1).view(np.uint32), ovs.view(np.uint32))


def assert_attention_matches_oracle(got, q, gk, gv, gks, gvs, n_new, clen, hq, hkv, d):
    scale = np.float32(1.0 / np.sqrt(d))
    want = O.attention_f32(q, gk, gv, gks, gvs, n_new, clen, hq, hkv, d, scale, NTHREADS)
    mx, mean = O.bf16_err(got.reshape(want.shape), want)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


@pytest.mark.parametrize("total,block", [(1500, 64), (3000, 32), (777, 256)])
def test_paged_append_bytes(total, block):
    hkv, d = 8, 128
    cont, paged, _, table, k, v = make_pair(total, 32, hkv, d, block, total)
    gk, gv, gks, gvs = gather(paged, table, total, block)
    assert_bytes_match_oracle(gk, gv, gks, gvs, k, v, d)
    assert np.array_equal(gk, cont.k[0].cpu().numpy()[:total])
    assert np.array_equal(gv, cont.v[0].cpu().numpy()[:total])
    assert np.array_equal(gks.view(np.uint32), cont.k_scale[0].cpu().numpy()[:total].view(np.uint32))
    assert np.array_equal(gvs.view(np.uint32), cont.v_scale[0].cpu().numpy()[:total].view(np.uint32))


@pytest.mark.parametrize("total,block,splits,d", [
    (35, 32, None, 128), (2041, 64, None, 128), (8196, 128, None, 128), (5000, 32, 64, 128),
    (300, 64, 7, 128),
    # long per-wave streams (nontemporal loads, the paged reload past a wave's
    # last tile): grouped workgroups at 64 splits and one wave per unit, and
    # the whole-row K layouts of head_dim 64 and 256
    (40000, 64, 64, 128), (20000, 32, None, 64), (12000, 128, 64, 64), (30000, 64, None, 256),
    (12000, 32, 64, 256),
])
def test_paged_decode_equals_contiguous(total, block, splits, d):
    paged_decode_case(total, block, splits, d, 24, 8)


@pytest.mark.parametrize("total,block,splits,d,hq,hkv", [
    (5000, 64, None, 128, 64, 2), (3001, 32, 16, 256, 16, 1), (900, 128, 7, 64, 96, 2),
])
def test_paged_decode_q_blocks(total, block, splits, d, hq, hkv):
    """Groups wider than 16 q heads (blocks of q heads reading one cache head)
    through the block table."""
    paged_decode_case(total, block, splits, d, hq, hkv)


def paged_decode_case(total, block, splits, d, hq, hkv):
    cont, paged, bt, table, _, _ = make_pair(total, hq, hkv, d, block, 10 + total)
    cfg = R.AttnConfig.for_heads(hq, hkv, d)
    be = R.AdaptiveAttention(cfg, splits)
    qh = O.normal_bf16((hq, d), 20 + total)
    q = bf16_dev(qh)
    o1 = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    o2 = torch.empty_like(o1)
    step(f"paged decode total={total} block={block} splits={be.num_splits}")
    be.run(o1, q, cont.view(0), 1, int_dev(total - 1))
    be.run(o2, q, paged.view(0, bt), 1, int_dev(total - 1))
    sync()
    got = bf16_host(o2)
    assert_attention_matches_oracle(got, qh, *gather(paged, table, total, block), 1, total - 1,
                                    hq, hkv, d)
    assert np.array_equal(bf16_host(o1), got)


@pytest.mark.parametrize("total,block,hq,hkv", [(2041, 64, 24, 8), (9000, 32, 24, 8),
                                                (3000, 64, 64, 2)])
def test_paged_fused_append_decode_equals_contiguous(total, block, hq, hkv):
    d = 128
    cont, paged, bt, table, k, v = make_pair(total - 1, hq, hkv, d, block, 30 + total)
    cfg = R.AttnConfig.for_heads(hq, hkv, d)
    be = R.AdaptiveAttention(cfg)
    qh = O.normal_bf16((hq, d), 40 + total)
    q = bf16_dev(qh)
    knh = O.normal_bf16((hkv, d), 41)
    vnh = O.normal_bf16((hkv, d), 42)
    kn, vn = bf16_dev(knh), bf16_dev(vnh)
    o1 = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    o2 = torch.empty_like(o1)
    step(f"paged fused append+decode total={total} block={block}")
    be.run_decode_append(o1, q, cont.slabs(0), kn, vn, int_dev(total - 1))
    be.run_decode_append(o2, q, paged.slabs(0, bt), kn, vn, int_dev(total - 1))
    sync()
    got = bf16_host(o2)
    assert np.array_equal(bf16_host(o1), got)
    gk, gv, gks, gvs = gather(paged, table, total, block)
    # The appended token's row is the oracle quantizer's, like every earlier row.
    assert_bytes_match_oracle(gk, gv, gks, gvs, np.concatenate([k, knh[None]]),
                              np.concatenate([v, vnh[None]]), d)
    assert np.array_equal(gk, cont.k[0].cpu().numpy()[:total])
    assert np.array_equal(gks.view(np.uint32), cont.k_scale[0].cpu().numpy()[:total].view(np.uint32))
    assert_attention_matches_oracle(got, qh, gk, gv, gks, gvs, 1, total - 1, hq, hkv, d)


# Workgroup shapes on 256 compute units: 1021 and 3000 @ 2237 take the
# key-split kernel, 200 (two 128-row blocks per head, whole grid resident) the
# 4-wave kernel with heavy/light pairing, 2500 the 4-wave kernel over two
# rounds (early-issue prologue), 4096 the 8-wave kernel.
@pytest.mark.parametrize("total,clen,block", [(1021, 0, 64), (3000, 2237, 32), (4096, 0, 128),
                                              (200, 0, 32), (1300, 1100, 64), (2500, 0, 64)])
def test_paged_prefill_equals_contiguous(total, clen, block):
    hq, hkv, d = 32, 8, 128
    cont, paged, bt, table, _, _ = make_pair(total, hq, hkv, d, block, 50 + total)
    cfg = R.AttnConfig.for_heads(hq, hkv, d)
    be = R.AdaptiveAttention(cfg)
    n = total - clen
    qh = O.normal_bf16((n, hq, d), 60 + total)
    q = bf16_dev(qh)
    o1 = torch.empty((n, hq, d), dtype=torch.bfloat16, device=DEV)
    o2 = torch.empty_like(o1)
    step(f"paged prefill total={total} clen={clen} block={block}")
    be.run(o1, q, cont.view(0), n, int_dev(clen))
    be.run(o2, q, paged.view(0, bt), n, int_dev(clen))
    sync()
    got = bf16_host(o2)
    assert_attention_matches_oracle(got, qh, *gather(paged, table, total, block), n, clen,
                                    hq, hkv, d)
    assert np.array_equal(bf16_host(o1), got)
