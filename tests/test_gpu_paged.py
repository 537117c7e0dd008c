"""Paged KV layout (no reference counterpart; the reference README plans paged
attention, README.md:142-143): a paged cache with a shuffled block table must
hold, after gathering, the bytes the contiguous cache holds, and decode /
fused append+decode / prefill over it must return exactly the contiguous
results (same data, same order of work)."""
import numpy as np
import pytest
import torch

import oracle_lib as O
import runtherder_amd as R
from gpu_util import DEV, bf16_dev, bf16_host, i32_dev, int_dev, step, sync

pytestmark = pytest.mark.gpu


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
    return cont, paged, bt, table


def gather(paged, table, total, block):
    rows = np.concatenate([np.arange(b * block, (b + 1) * block) for b in table])[:total]
    return (paged.k[0].cpu().numpy()[rows], paged.v[0].cpu().numpy()[rows],
            paged.k_scale[0].cpu().numpy()[rows], paged.v_scale[0].cpu().numpy()[rows])


@pytest.mark.parametrize("total,block", [(1500, 64), (3000, 32), (777, 256)])
def test_paged_append_bytes(total, block):
    hkv, d = 8, 128
    cont, paged, _, table = make_pair(total, 32, hkv, d, block, total)
    gk, gv, gks, gvs = gather(paged, table, total, block)
    assert np.array_equal(gk, cont.k[0].cpu().numpy()[:total])
    assert np.array_equal(gv, cont.v[0].cpu().numpy()[:total])
    assert np.array_equal(gks.view(np.uint32), cont.k_scale[0].cpu().numpy()[:total].view(np.uint32))
    assert np.array_equal(gvs.view(np.uint32), cont.v_scale[0].cpu().numpy()[:total].view(np.uint32))


@pytest.mark.parametrize("total,block,splits", [(35, 32, None), (2041, 64, None), (8196, 128, None),
                                                (5000, 32, 64), (300, 64, 7)])
def test_paged_decode_equals_contiguous(total, block, splits):
    hq, hkv, d = 24, 8, 128
    cont, paged, bt, _ = make_pair(total, hq, hkv, d, block, 10 + total)
    cfg = R.AttnConfig.for_heads(hq, hkv, d)
    be = R.AdaptiveAttention(cfg, splits)
    q = bf16_dev(O.normal_bf16((hq, d), 20 + total))
    o1 = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    o2 = torch.empty_like(o1)
    step(f"paged decode total={total} block={block} splits={be.num_splits}")
    be.run(o1, q, cont.view(0), 1, int_dev(total - 1))
    be.run(o2, q, paged.view(0, bt), 1, int_dev(total - 1))
    sync()
    assert np.array_equal(bf16_host(o1), bf16_host(o2))


@pytest.mark.parametrize("total,block", [(2041, 64), (9000, 32)])
def test_paged_fused_append_decode_equals_contiguous(total, block):
    hq, hkv, d = 24, 8, 128
    cont, paged, bt, table = make_pair(total - 1, hq, hkv, d, block, 30 + total)
    cfg = R.AttnConfig.for_heads(hq, hkv, d)
    be = R.AdaptiveAttention(cfg)
    q = bf16_dev(O.normal_bf16((hq, d), 40 + total))
    kn = bf16_dev(O.normal_bf16((hkv, d), 41))
    vn = bf16_dev(O.normal_bf16((hkv, d), 42))
    o1 = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    o2 = torch.empty_like(o1)
    step(f"paged fused append+decode total={total} block={block}")
    be.run_decode_append(o1, q, cont.view(0), kn, vn, int_dev(total - 1))
    be.run_decode_append(o2, q, paged.view(0, bt), kn, vn, int_dev(total - 1))
    sync()
    assert np.array_equal(bf16_host(o1), bf16_host(o2))
    gk, _, gks, _ = gather(paged, table, total, block)
    assert np.array_equal(gk, cont.k[0].cpu().numpy()[:total])
    assert np.array_equal(gks.view(np.uint32), cont.k_scale[0].cpu().numpy()[:total].view(np.uint32))


@pytest.mark.parametrize("total,clen,block", [(1021, 0, 64), (3000, 2237, 32), (4096, 0, 128)])
def test_paged_prefill_equals_contiguous(total, clen, block):
    hq, hkv, d = 32, 8, 128
    cont, paged, bt, _ = make_pair(total, hq, hkv, d, block, 50 + total)
    cfg = R.AttnConfig.for_heads(hq, hkv, d)
    be = R.AdaptiveAttention(cfg)
    n = total - clen
    q = bf16_dev(O.normal_bf16((n, hq, d), 60 + total))
    o1 = torch.empty((n, hq, d), dtype=torch.bfloat16, device=DEV)
    o2 = torch.empty_like(o1)
    step(f"paged prefill total={total} clen={clen} block={block}")
    be.run(o1, q, cont.view(0), n, int_dev(clen))
    be.run(o2, q, paged.view(0, bt), n, int_dev(clen))
    sync()
    assert np.array_equal(bf16_host(o1), bf16_host(o2))
