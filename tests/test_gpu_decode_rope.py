"""The fused decode step: RoPE of q and of the new k row, the FP8 append and the
split-K decode in one call (no reference counterpart; replaces the per-layer
sequence rope_bf16 -> KVCache::append -> AttentionBackend::run of reference
src/model/supported/llama/llama3.cu:228-234).

Checked against the GPU's own two-step sequence (rth_rope_bf16 on copies of q
and k, then rth_attn_decode_append_split on the rotated rows): cache bytes and
scales bit-identical, q and k_new left unrotated, outputs bit-identical. Against the
oracle: the rotated rows equal O.rope_apply_bf16 bit for bit, the new cache
row equals the oracle's quantizer on them, and the output is within max-abs
2e-2 / mean-abs 2e-3 of the oracle's attention."""
import numpy as np
import pytest
import torch

import oracle_lib as O
import runtherder_amd as R
from runtherder_amd import _ffi
from gpu_util import (DEV, NTHREADS, bf16_dev, bf16_host, f32_dev, i32_dev, int_dev, step,
                      sync, u8_dev)
from test_gpu_paged import gather, make_pair

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def assert_same_up_to_key_order(got, ref, d):
    """The RoPE / q-k-norm kernels and the plain fused append + decode attend
    to the appended key at the same point (head_dim <= 128: right behind the
    first cache tile's loads; 256: after the cache tiles), so the outputs
    agree bit for bit."""
    assert np.array_equal(got, ref), d


def inv_table(d, kind):
    if kind == "llama3":
        return O.rope_inv_freq_llama3(d, 5e5, 32.0, 1.0, 4.0, 8192)
    return O.rope_inv_freq_plain(d, 1e6)


@pytest.mark.parametrize("cache_len,hq,hkv,d,splits,kind,pos", [
    (8195, 24, 8, 128, None, "llama3", 8195),   # config 3 shape and position
    (0, 32, 8, 128, None, "plain", 0),          # first token: angle 0
    (700, 32, 8, 64, 16, "plain", 700),         # head_dim 64: partners 32 lanes apart
    (300, 16, 4, 256, 8, "llama3", 300),        # head_dim 256
    (2000, 64, 2, 128, 64, "plain", 2000),      # two blocks of 16 q heads per cache head
    (130, 16, 1, 256, 8, "plain", 130),         # MQA, head_dim 256, blocks of 8
    (5000, 32, 8, 128, 128, "plain", 131000),   # position far from cache_len
    (31, 8, 2, 128, 4, "llama3", 31),
])
def test_rope_decode_step_equals_two_step(cache_len, hq, hkv, d, splits, kind, pos):
    total = cache_len + 1
    splits = splits or R.default_num_splits(hkv)
    scale = np.float32(1.0 / np.sqrt(d))
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((total * hkv, d), 7000 + cache_len), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16((total * hkv, d), 8000 + cache_len), d)
    rows = slice(cache_len * hkv, total * hkv)
    k8[rows] = 0
    v8[rows] = 0
    ks[rows] = 0
    vs[rows] = 0
    q = O.normal_bf16((hq, d), 100 + hq + d)
    kn = O.normal_bf16((hkv, d), 200 + hkv + d)
    vn = O.normal_bf16((hkv, d), 300 + hkv + d)
    inv = inv_table(d, kind)
    posd, invd, cl = i32_dev(np.array([pos], np.int32)), f32_dev(inv), int_dev(cache_len)

    step(f"rope decode step ctx={total} hq={hq} hkv={hkv} d={d} splits={splits} pos={pos}")
    kc1, vc1, ks1, vs1 = u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs)
    qd, knd, vnd = bf16_dev(q), bf16_dev(kn), bf16_dev(vn)
    out1 = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    R.flash_decode_rope_append_split_bf16(out1, qd, kc1, vc1, ks1, vs1, knd, vnd, posd, invd,
                                          R.new_flash_split_scratch(hq, d, splits), splits, cl,
                                          hq, hkv, d, scale)

    kc2, vc2, ks2, vs2 = u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs)
    qr, knr = bf16_dev(q), bf16_dev(kn)
    R.rope_bf16(qr, knr, posd, invd, 1, hq, hkv, d)
    out2 = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    R.flash_decode_append_split_bf16(out2, qr, kc2, vc2, ks2, vs2, knr, bf16_dev(vn),
                                     R.new_flash_split_scratch(hq, d, splits), splits, cl, hq,
                                     hkv, d, scale)
    sync()

    assert np.array_equal(bf16_host(qd), q) and np.array_equal(bf16_host(knd), kn)
    for a, b in ((kc1, kc2), (vc1, vc2)):
        assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())
    for a, b in ((ks1, ks2), (vs1, vs2)):
        assert np.array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32))
    got = bf16_host(out1)
    assert_same_up_to_key_order(got, bf16_host(out2), d)

    q_rot = O.rope_apply_bf16(q[None], np.array([pos], np.int32), inv)[0]
    k_rot = O.rope_apply_bf16(kn[None], np.array([pos], np.int32), inv)[0]
    assert np.array_equal(bf16_host(qr), q_rot)
    wk, wks = O.quantize_kv_fp8(k_rot, d)
    gk, gks = kc1.cpu().numpy(), ks1.cpu().numpy()
    assert np.array_equal(gk[rows], wk)
    assert np.array_equal(gks[rows].view(np.uint32), wks.view(np.uint32))
    want = O.attention_f32(q_rot, gk, vc1.cpu().numpy(), gks, vs1.cpu().numpy(), 1, cache_len,
                           hq, hkv, d, scale, NTHREADS)
    mx, mean = O.bf16_err(got, want[0])
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


@pytest.mark.parametrize("total,block,hq,hkv,d", [(2041, 64, 24, 8, 128), (700, 32, 64, 2, 128),
                                                  (300, 128, 16, 4, 256)])
def test_paged_rope_decode_step(total, block, hq, hkv, d):
    """Through the block table: equals the contiguous cache's fused step bit for
    bit, and the contiguous two-step sequence."""
    pos = total - 1
    cont, paged, bt, table, k, v = make_pair(total - 1, hq, hkv, d, block, 90 + total)
    cfg = R.AttnConfig.for_heads(hq, hkv, d)
    be = R.AdaptiveAttention(cfg)
    q = O.normal_bf16((hq, d), 91 + total)
    kn = O.normal_bf16((hkv, d), 92 + total)
    vn = O.normal_bf16((hkv, d), 93 + total)
    inv = inv_table(d, "llama3")
    posd, invd, cl = i32_dev(np.array([pos], np.int32)), f32_dev(inv), int_dev(total - 1)
    step(f"paged rope decode step total={total} block={block} hq={hq} hkv={hkv} d={d}")
    o_paged = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    o_cont = torch.empty_like(o_paged)
    be.run_decode_rope_append(o_paged, bf16_dev(q), paged.slabs(0, bt), bf16_dev(kn),
                              bf16_dev(vn), posd, invd, cl)
    be.run_decode_rope_append(o_cont, bf16_dev(q), cont.slabs(0), bf16_dev(kn), bf16_dev(vn),
                              posd, invd, cl)
    sync()
    got = bf16_host(o_paged)
    assert np.array_equal(got, bf16_host(o_cont))
    gk, gv, gks, gvs = gather(paged, table, total, block)
    assert np.array_equal(gk, cont.k[0].cpu().numpy()[:total])
    assert np.array_equal(gks.view(np.uint32),
                          cont.k_scale[0].cpu().numpy()[:total].view(np.uint32))
    q_rot = O.rope_apply_bf16(q[None], np.array([pos], np.int32), inv)[0]
    want = O.attention_f32(q_rot, gk, gv, gks, gvs, 1, total - 1, hq, hkv, d,
                           np.float32(1.0 / np.sqrt(d)), NTHREADS)
    mx, mean = O.bf16_err(got, want[0])
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


def test_rope_decode_step_rejects_valu_shapes():
    """Shapes without the MFMA decode (head_dim 32 here) fail with an error
    instead of running a different sequence."""
    hq, hkv, d = 8, 2, 32
    out = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    z8 = torch.zeros((16 * hkv, d), dtype=torch.uint8, device=DEV)
    zs = torch.zeros((16 * hkv,), dtype=torch.float32, device=DEV)
    zb = torch.zeros((hkv, d), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_ffi.RthError) as e:
        R.flash_decode_rope_append_split_bf16(
            out, torch.zeros((hq, d), dtype=torch.bfloat16, device=DEV), z8, z8.clone(), zs,
            zs.clone(), zb, zb.clone(), int_dev(0), f32_dev(np.ones(d // 2, np.float32)),
            R.new_flash_split_scratch(hq, d, 4), 4, int_dev(3), hq, hkv, d, 0.1)
    assert "RoPE decode step" in str(e.value)


@pytest.mark.parametrize("cache_len,hq,hkv,d,splits,pos", [
    (8195, 32, 8, 128, None, 8195),    # Qwen3-8B shape
    (0, 32, 8, 128, None, 0),
    (700, 16, 4, 64, 16, 700),
    (300, 16, 4, 256, 8, 300),
    (2000, 64, 2, 128, 64, 2000),      # q blocks of 16
    (130, 16, 1, 256, 8, 130),
])
def test_qk_norm_rope_decode_step_equals_unfused(cache_len, hq, hkv, d, splits, pos):
    """Qwen3 order (qwen3.cu:189-202): rmsnorm per head of q and k, RoPE,
    append, decode. Reference: rth_rmsnorm_bf16 and rth_rope_bf16 on copies,
    then the fused append + decode on the transformed rows."""
    eps = 1e-6
    total = cache_len + 1
    splits = splits or R.default_num_splits(hkv)
    scale = np.float32(1.0 / np.sqrt(d))
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((total * hkv, d), 7100 + cache_len), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16((total * hkv, d), 8100 + cache_len), d)
    rows = slice(cache_len * hkv, total * hkv)
    for a in (k8, v8, ks, vs):
        a[rows] = 0
    q = O.normal_bf16((hq, d), 110 + hq + d)
    kn = O.normal_bf16((hkv, d), 210 + hkv + d)
    vn = O.normal_bf16((hkv, d), 310 + hkv + d)
    qg = O.normal_bf16((d,), 410 + d)
    kg = O.normal_bf16((d,), 510 + d)
    inv = inv_table(d, "plain")
    posd, invd, cl = i32_dev(np.array([pos], np.int32)), f32_dev(inv), int_dev(cache_len)
    qgd, kgd = bf16_dev(qg), bf16_dev(kg)

    step(f"qk-norm rope decode step ctx={total} hq={hq} hkv={hkv} d={d} splits={splits}")
    kc1, vc1, ks1, vs1 = u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs)
    qd, knd = bf16_dev(q), bf16_dev(kn)
    out1 = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    R.flash_decode_qk_norm_rope_append_split_bf16(out1, qd, kc1, vc1, ks1, vs1, knd, bf16_dev(vn),
                                                  qgd, kgd, eps, posd, invd,
                                                  R.new_flash_split_scratch(hq, d, splits),
                                                  splits, cl, hq, hkv, d, scale)

    kc2, vc2, ks2, vs2 = u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs)
    qr, knr = bf16_dev(q), bf16_dev(kn)
    R.rmsnorm_bf16(qr, qr, qgd, hq, d, eps)
    R.rmsnorm_bf16(knr, knr, kgd, hkv, d, eps)
    R.rope_bf16(qr, knr, posd, invd, 1, hq, hkv, d)
    out2 = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    R.flash_decode_append_split_bf16(out2, qr, kc2, vc2, ks2, vs2, knr, bf16_dev(vn),
                                     R.new_flash_split_scratch(hq, d, splits), splits, cl, hq,
                                     hkv, d, scale)
    sync()

    assert np.array_equal(bf16_host(qd), q) and np.array_equal(bf16_host(knd), kn)
    for a, b in ((kc1, kc2), (vc1, vc2)):
        assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())
    for a, b in ((ks1, ks2), (vs1, vs2)):
        assert np.array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32))
    got = bf16_host(out1)
    assert_same_up_to_key_order(got, bf16_host(out2), d)

    lanes = R.rmsnorm_lanes(d)
    q_t = O.rope_apply_bf16(O.rmsnorm_bf16(q, qg, eps, lanes)[None], np.array([pos], np.int32),
                            inv)[0]
    k_t = O.rope_apply_bf16(O.rmsnorm_bf16(kn, kg, eps, lanes)[None],
                            np.array([pos], np.int32), inv)[0]
    assert np.array_equal(bf16_host(qr), q_t)
    wk, wks = O.quantize_kv_fp8(k_t, d)
    gk, gks = kc1.cpu().numpy(), ks1.cpu().numpy()
    assert np.array_equal(gk[rows], wk)
    assert np.array_equal(gks[rows].view(np.uint32), wks.view(np.uint32))
    want = O.attention_f32(q_t, gk, vc1.cpu().numpy(), gks, vs1.cpu().numpy(), 1, cache_len,
                           hq, hkv, d, scale, NTHREADS)
    mx, mean = O.bf16_err(got, want[0])
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (mx, mean)


def test_paged_qk_norm_rope_decode_step():
    total, block, hq, hkv, d = 1500, 64, 32, 8, 128
    eps, pos = 1e-6, 1499
    cont, paged, bt, table, _, _ = make_pair(total - 1, hq, hkv, d, block, 77)
    be = R.AdaptiveAttention(R.AttnConfig.for_heads(hq, hkv, d))
    q = bf16_dev(O.normal_bf16((hq, d), 78))
    kn, vn = bf16_dev(O.normal_bf16((hkv, d), 79)), bf16_dev(O.normal_bf16((hkv, d), 80))
    qg, kg = bf16_dev(O.normal_bf16((d,), 81)), bf16_dev(O.normal_bf16((d,), 82))
    posd, invd, cl = i32_dev(np.array([pos], np.int32)), f32_dev(inv_table(d, "plain")), \
        int_dev(total - 1)
    step("paged qk-norm rope decode step")
    o_p = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    o_c = torch.empty_like(o_p)
    be.run_decode_qk_norm_rope_append(o_p, q, paged.slabs(0, bt), kn, vn, qg, kg, eps, posd, invd,
                                      cl)
    be.run_decode_qk_norm_rope_append(o_c, q, cont.slabs(0), kn, vn, qg, kg, eps, posd, invd, cl)
    sync()
    assert np.array_equal(bf16_host(o_p), bf16_host(o_c))
    gk, _, gks, _ = gather(paged, table, total, block)
    assert np.array_equal(gk, cont.k[0].cpu().numpy()[:total])
    assert np.array_equal(gks.view(np.uint32),
                          cont.k_scale[0].cpu().numpy()[:total].view(np.uint32))


def test_rope_decode_steps_in_a_graph():
    """Four fused RoPE decode steps of one layer captured in a HIP graph with a
    device-side position advance (rth_advance_position), replayed twice with
    eager work in between: every replay's outputs and cache rows equal the
    same steps run eagerly."""
    hq, hkv, d, depth, steps = 24, 8, 128, 3000, 4
    inv = f32_dev(inv_table(d, "llama3"))
    k8, ks = O.quantize_kv_fp8(O.normal_bf16(((depth + steps) * hkv, d), 61), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16(((depth + steps) * hkv, d), 62), d)
    q = bf16_dev(O.normal_bf16((steps, hq, d), 63))
    kn = bf16_dev(O.normal_bf16((steps, hkv, d), 64))
    vn = bf16_dev(O.normal_bf16((steps, hkv, d), 65))
    splits = R.default_num_splits(hkv)
    be = R.AdaptiveAttention(R.AttnConfig.for_heads(hq, hkv, d), splits)

    def fresh():
        return u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs)

    def run(view_k, view_v, view_ks, view_vs, out, pos, stream=None):
        for s in range(steps):
            R.flash_decode_rope_append_split_bf16(out[s], q[s], view_k, view_v, view_ks, view_vs,
                                                  kn[s], vn[s], pos, inv, be.partial, splits,
                                                  pos, hq, hkv, d, be.config.scale, stream)
            R.advance_position(pos, 1, stream)
        R.advance_position(pos, -steps, stream)

    step("rope decode steps, eager")
    ek = fresh()
    e_out = torch.empty((steps, hq, d), dtype=torch.bfloat16, device=DEV)
    run(*ek, e_out, int_dev(depth))
    sync()

    gk = fresh()
    g_out = torch.zeros_like(e_out)
    g_pos = int_dev(depth)
    stream = torch.cuda.Stream()
    sync()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        run(*gk, g_out, g_pos, stream.cuda_stream)
    for rep in range(2):
        step(f"rope decode steps, graph replay {rep}")
        g_out.zero_()
        graph.replay()
        sync()
        assert np.array_equal(bf16_host(g_out), bf16_host(e_out))
        for a, b in zip(gk, ek):
            assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())
        torch.zeros((1 << 20,), device=DEV).sum().item()   # eager work between replays


@pytest.mark.parametrize("d", [64, 128, 256])
def test_decode_steps_special_values(d):
    """The RoPE and Qwen3 decode steps on extreme rows: k rows of zeros, of
    bf16 subnormals only, of the largest finite values (their rotation
    overflows to inf) and of mixed huge and tiny values; v rows with NaN and
    +-inf entries as well. The cache codes and scales equal the oracle's
    RMSNorm -> RoPE -> quantizer pipeline bit for bit (the attention output is
    not checked: an inf or NaN key makes it non-finite by design)."""
    hq, hkv, cache_len, splits, pos, eps = 32, 8, 500, 32, 777, 1e-6
    scale = np.float32(1.0 / np.sqrt(d))
    total = cache_len + 1
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((total * hkv, d), 9100 + d), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16((total * hkv, d), 9200 + d), d)
    rows = slice(cache_len * hkv, total * hkv)
    q = O.normal_bf16((hq, d), 9300 + d)
    kn = O.normal_bf16((hkv, d), 9400 + d)
    vn = O.normal_bf16((hkv, d), 9500 + d)
    for x in (kn, vn):
        x[0, :] = 0
        x[1, :] = np.arange(1, d + 1, dtype=np.uint16)
        x[2, ::2], x[2, 1::2] = 0x7F7F, 0xFF7F
        x[3, ::3] = 0x7F00
    vn[4, 3], vn[4, 9], vn[5, 0] = 0x7FC0, 0x7F80, 0xFF80
    qg = O.normal_bf16((d,), 9600 + d)
    kg = O.normal_bf16((d,), 9700 + d)
    inv = inv_table(d, "plain")
    posd, invd, cl = i32_dev(np.array([pos], np.int32)), f32_dev(inv), int_dev(cache_len)
    p = np.array([pos], np.int32)
    lanes = R.rmsnorm_lanes(d)
    wv, wvs = O.quantize_kv_fp8(vn, d)
    for norm in (False, True):
        step(f"decode step special values d={d} norm={norm}")
        kc, vc, ksd, vsd = u8_dev(k8), u8_dev(v8), f32_dev(ks), f32_dev(vs)
        out = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
        part = R.new_flash_split_scratch(hq, d, splits)
        if norm:
            R.flash_decode_qk_norm_rope_append_split_bf16(
                out, bf16_dev(q), kc, vc, ksd, vsd, bf16_dev(kn), bf16_dev(vn), bf16_dev(qg),
                bf16_dev(kg), eps, posd, invd, part, splits, cl, hq, hkv, d, scale)
            k_t = O.rope_apply_bf16(O.rmsnorm_bf16(kn, kg, eps, lanes)[None], p, inv)[0]
        else:
            R.flash_decode_rope_append_split_bf16(out, bf16_dev(q), kc, vc, ksd, vsd,
                                                  bf16_dev(kn), bf16_dev(vn), posd, invd, part,
                                                  splits, cl, hq, hkv, d, scale)
            k_t = O.rope_apply_bf16(kn[None], p, inv)[0]
        sync()
        wk, wks = O.quantize_kv_fp8(k_t, d)
        assert np.array_equal(kc.cpu().numpy()[rows], wk)
        assert np.array_equal(ksd.cpu().numpy()[rows].view(np.uint32), wks.view(np.uint32))
        assert np.array_equal(vc.cpu().numpy()[rows], wv)
        assert np.array_equal(vsd.cpu().numpy()[rows].view(np.uint32), wvs.view(np.uint32))
