"""The reference call sequence (KVCache.append -> view -> backend.run, per
layer, reference src/model/supported/llama/llama3.cu:232-234) through the
Python mirror of the interface, and a multi-step decode captured in one HIP
graph (device-side position advance), replayed several times against eager."""
import numpy as np
import pytest
import torch

import oracle_lib as O
import runtherder_amd as R
from gpu_util import DEV, NTHREADS, bf16_dev, bf16_host, host, int_dev, step, sync

pytestmark = pytest.mark.gpu

HQ, HKV, D, L = 24, 8, 128, 4


def layer_inputs(n, layer, tag):
    q = O.normal_bf16((n, HQ, D), 10_000 * tag + 10 * layer + 1)
    k = O.normal_bf16((n, HKV, D), 10_000 * tag + 10 * layer + 2)
    v = O.normal_bf16((n, HKV, D), 10_000 * tag + 10 * layer + 3)
    return q, k, v


@pytest.mark.parametrize("kind", [R.BackendKind.Adaptive, R.BackendKind.Naive])
def test_prefill_then_decode_sequence(kind):
    cfg = R.AttnConfig.for_heads(HQ, HKV, D)
    backend = R.make_attention_backend(kind, cfg)
    cache = R.KVCache(L, 512, HKV, D)
    pos = int_dev(0)
    hist = {l: ([], [], []) for l in range(L)}
    start = 0
    for it, n in enumerate([150, 90, 1, 1, 1]):
        pos.fill_(start)
        for l in range(L):
            q, k, v = layer_inputs(n, l, it)
            hist[l][0].append(q); hist[l][1].append(k); hist[l][2].append(v)
            out = torch.empty((n, HQ, D), dtype=torch.bfloat16, device=DEV)
            step(f"{kind.name} layer={l} start={start} n={n}")
            cache.append(l, bf16_dev(k), bf16_dev(v), n, pos)
            backend.run(out, bf16_dev(q), cache.view(l), n, pos)
            sync()
            kall = np.concatenate(hist[l][1]).reshape(-1, D)
            vall = np.concatenate(hist[l][2]).reshape(-1, D)
            k8, ks = O.quantize_kv_fp8(kall, D)
            v8, vs = O.quantize_kv_fp8(vall, D)
            view = cache.view(l)
            rows = (start + n) * HKV
            assert np.array_equal(host(view.k).reshape(-1, D)[:rows], k8)
            assert np.array_equal(host(view.v_scale).reshape(-1)[:rows], vs)
            want = O.attention_f32(q, k8, v8, ks, vs, n, start, HQ, HKV, D, cfg.scale, NTHREADS)
            mx, mean = O.bf16_err(bf16_host(out), want)
            assert mx <= 2e-2 and mean <= 2e-3, (l, start, n, mx, mean)
        start += n


def test_decode_steps_in_one_hip_graph():
    steps, depth = 16, 300
    cfg = R.AttnConfig.for_heads(HQ, HKV, D)
    backend = R.AdaptiveAttention(cfg)
    cache = R.KVCache(L, depth + steps, HKV, D)
    pos = int_dev(0)
    hist_k = {l: [] for l in range(L)}
    hist_v = {l: [] for l in range(L)}
    for l in range(L):
        _, k, v = layer_inputs(depth, l, 99)
        hist_k[l].append(k); hist_v[l].append(v)
        cache.append(l, bf16_dev(k), bf16_dev(v), depth, pos)
    qs = [[layer_inputs(1, l, 500 + s) for l in range(L)] for s in range(steps)]
    qd = [[tuple(bf16_dev(a) for a in qs[s][l]) for l in range(L)] for s in range(steps)]
    outs = torch.zeros((steps, L, HQ, D), dtype=torch.bfloat16, device=DEV)

    def run_steps():
        for s in range(steps):
            for l in range(L):
                q, k, v = qd[s][l]
                cache.append(l, k, v, 1, pos)
                backend.run(outs[s, l], q, cache.view(l), 1, pos)
            R.advance_position(pos, 1)

    step("graph eager reference")
    pos.fill_(depth)
    run_steps()
    sync()
    eager = bf16_host(outs).copy()

    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    pos.fill_(depth)
    sync()
    step("graph capture")
    with torch.cuda.graph(g, stream=stream):
        run_steps()
    for rep in range(3):
        outs.zero_()
        pos.fill_(depth)
        sync()
        step(f"graph replay {rep}")
        g.replay()
        sync()
        assert np.array_equal(bf16_host(outs), eager), rep
        assert int(pos.item()) == depth + steps
        torch.cuda.synchronize()
        _ = (outs.float() * 2).sum().item()  # unrelated eager work between replays

    # oracle check of the last step of every layer
    for l in range(L):
        kall = np.concatenate(hist_k[l] + [qs[s][l][1] for s in range(steps)]).reshape(-1, D)
        vall = np.concatenate(hist_v[l] + [qs[s][l][2] for s in range(steps)]).reshape(-1, D)
        k8, ks = O.quantize_kv_fp8(kall, D)
        v8, vs = O.quantize_kv_fp8(vall, D)
        want = O.attention_f32(qs[-1][l][0], k8, v8, ks, vs, 1, depth + steps - 1, HQ, HKV, D,
                               cfg.scale, NTHREADS)
        mx, mean = O.bf16_err(eager[-1, l], want[0])
        assert mx <= 2e-2 and mean <= 2e-3, (l, mx, mean)


def test_config3_28_layer_128_step_graph():
    """BASELINE config 3 at depth 8196: 28 layers x 128 decode steps (fused
    one-token append + split-K decode per layer, device-side position advance)
    captured in one HIP graph. After one replay, every appended cache row
    equals the oracle quantizer's bytes and the last step of all 28 layers
    matches the oracle's attention over the whole cache."""
    layers, steps, depth = 28, 128, 8195
    cfg = R.AttnConfig.for_heads(HQ, HKV, D)
    backend = R.AdaptiveAttention(cfg)
    cache = R.KVCache(layers, depth + steps, HKV, D)
    pos = int_dev(0)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(8196)
    step("config3 graph: history fill")
    for l in range(layers):
        k = torch.randn((depth, HKV, D), generator=gen, device=DEV).to(torch.bfloat16)
        v = torch.randn((depth, HKV, D), generator=gen, device=DEV).to(torch.bfloat16)
        cache.append(l, k, v, depth, pos)
    qs = torch.randn((steps, layers, HQ, D), generator=gen, device=DEV).to(torch.bfloat16)
    kn = torch.randn((steps, layers, HKV, D), generator=gen, device=DEV).to(torch.bfloat16)
    vn = torch.randn((steps, layers, HKV, D), generator=gen, device=DEV).to(torch.bfloat16)
    outs = torch.zeros((steps, layers, HQ, D), dtype=torch.bfloat16, device=DEV)
    sync()
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    step("config3 graph: capture")
    with torch.cuda.graph(g, stream=stream):
        for s in range(steps):
            for l in range(layers):
                backend.run_decode_append(outs[s, l], qs[s, l], cache.slabs(l), kn[s, l],
                                          vn[s, l], pos)
            R.advance_position(pos, 1)
    pos.fill_(depth)
    sync()
    step("config3 graph: replay")
    g.replay()
    sync()
    assert int(pos.item()) == depth + steps
    kn_h, vn_h = bf16_host(kn), bf16_host(vn)
    q_last = bf16_host(qs[-1])
    out_last = bf16_host(outs[-1])
    for l in range(layers):
        view = cache.view(l)
        k8, v8 = host(view.k).reshape(-1, D), host(view.v).reshape(-1, D)
        ks, vs = host(view.k_scale).reshape(-1), host(view.v_scale).reshape(-1)
        rows = slice(depth * HKV, (depth + steps) * HKV)
        wk, wks = O.quantize_kv_fp8(kn_h[:, l].reshape(-1, D), D)
        wv, wvs = O.quantize_kv_fp8(vn_h[:, l].reshape(-1, D), D)
        assert np.array_equal(k8[rows], wk) and np.array_equal(v8[rows], wv), l
        assert np.array_equal(ks[rows].view(np.uint32), wks.view(np.uint32)), l
        assert np.array_equal(vs[rows].view(np.uint32), wvs.view(np.uint32)), l
        want = O.attention_f32(q_last[l], k8, v8, ks, vs, 1, depth + steps - 1, HQ, HKV, D,
                               cfg.scale, NTHREADS)
        mx, mean = O.bf16_err(out_last[l], want[0])
        assert mx <= 2e-2 and mean <= 2e-3, (l, mx, mean)
