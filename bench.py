#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one GPU).

Headline: decode attention HBM GB/s at 8K context (a
Llama-3.2-3B-shaped 28-layer decode, 24 Q / 8 KV heads, head_dim 128, FP8 E4M3
KV cache prefilled with quantized N(0,1), one token per step: per layer the
fused K/V append then the split-K flash decode, 128 steps captured in one HIP
graph). A "step" is one decode token through all 28 layers. Secondary: causal
prefill attention TFLOP/s at 4096 tokens (config 4: 32 Q / 8 KV heads, RoPE'd
N(0,1) inputs, FP8 writeback).

Algorithmic units (no credit for re-reads or scratch):
  decode bytes / call  = ctx*Hkv*D*2 + ctx*Hkv*8 + Hq*D*4
  prefill flops / call = 4*Hq*D*P, P = n*clen + n*(n+1)/2

Timed steps are exactly --steps (full 128-step graphs plus one graph of the
remainder), after exactly --warmup untimed steps. The line also carries the
roofline of the decode call at 32768 and 131072 keys and of prefill at 8192
and 16384 tokens ("target_range"), and CPU baselines for decode (GB/s) and
prefill (GFLOP/s).

Prints one JSON line. Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import math
import statistics
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0         # MI355X HBM3E, AMD published
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA, AMD published
GRAPH_STEPS = 128


def decode_bytes(ctx: int, hq: int, hkv: int, d: int) -> int:
    return ctx * hkv * d * 2 + ctx * hkv * 8 + hq * d * 4


def append_bytes(hkv: int, d: int) -> int:
    """The fused call's one-token append: k_new, v_new bf16 in, E4M3 codes
    and fp32 scales out."""
    return hkv * d * 2 * 2 + hkv * d * 2 + hkv * 8


def prefill_flops(n: int, clen: int, hq: int, d: int) -> int:
    pairs = n * clen + n * (n + 1) // 2
    return 4 * hq * d * pairs


class EventTimer:
    """HIP events on the stream the kernels run on."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream
        self.a = torch.cuda.Event(enable_timing=True)
        self.b = torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        self.a.record(self.stream)
        return self

    def __exit__(self, *exc):
        self.b.record(self.stream)
        self.b.synchronize()
        self.ms = self.a.elapsed_time(self.b)


def graph_us(torch, stream, fn, iters, replays=5):
    """Microseconds per call of fn, captured iters times in one HIP graph and
    timed over `replays` replays (one warm replay first), median of them: the
    kernels back to back, without the host launch rate of an eager loop, and
    one disturbed replay does not move the figure."""
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()   # work queued on other streams lands first
    times = []
    with torch.cuda.stream(stream):
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=stream):
            for _ in range(iters):
                fn()
        g.replay()
        for _ in range(replays):
            with EventTimer(torch, stream) as t:
                g.replay()
            times.append(t.ms)
    torch.cuda.synchronize()
    return statistics.median(times) * 1e3 / iters


def bench_decode(torch, R, args, stream):
    hq, hkv, d, L = 24, 8, 128, 28
    ctx0 = args.ctx                          # keys attended at the first step
    depth = ctx0 - 1                         # history prefilled before step 0
    max_seq = depth + GRAPH_STEPS + 1
    scale = 1.0 / math.sqrt(d)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)

    cache = R.KVCache(L, max_seq, hkv, d, device=dev)
    backend = R.AdaptiveAttention(R.AttnConfig(hq, hkv, d, scale))
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    chunk = 4096
    torch.cuda.synchronize()   # the allocations above are initialized on the default stream
    with torch.cuda.stream(stream):
        for l in range(L):
            for s0 in range(0, depth, chunk):
                n = min(chunk, depth - s0)
                k = torch.randn((n, hkv, d), generator=gen, device=dev).to(torch.bfloat16)
                v = torch.randn((n, hkv, d), generator=gen, device=dev).to(torch.bfloat16)
                pos.fill_(s0)
                cache.append(l, k, v, n, pos)
        # per-step, per-layer new token: q, k, v (distinct per step and layer)
        qs = torch.randn((GRAPH_STEPS, L, hq, d), generator=gen, device=dev).to(torch.bfloat16)
        ks = torch.randn((GRAPH_STEPS, L, hkv, d), generator=gen, device=dev).to(torch.bfloat16)
        vs = torch.randn((GRAPH_STEPS, L, hkv, d), generator=gen, device=dev).to(torch.bfloat16)
        out = torch.empty((GRAPH_STEPS, L, hq, d), dtype=torch.bfloat16, device=dev)
        pos.fill_(depth)
    torch.cuda.synchronize()

    def run_steps(fused, n_steps):
        for s in range(n_steps):
            for l in range(L):
                if fused:
                    backend.run_decode_append(out[s, l], qs[s, l], cache.slabs(l), ks[s, l],
                                              vs[s, l], pos)
                else:
                    cache.append(l, ks[s, l], vs[s, l], 1, pos)
                    backend.run(out[s, l], qs[s, l], cache.view(l), 1, pos)
            R.advance_position(pos, 1)
        R.advance_position(pos, -n_steps)   # replays are idempotent

    # Exactly args.steps timed steps (and args.warmup untimed ones): full
    # 128-step graphs plus one graph of the remainder.
    steps = max(1, args.steps)
    step_bytes = [sum(decode_bytes(ctx0 + s, hq, hkv, d) for _ in range(L))
                  for s in range(GRAPH_STEPS)]
    full, rem = divmod(steps, GRAPH_STEPS)
    total_bytes = full * sum(step_bytes) + sum(step_bytes[:rem])
    w_full, w_rem = divmod(max(0, args.warmup), GRAPH_STEPS)
    timed = {}
    for fused in (False, True):
        graphs = {}
        for n in {GRAPH_STEPS, rem, w_rem} - {0}:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                run_steps(fused, n)
            graphs[n] = g
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for _ in range(w_full):
                graphs[GRAPH_STEPS].replay()
            if w_rem:
                graphs[w_rem].replay()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            with EventTimer(torch, stream) as t:
                for _ in range(full):
                    graphs[GRAPH_STEPS].replay()
                if rem:
                    graphs[rem].replay()
        torch.cuda.synchronize()
        timed[fused] = t.ms
        del graphs
    ms_per_step = timed[True] / steps
    value_gbs = total_bytes / (timed[True] * 1e-3) / 1e9
    unfused_gbs = total_bytes / (timed[False] * 1e-3) / 1e9

    # Dominant kernels alone: the headline step's call (the fused K/V append +
    # split kernel, then the merge kernel) once per layer, rotating over the
    # 28 layers (defeats the 256 MB Infinity Cache), captured back to back in
    # a graph and timed with HIP events on its stream. Every call appends at
    # row `depth` (rewritten each time) and attends to depth + 1 keys.
    n_launch = L * 20
    kgraph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        pos.fill_(depth)
        torch.cuda.synchronize()
        with torch.cuda.graph(kgraph, stream=stream):
            for i in range(n_launch):
                l = i % L
                backend.run_decode_append(out[0, l], qs[0, l], cache.slabs(l), ks[0, l],
                                          vs[0, l], pos)
        kgraph.replay()
        torch.cuda.synchronize()
        with EventTimer(torch, stream) as tk:
            kgraph.replay()
    torch.cuda.synchronize()
    kern_us = tk.ms * 1e3 / n_launch
    kbytes = decode_bytes(depth + 1, hq, hkv, d) + append_bytes(hkv, d)
    achieved = kbytes / (kern_us * 1e-6) / 1e9

    # The same steps with RoPE in them (the engine's per-layer sequence
    # rope -> append -> run): the fused RoPE entry (2 launches per layer),
    # rope_bf16 + the fused append/decode (3), and the reference's order
    # rope_bf16 + append + run (4). One 128-step graph each, replayed twice
    # after one warmup replay. Measured after the kernel loop above and on
    # copies of q and k, which the unfused orders rotate (and normalize) in
    # place.
    inv = (5e5 ** (-torch.arange(0, d, 2, dtype=torch.float64, device=dev) / d)).float()
    qg = torch.randn((d,), generator=gen, device=dev).to(torch.bfloat16)
    kg = torch.randn((d,), generator=gen, device=dev).to(torch.bfloat16)
    eps = 1e-6
    torch.cuda.synchronize()

    with torch.cuda.stream(stream):
        qs_r, ks_r = qs.clone(), ks.clone()
    torch.cuda.synchronize()

    def run_rope_steps(mode, n_steps):
        for s in range(n_steps):
            for l in range(L):
                q, k, v, o, view = qs_r[s, l], ks_r[s, l], vs[s, l], out[s, l], cache.slabs(l)
                if mode == "fused":
                    backend.run_decode_rope_append(o, q, view, k, v, pos, inv, pos)
                elif mode == "rope+fused":
                    R.rope_bf16(q, k, pos, inv, 1, hq, hkv, d)
                    backend.run_decode_append(o, q, view, k, v, pos)
                elif mode == "qwen_fused":
                    backend.run_decode_qk_norm_rope_append(o, q, view, k, v, qg, kg, eps, pos,
                                                           inv, pos)
                elif mode == "qwen_three":
                    R.qk_norm_rope_append_fp8(q, view.k, view.v, view.k_scale, view.v_scale, k,
                                              v, qg, kg, eps, pos, inv, pos, 1, hq, hkv, d)
                    backend.run(o, q, view, 1, pos)
                elif mode == "qwen_reference":
                    R.rmsnorm_bf16(q, q, qg, hq, d, eps)
                    R.rmsnorm_bf16(k, k, kg, hkv, d, eps)
                    R.rope_bf16(q, k, pos, inv, 1, hq, hkv, d)
                    cache.append(l, k, v, 1, pos)
                    backend.run(o, q, view, 1, pos)
                else:
                    R.rope_bf16(q, k, pos, inv, 1, hq, hkv, d)
                    cache.append(l, k, v, 1, pos)
                    backend.run(o, q, view, 1, pos)
            R.advance_position(pos, 1)
        R.advance_position(pos, -n_steps)

    rope_ms = {}
    for mode in ("fused", "rope+fused", "reference", "qwen_fused", "qwen_three",
                 "qwen_reference"):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            run_rope_steps(mode, GRAPH_STEPS)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            g.replay()
            torch.cuda.synchronize()
            with EventTimer(torch, stream) as t:
                g.replay()
                g.replay()
        torch.cuda.synchronize()
        rope_ms[mode] = t.ms / (2 * GRAPH_STEPS)
        del g

    return {
        "value": value_gbs, "ms_per_step": ms_per_step, "steps": steps,
        "unfused_value": unfused_gbs, "unfused_ms_per_step": timed[False] / steps,
        "rope_ms_per_step": rope_ms, "rope_step_bytes": sum(step_bytes) / GRAPH_STEPS,
        "warmup": max(0, args.warmup), "ctx": ctx0, "splits": backend.num_splits,
        "kernel_us": kern_us, "kernel_bytes": kbytes, "kernel_gbs": achieved,
        "cache": cache, "qs": qs, "depth": depth, "hq": hq, "hkv": hkv, "d": d,
        "scale": scale, "out": out, "backend": backend, "pos": pos,
    }


def bench_prefill(torch, R, stream, n=4096, iters=None):
    """Prefill calls timed back to back after ~30 ms of warmup calls (the
    clock settles under the MFMA load), over ~60 ms unless iters is given."""
    hq, hkv, d = 32, 8, 128
    scale = 1.0 / math.sqrt(d)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(4321)
    cache = R.KVCache(1, n, hkv, d, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()   # pos is written on the default stream
    with torch.cuda.stream(stream):
        q = torch.randn((n, hq, d), generator=gen, device=dev).to(torch.bfloat16)
        k = torch.randn((n, hkv, d), generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn((n, hkv, d), generator=gen, device=dev).to(torch.bfloat16)
        out = torch.empty((n, hq, d), dtype=torch.bfloat16, device=dev)
        view = cache.view(0)
        cache.append(0, k, v, n, pos)
        fl = prefill_flops(n, 0, hq, d)
        call_s = fl / 0.9e15                  # ~ one call at 900 TFLOP/s
        warm = max(3, int(0.03 / call_s))
        if iters is None:
            iters = max(5, int(0.06 / call_s))
        for _ in range(warm):
            R.flash_prefill_bf16(out, q, view.k, view.v, view.k_scale, view.v_scale, n, pos,
                                 hq, hkv, d, scale)
        torch.cuda.synchronize()
        with EventTimer(torch, stream) as t:
            for _ in range(iters):
                R.flash_prefill_bf16(out, q, view.k, view.v, view.k_scale, view.v_scale, n,
                                     pos, hq, hkv, d, scale)
    torch.cuda.synchronize()
    us = t.ms * 1e3 / iters
    fl = prefill_flops(n, 0, hq, d)
    tflops = fl / (us * 1e-6) / 1e12
    app_us = graph_us(torch, stream, lambda: cache.append(0, k, v, n, pos), 50)
    app_bytes = n * hkv * d * 4 + n * hkv * d * 2 + n * hkv * 8
    return {"n": n, "us": us, "flops": fl, "tflops": tflops, "append_us": app_us,
            "append_gbs": app_bytes / (app_us * 1e-6) / 1e9}


def bench_rope_append(torch, R, stream, n=4096, iters=20):
    """Config-4 shapes (32Q/8KV, head_dim 128). Llama order: RoPE on q and k
    then the K/V append as two launches (rope_bf16 + append) against the fused
    entry. Qwen3 order: per-head RMSNorm of q and of k, RoPE, append (four
    launches) against the fused entry. Algorithmic bytes of a fused call: q
    read and written, k and v read, E4M3 codes and scales written."""
    hq, hkv, d = 32, 8, 128
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    cache = R.KVCache(1, n, hkv, d, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    positions = torch.arange(n, dtype=torch.int32, device=dev)
    inv = (1e6 ** (-torch.arange(0, d, 2, dtype=torch.float64, device=dev) / d)).float()
    eps = 1e-6
    torch.cuda.synchronize()   # pos, positions, inv are written on the default stream
    with torch.cuda.stream(stream):
        q = torch.randn((n, hq, d), generator=gen, device=dev).to(torch.bfloat16)
        k = torch.randn((n, hkv, d), generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn((n, hkv, d), generator=gen, device=dev).to(torch.bfloat16)
        qn = torch.randn((d,), generator=gen, device=dev).to(torch.bfloat16)
        kn = torch.randn((d,), generator=gen, device=dev).to(torch.bfloat16)

        def llama_two_step():
            R.rope_bf16(q, k, positions, inv, n, hq, hkv, d)
            cache.append(0, k, v, n, pos)

        def llama_fused():
            cache.append_rope(0, q, k, v, n, positions, inv, pos, hq)

        def qwen_unfused():
            R.rmsnorm_bf16(q, q, qn, n * hq, d, eps)
            R.rmsnorm_bf16(k, k, kn, n * hkv, d, eps)
            R.rope_bf16(q, k, positions, inv, n, hq, hkv, d)
            cache.append(0, k, v, n, pos)

        def qwen_fused():
            cache.append_qk_norm_rope(0, q, k, v, n, qn, kn, eps, positions, inv, pos, hq)

    res = {}
    for name, fn in (("two_step_us", llama_two_step), ("fused_us", llama_fused),
                     ("qwen_unfused_us", qwen_unfused), ("qwen_fused_us", qwen_fused)):
        res[name] = round(graph_us(torch, stream, fn, iters), 2)
    fused_bytes = n * hq * d * 4 + n * hkv * d * 4 + n * hkv * d * 2 + n * hkv * 8
    res.update({"n": n, "fused_bytes": fused_bytes,
                "fused_gbs": round(fused_bytes / (res["fused_us"] * 1e-6) / 1e9, 1),
                "qwen_fused_gbs": round(fused_bytes / (res["qwen_fused_us"] * 1e-6) / 1e9, 1)})
    return res


def bench_few_token_prefill(torch, R, stream, iters=10):
    """A causal prefill call of a few tokens after a long cache (32Q/8KV,
    head_dim 128): the flash prefill kernel (rth_attn_prefill, one workgroup
    per q tile walking every key, as the reference's) against
    AdaptiveAttention.run, which routes 2..256 tokens to the split-K prefill
    over its scratch (rth_attn_prefill_split)."""
    hq, hkv, d = 32, 8, 128
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    res = []
    be = R.AdaptiveAttention(R.AttnConfig.for_heads(hq, hkv, d))
    for clen in (8192, 32768):
        total = clen + 512
        cache = R.KVCache(1, total, hkv, d, device=dev)
        p0 = torch.zeros(1, dtype=torch.int32, device=dev)
        cl = torch.full((1,), clen, dtype=torch.int32, device=dev)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            k = torch.randn((total, hkv, d), generator=gen, device=dev).to(torch.bfloat16)
            v = torch.randn((total, hkv, d), generator=gen, device=dev).to(torch.bfloat16)
            cache.append(0, k, v, total, p0)
            view = cache.view(0)
            for n in (4, 16, 128, 256):
                q = torch.randn((n, hq, d), generator=gen, device=dev).to(torch.bfloat16)
                out = torch.empty_like(q)

                def flash():
                    R.flash_prefill_bf16(out, q, view.k, view.v, view.k_scale, view.v_scale, n,
                                         cl, hq, hkv, d, d ** -0.5)

                def adaptive():
                    be.run(out, q, view, n, cl)
                fu = graph_us(torch, stream, flash, iters)
                au = graph_us(torch, stream, adaptive, iters)
                res.append({"clen": clen, "n_new": n, "flash_prefill_us": round(fu, 2),
                            "adaptive_split_us": round(au, 2), "speedup": round(fu / au, 1)})
            # A chunk beyond the backend's routes through the entry itself:
            # the flash prefill over key runs, about two rounds of workgroups.
            cus = torch.cuda.get_device_properties(dev).multi_processor_count
            for n in (512,):
                q = torch.randn((n, hq, d), generator=gen, device=dev).to(torch.bfloat16)
                out = torch.empty_like(q)
                splits = max(1, min(16, 2 * cus // (((n + 127) // 128) * hq)))
                part = R.new_flash_split_scratch(n * hq, d, splits, device=dev)

                def flash():
                    R.flash_prefill_bf16(out, q, view.k, view.v, view.k_scale, view.v_scale, n,
                                         cl, hq, hkv, d, d ** -0.5)

                def keysplit():
                    R.flash_prefill_split_bf16(out, q, view.k, view.v, view.k_scale,
                                               view.v_scale, part, splits, n, cl, hq, hkv, d,
                                               d ** -0.5)
                fu = graph_us(torch, stream, flash, iters)
                su = graph_us(torch, stream, keysplit, iters)
                res.append({"clen": clen, "n_new": n, "flash_prefill_us": round(fu, 2),
                            "entry_key_runs_us": round(su, 2), "splits": splits,
                            "speedup": round(fu / su, 1)})
        del cache
    return res


def decode_kernel_sweep(torch, R, stream, points, quiet=False):
    """Per-call decode time of the headline step's call (the fused one-token
    K/V append + split kernel, then the merge kernel) at several context
    depths, rotating over enough layers that the working set exceeds the
    256 MB Infinity Cache; every call appends at row ctx - 1 (rewritten each
    time) and attends to ctx keys. points: (hq, hkv, ctx, splits or None)."""
    res = []
    d = 128
    dev = torch.device("cuda:0")
    for hq, hkv, ctx, splits in points:
        per_layer = ctx * hkv * d * 2 + ctx * hkv * 8
        L = max(2, min(28, math.ceil(600e6 / per_layer)))
        cache = R.KVCache(L, ctx, hkv, d, device=dev)
        cache.k.random_(0, 126)
        cache.v.random_(0, 126)
        cache.k_scale.uniform_(0.001, 0.01)
        cache.v_scale.uniform_(0.001, 0.01)
        backend = R.AdaptiveAttention(R.AttnConfig(hq, hkv, d, 1.0 / math.sqrt(d)),
                                      num_splits=splits)
        q = torch.randn((L, hq, d), device=dev).to(torch.bfloat16)
        kn = torch.randn((L, hkv, d), device=dev).to(torch.bfloat16)
        out = torch.empty((L, hq, d), dtype=torch.bfloat16, device=dev)
        pos = torch.full((1,), ctx - 1, dtype=torch.int32, device=dev)
        n = L * max(2, math.ceil(200 / L))
        torch.cuda.synchronize()   # the fills above run on the default stream
        with torch.cuda.stream(stream):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for i in range(n):
                    backend.run_decode_append(out[i % L], q[i % L], cache.slabs(i % L),
                                              kn[i % L], kn[i % L], pos)
            g.replay()
            torch.cuda.synchronize()
            with EventTimer(torch, stream) as t:
                g.replay()
        torch.cuda.synchronize()
        us = t.ms * 1e3 / n
        nbytes = decode_bytes(ctx, hq, hkv, d) + append_bytes(hkv, d)
        res.append({"hq": hq, "hkv": hkv, "ctx": ctx, "splits": backend.num_splits,
                    "layers": L, "us": round(us, 2), "gbs": round(nbytes / us / 1e3, 1),
                    "frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4)})
        if not quiet:
            print(json.dumps({"decode_sweep": res[-1]}), flush=True)
        del cache, backend, q, kn, out
        torch.cuda.empty_cache()
    return res


def prefill_sweep(torch, R, stream, ns):
    out = []
    for n in ns:
        pf = bench_prefill(torch, R, stream, n=n)
        out.append({"n": n, "us": round(pf["us"], 1), "tflops": round(pf["tflops"], 1),
                    "frac": round(pf["tflops"] / PEAK_BF16_TFLOPS, 4)})
        print(json.dumps({"prefill_sweep": out[-1]}), flush=True)
        torch.cuda.empty_cache()
    return out


COPY_BYTES = 256 << 20


def copy_calibration(torch, stream):
    """Plain device copy of COPY_BYTES (read COPY_BYTES, write COPY_BYTES), the
    reference for scaling FETCH_SIZE / WRITE_SIZE counter readings."""
    a = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda:0").random_()
    b = torch.empty_like(a)
    with torch.cuda.stream(stream):
        for _ in range(5):
            b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "launches": 5}), flush=True)
    return 0


def eager_kernels(torch, R, stream, args):
    """The bench's kernels launched eagerly (no graph) so a profiler attributes
    counters per dispatch: 56 decode calls at ctx args.ctx rotating over 28
    layers (args.hq q heads / 8 kv heads, args.splits splits), 28 one-token
    appends, and 3 prefill calls at 4096."""
    hq, hkv, d, L = args.hq, 8, 128, 28
    ctx = args.ctx
    dev = torch.device("cuda:0")
    cache = R.KVCache(L, ctx, hkv, d, device=dev)
    cache.k.random_(0, 126)
    cache.v.random_(0, 126)
    cache.k_scale.uniform_(0.001, 0.01)
    cache.v_scale.uniform_(0.001, 0.01)
    backend = R.AdaptiveAttention(R.AttnConfig(hq, hkv, d, 1.0 / math.sqrt(d)),
                                  num_splits=args.splits)
    q = torch.randn((L, hq, d), device=dev).to(torch.bfloat16)
    kn = torch.randn((L, hkv, d), device=dev).to(torch.bfloat16)
    out = torch.empty((L, hq, d), dtype=torch.bfloat16, device=dev)
    pos = torch.full((1,), ctx - 1, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()   # the fills above run on the default stream
    with torch.cuda.stream(stream):
        for i in range(2 * L):
            l = i % L
            if args.fused:
                backend.run_decode_append(out[l], q[l], cache.slabs(l), kn[l], kn[l], pos)
                continue
            if i < L:
                cache.append(l, kn[l], kn[l], 1, pos)
            backend.run(out[l], q[l], cache.view(l), 1, pos)
    torch.cuda.synchronize()
    del cache
    bench_prefill(torch, R, stream, n=args.prefill_n, iters=3)
    print(json.dumps({"eager_kernels": "done", "ctx": ctx}), flush=True)
    return 0


def profile_traffic(name="decode_attn_8k_pmc_traffic.md"):
    """HBM bytes per decode call from a committed PMC summary, if present."""
    f = ROOT / "profiles" / name
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("hbm_bytes_per_decode_call:"):
            return int(float(line.split(":", 1)[1]))
    return None


def host_cores():
    """Threads for the CPU baselines: every core this process may run on (the
    affinity mask), capped by a cgroup CPU quota when one is set; plus the
    machine's CPU count (nproc) for the record."""
    nproc = os.cpu_count() or 1
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = nproc
    quota = None
    try:
        q, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            quota = max(1, int(int(q) // int(period)))
    except (OSError, ValueError):
        pass
    cores = min(usable, quota) if quota else usable
    return max(1, cores), nproc, quota


def cpu_baseline(torch, dec, budget_s=10.0):
    """The oracle (C restatement of the reference's naive fp32 attention,
    reference src/kernels/attention.cu:34-91) on host threads: the same decode
    (ctx, 24Q/8KV, same FP8 cache bytes and queries) cycling over the 28
    layers until about budget_s seconds of CPU time are spent."""
    sys.path.insert(0, str(ROOT / "tests"))
    import numpy as np
    import oracle_lib as O

    usable, nproc, quota = host_cores()
    hq, hkv, d, depth = dec["hq"], dec["hkv"], dec["d"], dec["depth"]
    # the oracle runs one thread per (token, q head) row at most, 256 at most
    cores = min(usable, hq, 256)
    cache = dec["cache"]
    keys = depth + 1
    host = []
    for layer in range(28):
        view = cache.view(layer)
        host.append((dec["qs"][0, layer].view(torch.int16).cpu().numpy().view(np.uint16),
                     view.k[:keys].cpu().numpy().reshape(-1, d),
                     view.v[:keys].cpu().numpy().reshape(-1, d),
                     view.k_scale[:keys].cpu().numpy().reshape(-1),
                     view.v_scale[:keys].cpu().numpy().reshape(-1)))
    calls, t_total = 0, 0.0
    while t_total < budget_s and calls < 28 * 400:
        q, k8, v8, ks, vs = host[calls % 28]
        t0 = time.perf_counter()
        O.attention_f32(q, k8, v8, ks, vs, 1, depth, hq, hkv, d, np.float32(dec["scale"]), cores)
        t_total += time.perf_counter() - t0
        calls += 1
    nbytes = calls * decode_bytes(keys, hq, hkv, d)
    return {"value": round(nbytes / t_total / 1e9, 3), "unit": "GB/s", "cores": cores,
            "usable_cores": usable, "nproc": nproc, "cgroup_cpu_quota": quota, "kind": "port",
            "sample": f"{calls} decode calls (cycling the 28 layers) at ctx {keys}, 24Q/8KV, "
                      f"fp32 two-pass naive attention over the same FP8 cache bytes and queries, "
                      f"{t_total:.1f} s on {cores} threads"}


def cpu_prefill_baseline(budget_s=6.0):
    """The oracle's naive fp32 causal attention (reference
    src/kernels/attention.cu:34-91) on config 2's shape (n=1021, 24Q/8KV,
    head_dim 128, FP8 cache from the oracle's quantizer) on host threads,
    repeated for about budget_s seconds; GFLOP/s in the algorithmic units of
    the GPU prefill figure."""
    sys.path.insert(0, str(ROOT / "tests"))
    import numpy as np
    import oracle_lib as O

    usable, nproc, quota = host_cores()
    n, hq, hkv, d = 1021, 24, 8, 128
    cores = min(usable, n * hq, 256)
    q = O.normal_bf16((n, hq, d), 71)
    k8, ks = O.quantize_kv_fp8(O.normal_bf16((n * hkv, d), 72), d)
    v8, vs = O.quantize_kv_fp8(O.normal_bf16((n * hkv, d), 73), d)
    scale = np.float32(1.0 / math.sqrt(d))
    calls, t_total = 0, 0.0
    while t_total < budget_s and calls < 200:
        t0 = time.perf_counter()
        O.attention_f32(q, k8, v8, ks, vs, n, 0, hq, hkv, d, scale, cores)
        t_total += time.perf_counter() - t0
        calls += 1
    fl = calls * prefill_flops(n, 0, hq, d)
    return {"value": round(fl / t_total / 1e9, 2), "unit": "GFLOP/s", "cores": cores,
            "usable_cores": usable, "nproc": nproc, "cgroup_cpu_quota": quota, "kind": "port", "ms_per_call": round(1e3 * t_total / calls, 1),
            "sample": f"{calls} calls of config 2 (n=1021, 24Q/8KV, causal, clen 0), fp32 "
                      f"two-pass naive attention over the FP8 cache, {t_total:.1f} s on "
                      f"{cores} threads"}


def extra_rooflines(torch, R, stream):
    """The north star's target ranges beyond the headline points, each with
    its roofline: decode per call at ctx 32768 (config 3, 24Q/8KV, default
    splits) and 131072 (config 5, 32Q/8KV, the config's 64 splits; per-head
    scales do not change the work), prefill at 8192 and 16384 (config 4)."""
    out = []
    for hq, hkv, ctx, splits, cfg in ((24, 8, 32768, None, "config3"),
                                      (32, 8, 131072, 64, "config5"),
                                      (32, 8, 131072, None, "config5 default splits")):
        pt = decode_kernel_sweep(torch, R, stream, [(hq, hkv, ctx, splits)], quiet=True)[0]
        out.append({"kind": "decode", "workload": f"{cfg}: fused one-token append + decode "
                                                  f"{hq}Q/{hkv}KV ctx {ctx}, {pt['splits']} splits",
                    "us": pt["us"],
                    "roofline": {"bound": "hbm", "achieved": pt["gbs"], "peak": PEAK_HBM_GBS,
                                 "unit": "GB/s", "frac": pt["frac"],
                                 "bytes_per_launch": decode_bytes(ctx, hq, hkv, 128)
                                 + append_bytes(hkv, 128),
                                 "traffic": (profile_traffic("decode_attn_128k_pmc_traffic.md")
                                             if (ctx == 131072 and splits == 64) else None)}})
    for n in (8192, 16384):
        pf = bench_prefill(torch, R, stream, n=n)
        out.append({"kind": "prefill", "workload": f"config4: prefill 32Q/8KV n={n}, clen 0",
                    "us": round(pf["us"], 1),
                    "roofline": {"bound": "mfma", "achieved": round(pf["tflops"], 1),
                                 "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(pf["tflops"] / PEAK_BF16_TFLOPS, 4),
                                 "flops_per_launch": pf["flops"]}})
        torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--ctx", type=int, default=8196)
    ap.add_argument("--prefill-n", type=int, default=4096)
    ap.add_argument("--hq", type=int, default=24, help="--mode kernels: q heads of the decode")
    ap.add_argument("--splits", type=int, default=None,
                    help="--mode kernels: decode split count (default: the backend's)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--fused", action="store_true",
                    help="--mode kernels: decode calls through the fused append + decode entry "
                         "(the headline step's call) instead of append then run")
    ap.add_argument("--decode-kernel", choices=("auto", "valu"), default="auto",
                    help="valu: run every decode call on the VALU split kernel (A/B against "
                         "the MFMA kernel with --mode kernels or --sweep decode)")
    ap.add_argument("--sweep", nargs="?", const="all", choices=("all", "decode", "prefill", "few"),
                    help="per-call decode and/or prefill sweeps over the BASELINE depths; few: "
                         "the few-token prefill comparison alone")
    ap.add_argument("--mode", choices=("full", "kernels", "copy"), default="full",
                    help="kernels: eager launches of the bench kernels only (for "
                         "rocprofv3 --pmc); copy: a 256 MiB device copy (PMC "
                         "calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (the attention hot path is single-GPU); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2

    import torch
    import runtherder_amd as R

    R._ffi.load()
    if args.decode_kernel == "valu":
        R.set_decode_kernel(R.DECODE_VALU)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    if args.mode == "copy":
        return copy_calibration(torch, stream)
    if args.mode == "kernels":
        return eager_kernels(torch, R, stream, args)
    if args.sweep == "few":
        for p in bench_few_token_prefill(torch, R, stream):
            print(json.dumps({"prefill_after_long_cache": p}), flush=True)
        return 0
    if args.sweep:
        if args.sweep != "prefill":
            decode_kernel_sweep(torch, R, stream, [(24, 8, 35, None), (24, 8, 2041, None),
                                                   (24, 8, 8196, None), (24, 8, 32768, None),
                                                   (32, 8, 131072, None), (32, 8, 131072, 64)])
        if args.sweep != "decode":
            prefill_sweep(torch, R, stream, [1021, 2048, 4096, 8192, 16384])
        return 0
    dec = bench_decode(torch, R, args, stream)
    pf = bench_prefill(torch, R, stream, n=args.prefill_n)
    ra = bench_rope_append(torch, R, stream, n=args.prefill_n)
    few = bench_few_token_prefill(torch, R, stream)
    extra = extra_rooflines(torch, R, stream)
    cpu = None if args.no_cpu else cpu_baseline(torch, dec)
    cpu_pf = None if args.no_cpu else cpu_prefill_baseline()

    line = {
        "metric": "decode attn HBM GB/s (% peak) @8K ctx; prefill attn TFLOP/s @4K tok",
        "value": round(dec["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": dec["steps"],
        "warmup": dec["warmup"],
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3-kv/decode-bf16-mfma/prefill-fp8(qk,two-part-e4m3-q-split:exact>=2^-14-of-row-max)+f16(pv)-mfma/fp32-acc",
        "data": "synthetic: N(0,1) bf16 q/k/v, k/v quantized to FP8 E4M3 by the append kernel",
        "config": {
            "workload": "config3: 28-layer Llama-3.2-3B-shaped decode attention, 24Q/8KV, "
                        "head_dim 128, ctx 8196..8323, per layer one-token K/V append + "
                        "split-K decode through the fused append+decode entry (2 kernels), "
                        "128 steps per HIP graph",
            "ctx": dec["ctx"], "layers": 28, "num_splits": dec["splits"],
            "parallelism": "single GPU",
        },
        "percent_of_peak": round(100.0 * dec["value"] / PEAK_HBM_GBS, 2),
        "roofline": {
            "bound": "hbm", "achieved": round(dec["kernel_gbs"], 1), "peak": PEAK_HBM_GBS,
            "unit": "GB/s", "frac": round(dec["kernel_gbs"] / PEAK_HBM_GBS, 4),
            "traffic": profile_traffic(),
            "kernel": "flash_decode_kernel<128, true, false> + flash_decode_combine_kernel<128> (one fused append + decode call)",
            "kernel_us": round(dec["kernel_us"], 3), "bytes_per_launch": dec["kernel_bytes"],
        },
        "prefill": {
            "metric": "prefill attn TFLOP/s @4K tok",
            "workload": f"config4: 32Q/8KV head_dim 128 causal prefill, n={pf['n']}, clen 0",
            "value": round(pf["tflops"], 1), "unit": "TFLOP/s", "us": round(pf["us"], 1),
            "roofline": {"bound": "mfma", "achieved": round(pf["tflops"], 1),
                         "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pf["tflops"] / PEAK_BF16_TFLOPS, 4),
                         "flops_per_launch": pf["flops"]},
            "append_us": round(pf["append_us"], 2), "append_gbs": round(pf["append_gbs"], 1),
            "cpu_baseline": cpu_pf,
        },
        "target_range": extra,
        "rope_append": dict(ra, workload="config4 shapes: RoPE(q,k) + K/V FP8 append (and the "
                                         "Qwen3 q/k RMSNorm before it), fused entries vs the "
                                         "unfused launch sequences"),
        "prefill_after_long_cache": {
            "unit": "us per call", "points": few,
            "workload": "32Q/8KV head_dim 128: n_new = 4 / 16 / 128 / 256 / 512 tokens after 8192 / 32768 "
                        "cached keys; the flash prefill kernel vs AdaptiveAttention.run "
                        "(split-K decode over (token block, kv head) units for 2..80 tokens, the "
                        "flash prefill over key runs for 81..256); 512 tokens through "
                        "rth_attn_prefill_split (key runs, ~2 rounds of workgroups)"},
        "decode_step_unfused": {
            "value": round(dec["unfused_value"], 1), "unit": "GB/s",
            "ms_per_step": round(dec["unfused_ms_per_step"], 4),
            "workload": "the same steps as KVCache.append then AdaptiveAttention.run (3 kernels "
                        "per layer, the reference's call sequence)",
        },
        "decode_step_rope": {
            "unit": "ms/step (28 layers)",
            "fused": round(dec["rope_ms_per_step"]["fused"], 4),
            "rope_then_fused_append_decode": round(dec["rope_ms_per_step"]["rope+fused"], 4),
            "reference_order": round(dec["rope_ms_per_step"]["reference"], 4),
            "fused_gbs": round(dec["rope_step_bytes"] / (dec["rope_ms_per_step"]["fused"] * 1e-3)
                               / 1e9, 1),
            "workload": "the decode steps with RoPE (theta 5e5) of q and the new k: "
                        "rth_attn_decode_rope_append_split (2 kernels per layer) vs rope_bf16 + "
                        "the fused append/decode (3) vs rope_bf16 + append + run (4, the "
                        "reference's order); 128-step graphs",
        },
        "decode_step_qk_norm_rope": {
            "unit": "ms/step (28 layers)",
            "fused": round(dec["rope_ms_per_step"]["qwen_fused"], 4),
            "qk_norm_rope_append_then_run": round(dec["rope_ms_per_step"]["qwen_three"], 4),
            "reference_order": round(dec["rope_ms_per_step"]["qwen_reference"], 4),
            "workload": "the same steps in Qwen3's order (per-head RMSNorm of q and k, RoPE, "
                        "append, run; qwen3.cu:189-202): "
                        "rth_attn_decode_qk_norm_rope_append_split (2 kernels per layer) vs "
                        "rth_qk_norm_rope_append_fp8 + run (3) vs rmsnorm x2 + rope + append + "
                        "run (6); 24Q/8KV head shape as above",
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
