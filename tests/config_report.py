"""Per-configuration report for BASELINE.md's results table (run on the
MI355X box: `python tests/config_report.py`). Test infrastructure: the oracle
(CPU restatement of the reference's attention and quantizer) times the CPU
column and checks parity; the GPU column times the HIP path through the C ABI
(HIP events around graph replays or back-to-back calls). For the large
prefills the CPU time is measured on a block of rows and scaled by the
causal pair count, and parity is checked on the heaviest 256 rows."""
from __future__ import annotations

import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import oracle_lib as O  # noqa: E402
import runtherder_amd as R  # noqa: E402

DEV = "cuda:0"


def usable_cores():
    """Every core this process may run on (the affinity mask), capped by a
    cgroup CPU quota when one is set, and by the oracle's 256-thread limit."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    try:
        q, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            n = min(n, max(1, int(q) // int(period)))
    except (OSError, ValueError):
        pass
    return max(1, min(n, 256))


THREADS = usable_cores()
PEAK_HBM, PEAK_MFMA = 8000.0, 2500.0


def bf(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(
        torch.bfloat16).to(DEV)


def u8(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(DEV)


def f32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV)


def ival(x):
    return torch.tensor([x], dtype=torch.int32, device=DEV)


def hostbf(t):
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def gpu_us(fn, iters=50, graph=True):
    # The side stream must not start before the default stream's pending work
    # (cache fills, position writes) has finished.
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        fn()
        torch.cuda.synchronize()
        if graph:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for _ in range(iters):
                    fn()
            g.replay()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(s)
            g.replay()
            b.record(s)
        else:
            for _ in range(3):
                fn()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(s)
            for _ in range(iters):
                fn()
            b.record(s)
    b.synchronize()
    return a.elapsed_time(b) * 1e3 / iters


def cpu_ms(fn, reps=3):
    best = math.inf
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
    return best * 1e3


def dec_bytes(ctx, hq, hkv, d):
    return ctx * hkv * d * 2 + ctx * hkv * 8 + hq * d * 4


def pf_flops(n, clen, hq, d):
    return 4 * hq * d * (n * clen + n * (n + 1) // 2)


def err(got, want):
    mx, mean = O.bf16_err(got, want)
    return f"{mx:.1e} / {mean:.1e}"


rows = []


def decode_case(name, ctx, hq, hkv, d, splits, per_head=False, per_tensor=False, layers=1):
    scale = np.float32(1.0 / np.sqrt(d))
    q = O.normal_bf16((hq, d), 11)
    kx = O.normal_bf16((ctx * hkv, d), 12)
    vx = O.normal_bf16((ctx * hkv, d), 13)
    if per_tensor:
        kt = np.float32(np.abs(O.bf16_to_f32(kx)).max()) / np.float32(448)
        vt = np.float32(np.abs(O.bf16_to_f32(vx)).max()) / np.float32(448)
        ks, vs = np.full(ctx * hkv, kt, np.float32), np.full(ctx * hkv, vt, np.float32)
    elif per_head:
        ks = np.tile(O.uniform_f32(hkv, 0.01, 0.1, 52), ctx).astype(np.float32)
        vs = np.tile(O.uniform_f32(hkv, 0.01, 0.1, 53), ctx).astype(np.float32)
    if per_tensor or per_head:
        k8, v8 = O.quantize_kv_fp8_scaled(kx, ks, d), O.quantize_kv_fp8_scaled(vx, vs, d)
    else:
        k8, ks = O.quantize_kv_fp8(kx, d)
        v8, vs = O.quantize_kv_fp8(vx, d)
    splits = splits or R.default_num_splits(hkv)
    out = torch.empty((hq, d), dtype=torch.bfloat16, device=DEV)
    part = R.new_flash_split_scratch(hq, d, splits)
    tq, tk, tv, tks, tvs, pos = bf(q), u8(k8), u8(v8), f32(ks), f32(vs), ival(ctx - 1)
    call = lambda: R.flash_decode_split_bf16(out, tq, tk, tv, tks, tvs, part, splits, pos, hq,
                                             hkv, d, scale)
    us = gpu_us(call, iters=100)
    torch.cuda.synchronize()
    want = O.attention_f32(q, k8, v8, ks, vs, 1, ctx - 1, hq, hkv, d, scale, THREADS)
    c_ms = cpu_ms(lambda: O.attention_f32(q, k8, v8, ks, vs, 1, ctx - 1, hq, hkv, d, scale,
                                          THREADS))
    nb = dec_bytes(ctx, hq, hkv, d) * layers
    rows.append({"config": name, "cpu_ms": c_ms * layers, "cpu_rate": nb / (c_ms * layers) / 1e6,
                 "gpu_us": us * layers, "gpu_rate": nb / (us * layers) / 1e3,
                 "frac": nb / (us * layers) / 1e3 / PEAK_HBM, "unit": "GB/s",
                 "parity": err(hostbf(out), want[0]) + (f", {splits} splits" if splits else "")})
    print(json.dumps(rows[-1]), flush=True)


def prefill_case(name, n, clen, hq, hkv, d, rope_llama3=None, block=256):
    scale = np.float32(1.0 / np.sqrt(d))
    total = clen + n
    q = O.normal_bf16((n, hq, d), 21)
    k = O.normal_bf16((n, hkv, d), 22)
    v = O.normal_bf16((n, hkv, d), 23)
    if rope_llama3:
        inv = O.rope_inv_freq_llama3(d, 5e5, 32.0, 1.0, 4.0, 8192)
        pos = np.arange(clen, total, dtype=np.int32)
        q, k = O.rope_apply_bf16(q, pos, inv), O.rope_apply_bf16(k, pos, inv)
    cache = R.KVCache(1, total, hkv, d, device=DEV)
    view = cache.view(0)
    if clen:
        hk = O.normal_bf16((clen * hkv, d), 24)
        hv = O.normal_bf16((clen * hkv, d), 25)
        pks = np.tile(O.uniform_f32(hkv, 0.01, 0.1, 26), clen).astype(np.float32)
        pvs = np.tile(O.uniform_f32(hkv, 0.01, 0.1, 27), clen).astype(np.float32)
        R.quantize_kv_fp8_scaled(view.k.view(-1, d)[: clen * hkv], f32(pks), bf(hk), ival(0), 1,
                                 clen * hkv, d)
        R.quantize_kv_fp8_scaled(view.v.view(-1, d)[: clen * hkv], f32(pvs), bf(hv), ival(0), 1,
                                 clen * hkv, d)
        view.k_scale.view(-1)[: clen * hkv].copy_(torch.from_numpy(pks))
        view.v_scale.view(-1)[: clen * hkv].copy_(torch.from_numpy(pvs))
    tq, tk, tv, p0 = bf(q), bf(k), bf(v), ival(clen)
    out = torch.empty((n, hq, d), dtype=torch.bfloat16, device=DEV)
    app = lambda: cache.append(0, tk, tv, n, p0)
    pf = lambda: R.flash_prefill_bf16(out, tq, view.k, view.v, view.k_scale, view.v_scale, n, p0,
                                      hq, hkv, d, scale)
    app()
    pf()
    torch.cuda.synchronize()
    k8, v8 = view.k.cpu().numpy().reshape(-1, d), view.v.cpu().numpy().reshape(-1, d)
    ks, vs = view.k_scale.cpu().numpy().reshape(-1), view.v_scale.cpu().numpy().reshape(-1)
    wk, wks = O.quantize_kv_fp8(k, d)
    bytes_ok = np.array_equal(k8[clen * hkv:], wk) and np.array_equal(
        ks[clen * hkv:].view(np.uint32), wks.view(np.uint32))
    fl = pf_flops(n, clen, hq, d)
    pf_us = gpu_us(pf, iters=max(5, int(0.05 / (fl / 0.9e15))), graph=False)
    app_us = gpu_us(app, iters=20)
    got = hostbf(out)
    r0 = max(0, n - block)
    want = O.attention_f32(q[r0:], k8, v8, ks, vs, n - r0, clen + r0, hq, hkv, d, scale, THREADS)
    # CPU: the oracle on rows r0..n-1 (plus the quantizer), scaled by the
    # causal pair count of the whole call.
    c_blk = cpu_ms(lambda: O.attention_f32(q[r0:], k8, v8, ks, vs, n - r0, clen + r0, hq, hkv, d,
                                           scale, THREADS), reps=1)
    c_q = cpu_ms(lambda: (O.quantize_kv_fp8(k, d), O.quantize_kv_fp8(v, d)), reps=1)
    blk_pairs = (n - r0) * (clen + r0) + ((n - r0) * (n - r0 + 1)) // 2 + (n - r0) * 0
    scale_f = (n * clen + n * (n + 1) // 2) / blk_pairs
    c_ms = c_blk * scale_f + c_q
    rows.append({"config": name, "cpu_ms": c_ms, "cpu_rate": fl / (c_ms * 1e-3) / 1e9,
                 "gpu_us": app_us + pf_us, "prefill_us": pf_us, "append_us": app_us,
                 "gpu_rate": fl / (pf_us * 1e-6) / 1e12, "frac": fl / (pf_us * 1e-6) / 1e12 /
                 PEAK_MFMA, "unit": "TFLOP/s (prefill) / GFLOP/s (CPU)",
                 "parity": err(got[r0:], want) + (" (rows %d..%d)" % (r0, n - 1) if r0 else "")
                 + ("; FP8 bytes bit-exact" if bytes_ok else "; FP8 BYTES DIFFER"),
                 "cpu_scaled": r0 > 0})
    print(json.dumps(rows[-1]), flush=True)
    del cache, view
    torch.cuda.empty_cache()


def config3_step(ctx):
    """One decode step of the 28-layer config (fused append + decode per
    layer) from a graph of 16 steps; parity on the last layer of the last
    step."""
    hq, hkv, d, L, steps = 24, 8, 128, 28, 16
    depth = ctx - 1
    scale = np.float32(1.0 / np.sqrt(d))
    cache = R.KVCache(L, depth + steps, hkv, d, device=DEV)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(ctx)
    pos = ival(0)
    for l in range(L):
        for s0 in range(0, depth, 4096):
            m = min(4096, depth - s0)
            pos.fill_(s0)
            cache.append(l, torch.randn((m, hkv, d), generator=gen, device=DEV).to(torch.bfloat16),
                         torch.randn((m, hkv, d), generator=gen, device=DEV).to(torch.bfloat16),
                         m, pos)
    be = R.AdaptiveAttention(R.AttnConfig(hq, hkv, d, float(scale)))
    qs = torch.randn((steps, L, hq, d), generator=gen, device=DEV).to(torch.bfloat16)
    kn = torch.randn((steps, L, hkv, d), generator=gen, device=DEV).to(torch.bfloat16)
    vn = torch.randn((steps, L, hkv, d), generator=gen, device=DEV).to(torch.bfloat16)
    outs = torch.empty((steps, L, hq, d), dtype=torch.bfloat16, device=DEV)

    def run():
        for s in range(steps):
            for l in range(L):
                be.run_decode_append(outs[s, l], qs[s, l], cache.slabs(l), kn[s, l], vn[s, l], pos)
            R.advance_position(pos, 1)
        R.advance_position(pos, -steps)

    pos.fill_(depth)
    us_step = gpu_us(run, iters=4) / steps
    pos.fill_(depth)
    run()
    torch.cuda.synchronize()
    view = cache.view(L - 1)
    keys = depth + steps
    k8, v8 = view.k.cpu().numpy().reshape(-1, d), view.v.cpu().numpy().reshape(-1, d)
    ks, vs = view.k_scale.cpu().numpy().reshape(-1), view.v_scale.cpu().numpy().reshape(-1)
    qh = hostbf(qs[-1, L - 1])
    want = O.attention_f32(qh, k8, v8, ks, vs, 1, keys - 1, hq, hkv, d, scale, THREADS)
    c = cpu_ms(lambda: O.attention_f32(qh, k8, v8, ks, vs, 1, keys - 1, hq, hkv, d, scale,
                                       THREADS))
    nb = L * dec_bytes(ctx, hq, hkv, d)
    rows.append({"config": f"3 @ {ctx} (28-layer step)", "cpu_ms": c * L,
                 "cpu_rate": nb / (c * L) / 1e6, "gpu_us": us_step,
                 "gpu_rate": nb / us_step / 1e3, "frac": nb / us_step / 1e3 / PEAK_HBM,
                 "unit": "GB/s", "parity": err(hostbf(outs[-1, L - 1]), want[0]) +
                 ", last step, layer 27"})
    print(json.dumps(rows[-1]), flush=True)
    del cache
    torch.cuda.empty_cache()


def main():
    R._ffi.load()
    decode_case("1: decode ctx 511", 511, 24, 8, 128, None, per_tensor=True)
    prefill_case("2: prefill 1021 (RoPE llama3)", 1021, 0, 24, 8, 128, rope_llama3=True,
                 block=1021)
    config3_step(8196)
    config3_step(32768)
    prefill_case("4 @ 4096", 4096, 0, 32, 8, 128)
    prefill_case("4 @ 16384", 16384, 0, 32, 8, 128)
    decode_case("5: decode 128K, 64 splits, per-head scales", 131072, 32, 8, 128, 64,
                per_head=True)
    prefill_case("5: chunk 4096 @ 126976", 4096, 126976, 32, 8, 128, block=64)
    lines = [f"| config | CPU ms ({THREADS} threads, nproc {os.cpu_count()}) | CPU rate | GPU us | GPU rate | % of peak | "
             "parity (max / mean abs) |", "|---|---|---|---|---|---|---|"]
    for r in rows:
        dec = r["unit"] == "GB/s"
        cpu_rate = f"{r['cpu_rate']:.2f} GB/s" if dec else f"{r['cpu_rate']:.1f} GFLOP/s"
        gpu_rate = f"{r['gpu_rate']:.0f} GB/s" if dec else f"{r['gpu_rate']:.0f} TFLOP/s"
        gus = f"{r['gpu_us']:.1f}" if dec else (f"{r['prefill_us']:.1f} + {r['append_us']:.1f} "
                                                 f"(append)")
        cms = f"{r['cpu_ms']:.1f}" + (" (scaled)" if r.get("cpu_scaled") else "")
        lines.append(f"| {r['config']} | {cms} | {cpu_rate} | {gus} | {gpu_rate} | "
                     f"{100 * r['frac']:.1f} % | {r['parity']} |")
    md = "\n".join(lines)
    print(md)
    out = ROOT / "gpurun_out"
    out.mkdir(exist_ok=True)
    (out / "config_report.md").write_text(md + "\n")


if __name__ == "__main__":
    main()
