#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

Primary line (the metric's decode half): W4A8 decode projection set of a
Qwen3-4B-shaped layer (qkv 2560x6144, o 4096x2560, fused gate_up 2560x19456 +
SwiGLU -> down 9728x2560), M=1, 36 layers with distinct seeded weights, fp16
activations resident in HBM. value = algorithmic bytes / wall time (GB/s).

Secondary workloads (same JSON line, "secondary"): M=4 decode, the M=4096
W8A8/W4A8 prefill projection set x36 + lm_head (int8 TOPS), the M=512 FFN
block x36, the M=128 W8A8 up projection, the 35B-A3B-class MoE at T=512
and T=1, the attention lines, and the PCIe-inclusive rates of the reference's
host-buffer signatures (decode set and M=128 up projection).

Timing (every workload): the step runs eagerly (host launches between two
synchronizations) and as a HIP graph replay (checked bit-exact against eager
runs) between two HIP events; the faster valid one is used, both are reported.
roofline: the dominant kernel's algorithmic bytes (or ops) per launch over its
average launch time: 36 back-to-back launches of that kernel alone (distinct
layers' weights) captured in a graph and timed with HIP events on the replay
stream.
cpu_baseline: the C oracle (OpenMP) on a bounded sample of the same workload
on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "int8 TOPS (% MFMA peak) at M=512/4096 prefill; HBM GB/s at M=1 decode"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0

# Qwen3-4B layer shapes
H, Q, KV, F, LAYERS, VOCAB = 2560, 4096, 1024, 9728, 36, 151936


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def torch_setup():
    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    return torch


class Gen:
    """Seeded device-side generators (torch's Philox on cuda) per tensor name."""

    def __init__(self, torch, config):
        self.torch = torch
        self.config = config

    def gen(self, name):
        g = self.torch.Generator(device="cuda")
        h = 0x5EED0000 + self.config
        for c in name:
            h = (h * 1000003 + ord(c)) & 0xFFFFFFFFFFFF
        g.manual_seed(h)
        return g

    def codes(self, name, bits, k, n):
        lo, hi = (-8, 8) if bits == 4 else (-127, 128)
        return self.torch.randint(lo, hi, (k, n), dtype=self.torch.int8, device="cuda", generator=self.gen(name))

    def scales(self, name, n):
        return (self.torch.rand(n, device="cuda", generator=self.gen(name + "/s")) * 0.009 + 0.001).float()

    def acts(self, name, rows, k, outliers):
        t = self.torch
        g = self.gen(name)
        x = t.randn(rows, k, device="cuda", generator=g)
        if outliers:
            cols = t.randperm(k, device="cuda", generator=g)[: int(math.ceil(0.005 * k))]
            x[:, cols] *= 20.0
        return x.half()


def lin_bytes(bits, k, n, rows):
    """Algorithmic bytes of one linear: weights at storage width + f32 scales +
    fp16 activations in and out."""
    return k * n * bits // 8 + 4 * n + 2 * rows * (k + n)


def time_steps(torch, step, steps, warmup):
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1000.0 / steps


def best_time(torch, step, steps, warmup, check):
    """Eager launches and a HIP-graph replay of the same step (replays checked
    bit-exact against eager runs); the faster valid one is the step time."""
    ms_eager = time_steps(torch, step, steps, warmup)
    ms_graph, ok = graph_time(torch, step, steps, check)
    return (min(ms_eager, ms_graph) if ok else ms_eager), ms_eager, ms_graph, ok


def graph_time(torch, fn, reps, check=None):
    """Capture fn() into a HIP graph and time `reps` replays between two events
    recorded on the replay stream. check(): called after an eager run and after
    a replay; both results must be identical (graph replay correctness)."""
    eager_ref = None
    fn()
    torch.cuda.synchronize()
    if check is not None:
        eager_ref = check()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            fn()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    ok = True
    if check is not None:
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            got = check()
            ok = ok and all(torch.equal(a, b) for a, b in zip(eager_ref, got))
            fn()  # eager work between replays
            torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    cur = torch.cuda.current_stream()
    e0.record(cur)
    for _ in range(reps):
        g.replay()
    e1.record(cur)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps, ok


# HBM bytes per launch of the dominant decode kernel (gate_up GEMV, M=1), from
# two rocprofv3 counter runs of `bench.py --traffic-probe` (FETCH_SIZE, then
# WRITE_SIZE, KiB per dispatch, median over 108 dispatches), each scaled by
# what the same counter reads for a 268,435,456-byte device copy in the same
# run: FETCH_SIZE 131,090.2 KiB (factor 2.0), WRITE_SIZE 262,144 KiB (factor 1.0).
# Summary and commands: profiles/traffic_gemv_gate_up_m1.txt.
TRAFFIC_GEMV_GATE_UP_M1 = int(round((12431.0 * 2.0 + 81.0625 * 1.0) * 1024))


def roofline(achieved, bound, kernel, avg_us, work, launches, method, traffic=None):
    if bound == "hbm":
        peak, unit = HBM_PEAK_GBS, "GB/s"
    else:
        peak, unit = INT8_PEAK_TOPS, "TFLOP/s"
    return {"bound": bound, "kernel": kernel, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic, "avg_us": round(avg_us, 3),
            "work_per_launch": work, "launches": launches, "method": method}


# ---------------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------------

class DenseLayers:
    """36 layers of qkv / o / gate_up / down weights and shared workspaces."""

    def __init__(self, torch, ctx, gen, rows, bits, layers=LAYERS, outliers=False, tag="dec"):
        from open_rknpu2_lm_infer_amd import device as D
        self.torch, self.ctx, self.rows, self.layers = torch, ctx, rows, layers
        qkv_b, o_b, gu_b, dn_b = bits
        self.w = []
        self.host0 = None
        for l in range(layers):
            mats = {}
            for name, b, k, n in (("qkv", qkv_b, H, Q + 2 * KV), ("o", o_b, Q, H), ("gate_up", gu_b, H, 2 * F),
                                  ("down", dn_b, F, H)):
                codes = gen.codes(f"{tag}/l{l}/{name}", b, k, n)
                scales = gen.scales(f"{tag}/l{l}/{name}", n)
                mats[name] = ctx.weights(b, codes, scales)
                if l == 0:
                    if self.host0 is None:
                        self.host0 = {}
                    self.host0[name] = (b, codes.cpu().numpy(), scales.cpu().numpy())
                del codes, scales
            self.w.append(mats)
        self.x_qkv = gen.acts(f"{tag}/x_qkv", rows, H, outliers)
        self.x_o = gen.acts(f"{tag}/x_o", rows, Q, outliers)
        self.x_ffn = gen.acts(f"{tag}/x_ffn", rows, H, outliers)
        self.y_qkv = torch.empty(rows, Q + 2 * KV, dtype=torch.float16, device="cuda")
        self.y_o = torch.empty(rows, H, dtype=torch.float16, device="cuda")
        self.y_ffn = torch.empty(rows, H, dtype=torch.float16, device="cuda")
        w0 = self.w[0]
        self.ws = {name: ctx.workspace(w0[name].bits, rows, w0[name].k, w0[name].n) for name in w0}
        self.D = D

    def step(self):
        D, ctx, r = self.D, self.ctx, self.rows
        for mats in self.w:
            D.linear(ctx, mats["qkv"], self.x_qkv, self.y_qkv, r, ws=self.ws["qkv"])
            D.linear(ctx, mats["o"], self.x_o, self.y_o, r, ws=self.ws["o"])
            D.ffn(ctx, mats["gate_up"], mats["down"], self.x_ffn, self.y_ffn, r, gws=self.ws["gate_up"],
                  dws=self.ws["down"])

    def bytes_per_layer(self):
        w0, r = self.w[0], self.rows
        return sum(lin_bytes(w0[n].bits, w0[n].k, w0[n].n, r) for n in w0)

    def ops_per_layer(self):
        w0 = self.w[0]
        return sum(2.0 * self.rows * w0[n].k * w0[n].n for n in w0)


def cpu_decode_baseline(layer0, rows, budget_s=10.0):
    """Oracle (C, OpenMP) on layer 0's decode set, repeated for ~budget_s."""
    import numpy as np
    from oracle import oracle
    g = np.random.default_rng(1)
    x = g.standard_normal((rows, H)).astype(np.float16).astype(np.float32)
    xo = g.standard_normal((rows, Q)).astype(np.float16).astype(np.float32)
    qkv, o, gu, dn = (layer0[n] for n in ("qkv", "o", "gate_up", "down"))
    bytes_layer = sum(lin_bytes(b, c.shape[0], c.shape[1], rows) for b, c, _ in (qkv, o, gu, dn))
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.linear(qkv[1], qkv[2], x)
        oracle.linear(o[1], o[2], xo)
        oracle.ffn(gu[1], gu[2], dn[1], dn[2], x)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {"value": round(bytes_layer * reps / el / 1e9, 3), "unit": "GB/s", "cores": oracle.threads(),
            "kind": "port",
            "sample": f"layer 0 of 36, M={rows} decode set (qkv, o, gate_up+SwiGLU->requant->down), "
                      f"{reps} repetitions in {el:.1f} s; same algorithmic-byte count as the GPU line"}


def run_decode(torch, ctx, rows, steps, warmup, want_cpu, want_roofline=True):
    from open_rknpu2_lm_infer_amd import device as D
    gen = Gen(torch, 1)
    log(f"[bench] decode M={rows}: creating 36 layers of W4 weights")
    t = DenseLayers(torch, ctx, gen, rows, (4, 4, 4, 4), tag=f"dec{rows}")
    nbytes = t.bytes_per_layer() * LAYERS
    ms_eager = time_steps(torch, t.step, steps, warmup)
    check = lambda: [t.y_qkv.clone(), t.y_o.clone(), t.y_ffn.clone()]
    ms_graph, ok = graph_time(torch, t.step, steps, check)
    ms = min(ms_graph, ms_eager) if ok else ms_eager
    out = {"ms_per_step": ms, "value": nbytes / (ms * 1e-3) / 1e9, "bytes_per_step": nbytes,
           "ms_eager": ms_eager, "ms_graph": ms_graph, "graph_matches_eager": ok}
    log(f"[bench] decode M={rows}: eager {ms_eager:.3f} ms/step, graph {ms_graph:.3f} ms/step "
        f"(replay bit-exact: {ok}) -> {out['value']:.1f} GB/s")
    if want_roofline:
        # Dominant kernel: the gate_up GEMV (25 MB of W4 weights per launch),
        # the same kernel the fused FFN launches. 36 launches on distinct
        # layers' weights, graph-captured, between two events.
        gu = [mats["gate_up"] for mats in t.w]
        mid = torch.empty(rows, F, dtype=torch.float16, device="cuda")
        ws = t.ws["gate_up"]
        def gu_run():
            for w in gu:
                D.linear(ctx, w, t.x_ffn, mid, rows, swiglu=True, ws=ws)
        ms_gu, _ = graph_time(torch, gu_run, steps)
        per_launch_us = ms_gu * 1e3 / len(gu)
        work = lin_bytes(4, H, 2 * F, rows)
        out["roofline"] = roofline(work / (per_launch_us * 1e-6) / 1e9, "hbm",
                                   f"gemv_kernel<__half,{rows if rows in (1, 2, 4) else 8},4,SwiGLU> "
                                   f"gate_up 2560x19456 W4, M={rows}", per_launch_us, work, len(gu) * steps,
                                   "graph of 36 back-to-back launches (distinct weights), HIP events on the replay stream",
                                   TRAFFIC_GEMV_GATE_UP_M1 if rows == 1 else None)
        log(f"[bench] decode roofline: {out['roofline']}")
    if want_cpu:
        log("[bench] cpu baseline (oracle) on layer 0 ...")
        out["cpu_baseline"] = cpu_decode_baseline(t.host0, rows)
        log(f"[bench] cpu baseline: {out['cpu_baseline']}")
    del t
    return out


def run_prefill(torch, ctx, rows, steps, warmup):
    """Config 3: M=4096, qkv/o/down W8A8, gate_up W4A8, 36 layers + lm_head W8."""
    from open_rknpu2_lm_infer_amd import device as D
    gen = Gen(torch, 3)
    log(f"[bench] prefill M={rows}: creating 36 layers + lm_head")
    t = DenseLayers(torch, ctx, gen, rows, (8, 8, 4, 8), outliers=True, tag="pf")
    head = ctx.weights(8, gen.codes("pf/lm_head", 8, H, VOCAB), gen.scales("pf/lm_head", VOCAB))
    y_head = torch.empty(rows, VOCAB, dtype=torch.float16, device="cuda")
    ws_head = ctx.workspace(8, rows, H, VOCAB)

    def step():
        t.step()
        D.linear(ctx, head, t.x_qkv, y_head, rows, ws=ws_head)

    ms, ms_eager, ms_graph, ok = best_time(torch, step, steps, warmup,
                                           lambda: [t.y_qkv.clone(), t.y_ffn.clone(), y_head.clone()])
    ops = t.ops_per_layer() * LAYERS + 2.0 * rows * H * VOCAB
    # dominant kernel: the W4 gate_up GEMM with fused SwiGLU, 36 launches on
    # the 36 layers' weights in a graph; each linear also launches its
    # activation quantization (about 5% of the pair), which the time includes.
    gu = [mats["gate_up"] for mats in t.w]
    mid = torch.empty(rows, F, dtype=torch.float16, device="cuda")
    def gu_run():
        for w in gu:
            D.linear(ctx, w, t.x_ffn, mid, rows, swiglu=True, ws=t.ws["gate_up"])
    ms_gu, _ = graph_time(torch, gu_run, max(2, steps // 2))
    per_us = ms_gu * 1e3 / len(gu)
    launches = len(gu)
    work = 2.0 * rows * H * 2 * F
    res = {"workload": f"prefill M={rows}: Qwen3-4B qkv/o/down W8A8 + gate_up W4A8 (+SwiGLU) x36 + lm_head W8A8",
           "value": round(ops / (ms * 1e-3) / 1e12, 2), "unit": "TOPS", "ms_per_step": round(ms, 3),
           "frac_of_int8_peak": round(ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
           "ms_eager": round(ms_eager, 3), "ms_graph": round(ms_graph, 3), "graph_matches_eager": ok,
           "roofline": roofline(work / (per_us * 1e-6) / 1e12, "mfma",
                                f"gemm_kernel<128,128,2,2,W4,SwiGLU> gate_up 2560x19456, M={rows}", per_us, work,
                                launches, "graph of 36 back-to-back quantization + GEMM launch pairs, HIP events "
                                "on the replay stream"),
           "vendor_ref": vendor_int8_gemm(torch, rows, H, 2 * F)}
    log(f"[bench] prefill: {res['value']} TOPS ({ms:.2f} ms/step); vendor int8 GEMM {res['vendor_ref']}")
    del t, head
    return res


def vendor_int8_gemm(torch, m, k, n, reps=20):
    """Context for the MFMA roofline: the vendor library's plain int8 GEMM
    (torch._int_mm -> hipBLASLt, int32 out, no quantization, dequant or
    SwiGLU) on the same M, K, N, timed with HIP events on the current stream."""
    try:
        a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device="cuda")
        b = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda").t()
        for _ in range(3):
            torch._int_mm(a, b)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            torch._int_mm(a, b)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        return {"op": f"torch._int_mm int8 [{m}x{k}] x [{k}x{n}] -> int32", "us": round(us, 1),
                "tops": round(2.0 * m * k * n / (us * 1e-6) / 1e12, 1)}
    except Exception as ex:  # library without an int8 GEMM: reported, not fatal
        return {"op": "torch._int_mm", "error": str(ex)[:120]}


def run_ffn512(torch, ctx, steps, warmup, rows=512):
    """Config 2: M=512 W4A8 gate_up -> SwiGLU -> requant -> W8A8 down, 36 layers."""
    from open_rknpu2_lm_infer_amd import device as D
    gen = Gen(torch, 2)
    layers = []
    for l in range(LAYERS):
        layers.append((ctx.weights(4, gen.codes(f"ffn/l{l}/gu", 4, H, 2 * F), gen.scales(f"ffn/l{l}/gu", 2 * F)),
                       ctx.weights(8, gen.codes(f"ffn/l{l}/dn", 8, F, H), gen.scales(f"ffn/l{l}/dn", H))))
    x = gen.acts("ffn/x", rows, H, True)
    y = torch.empty(rows, H, dtype=torch.float16, device="cuda")
    gws = ctx.workspace(4, rows, H, 2 * F)
    dws = ctx.workspace(8, rows, F, H)

    def step():
        for gu, dn in layers:
            D.ffn(ctx, gu, dn, x, y, rows, gws=gws, dws=dws)

    ms, ms_eager, ms_graph, ok = best_time(torch, step, steps, warmup, lambda: [y.clone()])
    ops = LAYERS * 2.0 * rows * (H * 2 * F + F * H)
    res = {"workload": "FFN block M=512: W4A8 gate_up 2560->2x9728 + SwiGLU + requant + W8A8 down, 36 layers",
           "value": round(ops / (ms * 1e-3) / 1e12, 2), "unit": "TOPS", "ms_per_step": round(ms, 3),
           "frac_of_int8_peak": round(ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
           "ms_eager": round(ms_eager, 3), "ms_graph": round(ms_graph, 3), "graph_matches_eager": ok}
    log(f"[bench] ffn512: {res['value']} TOPS")
    del layers
    return res


def run_up128(torch, ctx, steps, warmup, rows=128):
    """Config 0: single W8A8 linear M=128 K=2560 N=9728, outlier channels."""
    from open_rknpu2_lm_infer_amd import device as D
    gen = Gen(torch, 0)
    w = ctx.weights(8, gen.codes("up/w", 8, H, F), gen.scales("up/w", F))
    x = gen.acts("up/x", rows, H, True)
    y = torch.empty(rows, F, dtype=torch.float16, device="cuda")
    ws = ctx.workspace(8, rows, H, F)
    step = lambda: D.linear(ctx, w, x, y, rows, ws=ws)
    ms, _, _, _ = best_time(torch, step, steps * 10, warmup, lambda: [y.clone()])
    ops = 2.0 * rows * H * F
    return {"workload": "W8A8 linear M=128 K=2560 N=9728 (Qwen3-4B FFN up)", "value": round(ops / (ms * 1e-3) / 1e12, 2),
            "unit": "TOPS", "ms_per_step": round(ms, 4),
            "gbs": round(lin_bytes(8, H, F, rows) / (ms * 1e-3) / 1e9, 1)}


def run_host_abi(layers=4, reps=20):
    """The reference's own host-buffer signatures, through the host mirror of
    src/npu.rs: rk_npu_w4a8_run_f32 / rk_npu_w4a8_run_swiglu_f32 (decode set,
    M=1, `layers` distinct layers, the f32 SwiGLU middle handed back to the
    host and into the down projection as the reference's callers do) and
    rk_npu_f32i8f32_run_dynamic (W8A8 M=128 up projection). A and C are host
    f32 buffers copied in and out before each call returns, so these rates
    include PCIe and the per-call synchronization; they are reported beside
    the HBM-resident lines, never as the headline value."""
    import numpy as np
    from open_rknpu2_lm_infer_amd import npu
    g = np.random.default_rng(0x5EED0001)
    backend = npu.Backend(npu.ModelOptions(chunk=256))

    def qm(bits, k, n):
        lo, hi = (-8, 8) if bits == 4 else (-127, 128)
        return npu.QuantMatrix(bits, k, n, g.integers(lo, hi, size=(k, n), dtype=np.int8),
                               g.uniform(0.001, 0.01, n).astype(np.float32))

    shapes = (("qkv", H, Q + 2 * KV), ("o", Q, H), ("gate_up", H, 2 * F), ("down", F, H))
    lay = [{name: backend.load(qm(4, k, n)) for name, k, n in shapes} for _ in range(layers)]
    x = g.standard_normal((1, H)).astype(np.float16).astype(np.float32)
    xo = g.standard_normal((1, Q)).astype(np.float16).astype(np.float32)
    y_qkv, y_o = np.empty((1, Q + 2 * KV), np.float32), np.empty((1, H), np.float32)
    mid, y_ffn = np.empty((1, F), np.float32), np.empty((1, H), np.float32)

    def step():
        for L in lay:
            L["qkv"].run(x, y_qkv, 1)
            L["o"].run(xo, y_o, 1)
            assert L["gate_up"].run_swiglu(x, mid, 1)
            L["down"].run(mid, y_ffn, 1)

    for _ in range(3):
        step()
    t0 = time.perf_counter()
    for _ in range(reps):
        step()
    us_layer = (time.perf_counter() - t0) * 1e6 / (reps * layers)
    bytes_layer = sum(lin_bytes(4, k, n, 1) for _, k, n in shapes)
    del lay
    up = backend.load(qm(8, H, F))
    xu = g.standard_normal((128, H)).astype(np.float32)
    xu[:, g.choice(H, math.ceil(0.005 * H), replace=False)] *= 20.0
    xu = xu.astype(np.float16).astype(np.float32)
    yu = np.empty((128, F), np.float32)
    for _ in range(3):
        up.run(xu, yu, 128)
    t0 = time.perf_counter()
    for _ in range(reps * 5):
        up.run(xu, yu, 128)
    us_up = (time.perf_counter() - t0) * 1e6 / (reps * 5)
    res = [{"workload": f"host-buffer C ABI (rk_npu_w4a8_run_f32 / _run_swiglu_f32, f32 A and C in host memory): "
                        f"decode M=1 W4A8 set, {layers} layers",
            "value": round(bytes_layer / (us_layer * 1e-6) / 1e9, 1), "unit": "GB/s", "us_per_layer": round(us_layer, 2),
            "note": "PCIe-inclusive, one synchronization per call"},
           {"workload": "host-buffer C ABI (rk_npu_f32i8f32_run_dynamic): W8A8 linear M=128 K=2560 N=9728",
            "value": round(2.0 * 128 * H * F / (us_up * 1e-6) / 1e12, 2), "unit": "TOPS", "us_per_call": round(us_up, 2),
            "note": "PCIe-inclusive: 1.3 MB of f32 A in, 5.0 MB of f32 C out per call"}]
    log(f"[bench] host ABI: {res[0]['value']} GB/s decode ({us_layer:.1f} us/layer), "
        f"{res[1]['value']} TOPS up M=128 ({us_up:.1f} us/call)")
    return res


def run_moe(torch, ctx, steps, warmup, tokens_list=(512, 1)):
    """Config 4: hidden 2048, 128 experts, top-8, I=768, routed W4 gate_up +
    W8 down; shared W8 FFN of intermediate 2048 through the dense path."""
    import ctypes

    import numpy as np

    from open_rknpu2_lm_infer_amd import _ffi as F_
    from open_rknpu2_lm_infer_amd import device as D
    from open_rknpu2_lm_infer_amd import npu
    from oracle import oracle
    h, inter, experts, top, sh_inter = 2048, 768, 128, 8, 2048
    g = np.random.default_rng(0x5EED0004)
    L = F_.lib()
    keep, arr = [], (F_.rk_npu_moe_w8_expert * experts)()
    for e in range(experts):
        gc = g.integers(-8, 8, (h, 2 * inter), dtype=np.int8)
        gs = g.uniform(0.001, 0.01, 2 * inter).astype(np.float32)
        dc = g.integers(-127, 128, (inter, h), dtype=np.int8)
        ds = g.uniform(0.001, 0.01, h).astype(np.float32)
        keep.append((gc, gs, dc, ds))
        arr[e] = F_.rk_npu_moe_w8_expert(gc.ctypes.data_as(F_.i8p), gs.ctypes.data_as(F_.f32p),
                                         dc.ctypes.data_as(F_.i8p), ds.ctypes.data_as(F_.f32p))
    max_t = max(tokens_list)
    cfg = F_.rk_npu_moe_w8_config()
    L.rk_npu_moe_w8_config_init(ctypes.byref(cfg), h, inter, experts, 0, top, max_t)
    bank = npu._Handle(L.rk_npu_moe_w4w8_weights_create(ctx.domain, ctypes.byref(cfg.weights), arr),
                       L.rk_npu_moe_w8_weights_free, "MoE bank", ctx.shared)
    work = npu._Handle(L.rk_npu_moe_w4w8_workspace_create(ctx.domain, ctypes.byref(cfg)),
                       L.rk_npu_moe_w8_workspace_free, "MoE workspace", ctx.shared)
    del keep, arr
    gen = Gen(torch, 4)
    sgu = ctx.weights(8, gen.codes("moe/sh/gu", 8, h, 2 * sh_inter), gen.scales("moe/sh/gu", 2 * sh_inter))
    sdn = ctx.weights(8, gen.codes("moe/sh/dn", 8, sh_inter, h), gen.scales("moe/sh/dn", h))
    results = []
    for T in tokens_list:
        logits = g.standard_normal((T, experts)).astype(np.float32)
        ids = np.zeros((T, top), np.int32)
        rw = np.zeros((T, top), np.float32)
        for r in range(T):
            ids[r], rw[r] = oracle.routes(logits[r], top)
        x = torch.from_numpy(g.standard_normal((T, h)).astype(np.float32)).cuda()
        d_ids = torch.from_numpy(ids).cuda()
        d_rw = torch.from_numpy(rw).cuda()
        y = torch.empty(T, h, dtype=torch.float32, device="cuda")
        ys = torch.empty(T, h, dtype=torch.float16, device="cuda")
        xs = x.half()
        gws = ctx.workspace(8, T, h, 2 * sh_inter)
        dws = ctx.workspace(8, T, sh_inter, h)

        def step():
            rc = L.rk_npu_hip_moe_run(work.raw, bank.raw, T, ctypes.c_void_p(x.data_ptr()),
                                      ctypes.c_void_p(d_ids.data_ptr()), ctypes.c_void_p(d_rw.data_ptr()),
                                      ctypes.c_void_p(y.data_ptr()), D.current_stream())
            npu.check(rc, "MoE run")
            D.ffn(ctx, sgu, sdn, xs, ys, T, gws=gws, dws=dws)

        ms, ms_eager, ms_graph, ok = best_time(torch, step, steps * (10 if T == 1 else 1), warmup,
                                               lambda: [y.clone(), ys.clone()])
        routed_ops = 2.0 * T * top * (h * 2 * inter + inter * h)
        shared_ops = 2.0 * T * (h * 2 * sh_inter + sh_inter * h)
        routed_bytes = min(experts, T * top) * (h * 2 * inter // 2 + 4 * 2 * inter + inter * h + 4 * h)
        shared_bytes = h * 2 * sh_inter + 4 * 2 * sh_inter + sh_inter * h + 4 * h
        res = {"workload": f"MoE 35B-A3B-class T={T}: h2048 E128 top8 I768 W4 gate_up + W8 down, shared W8 FFN I2048",
               "ms_per_step": round(ms, 4), "ms_eager": round(ms_eager, 4), "ms_graph": round(ms_graph, 4),
               "graph_matches_eager": ok}
        if T >= 64:
            res.update(value=round((routed_ops + shared_ops) / (ms * 1e-3) / 1e12, 2), unit="TOPS")
        else:
            res.update(value=round((routed_bytes + shared_bytes) / (ms * 1e-3) / 1e9, 1), unit="GB/s")
        log(f"[bench] moe T={T}: {res['value']} {res['unit']} ({ms:.3f} ms)")
        results.append(res)
    return results


def run_attention(torch, ctx, steps, layers=36, length=4096):
    """FP16 GQA attention (Qwen3-4B geometry: 32 query heads over 8 KV heads,
    head_dim 128) over per-layer KV caches of `length` rows, through the
    device entry points: a decode step (one query row per layer at the last
    position: every cached row read) in GB/s of K/V bytes, and a prefill block
    (128 query rows per layer ending at the last position, causal) in TFLOP/s
    of the QK and PV products. One cache per layer, so the K/V reads of a step
    (36 x 16.8 MB) come from HBM, not from the 256 MB last-level cache."""
    import ctypes
    from open_rknpu2_lm_infer_amd import _ffi as F
    L = F.lib()
    qh, kh, d = 32, 8, 128
    cfg = F.rk_npu_attention_f16_config()
    L.rk_npu_attention_f16_config_init(ctypes.byref(cfg))
    cfg.query_heads, cfg.kv_heads, cfg.head_dim = qh, kh, d
    cfg.softmax_scale = d ** -0.5
    cfg.max_query_rows, cfg.max_capacity, cfg.initial_capacity = 128, length, length
    ws = ctypes.c_void_p()
    assert L.rk_npu_attention_f16_prepare(ctx.domain, ctypes.byref(cfg), ctypes.byref(ws)) == 0
    caches = []
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    kd = torch.randn((kh, length, d), generator=g, device="cuda", dtype=torch.float32).half()
    vd = torch.randn((kh, length, d), generator=g, device="cuda", dtype=torch.float32).half()
    try:
        for _ in range(layers):
            c = ctypes.c_void_p()
            assert L.rk_npu_attention_f16_cache_create(ctx.domain, ctypes.byref(cfg), ctypes.byref(c)) == 0
            caches.append(c)
            assert L.rk_npu_hip_attention_cache_append(c, kd.data_ptr(), vd.data_ptr(), length,
                                                       torch.cuda.current_stream().cuda_stream) == 0
        torch.cuda.synchronize()
        q = torch.randn((qh, 128, d), generator=g, device="cuda", dtype=torch.float32).half()
        out = torch.empty((qh, 128, d), dtype=torch.float32, device="cuda")
        res = []
        for rows, name in ((1, "decode"), (128, "prefill")):
            pos = length - rows
            qr = q[:, :rows].contiguous()
            o = out[:, :rows].contiguous()

            def step():
                st = torch.cuda.current_stream().cuda_stream
                for c in caches:
                    L.rk_npu_hip_attention_run(ws, c, qr.data_ptr(), rows, pos, o.data_ptr(), 0, st)

            assert L.rk_npu_hip_attention_run(ws, caches[0], qr.data_ptr(), rows, pos, o.data_ptr(), 0,
                                              torch.cuda.current_stream().cuda_stream) == 0
            ms, ms_eager, ms_graph, ok = best_time(torch, step, steps, 2, lambda: [o.clone()])
            if rows == 1:
                kv_bytes = layers * 2 * kh * length * d * 2
                res.append({"workload": f"attention decode: GQA 32/8 heads, d=128, {length} cached rows, 1 query row, "
                                        f"{layers} layers", "value": round(kv_bytes / (ms * 1e-3) / 1e9, 1),
                            "unit": "GB/s", "ms_per_step": round(ms, 4), "us_per_layer": round(ms * 1e3 / layers, 2),
                            "graph_matches_eager": ok})
            else:
                keys = sum(pos + r + 1 for r in range(rows))
                flops = layers * 4.0 * qh * d * keys
                res.append({"workload": f"attention prefill: GQA 32/8 heads, d=128, {rows} query rows ending at "
                                        f"{length} cached rows, causal, {layers} layers",
                            "value": round(flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
                            "ms_per_step": round(ms, 4), "us_per_layer": round(ms * 1e3 / layers, 2),
                            "graph_matches_eager": ok})
        return res
    finally:
        torch.cuda.synchronize()
        for c in caches:
            L.rk_npu_attention_f16_cache_free(c)
        L.rk_npu_attention_f16_workspace_free(ws)


def traffic_probe(torch, ctx, rows=1, reps=3):
    """Workload for the HBM-traffic counter runs (no timing): a plain 256 MiB
    device copy (known bytes: the calibration of FETCH_SIZE / WRITE_SIZE) and
    the decode gate_up GEMV on 36 layers' distinct weights."""
    from open_rknpu2_lm_infer_amd import device as D
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").random_(0, 256)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    gen = Gen(torch, 1)
    t = DenseLayers(torch, ctx, gen, rows, (4, 4, 4, 4), tag=f"dec{rows}")
    mid = torch.empty(rows, F, dtype=torch.float16, device="cuda")
    for _ in range(reps):
        for mats in t.w:
            D.linear(ctx, mats["gate_up"], t.x_ffn, mid, rows, swiglu=True, ws=t.ws["gate_up"])
    torch.cuda.synchronize()
    log(f"[bench] traffic probe: copy 268435456 B x{reps}, gate_up GEMV x{reps * LAYERS} "
        f"({lin_bytes(4, H, 2 * F, rows)} algorithmic B each)")


def run_probes(torch, ctx, reps=20):
    """Ceilings measured on this box with the library's roofline probes
    (rk_npu_hip_mfma_probe, rk_npu_hip_stream_probe), beside the decode
    projections' own per-launch times in the same setting: 36 launches on 36
    distinct buffers / weight sets captured in a graph, HIP events on the
    replay stream, so every read comes from HBM."""
    import ctypes
    from open_rknpu2_lm_infer_amd import _ffi as FFI
    from open_rknpu2_lm_infer_amd import device as D
    L = FFI.lib()
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    res = {"mfma_int8": [], "hbm_read": [], "decode_kernels": []}
    sink = torch.empty(4096 * 256, dtype=torch.int32, device="cuda")
    for blocks in (256, 512, 1024, 2048):
        iters = 512
        def fn():
            npu_check(L.rk_npu_hip_mfma_probe(blocks, iters, ctypes.c_void_p(sink.data_ptr()), cur()), "mfma probe")
        ms, _ = graph_time(torch, fn, reps)
        ops = blocks * 4 * iters * 8 * 65536
        res["mfma_int8"].append({"blocks": blocks, "waves_per_simd": blocks // 256, "us": round(ms * 1e3, 2),
                                 "tops": round(ops / (ms * 1e-3) / 1e12, 1)})
        log(f"[probe] mfma blocks={blocks}: {res['mfma_int8'][-1]['tops']} TOPS")
    gen = Gen(torch, 1)
    t = DenseLayers(torch, ctx, gen, 1, (4, 4, 4, 4), tag="dec1")
    # per projection: (name, K, N, GEMV grid, GEMV threads per block)
    shapes = (("qkv", H, Q + 2 * KV, (Q + 2 * KV) // 8, 256), ("o", Q, H, H // 8, 256),
              ("gate_up", H, 2 * F, 2 * F // 16, 320), ("down", F, H, 4 * H // 8, 256))
    sinkb = torch.empty(1 << 20, dtype=torch.int32, device="cuda")
    for name, k, n, grid, threads in shapes:
        nbytes = lin_bytes(4, k, n, 1)
        bufs = [torch.empty(k * n // 2 + 4 * n, dtype=torch.uint8, device="cuda") for _ in range(LAYERS)]
        row = {"projection": name, "bytes": nbytes, "gemv_grid": [grid, threads]}
        for label, blocks, thr, read in (("empty launch, GEMV grid", grid, threads, 0),
                                         ("read, GEMV grid", grid, threads, 1),
                                         ("read, 256x512", 256, 512, 1), ("read, 512x512", 512, 512, 1),
                                         ("read, 1024x256", 1024, 256, 1), ("read, 2048x256", 2048, 256, 1)):
            def fn():
                for b in bufs:
                    npu_check(L.rk_npu_hip_stream_probe(ctypes.c_void_p(b.data_ptr()), b.numel(), blocks, thr, read,
                                                        ctypes.c_void_p(sinkb.data_ptr()), cur()), "stream probe")
            ms, _ = graph_time(torch, fn, reps)
            us = ms * 1e3 / LAYERS
            row[label] = {"us": round(us, 3), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1) if read else None}
        del bufs
        mats = [m[name] for m in t.w]
        if name == "down":
            def fn():
                for m in t.w:
                    D.ffn(ctx, m["gate_up"], m["down"], t.x_ffn, t.y_ffn, 1, gws=t.ws["gate_up"], dws=t.ws["down"])
            ms_ffn, _ = graph_time(torch, fn, reps)
            row["FFN call (gate_up launch + down launch)"] = {"us": round(ms_ffn * 1e3 / LAYERS, 3)}
            with D.plan_switch("HM_FFN_FUSED", 1):
                ms_one, _ = graph_time(torch, fn, reps)
            row["FFN call as one launch (HM_FFN_FUSED=1)"] = {"us": round(ms_one * 1e3 / LAYERS, 3)}
        else:
            x = t.x_o if name == "o" else t.x_ffn
            y = torch.empty(1, n // 2 if name == "gate_up" else n, dtype=torch.float16, device="cuda")
            def fn():
                for w in mats:
                    D.linear(ctx, w, x, y, 1, swiglu=(name == "gate_up"), ws=t.ws[name])
            ms, _ = graph_time(torch, fn, reps)
            us = ms * 1e3 / LAYERS
            row["library call"] = {"us": round(us, 3), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)}
        res["hbm_read"].append(row)
        log(f"[probe] {name}: {row}")
    del t
    return res


def npu_check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: rc {rc}")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--primary-only", action="store_true", help="skip the secondary workloads")
    ap.add_argument("--decode-rows", type=int, default=1,
                    help="rows of the primary decode line (1 is the metric's configuration)")
    ap.add_argument("--only", choices=["prefill", "ffn512", "up128", "moe", "attention", "host"],
                    help="run one secondary workload alone and print its result (for profiling)")
    ap.add_argument("--probes", action="store_true",
                    help="only measure the ceilings (MFMA int8 rate, HBM read floors per decode projection)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only run the workload of the FETCH_SIZE / WRITE_SIZE counter runs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    torch = torch_setup()
    from open_rknpu2_lm_infer_amd import device as D
    ctx = D.DeviceContext(0)
    if args.traffic_probe:
        traffic_probe(torch, ctx)
        return
    if args.probes:
        print(json.dumps(run_probes(torch, ctx)), flush=True)
        return
    if args.only:
        steps = max(4, args.steps // 2)
        res = {"prefill": lambda: run_prefill(torch, ctx, 4096, steps, 2),
               "ffn512": lambda: run_ffn512(torch, ctx, steps, 2),
               "up128": lambda: run_up128(torch, ctx, args.steps, args.warmup),
               "moe": lambda: run_moe(torch, ctx, steps, 2),
               "attention": lambda: run_attention(torch, ctx, steps),
               "host": lambda: run_host_abi()}[args.only]()
        print(json.dumps(res), flush=True)
        return
    primary = run_decode(torch, ctx, args.decode_rows, args.steps, args.warmup, not args.no_cpu_baseline)
    secondary = []
    if not args.primary_only:
        m4 = run_decode(torch, ctx, 4, args.steps, args.warmup, False, want_roofline=True)
        secondary.append({"workload": "decode M=4 (MTP/draft verify), same W4A8 set x36",
                          "value": round(m4["value"], 1), "unit": "GB/s", "ms_per_step": round(m4["ms_per_step"], 4),
                          "roofline": m4["roofline"]})
        secondary.append(run_prefill(torch, ctx, 4096, max(4, args.steps // 2), 2))
        secondary.append(run_ffn512(torch, ctx, max(4, args.steps // 2), 2))
        secondary.append(run_up128(torch, ctx, args.steps, args.warmup))
        secondary.extend(run_host_abi())
        secondary.extend(run_moe(torch, ctx, max(4, args.steps // 2), 2))
        secondary.extend(run_attention(torch, ctx, max(4, args.steps // 2)))
    for s in secondary:
        s.pop("kernels", None)
        if "roofline" in s:
            s["roofline"].pop("work_per_launch", None)
    roof = dict(primary["roofline"])
    roof.pop("work_per_launch", None)
    config_extra = {"ms_eager": round(primary["ms_eager"], 4), "ms_graph": round(primary["ms_graph"], 4),
                    "graph_matches_eager": primary["graph_matches_eager"]}
    line = {
        "metric": METRIC,
        "value": round(primary["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(primary["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded random W4 codes in [-8,7], f32 scales U(0.001,0.01), fp16 N(0,1) activations)",
        "config": {"workload": "decode: Qwen3-4B-shaped W4A8 projection set (qkv 2560x6144, o 4096x2560, "
                               f"gate_up 2560x19456 + SwiGLU -> down 9728x2560), M={args.decode_rows}, 36 layers",
                   "rows": args.decode_rows, "layers": 36, "weight_bits": 4, "activations": "fp16 in/out, per-token dynamic int8",
                   "bytes_per_step": primary["bytes_per_step"], "parallelism": "single GPU",
                   "timing": "faster of eager launches and HIP graph replay of the same step "
                             "(replay checked bit-exact vs eager)", **config_extra},
        "roofline": roof,
        "cpu_baseline": primary.get("cpu_baseline"),
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
