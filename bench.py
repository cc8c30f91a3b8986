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
host-buffer signatures (decode set, M=128 up projection, decode attention).

Timing (every workload): the step runs eagerly (host launches between two
synchronizations) and as a HIP graph replay (checked bit-exact against eager
runs) between two HIP events; the faster valid one is used, both are reported.
roofline: the dominant kernel's algorithmic bytes (or ops) per launch over its
average launch time: 36 back-to-back launches of that kernel alone (distinct
layers' weights) captured in a graph and timed with HIP events on the replay
stream. `--roofline-only` runs only these passes (every line's, and the
per-projection passes of the decode and prefill sets), so a kernel-trace
profile of that command holds the same launches; `--summarize-trace CSV`
turns such a trace into per-kernel averages.
cpu_baseline: the C oracle (OpenMP) on a bounded sample of the same workload
on this host's cores: one warm-up, then the median of at least 5 timed
repetitions, with the CPU model, the cores visible to the process and the
OpenMP thread count.
"""
from __future__ import annotations

import argparse
import csv
import functools
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "int8 TOPS (% MFMA peak) at M=512/4096 prefill; HBM GB/s at M=1 decode"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
F16_PEAK_TFLOPS = 2500.0

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


# HBM bytes per launch of the dominant decode kernel (the gate_up GEMV) at
# M=1 and M=4, from two rocprofv3 counter runs of `bench.py --traffic-probe`
# (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch, medians over 216
# dispatches), each scaled by what the same counter reads for the run's
# 268,435,456-byte device copy: FETCH_SIZE 131,083.5 KiB (factor 2.0),
# WRITE_SIZE 262,144 KiB (factor 1.0). Commands and every decode GEMV's
# figures: profiles/traffic_decode_gemv_m1_m4.txt.
TRAFFIC_GEMV_GATE_UP = {1: int(round((12429.5 * 2.0 + 81.1 * 1.0) * 1024)),
                        4: int(round((12466.5 * 2.0 + 304.0 * 1.0) * 1024))}


ROOF_METHOD = "graph of 36 back-to-back launches (distinct weights), HIP events on the replay stream"


def roofline(achieved, bound, kernel, avg_us, work, launches, method=ROOF_METHOD, traffic=None, peak=None):
    if bound == "hbm":
        peak, unit = peak or HBM_PEAK_GBS, "GB/s"
    else:
        peak, unit = peak or INT8_PEAK_TOPS, "TFLOP/s"
    return {"bound": bound, "kernel": kernel, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic, "avg_us": round(avg_us, 3),
            "work_per_launch": work, "launches": launches, "method": method}


def roof_of(bound, kernel, work, us, launches, method=ROOF_METHOD, traffic=None, peak=None):
    """roofline() from algorithmic work per launch (bytes for "hbm", ops for
    "mfma") and the average launch time in microseconds."""
    scale = 1e9 if bound == "hbm" else 1e12
    return roofline(work / (us * 1e-6) / scale, bound, kernel, us, work, launches, method, traffic, peak)


def per_launch_us(torch, fns, reps):
    """Average time per launch of the calls fns[i]() (each one library call,
    normally on its own weights), captured back to back in one HIP graph and
    replayed `reps` times between two HIP events on the replay stream."""
    def run():
        for f in fns:
            f()
    ms, _ = graph_time(torch, run, reps)
    return ms * 1e3 / len(fns)


def cpu_info():
    """The host facts every CPU baseline carries: CPU model name, cores
    visible to this process (and in the machine), the oracle's OpenMP threads."""
    from oracle import oracle
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "nproc": len(os.sched_getaffinity(0)), "cpu_count": os.cpu_count(),
            "omp_threads": oracle.threads(), "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}


def cpu_median(fn, budget_s, min_reps=5):
    """One warm-up call, then timed calls until both `min_reps` calls and
    `budget_s` seconds are done: (median seconds per call, calls timed)."""
    fn()
    times, t_start = [], time.perf_counter()
    while len(times) < min_reps or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline(value, unit, sec, reps, sample, **extra):
    info = cpu_info()
    return {"value": round(value, 3), "unit": unit, "cores": info["omp_threads"], "kind": "port",
            "sample": sample, "ms": round(sec * 1e3, 3), "reps": reps, **extra, **info}


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
        """One pass over the 36 layers with a layer's data flow: qkv's output
        feeds o (its first rows x 4096 values standing in for the attention
        output) and o's output feeds the FFN, so every launch reads what the
        one before it wrote. Each layer's qkv reads the same fixed input: fed
        the previous layer's FFN output instead, without the model's RMSNorm
        (not part of this path), random weights and the SwiGLU's squaring take
        the values to zero or to overflow within a few layers, and zero data
        lets the matrix cores hold a higher clock (an M=4096 step measured
        19.1 ms against 20.3 ms), which would not be the workload."""
        for mats in self.w:
            self.layer(mats)

    def layer(self, mats):
        D, ctx, r = self.D, self.ctx, self.rows
        attn = self.y_qkv.view(-1)[:r * Q].view(r, Q)
        D.linear(ctx, mats["qkv"], self.x_qkv, self.y_qkv, r, ws=self.ws["qkv"])
        D.linear(ctx, mats["o"], attn, self.y_o, r, ws=self.ws["o"])
        D.ffn(ctx, mats["gate_up"], mats["down"], self.y_o, self.y_ffn, r, gws=self.ws["gate_up"],
              dws=self.ws["down"])

    def magnitudes(self):
        """max |value| of the three outputs after a step (the data stays in range)."""
        return [round(float(t.float().abs().max()), 3) for t in (self.y_qkv, self.y_o, self.y_ffn)]

    def bytes_per_layer(self):
        w0, r = self.w[0], self.rows
        return sum(lin_bytes(w0[n].bits, w0[n].k, w0[n].n, r) for n in w0)

    def ops_per_layer(self):
        w0 = self.w[0]
        return sum(2.0 * self.rows * w0[n].k * w0[n].n for n in w0)


def cpu_decode_baseline(layer0, rows, budget_s=10.0):
    """Oracle (C, OpenMP) on layer 0's decode set, timed as cpu_median()."""
    import numpy as np
    from oracle import oracle
    g = np.random.default_rng(1)
    x = g.standard_normal((rows, H)).astype(np.float16).astype(np.float32)
    xo = g.standard_normal((rows, Q)).astype(np.float16).astype(np.float32)
    qkv, o, gu, dn = (layer0[n] for n in ("qkv", "o", "gate_up", "down"))
    bytes_layer = sum(lin_bytes(b, c.shape[0], c.shape[1], rows) for b, c, _ in (qkv, o, gu, dn))

    def one():
        oracle.linear(qkv[1], qkv[2], x)
        oracle.linear(o[1], o[2], xo)
        oracle.ffn(gu[1], gu[2], dn[1], dn[2], x)

    sec, reps = cpu_median(one, budget_s)
    return cpu_baseline(bytes_layer / sec / 1e9, "GB/s", sec, reps,
                        f"layer 0 of 36, M={rows} decode set (qkv, o, gate_up+SwiGLU->requant->down); "
                        f"same algorithmic-byte count as the GPU line; ms is per layer",
                        ms_step_x36=round(sec * 1e3 * LAYERS, 2))


def decode_passes(torch, ctx, t, reps):
    """Per-projection launch times of a decode set (36 launches each, one per
    layer, in a graph): qkv, o, gate_up (+SwiGLU, fp16 out) and the FFN call
    (gate_up + SwiGLU + row max, then the down launch that requantizes the
    middle); the down launch's time is the FFN call's minus gate_up's."""
    D, r = t.D, t.rows
    mid = torch.empty(r, F, dtype=torch.float16, device="cuda")
    specs = (
        ("qkv", lambda m: D.linear(ctx, m["qkv"], t.x_qkv, t.y_qkv, r, ws=t.ws["qkv"]),
         lin_bytes(4, H, Q + 2 * KV, r)),
        ("o", lambda m: D.linear(ctx, m["o"], t.x_o, t.y_o, r, ws=t.ws["o"]), lin_bytes(4, Q, H, r)),
        ("gate_up", lambda m: D.linear(ctx, m["gate_up"], t.x_ffn, mid, r, swiglu=True, ws=t.ws["gate_up"]),
         lin_bytes(4, H, 2 * F, r)),
        ("ffn call", lambda m: D.ffn(ctx, m["gate_up"], m["down"], t.x_ffn, t.y_ffn, r, gws=t.ws["gate_up"],
                                     dws=t.ws["down"]), lin_bytes(4, H, 2 * F, r) + lin_bytes(4, F, H, r)),
    )
    out = {}
    for name, fn, work in specs:
        calls = [functools.partial(fn, m) for m in t.w]
        us = per_launch_us(torch, calls, reps)
        out[name] = {"us": round(us, 3), "bytes": work, "gbs": round(work / us / 1e3, 1),
                     "frac_hbm": round(work / us / 1e3 / HBM_PEAK_GBS, 4)}
    us_dn = out["ffn call"]["us"] - out["gate_up"]["us"]
    dn = lin_bytes(4, F, H, r)
    out["down (ffn call - gate_up)"] = {"us": round(us_dn, 3), "bytes": dn, "gbs": round(dn / us_dn / 1e3, 1),
                                        "frac_hbm": round(dn / us_dn / 1e3 / HBM_PEAK_GBS, 4)}
    return out


def stream_read_us(torch, nbytes, reps=20, blocks=2048, threads=256):
    """One launch reading `nbytes` of device memory with the GEMV's 16-byte
    non-temporal loads (rk_npu_hip_stream_probe), on 36 distinct buffers
    launched back to back in a graph (so every read comes from HBM): average
    microseconds per launch."""
    import ctypes
    from open_rknpu2_lm_infer_amd import _ffi as FFI
    LP = FFI.probe_lib()
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(LAYERS)]
    sink = torch.empty(blocks, dtype=torch.int32, device="cuda")

    def fn():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for b in bufs:
            npu_check(LP.rk_npu_hip_stream_probe(ctypes.c_void_p(b.data_ptr()), nbytes, blocks, threads, 1,
                                                 ctypes.c_void_p(sink.data_ptr()), st), "stream probe")
    ms, _ = graph_time(torch, fn, reps)
    del bufs
    return ms * 1e3 / LAYERS


def run_decode(torch, ctx, rows, steps, warmup, want_cpu, want_roofline=True, timed=True, reps=None):
    gen = Gen(torch, 1)
    log(f"[bench] decode M={rows}: creating 36 layers of W4 weights")
    t = DenseLayers(torch, ctx, gen, rows, (4, 4, 4, 4), tag=f"dec{rows}")
    nbytes = t.bytes_per_layer() * LAYERS
    out = {"bytes_per_step": nbytes}
    if timed:
        ms_eager = time_steps(torch, t.step, steps, warmup)
        check = lambda: [t.y_qkv.clone(), t.y_o.clone(), t.y_ffn.clone()]
        ms_graph, ok = graph_time(torch, t.step, steps, check)
        ms = min(ms_graph, ms_eager) if ok else ms_eager
        out.update({"ms_per_step": ms, "value": nbytes / (ms * 1e-3) / 1e9, "ms_eager": ms_eager,
                    "ms_graph": ms_graph, "graph_matches_eager": ok})
        log(f"[bench] decode M={rows}: eager {ms_eager:.3f} ms/step, graph {ms_graph:.3f} ms/step "
            f"(replay bit-exact: {ok}) -> {out['value']:.1f} GB/s; max |qkv|, |o|, |ffn| {t.magnitudes()}")
    if want_roofline:
        # Dominant kernel: the gate_up GEMV (25 MB of W4 weights per launch).
        passes = decode_passes(torch, ctx, t, reps or steps)
        gu = passes["gate_up"]
        out["projections"] = passes
        out["roofline"] = roof_of("hbm", f"gemv_kernel (W4, SwiGLU epilogue) gate_up 2560x19456, M={rows}",
                                  gu["bytes"], gu["us"], LAYERS * (reps or steps),
                                  traffic=TRAFFIC_GEMV_GATE_UP.get(rows))
        # The measured ceiling of one launch of this size: a plain read of the
        # same bytes with the same loads, launched the same way.
        read_us = stream_read_us(torch, gu["bytes"])
        ceil = gu["bytes"] / (read_us * 1e-6) / 1e9
        out["roofline"]["measured_ceiling"] = {
            "value": round(ceil, 1), "unit": "GB/s", "frac": round(out["roofline"]["achieved"] / ceil, 4),
            "us": round(read_us, 3),
            "what": "one launch reading the same bytes with the GEMV's 16-byte non-temporal loads "
                    "(rk_npu_hip_stream_probe, 2048 x 256 threads), 36 distinct buffers back to back in a graph"}
        log(f"[bench] decode M={rows} projections: {passes}")
        log(f"[bench] decode roofline: {out['roofline']}")
    if want_cpu:
        log(f"[bench] cpu baseline (oracle) on layer 0, M={rows} ...")
        out["cpu_baseline"] = cpu_decode_baseline(t.host0, rows, 10.0 if rows == 1 else 4.0)
        log(f"[bench] cpu baseline: {out['cpu_baseline']}")
    del t
    return out


def prefill_passes(torch, ctx, t, head, y_head, ws_head, reps):
    """Per-projection launch times of the M=4096 set: each entry is 36
    back-to-back library calls (quantization launch + GEMM launch) on the 36
    layers' weights (the lm_head: 4 calls on its one weight set, 389 MB, more
    than the last-level cache holds), in a graph."""
    D, r = t.D, t.rows
    mid = torch.empty(r, F, dtype=torch.float16, device="cuda")
    specs = (
        ("qkv W8", lambda m: D.linear(ctx, m["qkv"], t.x_qkv, t.y_qkv, r, ws=t.ws["qkv"]), 2.0 * r * H * (Q + 2 * KV)),
        ("o W8", lambda m: D.linear(ctx, m["o"], t.x_o, t.y_o, r, ws=t.ws["o"]), 2.0 * r * Q * H),
        ("gate_up W4 +SwiGLU", lambda m: D.linear(ctx, m["gate_up"], t.x_ffn, mid, r, swiglu=True,
                                                  ws=t.ws["gate_up"]), 2.0 * r * H * 2 * F),
        ("ffn call (gate_up W4 + down W8)", lambda m: D.ffn(ctx, m["gate_up"], m["down"], t.x_ffn, t.y_ffn, r,
                                                            gws=t.ws["gate_up"], dws=t.ws["down"]),
         2.0 * r * (H * 2 * F + F * H)),
    )
    out = {}
    for name, fn, work in specs:
        us = per_launch_us(torch, [functools.partial(fn, m) for m in t.w], reps)
        out[name] = {"us": round(us, 2), "ops": work, "tops": round(work / us / 1e6, 1),
                     "frac_int8": round(work / us / 1e6 / INT8_PEAK_TOPS, 4)}
    us = per_launch_us(torch, [lambda: D.linear(ctx, head, t.x_qkv, y_head, r, ws=ws_head)] * 4, reps)
    work = 2.0 * r * H * VOCAB
    out["lm_head W8"] = {"us": round(us, 2), "ops": work, "tops": round(work / us / 1e6, 1),
                         "frac_int8": round(work / us / 1e6 / INT8_PEAK_TOPS, 4)}
    gu, fc = out["gate_up W4 +SwiGLU"], out["ffn call (gate_up W4 + down W8)"]
    us_dn, work = fc["us"] - gu["us"], 2.0 * r * F * H
    out["down W8 (ffn call - gate_up)"] = {"us": round(us_dn, 2), "ops": work, "tops": round(work / us_dn / 1e6, 1),
                                           "frac_int8": round(work / us_dn / 1e6 / INT8_PEAK_TOPS, 4)}
    return out


def cpu_prefill_baseline(t, head_host, x_rows, budget_s=8.0):
    """Oracle on a 64-row sample of layer 0 (qkv, o, FFN) and of the lm_head;
    ms_step_extrapolated = (36 x layer + lm_head) x 4096 / 64."""
    from oracle import oracle
    x, xo = x_rows
    (qb, qc, qs), (ob, oc, os_), (gb, gc, gs), (db, dc, ds) = (t.host0[n] for n in ("qkv", "o", "gate_up", "down"))

    def layer():
        oracle.linear(qc, qs, x)
        oracle.linear(oc, os_, xo)
        oracle.ffn(gc, gs, dc, ds, x)

    sec_l, reps_l = cpu_median(layer, budget_s / 2)
    sec_h, reps_h = cpu_median(lambda: oracle.linear(head_host[0], head_host[1], x), budget_s / 2)
    rows = x.shape[0]
    ops = 2.0 * rows * (H * (Q + 2 * KV) + Q * H + H * 2 * F + F * H) + 2.0 * rows * H * VOCAB
    sec = sec_l + sec_h
    return cpu_baseline(ops / sec / 1e12, "TOPS", sec, min(reps_l, reps_h),
                        f"{rows} of 4096 rows: layer 0 (qkv, o, gate_up+SwiGLU->requant->down) and the lm_head, "
                        f"medians {sec_l * 1e3:.1f} + {sec_h * 1e3:.1f} ms",
                        ms_step_extrapolated=round((LAYERS * sec_l + sec_h) * 1e3 * 4096 / rows, 1))


def run_prefill(torch, ctx, rows, steps, warmup, want_cpu=True, timed=True, reps=None):
    """Config 3: M=4096, qkv/o/down W8A8, gate_up W4A8, 36 layers + lm_head W8."""
    from open_rknpu2_lm_infer_amd import device as D
    gen = Gen(torch, 3)
    log(f"[bench] prefill M={rows}: creating 36 layers + lm_head")
    t = DenseLayers(torch, ctx, gen, rows, (8, 8, 4, 8), outliers=True, tag="pf")
    head_codes = gen.codes("pf/lm_head", 8, H, VOCAB)
    head_scales = gen.scales("pf/lm_head", VOCAB)
    head = ctx.weights(8, head_codes, head_scales)
    head_host = (head_codes.cpu().numpy(), head_scales.cpu().numpy()) if want_cpu else None
    del head_codes, head_scales
    y_head = torch.empty(rows, VOCAB, dtype=torch.float16, device="cuda")
    ws_head = ctx.workspace(8, rows, H, VOCAB)
    ops = t.ops_per_layer() * LAYERS + 2.0 * rows * H * VOCAB
    res = {"workload": f"prefill M={rows}: Qwen3-4B qkv/o/down W8A8 + gate_up W4A8 (+SwiGLU) x36 + lm_head W8A8"}
    if timed:
        def step():
            t.step()
            D.linear(ctx, head, t.y_ffn, y_head, rows, ws=ws_head)  # the last layer's output feeds the lm_head

        ms, ms_eager, ms_graph, ok = best_time(torch, step, steps, warmup,
                                               lambda: [t.y_qkv.clone(), t.y_ffn.clone(), y_head.clone()])
        res.update({"value": round(ops / (ms * 1e-3) / 1e12, 2), "unit": "TOPS", "ms_per_step": round(ms, 3),
                    "frac_of_int8_peak": round(ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
                    "ms_eager": round(ms_eager, 3), "ms_graph": round(ms_graph, 3), "graph_matches_eager": ok})
    # dominant kernel: the W4 gate_up GEMM with fused SwiGLU; each library
    # call also launches its activation quantization, which the time includes.
    passes = prefill_passes(torch, ctx, t, head, y_head, ws_head, reps or max(2, steps // 2))
    gu = passes["gate_up W4 +SwiGLU"]
    res["projections"] = passes
    res["roofline"] = roof_of("mfma", f"gemm_kernel (W4, SwiGLU epilogue) gate_up 2560x19456, M={rows}, "
                                      "with its quantization launch", gu["ops"], gu["us"],
                              LAYERS * (reps or max(2, steps // 2)),
                              method="graph of 36 back-to-back quantization + GEMM launch pairs (distinct weights), "
                                     "HIP events on the replay stream")
    if timed:
        # The int8 rate the chip sustains from registers on full-range operands
        # (no memory traffic; the clock settles where the power limit puts it):
        # the measured ceiling beside the published dense figure.
        from open_rknpu2_lm_infer_amd import _ffi as FFI
        ceil = mfma_rand_rate(torch, FFI.probe_lib(), 2048)
        res["roofline"]["measured_ceiling"] = {
            "value": round(ceil, 1), "unit": "TOPS", "frac": round(res["roofline"]["achieved"] / ceil, 4),
            "what": "int8 MFMA from registers, random operands, 8 waves/SIMD, sustained (rk_npu_hip_mfma_rand_probe)"}
        res["vendor_ref"] = vendor_int8_gemm(torch, rows, H, 2 * F)
        log(f"[bench] prefill: {res['value']} TOPS ({ms:.2f} ms/step); vendor int8 GEMM {res['vendor_ref']}; "
            f"max |qkv|, |o|, |ffn| {t.magnitudes()}")
    log(f"[bench] prefill projections: {passes}")
    if want_cpu:
        xs = t.x_qkv[:64].float().cpu().numpy(), t.x_o[:64].float().cpu().numpy()
        res["cpu_baseline"] = cpu_prefill_baseline(t, head_host, xs)
        log(f"[bench] prefill cpu baseline: {res['cpu_baseline']}")
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


def run_ffn512(torch, ctx, steps, warmup, rows=512, want_cpu=True, timed=True, reps=None):
    """Config 2: M=512 W4A8 gate_up -> SwiGLU -> requant -> W8A8 down, 36 layers."""
    from open_rknpu2_lm_infer_amd import device as D
    gen = Gen(torch, 2)
    layers, host0 = [], None
    for l in range(LAYERS):
        gc, gs = gen.codes(f"ffn/l{l}/gu", 4, H, 2 * F), gen.scales(f"ffn/l{l}/gu", 2 * F)
        dc, ds = gen.codes(f"ffn/l{l}/dn", 8, F, H), gen.scales(f"ffn/l{l}/dn", H)
        if l == 0 and want_cpu:
            host0 = [v.cpu().numpy() for v in (gc, gs, dc, ds)]
        layers.append((ctx.weights(4, gc, gs), ctx.weights(8, dc, ds)))
        del gc, gs, dc, ds
    x = gen.acts("ffn/x", rows, H, True)
    y = torch.empty(rows, H, dtype=torch.float16, device="cuda")
    gws = ctx.workspace(4, rows, H, 2 * F)
    dws = ctx.workspace(8, rows, F, H)
    ops_layer = 2.0 * rows * (H * 2 * F + F * H)
    res = {"workload": "FFN block M=512: W4A8 gate_up 2560->2x9728 + SwiGLU + requant + W8A8 down, 36 layers"}
    calls = [functools.partial(D.ffn, ctx, gu, dn, x, y, rows, gws=gws, dws=dws) for gu, dn in layers]
    if timed:
        def step():
            for c in calls:
                c()

        ms, ms_eager, ms_graph, ok = best_time(torch, step, steps, warmup, lambda: [y.clone()])
        ops = LAYERS * ops_layer
        res.update({"value": round(ops / (ms * 1e-3) / 1e12, 2), "unit": "TOPS", "ms_per_step": round(ms, 3),
                    "frac_of_int8_peak": round(ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
                    "ms_eager": round(ms_eager, 3), "ms_graph": round(ms_graph, 3), "graph_matches_eager": ok})
        log(f"[bench] ffn512: {res['value']} TOPS")
    n = reps or max(2, steps // 2)
    us = per_launch_us(torch, calls, n)
    res["roofline"] = roof_of("mfma", "FFN call M=512 (quantization + gate_up W4 GEMM + SwiGLU + requant + down W8 GEMM)",
                              ops_layer, us, LAYERS * n,
                              method="graph of 36 back-to-back FFN calls (distinct weights), HIP events on the "
                                     "replay stream")
    if want_cpu:
        xs = x[:64].float().cpu().numpy()
        from oracle import oracle
        sec, reps_c = cpu_median(lambda: oracle.ffn(host0[0], host0[1], host0[2], host0[3], xs), 4.0)
        res["cpu_baseline"] = cpu_baseline(2.0 * 64 * (H * 2 * F + F * H) / sec / 1e12, "TOPS", sec, reps_c,
                                           "64 of 512 rows of layer 0's FFN (gate_up+SwiGLU->requant->down)",
                                           ms_step_extrapolated=round(sec * 1e3 * LAYERS * rows / 64, 1))
        log(f"[bench] ffn512 cpu baseline: {res['cpu_baseline']}")
    del layers, calls
    return res


def run_up128(torch, ctx, steps, warmup, rows=128, want_cpu=True, timed=True, reps=None):
    """Config 0: single W8A8 linear M=128 K=2560 N=9728, outlier channels.
    Timed on 36 distinct weight copies launched back to back (900 MB, more
    than the last-level cache holds: every call reads its weights from HBM);
    the same call replayed on one weight set (25 MB, cache-resident) is
    reported beside it."""
    from open_rknpu2_lm_infer_amd import device as D
    gen = Gen(torch, 0)
    codes, scales = gen.codes("up/w", 8, H, F), gen.scales("up/w", F)
    ws_ = [ctx.weights(8, codes, scales) for _ in range(LAYERS)]
    host = (codes.cpu().numpy(), scales.cpu().numpy()) if want_cpu else None
    del codes, scales
    x = gen.acts("up/x", rows, H, True)
    y = torch.empty(rows, F, dtype=torch.float16, device="cuda")
    ws = ctx.workspace(8, rows, H, F)
    ops, nbytes = 2.0 * rows * H * F, lin_bytes(8, H, F, rows)
    n = reps or steps
    us = per_launch_us(torch, [functools.partial(D.linear, ctx, w, x, y, rows, ws=ws) for w in ws_], n)
    res = {"workload": "W8A8 linear M=128 K=2560 N=9728 (Qwen3-4B FFN up)",
           "value": round(ops / (us * 1e-6) / 1e12, 2), "unit": "TOPS", "ms_per_step": round(us * 1e-3, 4),
           "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
           "timing": "per call over 36 distinct weight copies in a graph (weights read from HBM)",
           "roofline": roof_of("hbm", "W8A8 linear M=128 (quantization + gemm_kernel), 2560x9728", nbytes, us,
                               LAYERS * n, method="graph of 36 back-to-back calls on distinct weight copies, HIP "
                                                  "events on the replay stream")}
    if timed:
        step = lambda: D.linear(ctx, ws_[0], x, y, rows, ws=ws)
        ms, _, _, _ = best_time(torch, step, steps * 10, warmup, lambda: [y.clone()])
        res["cache_resident_us"] = round(ms * 1e3, 2)
    if want_cpu:
        xh = x.float().cpu().numpy()
        from oracle import oracle
        sec, reps_c = cpu_median(lambda: oracle.linear(host[0], host[1], xh), 4.0)
        res["cpu_baseline"] = cpu_baseline(ops / sec / 1e12, "TOPS", sec, reps_c, "the whole call (128 rows)")
    log(f"[bench] up128: {res['value']} TOPS, {res['gbs']} GB/s per call from HBM")
    del ws_
    return res


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
    # Decode attention through the reference's host-buffer calls (as
    # Attention::run makes them: rk_npu_attention_f16_cache_append of the
    # token's K/V row, then rk_npu_attention_f16_run of its query), 32 query
    # heads over 8 KV heads, d = 128, at 4000 cached rows (loaded through the
    # host mirror's prefill chunks).
    att_backend = npu.Backend(npu.ModelOptions(chunk=256, context=4224))
    att = att_backend.attention(32, 8, 128, 128 ** -0.5)
    pos = 0
    while pos < 4000:
        rows = min(250, 4000 - pos)
        kv = g.standard_normal((rows, 8, 128)).astype(np.float32)
        att.run(g.standard_normal((rows, 32, 128)).astype(np.float32), kv, kv, np.empty((rows, 32, 128), np.float32),
                rows, pos)
        pos += rows
    # the two C calls per step on fp16 bits packed beforehand, as the
    # reference's caller hands them over (no Python-side conversion timed)
    from open_rknpu2_lm_infer_amd import _ffi as F_
    Lh = F_.lib()
    qa = g.standard_normal((32, 1, 128)).astype(np.float16).view(np.uint16)
    ka = g.standard_normal((8, 1, 128)).astype(np.float16).view(np.uint16)
    oa = np.empty((32, 1, 128), np.float32)
    ws_raw, cache_raw, ctx_raw = att_backend._attention.workspace.raw, att.cache.raw, att_backend.ctx
    steps = 100

    def att_step(p):
        npu.check(Lh.rk_npu_attention_f16_cache_append(ctx_raw, cache_raw, ka.ctypes.data, ka.ctypes.data, 1),
                  "append")
        npu.check(Lh.rk_npu_attention_f16_run(ctx_raw, ws_raw, cache_raw, qa.ctypes.data, 1, p, oa.ctypes.data,
                                              None, None), "run")

    for i in range(8):
        att_step(pos + i)
    t0 = time.perf_counter()
    for i in range(steps):
        att_step(pos + 8 + i)
    us_att = (time.perf_counter() - t0) * 1e6 / steps
    kv_bytes = 2 * 8 * 128 * 2 * (pos + 8 + steps // 2)  # K and V rows read per step (mean length)
    del att, att_backend
    res = [{"workload": f"host-buffer C ABI (rk_npu_w4a8_run_f32 / _run_swiglu_f32, f32 A and C in host memory): "
                        f"decode M=1 W4A8 set, {layers} layers",
            "value": round(bytes_layer / (us_layer * 1e-6) / 1e9, 1), "unit": "GB/s", "us_per_layer": round(us_layer, 2),
            "note": "PCIe-inclusive, one synchronization per call"},
           {"workload": "host-buffer C ABI (rk_npu_f32i8f32_run_dynamic): W8A8 linear M=128 K=2560 N=9728",
            "value": round(2.0 * 128 * H * F / (us_up * 1e-6) / 1e12, 2), "unit": "TOPS", "us_per_call": round(us_up, 2),
            "note": "PCIe-inclusive: 1.3 MB of f32 A in, 5.0 MB of f32 C out per call"},
           {"workload": "host-buffer C ABI (rk_npu_attention_f16_cache_append + rk_npu_attention_f16_run): decode "
                        "attention, GQA 32/8 heads, d=128, one token appended and attended at ~4000 cached rows",
            "value": round(kv_bytes / (us_att * 1e-6) / 1e9, 1), "unit": "GB/s", "us_per_layer": round(us_att, 2),
            "note": "K/V bytes read per step over the wall time of the two host calls (PCIe-inclusive)"}]
    log(f"[bench] host ABI: {res[0]['value']} GB/s decode ({us_layer:.1f} us/layer), "
        f"{res[1]['value']} TOPS up M=128 ({us_up:.1f} us/call), attention {us_att:.1f} us/layer")
    return res


def run_moe(torch, ctx, steps, warmup, tokens_list=(512, 1), want_cpu=True):
    """Config 4: hidden 2048, 128 experts, top-8, I=768, routed W4 gate_up +
    W8 down; shared W8 FFN of intermediate 2048 through the dense path.
    roofline: HBM, over the weight bytes one step must read (every expert a
    token routes to, plus the shared FFN) and the step's time."""
    import ctypes

    import numpy as np

    from open_rknpu2_lm_infer_amd import _ffi as F_
    from open_rknpu2_lm_infer_amd import device as D
    from open_rknpu2_lm_infer_amd import npu
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
    del arr
    if not want_cpu:
        del keep
    gen = Gen(torch, 4)
    sh = [gen.codes("moe/sh/gu", 8, h, 2 * sh_inter), gen.scales("moe/sh/gu", 2 * sh_inter),
          gen.codes("moe/sh/dn", 8, sh_inter, h), gen.scales("moe/sh/dn", h)]
    sgu = ctx.weights(8, sh[0], sh[1])
    sdn = ctx.weights(8, sh[2], sh[3])
    sh_host = [v.cpu().numpy() for v in sh] if want_cpu else None
    del sh
    results = []
    for T in tokens_list:
        logits = g.standard_normal((T, experts)).astype(np.float32)
        ids = np.zeros((T, top), np.int32)
        rw = np.zeros((T, top), np.float32)
        for r in range(T):
            ids[r], rw[r] = npu.routes(logits[r], top)  # the product mirror of the router
        x_host = g.standard_normal((T, h)).astype(np.float32)
        x = torch.from_numpy(x_host).cuda()
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
        parts = ("slot GEMVs W4 gate_up + W8 down, combine" if T == 1 else
                 "route, quantization into slot order, grouped W4 gate_up + W8 down GEMMs, combine")
        res["roofline"] = roof_of("hbm", f"MoE call T={T} ({parts}) + shared FFN call", routed_bytes + shared_bytes,
                                  ms * 1e3,
                                  steps * (10 if T == 1 else 1),
                                  method="whole step (one MoE call + one shared FFN call), faster of eager and "
                                         "graph replay; HIP events")
        if want_cpu:
            sample = min(T, 32)
            gu_l = [(c[0], c[1]) for c in keep]
            dn_l = [(c[2], c[3]) for c in keep]
            shared = ((sh_host[0], sh_host[1]), (sh_host[2], sh_host[3]))
            from oracle import oracle
            fn = lambda: oracle.moe(gu_l, dn_l, x_host[:sample], ids[:sample], rw[:sample], shared=shared)
            sec, reps_c = cpu_median(fn, 4.0)
            s_ops = (routed_ops + shared_ops) * sample / T
            s_bytes = (min(experts, len(set(ids[:sample].ravel().tolist()))) *
                       (h * 2 * inter // 2 + 4 * 2 * inter + inter * h + 4 * h) + shared_bytes)
            res["cpu_baseline"] = (cpu_baseline(s_ops / sec / 1e12, "TOPS", sec, reps_c,
                                                f"{sample} of {T} tokens (oracle MoE with the shared FFN)")
                                   if T >= 64 else
                                   cpu_baseline(s_bytes / sec / 1e9, "GB/s", sec, reps_c,
                                                "the whole call (oracle MoE with the shared FFN)"))
        log(f"[bench] moe T={T}: {res['value']} {res['unit']} ({ms:.3f} ms)")
        results.append(res)
    return results


def run_attention(torch, ctx, steps, layers=36, length=4096, want_cpu=True):
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
            us_layer = ms * 1e3 / layers
            if want_cpu:
                from oracle import oracle
                qn = qr.float().cpu().numpy()
                kn, vn = kd.float().cpu().numpy(), vd.float().cpu().numpy()
                sec, reps_c = cpu_median(lambda: oracle.attention(qn, kn, vn, d ** -0.5, pos, True), 3.0)
            if rows == 1:
                kv_layer = 2 * kh * length * d * 2
                kv_bytes = layers * kv_layer
                r_ = {"workload": f"attention decode: GQA 32/8 heads, d=128, {length} cached rows, 1 query row, "
                                  f"{layers} layers", "value": round(kv_bytes / (ms * 1e-3) / 1e9, 1),
                      "unit": "GB/s", "ms_per_step": round(ms, 4), "us_per_layer": round(us_layer, 2),
                      "graph_matches_eager": ok,
                      "roofline": roof_of("hbm", "attention decode call (split kernel + combine), one layer",
                                          kv_layer, us_layer, layers * steps,
                                          method="per layer of the step: 36 calls on distinct caches in the step, "
                                                 "faster of eager and graph replay; HIP events")}
                if want_cpu:
                    r_["cpu_baseline"] = cpu_baseline(kv_layer / sec / 1e9, "GB/s", sec, reps_c,
                                                      "one layer's call (float64 numpy oracle)")
            else:
                keys = sum(pos + r + 1 for r in range(rows))
                flops_layer = 4.0 * qh * d * keys
                flops = layers * flops_layer
                r_ = {"workload": f"attention prefill: GQA 32/8 heads, d=128, {rows} query rows ending at "
                                  f"{length} cached rows, causal, {layers} layers",
                      "value": round(flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
                      "ms_per_step": round(ms, 4), "us_per_layer": round(us_layer, 2),
                      "graph_matches_eager": ok,
                      "roofline": roof_of("mfma", "attention prefill call (f16 MFMA kernel + combine), one layer",
                                          flops_layer, us_layer, layers * steps, peak=F16_PEAK_TFLOPS,
                                          method="per layer of the step: 36 calls on distinct caches in the step, "
                                                 "faster of eager and graph replay; HIP events; peak: dense f16 MFMA")}
                if want_cpu:
                    r_["cpu_baseline"] = cpu_baseline(flops_layer / sec / 1e12, "TFLOP/s", sec, reps_c,
                                                      "one layer's call (float64 numpy oracle)")
            res.append(r_)
        return res
    finally:
        torch.cuda.synchronize()
        for c in caches:
            L.rk_npu_attention_f16_cache_free(c)
        L.rk_npu_attention_f16_workspace_free(ws)


def traffic_probe(torch, ctx, reps=3):
    """Workload for the HBM-traffic counter runs (no timing): a plain 256 MiB
    device copy (known bytes: the calibration of FETCH_SIZE / WRITE_SIZE),
    then, at M=1 and M=4, `reps` passes over 36 layers' distinct weights of
    each decode projection in turn (qkv, o, gate_up + SwiGLU, the FFN call),
    so every dispatch of a kernel reads its weights from HBM."""
    from open_rknpu2_lm_infer_amd import device as D
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").random_(0, 256)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    for rows in (1, 4):
        gen = Gen(torch, 1)
        t = DenseLayers(torch, ctx, gen, rows, (4, 4, 4, 4), tag=f"dec{rows}")
        mid = torch.empty(rows, F, dtype=torch.float16, device="cuda")
        r = rows
        calls = (lambda m: D.linear(ctx, m["qkv"], t.x_qkv, t.y_qkv, r, ws=t.ws["qkv"]),
                 lambda m: D.linear(ctx, m["o"], t.x_o, t.y_o, r, ws=t.ws["o"]),
                 lambda m: D.linear(ctx, m["gate_up"], t.x_ffn, mid, r, swiglu=True, ws=t.ws["gate_up"]),
                 lambda m: D.ffn(ctx, m["gate_up"], m["down"], t.x_ffn, t.y_ffn, r, gws=t.ws["gate_up"],
                                 dws=t.ws["down"]))
        for call in calls:
            for _ in range(reps):
                for m in t.w:
                    call(m)
            torch.cuda.synchronize()
        del t
        log(f"[bench] traffic probe M={rows}: qkv, o, gate_up, FFN call x{reps * LAYERS} each")
    log("[bench] traffic probe: copy 268435456 B x" + str(reps))


def lds_probe(torch, LP, cur, iters=4096):
    """LDS read bandwidth per CU (rk_npu_hip_lds_probe): one block per CU of
    4 or 8 waves, each wave streaming conflict-free 16-byte reads; bytes per
    shader-clock cycle per CU from the in-kernel cycle counts (median over the
    blocks), and the clock from the cycle and 100 MHz real-time counts."""
    import ctypes
    out = []
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.empty(cus * 8, dtype=torch.int32, device="cuda")
    clocks = torch.empty(cus * 2, dtype=torch.int64, device="cuda")
    for threads in (256, 512):
        for _ in range(2):  # the first launch warms the clock
            npu_check(LP.rk_npu_hip_lds_probe(cus, threads, iters, ctypes.c_void_p(sink.data_ptr()),
                                              ctypes.c_void_p(clocks.data_ptr()), cur()), "lds probe")
        torch.cuda.synchronize()
        c = clocks.view(cus, 2).cpu().tolist()
        cyc = statistics.median(r[0] for r in c)
        ticks = statistics.median(r[1] for r in c)
        nbytes = (threads // 64) * iters * 8 * 1024
        out.append({"waves_per_cu": threads // 64, "bytes_per_cu": nbytes, "cycles": int(cyc),
                    "bytes_per_clk_per_cu": round(nbytes / cyc, 1),
                    "clock_ghz": round(cyc / (ticks * 10.0), 3) if ticks else None})
        log(f"[probe] lds read {threads // 64} waves/CU: {out[-1]}")
    return out


LOAD_PROBE_SPANS = ((2 << 20, "2 MB (resident in each XCD's 4 MB L2)"),
                    (32 << 20, "32 MB (beyond the L2: the last-level cache)"),
                    (1 << 30, "1 GB (HBM)"))


def load_probe(torch, LP, cur, iters=512):
    """Global -> LDS load rate (rk_npu_hip_load_probe): every wave streams 1-KB
    chunks into its own LDS ring through the LDS DMA load the GEMM ring uses,
    8 loads in flight, from a source region resident in the L2, in the
    last-level cache, or in HBM; bytes per shader-clock cycle per CU (median
    block, times blocks per CU) and the aggregate rate over the launch."""
    import ctypes
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    out = []
    for span, where in LOAD_PROBE_SPANS:
        for threads, per_cu in ((512, 1), (256, 4)):
            blocks = cus * per_cu
            sink = torch.empty(blocks * threads // 64, dtype=torch.int32, device="cuda")
            clocks = torch.empty(blocks * 2, dtype=torch.int64, device="cuda")
            for _ in range(2):  # the first launch warms the caches and the clock
                npu_check(LP.rk_npu_hip_load_probe(blocks, threads, 8, 1, ctypes.c_void_p(src.data_ptr()), span, iters,
                                                   ctypes.c_void_p(sink.data_ptr()),
                                                   ctypes.c_void_p(clocks.data_ptr()), cur()), "load probe")
            torch.cuda.synchronize()
            c = clocks.view(blocks, 2).cpu().tolist()
            cyc = statistics.median(r[0] for r in c)
            ticks_max = max(r[1] for r in c)
            per_block = threads // 64 * iters * 1024
            out.append({"span": span, "where": where, "threads": threads, "blocks_per_cu": per_cu,
                        "bytes_per_clk_per_cu": round(per_block * per_cu / cyc, 1),
                        "tb_s": round(per_block * blocks / (ticks_max / 100e6) / 1e12, 2)})
            log(f"[probe] load {where} {threads}x{per_cu}/CU: {out[-1]}")
    del src
    return out


def mfma_rand_rate(torch, LP, blocks, warm_s=2.0, reps=20):
    """Sustained int8 MFMA rate on full-range operands (rk_npu_hip_mfma_rand_probe,
    `blocks` x 256 threads): replayed for warm_s seconds first, so the clock has
    settled where the chip's power limit puts it, then timed over `reps`
    replays of a graph of one launch."""
    import ctypes
    sink = torch.empty(blocks * 256, dtype=torch.int32, device="cuda")
    iters = 512
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def fn():
        npu_check(LP.rk_npu_hip_mfma_rand_probe(blocks, iters, ctypes.c_void_p(sink.data_ptr()), cur()), "mfma probe")
    t0 = time.time()
    while time.time() - t0 < warm_s:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
    ms, _ = graph_time(torch, fn, reps)
    return blocks * 4 * iters * 8 * 65536 / (ms * 1e-3) / 1e12


def power_probe(torch, ctx, LP, secs=4.0):
    """Socket power (amd-smi metric --power) and shader clock (rocm-smi -c),
    sampled every ~0.3 s while the GPU idles, runs the random-operand MFMA probe
    (8 waves per SIMD), and runs the M=4096 gate_up W4 GEMM + SwiGLU (a graph of
    8 calls on distinct weight copies) back to back for `secs` seconds each;
    medians per phase. Empty when the tools are missing."""
    import ctypes, functools, shutil, subprocess, threading
    from open_rknpu2_lm_infer_amd import device as D
    if not (shutil.which("amd-smi") and shutil.which("rocm-smi")):
        return []
    samples, phase, stop = [], ["idle"], [False]

    def sampler():
        while not stop[0]:
            try:
                o = subprocess.run(["amd-smi", "metric", "--power", "--json"], capture_output=True, text=True,
                                   timeout=10).stdout
                w = json.loads(o)["gpu_data"][0]["power"]["socket_power"]["value"]
                o = subprocess.run(["rocm-smi", "-c", "--json"], capture_output=True, text=True, timeout=10).stdout
                clk = next(iter(json.loads(o).values())).get("sclk clock speed:", "")
                samples.append((phase[0], float(w), int("".join(ch for ch in clk if ch.isdigit()) or 0)))
            except Exception:
                pass
            time.sleep(0.3)
    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    time.sleep(secs / 2)
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    sink = torch.empty(2048 * 256, dtype=torch.int32, device="cuda")
    gen = Gen(torch, 9)
    bits, m, k, n = 4, 4096, H, 2 * F
    codes, scales = gen.codes("pw/gu", bits, k, n), gen.scales("pw/gu", n)
    ws_ = [ctx.weights(bits, codes, scales) for _ in range(8)]
    del codes
    x = gen.acts("pw/gu/x", m, k, True)
    y = torch.empty(m, n // 2, dtype=torch.float16, device="cuda")
    wsp = ctx.workspace(bits, m, k, n)
    calls = [functools.partial(D.linear, ctx, w, x, y, m, swiglu=True, ws=wsp) for w in ws_]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for c in calls:
            c()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            for c in calls:
                c()
    torch.cuda.synchronize()
    phases = (("int8 MFMA, random operands, 8 waves/SIMD",
               lambda: npu_check(LP.rk_npu_hip_mfma_rand_probe(2048, 512, ctypes.c_void_p(sink.data_ptr()), cur()),
                                 "mfma probe"), 2048 * 4 * 512 * 8 * 65536),
              ("M=4096 gate_up 2560x19456 W4 GEMM + SwiGLU", g.replay, 8 * 2.0 * m * k * n))
    rates = {"idle": None}
    for name, fn, work in phases:
        fn()
        torch.cuda.synchronize()
        phase[0] = name
        t0, cnt = time.time(), 0
        while time.time() - t0 < secs:
            fn()
            cnt += 1
            if cnt % 8 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        rates[name] = work * cnt / (time.time() - t0) / 1e12
        phase[0] = "gap"
        time.sleep(1.0)
    stop[0] = True
    th.join()
    out = []
    for name in rates:
        w = sorted(x[1] for x in samples if x[0] == name)
        c = sorted(x[2] for x in samples if x[0] == name)
        if w:
            out.append({"phase": name, "watts": w[len(w) // 2], "sclk_mhz": c[len(c) // 2], "samples": len(w),
                        "tops": round(rates[name], 1) if rates[name] else None})
            log(f"[probe] power {out[-1]}")
    return out


def run_probes(torch, ctx, reps=20):
    """Ceilings measured on this GPU with the roofline probes of the
    measurement-only library libhip_probes.so (rk_npu_hip_mfma_probe,
    rk_npu_hip_stream_probe), beside the decode
    projections' own per-launch times in the same setting: 36 launches on 36
    distinct buffers / weight sets captured in a graph, HIP events on the
    replay stream, so every read comes from HBM."""
    import ctypes
    from open_rknpu2_lm_infer_amd import _ffi as FFI
    from open_rknpu2_lm_infer_amd import device as D
    L = FFI.lib()
    LP = FFI.probe_lib()
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    res = {"mfma_int8": [], "hbm_read": [], "decode_kernels": []}
    sink = torch.empty(4096 * 256, dtype=torch.int32, device="cuda")
    for blocks in (256, 512, 1024, 2048):
        iters = 512
        def fn():
            npu_check(LP.rk_npu_hip_mfma_probe(blocks, iters, ctypes.c_void_p(sink.data_ptr()), cur()), "mfma probe")
        ms, _ = graph_time(torch, fn, reps)
        ops = blocks * 4 * iters * 8 * 65536
        res["mfma_int8"].append({"blocks": blocks, "waves_per_simd": blocks // 256, "us": round(ms * 1e3, 2),
                                 "tops": round(ops / (ms * 1e-3) / 1e12, 1)})
        log(f"[probe] mfma blocks={blocks}: {res['mfma_int8'][-1]['tops']} TOPS")
    res["mfma_int8_random"] = []
    for blocks in (256, 512, 1024, 2048):
        res["mfma_int8_random"].append({"blocks": blocks, "waves_per_simd": blocks // 256,
                                        "tops": round(mfma_rand_rate(torch, LP, blocks), 1)})
        log(f"[probe] mfma random operands blocks={blocks}: {res['mfma_int8_random'][-1]['tops']} TOPS")
    res["lds_read"] = lds_probe(torch, LP, cur)
    res["load_rate"] = load_probe(torch, LP, cur)
    res["power"] = power_probe(torch, ctx, LP)
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
                    npu_check(LP.rk_npu_hip_stream_probe(ctypes.c_void_p(b.data_ptr()), b.numel(), blocks, thr, read,
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
    # The decode step against one layer's weights (50 MB, resident in the
    # 256 MB last-level cache) replayed 36 times: what the step would take if
    # its weight reads cost nothing beyond the cache.
    def layer0_x36():
        for _ in range(LAYERS):
            t.layer(t.w[0])
    ms_step, _ = graph_time(torch, t.step, reps)
    ms_warm, _ = graph_time(torch, layer0_x36, reps)
    nbytes = t.bytes_per_layer() * LAYERS
    res["decode_step_cache_warm"] = {
        "36 distinct layers (the bench step)": {"ms": round(ms_step, 4), "gbs": round(nbytes / ms_step / 1e6, 1)},
        "layer 0 x 36 (weights cache-resident)": {"ms": round(ms_warm, 4), "gbs": round(nbytes / ms_warm / 1e6, 1)}}
    log(f"[probe] decode step, cache-warm bound: {res['decode_step_cache_warm']}")
    del t
    torch.cuda.empty_cache()
    # One launch reading the decode step's whole weight volume (1.82 GB): the
    # HBM read rate a single stream sustains, the ceiling of a step whose
    # launches had no fixed cost.
    big = torch.empty(nbytes // 16 * 16, dtype=torch.uint8, device="cuda")
    res["hbm_read_step_volume"] = {"bytes": big.numel()}
    for blocks, thr in ((1024, 256), (2048, 256), (4096, 256), (1024, 512)):
        def fn():
            npu_check(LP.rk_npu_hip_stream_probe(ctypes.c_void_p(big.data_ptr()), big.numel(), blocks, thr, 1,
                                                ctypes.c_void_p(sinkb.data_ptr()), cur()), "stream probe")
        ms, _ = graph_time(torch, fn, 5)
        res["hbm_read_step_volume"][f"{blocks}x{thr}"] = {"ms": round(ms, 4), "gbs": round(big.numel() / ms / 1e6, 1)}
    log(f"[probe] one launch over the step's bytes: {res['hbm_read_step_volume']}")
    del big
    # The fixed cost of a launch against its grid: 36 launches of a kernel
    # that loads nothing, back to back in a graph (the decode GEMVs launch
    # 640-1280 blocks).
    res["launch_cost"] = []
    for blocks, thr in ((1, 64), (8, 256), (64, 256), (256, 256), (640, 256), (1280, 256), (2560, 256),
                        (5120, 256)):
        def fn():
            for _ in range(LAYERS):
                npu_check(LP.rk_npu_hip_stream_probe(ctypes.c_void_p(sinkb.data_ptr()), 0, blocks, thr, 0,
                                                    ctypes.c_void_p(sinkb.data_ptr()), cur()), "stream probe")
        ms, _ = graph_time(torch, fn, reps)
        res["launch_cost"].append({"blocks": blocks, "threads": thr, "us": round(ms * 1e3 / LAYERS, 3)})
    log(f"[probe] empty launches in a graph: {res['launch_cost']}")
    res["moe_t1_shared_in_bank"] = moe_shared_bank_t1(torch, ctx, reps * 10)
    log(f"[probe] MoE T=1 with the shared expert in the bank: {res['moe_t1_shared_in_bank']}")
    return res


def moe_shared_bank_t1(torch, ctx, steps):
    """One token through a MoE bank that holds the shared expert (h2048, 128
    experts, top-8, I768, W4 gate_up + W8 down, shared W8 expert of the same
    I): the shared down GEMV running the combine in its epilogue against the
    combine as its own launch (HM_GEMV_COMBINE=0); outputs compared bit for
    bit. Faster of eager and graph replay, HIP events."""
    import ctypes

    import numpy as np

    from open_rknpu2_lm_infer_amd import _ffi as F_
    from open_rknpu2_lm_infer_amd import device as D
    from open_rknpu2_lm_infer_amd import npu
    h, inter, experts, top = 2048, 768, 128, 8
    g = np.random.default_rng(0x5EED0004 + 1)
    L = F_.lib()
    keep, arr = [], (F_.rk_npu_moe_w8_expert * (experts + 1))()
    for e in range(experts + 1):
        lo = -8 if e < experts else -127  # routed gate_up W4, the shared expert W8
        gc = g.integers(lo, -lo, (h, 2 * inter), dtype=np.int8)
        gs = g.uniform(0.001, 0.01, 2 * inter).astype(np.float32)
        dc = g.integers(-127, 128, (inter, h), dtype=np.int8)
        ds = g.uniform(0.001, 0.01, h).astype(np.float32)
        keep.append((gc, gs, dc, ds))
        arr[e] = F_.rk_npu_moe_w8_expert(gc.ctypes.data_as(F_.i8p), gs.ctypes.data_as(F_.f32p),
                                         dc.ctypes.data_as(F_.i8p), ds.ctypes.data_as(F_.f32p))
    cfg = F_.rk_npu_moe_w8_config()
    L.rk_npu_moe_w8_config_init(ctypes.byref(cfg), h, inter, experts, 1, top, 1)
    bank = npu._Handle(L.rk_npu_moe_w4w8_weights_create(ctx.domain, ctypes.byref(cfg.weights), arr),
                       L.rk_npu_moe_w8_weights_free, "MoE bank", ctx.shared)
    work = npu._Handle(L.rk_npu_moe_w4w8_workspace_create(ctx.domain, ctypes.byref(cfg)),
                       L.rk_npu_moe_w8_workspace_free, "MoE workspace", ctx.shared)
    del arr, keep
    ids, rw = npu.routes(g.standard_normal(experts).astype(np.float32), top)
    ids, rw = np.asarray(ids, np.int32), np.asarray(rw, np.float32)
    x = torch.from_numpy(g.standard_normal((1, h)).astype(np.float32)).cuda()
    d_ids = torch.from_numpy(ids[None, :].astype(np.int32)).cuda()
    d_rw = torch.from_numpy(rw[None, :].astype(np.float32)).cuda()
    y = torch.empty(1, h, dtype=torch.float32, device="cuda")

    def step():
        npu_check(L.rk_npu_hip_moe_run(work.raw, bank.raw, 1, ctypes.c_void_p(x.data_ptr()),
                                       ctypes.c_void_p(d_ids.data_ptr()), ctypes.c_void_p(d_rw.data_ptr()),
                                       ctypes.c_void_p(y.data_ptr()), D.current_stream()), "MoE run")
    out, outs = {}, []
    for label, fuse in (("combine in the shared down GEMV", 1), ("combine as its own launch", 0)):
        with D.plan_switch("HM_GEMV_COMBINE", fuse):
            ms, ms_eager, ms_graph, ok = best_time(torch, step, steps, 10, lambda: [y.clone()])
            step()
            torch.cuda.synchronize()
            outs.append(y.cpu().numpy().copy())
        out[label] = {"us": round(ms * 1e3, 2), "eager_us": round(ms_eager * 1e3, 2),
                      "graph_us": round(ms_graph * 1e3, 2), "graph_matches_eager": ok}
    out["bit_identical"] = bool(np.array_equal(outs[0], outs[1]))
    return out


# GEMM shapes of the tile sweep: (name, bits, M, K, N, SwiGLU)
SWEEP_SHAPES = (("M128 up 2560x9728 W8", 8, 128, H, F, False), ("M512 gate_up 2560x19456 W4", 4, 512, H, 2 * F, True),
                ("M512 down 9728x2560 W8", 8, 512, F, H, False), ("M4096 qkv 2560x6144 W8", 8, 4096, H, Q + 2 * KV, False),
                ("M4096 o 4096x2560 W8", 8, 4096, Q, H, False),
                ("M4096 gate_up 2560x19456 W4", 4, 4096, H, 2 * F, True),
                ("M4096 down 9728x2560 W8", 8, 4096, F, H, False),
                ("M4096 lm_head 2560x151936 W8", 8, 4096, H, VOCAB, False))


def tile_sweep(torch, ctx, only=None, reps=5):
    """Every GEMM tile (HM_GEMM_VARIANT 0..5: 256x256, 256x128, 128x128, 64x128,
    32x128, 192x256) unsplit, and the split-K counts 2, 3, 4, 6, 8 (HM_SPLITS) of the
    128x128 and 64x128 tiles, plus the plan's own choice, on the GEMM shapes of
    the bench: one library call (quantization launch included) per distinct
    weight copy, enough copies that they exceed the last-level cache, in a
    graph. Workspaces are created under each setting so split partials fit."""
    from open_rknpu2_lm_infer_amd import device as D
    gen = Gen(torch, 7)
    configs = [(-1, 0)] + [(v, 1) for v in range(6)] + [(v, sp) for v in (2, 3) for sp in (2, 3, 4, 6, 8)]
    out = {}
    for name, bits, m, k, n, sw in SWEEP_SHAPES:
        if only and not any(o in name for o in only):
            continue
        copies = max(4, min(LAYERS, math.ceil(600e6 / (k * n * bits // 8))))
        codes, scales = gen.codes(name, bits, k, n), gen.scales(name, n)
        ws_ = [ctx.weights(bits, codes, scales) for _ in range(copies)]
        del codes
        x = gen.acts(name + "/x", m, k, True)
        y = torch.empty(m, n // 2 if sw else n, dtype=torch.float16, device="cuda")
        row = {}
        # one untimed pass first (the first timed setting of a shape read ~5%
        # slow), the plan's own choice timed last
        with D.plan_switch("HM_GEMM_VARIANT", -1):
            per_launch_us(torch, [functools.partial(D.linear, ctx, w, x, y, m, swiglu=sw, ws=ctx.workspace(bits, m, k, n))
                                  for w in ws_], 1)
        for v, sp in configs[1:] + configs[:1]:
            with D.plan_switch("HM_GEMM_VARIANT", v), D.plan_switch("HM_SPLITS", sp):
                wsp = ctx.workspace(bits, m, k, n, cached=False)
                us = per_launch_us(torch, [functools.partial(D.linear, ctx, w, x, y, m, swiglu=sw, ws=wsp)
                                           for w in ws_], reps)
            key = "plan" if v < 0 else f"tile{v}" + (f"/k{sp}" if sp > 1 else "")
            row[key] = round(us, 2)
        best = min(row, key=row.get)
        out[name] = {"us": row, "best": best, "tops_best": round(2.0 * m * k * n / row[best] / 1e6, 1),
                     "copies": copies}
        log(f"[sweep] {name}: best {best} {row[best]} us, plan {row['plan']} us")
        del ws_
        torch.cuda.empty_cache()
    return out


ROOF_REPS = 50  # graph replays per roofline pass (36 launches each)


def roofline_only(torch, ctx, which="all"):
    """Every line's roofline passes (or one line's) and nothing else: the
    launches of a kernel-trace profile of this command are the timed ones,
    apart from two eager warm-up calls per pass (fn() before capture and on
    the capture stream) and one warm replay."""
    out = {}
    if which in ("all", "decode"):
        for rows in (1, 4):
            r = run_decode(torch, ctx, rows, 0, 0, False, timed=False, reps=ROOF_REPS)
            out[f"decode M={rows}"] = {"projections": r["projections"], "roofline": r["roofline"]}
    if which in ("all", "prefill"):
        r = run_prefill(torch, ctx, 4096, 0, 0, want_cpu=False, timed=False, reps=4)
        out["prefill M=4096"] = {"projections": r["projections"], "roofline": r["roofline"]}
    if which in ("all", "ffn512"):
        out["ffn M=512"] = run_ffn512(torch, ctx, 0, 0, want_cpu=False, timed=False, reps=4)["roofline"]
    if which in ("all", "up128"):
        out["up M=128"] = run_up128(torch, ctx, 0, 0, want_cpu=False, timed=False, reps=20)["roofline"]
    return out


def summarize_trace(path, top=60):
    """Per (kernel, grid) launch statistics of a rocprofv3 --kernel-trace CSV
    (columns Kernel_Name, Grid_Size*, Workgroup_Size*, Start_Timestamp,
    End_Timestamp in ns): count, mean / median / p10 / p90 duration in us,
    ordered by total time. Grids are in work-items, as rocprofv3 writes them."""
    groups = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            name = row.get("Kernel_Name", "?")
            grid = row.get("Grid_Size_X") or row.get("Grid_Size") or "?"
            wg = row.get("Workgroup_Size_X") or row.get("Workgroup_Size") or "?"
            dur = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3
            groups.setdefault((name, grid, wg), []).append(dur)
    rows = sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:top]
    lines = [f"{'total_us':>12} {'count':>6} {'mean_us':>9} {'median':>9} {'p10':>9} {'p90':>9} {'grid':>9} {'wg':>4}  kernel"]
    for (name, grid, wg), d in rows:
        d.sort()
        q = lambda p: d[min(len(d) - 1, int(p * len(d)))]
        short = name if len(name) <= 150 else name[:147] + "..."
        lines.append(f"{sum(d):12.1f} {len(d):6d} {statistics.mean(d):9.3f} {statistics.median(d):9.3f} "
                     f"{q(0.1):9.3f} {q(0.9):9.3f} {grid:>9} {wg:>4}  {short}")
    return "\n".join(lines)


def summarize_counters(path, top=60):
    """Per (kernel, grid) medians of each counter of a rocprofv3 --pmc CSV
    (one row per dispatch and counter: Kernel_Name, Grid_Size, Counter_Name,
    Counter_Value), ordered by dispatch count then name."""
    groups = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            key = (row.get("Kernel_Name", "?"), row.get("Grid_Size") or row.get("Grid_Size_X") or "?")
            groups.setdefault(key, {}).setdefault(row["Counter_Name"], []).append(float(row["Counter_Value"]))
    items = sorted(groups.items(), key=lambda kv: (-max(len(v) for v in kv[1].values()), kv[0][0]))[:top]
    lines = []
    for (name, grid), counters in items:
        short = name if len(name) <= 150 else name[:147] + "..."
        vals = "  ".join(f"{c}={statistics.median(v):.1f}" for c, v in sorted(counters.items()))
        n = max(len(v) for v in counters.values())
        lines.append(f"{n:6d} grid={grid:>9}  {vals}  {short}")
    return "\n".join(lines)


# --- profiles/ --------------------------------------------------------------------
# `bench.py --profile NAME INPUT...` prints the whole text of one file under
# profiles/ from the outputs of the commands its header states (run from the
# repository root on one MI355X, rocprofv3 with TMPDIR=/tmp), so every table
# there is regenerated by committed code:
#   roofline  BENCH_JSON ROOF_JSON TRACE_CSV    -> roofline_passes_kernel_trace.txt
#   traffic   FETCH_CSV WRITE_CSV               -> traffic_decode_gemv_m1_m4.txt
#   gemm-counters PMC1_CSV PMC2_CSV PROBES_JSON -> counters_gemm_prefill_m4096.txt
#   probes    PROBES_JSON                       -> probes_hbm_read_floor_mfma_rate.txt
#   sweep     SWEEP_JSON                        -> gemm_tile_sweep.txt
#   moe       STATS_CSV MOE_JSON                -> moe_35b_a3b_t512_t1_kernel_stats.txt
#   attention STATS_CSV ATTN_JSON PMC1_CSV PMC2_CSV -> attention_gqa_decode_prefill_kernel_stats.txt

PROFILE_SETUP = "  cd /tmp && export TMPDIR=/tmp && cd <repo>"


def _last_json(path):
    for line in reversed(open(path).read().strip().splitlines()):
        if line.strip()[:1] in ("{", "["):
            return json.loads(line)
    raise ValueError(f"{path}: no JSON line")


def _kname(name):
    """A kernel's demangled name without the namespace and parameter list."""
    name = name[5:] if name.startswith("void ") else name
    name = name.replace("hm::", "")
    i = name.rfind("(")
    return name[:i] if i > 0 else name


def _trace(path):
    """(kernel, grid in work-items, workgroup) -> per-dispatch durations (us)
    of a rocprofv3 --kernel-trace CSV."""
    groups = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            grid = int(row.get("Grid_Size_X") or row.get("Grid_Size") or 0)
            wg = int(row.get("Workgroup_Size_X") or row.get("Workgroup_Size") or 0)
            d = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3
            groups.setdefault((_kname(row.get("Kernel_Name", "?")), grid, wg), []).append(d)
    return groups


def _pick(groups, must, grid):
    """The one group whose kernel name holds every string of `must` at this grid."""
    hits = [k for k in groups if k[1] == grid and all(m in k[0] for m in must)]
    if len(hits) != 1:
        raise ValueError(f"{must} grid {grid}: {len(hits)} matches {hits[:4]}")
    return hits[0]


def _counters(path):
    """Dispatch id -> ({counter: value}, kernel, grid, workgroup, duration us)
    of a rocprofv3 --pmc CSV."""
    disp = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            k = r["Dispatch_Id"]
            if k not in disp:
                dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
                disp[k] = ({}, _kname(r["Kernel_Name"]), int(r["Grid_Size"]), int(r.get("Workgroup_Size") or 0), dur)
            disp[k][0][r["Counter_Name"]] = float(r["Counter_Value"])
    return disp


def _sec(bench, prefix):
    return next(x for x in bench["secondary"] if x["workload"].startswith(prefix))


# Roofline passes: (label, [(name parts, grid)], work per call, bound,
# the bench line's avg_us, the --roofline-only output's avg_us). A pass whose
# library call is several launches adds their durations.
def _roof_passes(bench, roof):
    P, R = bench["projections"], roof["decode M=1"]["projections"]
    dn = "down (ffn call - gate_up)"
    return [
        ("decode M=1 qkv 2560x6144 W4", [(["gemv_kernel<__half, 1, 4, 0,"], 196608)], lin_bytes(4, H, Q + 2 * KV, 1),
         "hbm", P["qkv"]["us"], R["qkv"]["us"]),
        ("decode M=1 o 4096x2560 W4", [(["gemv_kernel<__half, 1, 4, 0,"], 81920)], lin_bytes(4, Q, H, 1), "hbm",
         P["o"]["us"], R["o"]["us"]),
        ("decode M=1 gate_up 2560x19456 W4 +SwiGLU (roofline kernel)",
         [(["gemv_kernel<__half, 1, 4, 2,"], 389120)], lin_bytes(4, H, 2 * F, 1), "hbm", P["gate_up"]["us"],
         R["gate_up"]["us"]),
        ("decode M=1 down 9728x2560 W4 (second launch of the FFN call)",
         [(["gemv_kernel<float, 1, 4, 0,", "true>"], 327680)], lin_bytes(4, F, H, 1), "hbm", P[dn]["us"], R[dn]["us"]),
        ("decode M=4 gate_up W4 +SwiGLU (quantization launch + GEMV)",
         [(["quant_rows_kernel<__half, 0,"], 1024), (["gemv_kernel<float, 4, 4, 2,"], 311296)],
         lin_bytes(4, H, 2 * F, 4), "hbm", _sec(bench, "decode M=4")["roofline"]["avg_us"],
         roof["decode M=4"]["roofline"]["avg_us"]),
        ("prefill M=4096 gate_up W4 +SwiGLU (quantization launch + GEMM)",
         [(["quant_tile_kernel<__half, 0,"], 262144), (["gemm_kernel<128, 128, 2, 2, 4, 2, true"], 1245184)],
         2.0 * 4096 * H * 2 * F, "mfma", _sec(bench, "prefill")["roofline"]["avg_us"],
         roof["prefill M=4096"]["roofline"]["avg_us"]),
        ("FFN M=512 call (quantization, gate_up GEMM, requant, down GEMM pieces, finish)",
         [(["quant_tile_kernel<__half, 0,"], 32768), (["gemm_kernel<64, 128, 2, 2, 4, 2, true"], 311296),
          (["quant_tile_kernel<float, 0,"], 32768), (["gemm_kernel<128, 128, 2, 2, 8, 0, true, 1>"], 61440),
          (["gemm_split_finish_kernel<8, 0>"], 20480)],
         2.0 * 512 * (H * 2 * F + F * H), "mfma", _sec(bench, "FFN block")["roofline"]["avg_us"],
         roof["ffn M=512"]["avg_us"]),
        ("M=128 W8A8 up 2560x9728 call (quantization launch + GEMM)",
         [(["quant_rows_kernel<__half, 0,"], 32768), (["gemm_kernel<64, 128, 2, 2, 8, 0, true, 0>"], 38912)],
         lin_bytes(8, H, F, 128), "hbm", _sec(bench, "W8A8 linear")["roofline"]["avg_us"],
         roof["up M=128"]["avg_us"]),
    ]


def profile_roofline(bench_json, roof_json, trace_csv):
    bench, roof, groups = _last_json(bench_json), _last_json(roof_json), _trace(trace_csv)
    out = ["Kernel trace of every roofline pass of bench.py, one MI355X (gfx950), one build.", "",
           "Commands (repository root):", PROFILE_SETUP,
           "  python3 bench.py > bench.json",
           "  rocprofv3 --kernel-trace --stats --output-format csv -d <out> -o roof -- python3 -u bench.py "
           "--roofline-only > roof.json",
           "  python3 bench.py --profile roofline bench.json roof.json <out>/<host>/<pid>_roof_kernel_trace.csv", "",
           "bench.py --roofline-only runs only the roofline passes: per pass, 36 library calls on 36 layers' distinct",
           "weights captured in one HIP graph and replayed (decode 50 times, prefill and FFN M=512 4 times, M=128",
           "20 times) after two eager calls; the trace holds those launches.",
           "  rocprof mean / median: per-dispatch kernel duration (begin to end) under the profiler, summed over the",
           "    launches of one library call;",
           "  events: the same launches' graph replay period (HIP events on the replay stream) in the profiled run;",
           "  bench: the bench line's avg_us (the same measurement without the profiler: what the line reports).",
           "frac = work per call / time / peak (8 TB/s HBM, or 5.0 POP/s dense int8).", "",
           f"{'pass':62} {'rocprof':>8} {'median':>8} {'events':>8} {'bench':>8} {'frac(rocprof)':>13} {'frac(bench)':>11}"]
    fr = {}
    for label, parts, work, bound, b_us, r_us in _roof_passes(bench, roof):
        keys = [_pick(groups, m, g) for m, g in parts]
        mean = sum(statistics.mean(groups[k]) for k in keys)
        med = sum(statistics.median(groups[k]) for k in keys)
        peak = 8e12 if bound == "hbm" else 5e15
        f_r, f_b = work / (mean * 1e-6) / peak, work / (b_us * 1e-6) / peak
        fr[label] = (mean, b_us, f_r, f_b)
        out.append(f"{label[:62]:62} {mean:8.3f} {med:8.3f} {r_us:8.3f} {b_us:8.3f} {f_r:13.4f} {f_b:11.4f}")
        out.append("    " + " + ".join(f"{k[0]} grid {k[1]} x{len(groups[k])}" for k in keys)
                   + f"; work {work:.6g} {'B' if bound == 'hbm' else 'ops'} per call")
    gu = next(v for k, v in fr.items() if "(roofline kernel)" in k)
    out += ["", "Reading:",
            f"- The bench line's roofline kernel (decode gate_up GEMV): {gu[1]:.3f} us per launch back to back in a",
            f"  graph (frac {gu[3]:.4f}), {gu[0]:.3f} us per dispatch under the profiler (frac {gu[2]:.4f}). The profiler",
            "  serializes dispatches (its graph period is the events column); without it one launch's drain overlaps",
            "  the next launch's start, which is how the launches run in the step. Both fractions are reported here;",
            "  the bench line's is the graph period's.",
            f"- The decode step as a whole: {bench['value']:.2f} GB/s, {bench['value'] / 8000:.4f} of 8 TB/s "
            f"({bench['ms_per_step']:.4f} ms per step of 36 layers).",
            "- Algorithmic bytes (hbm): weights at storage width + f32 column scales + fp16 activations in and out;",
            "  ops (mfma): 2*M*K*N.", "",
            "Per-kernel launch statistics of the whole trace (top 45 by total time):"]
    out += summarize_trace(trace_csv, top=45).splitlines()
    return "\n".join(out)


TRAFFIC_SPEC = [
    ("M=1 qkv 2560x6144", ["gemv_kernel<__half, 1, 4, 0,"], 196608, lin_bytes(4, H, Q + 2 * KV, 1)),
    ("M=1 o 4096x2560", ["gemv_kernel<__half, 1, 4, 0,"], 81920, lin_bytes(4, Q, H, 1)),
    ("M=1 gate_up 2560x19456 +SwiGLU", ["gemv_kernel<__half, 1, 4, 2,"], 389120, lin_bytes(4, H, 2 * F, 1)),
    ("M=1 down 9728x2560 (split K, f32 middle in)", ["gemv_kernel<float, 1, 4, 0,", "true>"], 327680,
     lin_bytes(4, F, H, 1)),
    ("M=4 qkv (rows quantized beforehand)", ["gemv_kernel<float, 4, 4, 0,"], 196608, lin_bytes(4, H, Q + 2 * KV, 4)),
    ("M=4 o", ["gemv_kernel<float, 4, 4, 0,"], 81920, lin_bytes(4, Q, H, 4)),
    ("M=4 gate_up +SwiGLU", ["gemv_kernel<float, 4, 4, 2,"], 311296, lin_bytes(4, H, 2 * F, 4)),
    ("M=4 down (512-thread blocks)", ["gemv_kernel<float, 4, 4, 0,"], 163840, lin_bytes(4, F, H, 4)),
]


def _per_kernel(disp, counter):
    """(kernel, grid) -> median of one counter over its dispatches."""
    groups = {}
    for vals, name, grid, _, _ in disp.values():
        if counter in vals:
            groups.setdefault((name, grid), []).append(vals[counter])
    return {k: (statistics.median(v), len(v)) for k, v in groups.items()}


def profile_traffic(fetch_csv, write_csv):
    fe, wr = _per_kernel(_counters(fetch_csv), "FETCH_SIZE"), _per_kernel(_counters(write_csv), "WRITE_SIZE")
    # the calibration copy: the dispatch writing 262,144 KiB
    cal = [k for k, (v, _) in wr.items() if abs(v - 262144.0) < 64.0 and "copy" in k[0].lower()]
    if len(cal) != 1:
        raise ValueError(f"calibration copy: {cal}")
    cf, cw = fe[cal[0]][0], wr[cal[0]][0]
    ff, fw = 262144.0 / cf, 262144.0 / cw
    out = ["HBM traffic of the decode GEMVs (M=1 and M=4, W4 weights, Qwen3-4B-shaped projections), one MI355X.", "",
           "Commands (repository root; two counter runs of the same workload, each in its own process):",
           PROFILE_SETUP,
           "  rocprofv3 --pmc FETCH_SIZE --output-format csv -d <out_fetch> -o run -- python3 -u bench.py --traffic-probe",
           "  rocprofv3 --pmc WRITE_SIZE --output-format csv -d <out_write> -o run -- python3 -u bench.py --traffic-probe",
           "  python3 bench.py --profile traffic <out_fetch>/<host>/<pid>_run_counter_collection.csv "
           "<out_write>/<host>/<pid>_run_counter_collection.csv", "",
           "--traffic-probe: a 268,435,456-byte device copy (calibration), then at M=1 and M=4 three passes over 36",
           "layers' distinct weights of each projection in turn (qkv, o, gate_up + SwiGLU, the FFN call), so every",
           "dispatch reads its weights from HBM. Values are KiB per dispatch, medians over the dispatches.",
           f"Calibration ({cal[0][0]}): FETCH_SIZE {cf:.1f} KiB and WRITE_SIZE {cw:.1f} KiB for 262,144 KiB read and",
           f"written: bytes = FETCH_SIZE x {ff:.3f} x 1024 + WRITE_SIZE x {fw:.3f} x 1024.", "",
           f"{'kernel (grid in work-items)':48} {'FETCH KiB':>10} {'WRITE KiB':>10} {'traffic B':>12} "
           f"{'algorithmic B':>14} {'ratio':>6}"]
    for label, must, grid, alg in TRAFFIC_SPEC:
        kf = [k for k in fe if k[1] == grid and all(m in k[0] for m in must)]
        kw = [k for k in wr if k[1] == grid and all(m in k[0] for m in must)]
        if len(kf) != 1 or len(kw) != 1:
            raise ValueError(f"{label}: {kf} {kw}")
        (f, n), (w, _) = fe[kf[0]], wr[kw[0]]
        t = f * ff * 1024 + w * fw * 1024
        out.append(f"{label:48} {f:10.1f} {w:10.1f} {t:12.0f} {alg:14d} {t / alg:6.3f}")
        out.append(f"    {kf[0][0]} grid {grid} ({n} dispatches)")
    out += ["", "Algorithmic bytes: weights at 4 bits + f32 column scales + fp16 activations in and out (the f32",
            "middle of the down projection and the row-max partials are not counted). A ratio near 1 means every",
            "weight byte is read from HBM once and nothing else of size is: the gap to the 8 TB/s roofline is time,",
            "not bytes. bench.py's primary roofline carries traffic = the M=1 gate_up row (TRAFFIC_GEMV_GATE_UP)."]
    return "\n".join(out)


GEMM_ROLES = [
    # (role, kernel, grid in work-items, o/down told apart by duration, ops,
    #  wave tile in 32x32 fragments (FM, FN), W4, block tile (BM, BN))
    ("qkv 2560x6144 W8 (1536 tiles of 128x128)", "gemm_kernel<128, 128, 2, 2, 8, 0, true, 0>", 393216, None,
     2.0 * 4096 * H * (Q + 2 * KV), 2, 2, False, 128, 128),
    ("o 4096x2560 W8 (220 tiles of 192x256)", "gemm_kernel<192, 256, 2, 4, 8, 0, true, 0>", 112640, "short",
     2.0 * 4096 * Q * H, 3, 2, False, 192, 256),
    ("gate_up 2560x19456 W4 +SwiGLU (4864 tiles)", "gemm_kernel<128, 128, 2, 2, 4, 2, true, 0>", 1245184, None,
     2.0 * 4096 * H * 2 * F, 2, 2, True, 128, 128),
    ("down 9728x2560 W8 (220 tiles of 192x256)", "gemm_kernel<192, 256, 2, 4, 8, 0, true, 0>", 112640, "long",
     2.0 * 4096 * F * H, 3, 2, False, 192, 256),
    ("lm_head 2560x151936 W8 (9504 tiles of 256x256)", "gemm_kernel<256, 256, 2, 4, 8, 0, true, 0>", 4866048, None,
     2.0 * 4096 * H * VOCAB, 4, 2, False, 256, 256),
]


# LDS bytes read per MFMA (v_mfma_i32_32x32x32_i8: a 32x32 A fragment and a
# 32x32 B fragment of one 32-k step) for a wave tile of FM x FN fragments:
# A 1 KB per row block, B 1 KB (W8) or 0.5 KB (W4, packed) per column block,
# shared by the wave's FM * FN MFMAs.
def _lds_per_mfma(fm, fn, w4):
    return (fm * 1024 + fn * (512 if w4 else 1024)) / (fm * fn)


def profile_gemm_counters(pmc1_csv, pmc2_csv, probes_json):
    r1, r2 = _counters(pmc1_csv), _counters(pmc2_csv)
    probes = _last_json(probes_json)
    lds_peak = max(x["bytes_per_clk_per_cu"] for x in probes.get("lds_read", [{"bytes_per_clk_per_cu": 0}]))

    def pick(disp, sub, grid, split):
        ks = [k for k, v in disp.items() if sub in v[1] and v[2] == grid]
        if split:
            durs = sorted(disp[k][4] for k in ks)
            cut = (durs[0] + durs[-1]) / 2
            ks = [k for k in ks if (disp[k][4] < cut) == (split == "short")]
        return ks

    med = lambda disp, ks, c: statistics.median(disp[k][0][c] for k in ks)
    out = ["Hardware counters of the M=4096 prefill GEMMs (Qwen3-4B-shaped set + lm_head), one MI355X.", "",
           "Commands (repository root; two counter runs, each in its own process, no tracing options):", PROFILE_SETUP,
           "  rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_WAIT_ANY SQ_INSTS_LDS SQ_WAVES "
           "GRBM_GUI_ACTIVE \\",
           "      --output-format csv -d <out1> -o run -- python3 -u bench.py --roofline-only prefill",
           "  rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_VALU SQ_INSTS_SALU SQ_INSTS_SMEM "
           "SQ_WAIT_INST_LDS GRBM_GUI_ACTIVE \\",
           "      --output-format csv -d <out2> -o run -- python3 -u bench.py --roofline-only prefill",
           "  python3 bench.py --probes > probes.json",
           "  python3 bench.py --profile gemm-counters <out1>/<host>/<pid>_run_counter_collection.csv "
           "<out2>/<host>/<pid>_run_counter_collection.csv probes.json", "",
           "Per-dispatch medians; counters are summed over the 8 XCDs (GRBM_GUI_ACTIVE / 8 is one XCD's busy cycles).",
           "  MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 x 1024 SIMDs);",
           "  clock = GRBM_GUI_ACTIVE / 8 / the dispatch's duration;",
           "  LDS util = SQ_LDS_IDX_ACTIVE / (GRBM_GUI_ACTIVE / 8 x 256 CUs) (rocprofv3's LdsUtil), in the run of pass 2;",
           "  LDS B/MFMA = LDS bytes the wave tile reads per v_mfma_i32_32x32x32_i8 (fragment geometry);",
           "  WAIT_ANY, WAIT_LDS = SQ_WAIT_ANY, SQ_WAIT_INST_LDS per SQ_WAVE_CYCLES; confl = SQ_LDS_BANK_CONFLICT /",
           "  SQ_LDS_IDX_ACTIVE; VALU/wave, LDS/wave = instructions per wave.",
           "The o and down GEMMs share one kernel and grid; their dispatches are told apart by duration.", "",
           "  load B/clk/CU = the GEMM's stage loads (every tile's A and B bytes for every 64-k stage) per clock",
           "  cycle per CU holding tiles (min(256, tiles)), at the clock of the same row.", "",
           f"{'GEMM (role)':44} {'dur us':>7} {'GHz':>5} {'POP/s':>6} {'MFMA':>5} {'load':>5} {'LDS util':>8} "
           f"{'B/MFMA':>6} {'WAIT_ANY':>8} {'WAIT_LDS':>8} {'confl':>6} {'VALU/wave':>9} {'LDS/wave':>8}"]
    for label, sub, grid, split, ops, fm, fn, w4, bm, bn in GEMM_ROLES:
        k1, k2 = pick(r1, sub, grid, split), pick(r2, sub, grid, split)
        if not k1 or not k2:
            raise ValueError(f"{label}: no dispatches")
        dur = statistics.median(r1[k][4] for k in k1)
        grbm = med(r1, k1, "GRBM_GUI_ACTIVE") / 8
        grbm2 = med(r2, k2, "GRBM_GUI_ACTIVE") / 8
        wc = med(r1, k1, "SQ_WAVE_CYCLES")
        waves = med(r1, k1, "SQ_WAVES")
        lds_act = med(r2, k2, "SQ_LDS_IDX_ACTIVE")
        tiles = grid // r1[k1[0]][3]
        load_bytes = ops / 2 * (1.0 / bn + (0.5 if w4 else 1.0) / bm)
        load = load_bytes / (grbm * min(256, tiles))
        out.append(f"{label:44} {dur:7.1f} {grbm / dur / 1e3:5.2f} {ops / (dur * 1e-6) / 1e15:6.2f} "
                   f"{med(r1, k1, 'SQ_VALU_MFMA_BUSY_CYCLES') / (grbm * 1024):5.3f} {load:5.1f} "
                   f"{lds_act / (grbm2 * 256):8.3f} "
                   f"{_lds_per_mfma(fm, fn, w4):6.0f} {med(r1, k1, 'SQ_WAIT_ANY') / wc:8.3f} "
                   f"{med(r2, k2, 'SQ_WAIT_INST_LDS') / wc:8.3f} {med(r2, k2, 'SQ_LDS_BANK_CONFLICT') / lds_act:6.3f} "
                   f"{med(r2, k2, 'SQ_INSTS_VALU') / waves:9.0f} {med(r1, k1, 'SQ_INSTS_LDS') / waves:8.0f}")
        out.append(f"    {sub} grid {grid} wg {r1[k1[0]][3]} ({len(k1)} + {len(k2)} dispatches)")
    mf = probes.get("mfma_int8", [])
    if mf:
        out += ["", "Ceilings on the same build (bench.py --probes): int8 MFMA from registers "
                + ", ".join(f"{x['tops'] / 1000:.2f} POP/s at {x['waves_per_simd']} waves/SIMD" for x in mf) + ";",
                "LDS reads (conflict-free 16-byte, one block per CU) "
                + ", ".join(f"{x['bytes_per_clk_per_cu']} B/clk/CU at {x['waves_per_cu']} waves/CU ({x['clock_ghz']} GHz)"
                            for x in probes.get("lds_read", [])) + "."]
    rnd = probes.get("mfma_int8_random", [])
    if rnd:
        out += ["int8 MFMA from registers on random operand bytes (the bit activity of real data): "
                + ", ".join(f"{x['tops'] / 1000:.2f} POP/s at {x['waves_per_simd']} waves/SIMD" for x in rnd)
                + " (the clock lowered by the board's power management)."]
    for r in probes.get("power", []):
        if r.get("tops"):
            out += [f"Power, {r['phase']}: {r['watts']:.0f} W at {r['sclk_mhz']} MHz ({r['tops'] / 1000:.2f} POP/s)."]
    lr = probes.get("load_rate", [])
    if lr:
        out += ["Global -> LDS loads (rk_npu_hip_load_probe, 8 in flight per wave), B/clk/CU: "
                + "; ".join(f"{x['where'].split(' (')[0]} {x['bytes_per_clk_per_cu']} ({x['threads'] // 64} waves x "
                            f"{x['blocks_per_cu']})" for x in lr) + " (sources resident in the L2, in the last-level "
                "cache, in HBM)."]
    out += ["", "Reading: LDS utilisation stays at about a fifth of the cycles and the measured LDS read rate",
            f"({lds_peak} B/clk/CU) is several times what the tiles ask for; bank conflicts are a few percent. The",
            "matrix cores idle on the rest: the per-stage barrier and the waits for each stage's loads. The stage",
            "loads arrive at a rate between the probe's L2-resident and last-level-cache rates: every stage waits",
            "for its slowest load, and a stage's loads include L2 misses."]
    return "\n".join(out)


def profile_probes(probes_json):
    d = _last_json(probes_json)
    out = ["Ceilings measured on one MI355X with the measurement library's probes (libhip_probes.so,",
           "csrc/probes.hip), beside the decode projections' own launches.", "",
           "Command (repository root):", PROFILE_SETUP, "  python3 bench.py --probes > probes.json",
           "  python3 bench.py --profile probes probes.json", "",
           "rk_npu_hip_mfma_probe: back-to-back independent v_mfma_i32_32x32x32_i8 from registers, no memory",
           "traffic (8 accumulators per wave), graph of one launch replayed 20 times:",
           " blocks waves/SIMD       us     TOPS"]
    for r in d["mfma_int8"]:
        out.append(f"{r['blocks']:7d} {r['waves_per_simd']:10d} {r['us']:8.2f} {r['tops']:8.1f}")
    tops = [r["tops"] for r in d["mfma_int8"]]
    out += ["", f"The int8 rate the chip holds is {min(tops) / 1000:.1f}-{max(tops) / 1000:.1f} POP/s "
            f"({min(tops) / 50:.0f}-{max(tops) / 50:.0f}% of the 5.0 POP/s dense figure) on these operands, whose bytes",
            "are mostly zero."]
    if d.get("mfma_int8_random"):
        out += ["", "rk_npu_hip_mfma_rand_probe: the same loop on full-range hashed operand bytes, a different operand",
                "pair per MFMA (the bit activity of a GEMM on real data), replayed for 2 s before it is timed:",
                " blocks waves/SIMD     TOPS"]
        for r in d["mfma_int8_random"]:
            out.append(f"{r['blocks']:7d} {r['waves_per_simd']:10d} {r['tops']:8.1f}")
    if d.get("power"):
        out += ["", "Socket power (amd-smi metric --power) and shader clock (rocm-smi -c), medians of samples every",
                "~0.3 s while each workload runs back to back for 4 s (board limit: 1400 W):"]
        for r in d["power"]:
            rate = f"{r['tops']:8.1f} TOPS" if r.get("tops") else " " * 13
            out.append(f"    {r['phase']:44} {r['watts']:7.0f} W {r['sclk_mhz']:6d} MHz {rate}")
    out += [""]
    out += [
            "rk_npu_hip_lds_probe: one block per CU, every wave streaming conflict-free 16-byte LDS reads (8 in",
            "flight); cycles and clock from the kernel's own s_memtime / s_memrealtime:"]
    for r in d.get("lds_read", []):
        out.append(f"    {r['waves_per_cu']} waves/CU: {r['bytes_per_clk_per_cu']} B/clk/CU at {r['clock_ghz']} GHz")
    if d.get("load_rate"):
        out += ["", "rk_npu_hip_load_probe: every wave streaming 1-KB chunks into its own LDS ring with the GEMM ring's",
                "LDS DMA load (global_load_lds_dwordx4), 8 in flight, from a region of the given size (each wave",
                "walking it from its own start); B/clk/CU from the kernel's cycle counts, TB/s over the launch:"]
        for r in d["load_rate"]:
            out.append(f"    {r['where']:46} {r['threads'] // 64} waves x {r['blocks_per_cu']} blocks/CU: "
                       f"{r['bytes_per_clk_per_cu']:6.1f} B/clk/CU {r['tb_s']:6.2f} TB/s")
    out += ["", "rk_npu_hip_stream_probe: one launch reading each projection's weight bytes (36 distinct buffers in",
            "a graph, so every read comes from HBM) with the GEMV's 16-byte non-temporal loads, at several grids;",
            "'empty' is the same grid with no loads (the launch's fixed cost); the projection's own GEMV launch",
            "is timed in the same way:"]
    best = {}
    for p in d["hbm_read"]:
        g = p["gemv_grid"]
        out.append(f"{p['projection']} ({p['bytes']} B, GEMV grid {g[0]} x {g[1]} threads):")
        reads = []
        for k, v in p.items():
            if isinstance(v, dict) and "us" in v:
                out.append(f"    {k:42} {v['us']:8.3f} us" + (f" {v['gbs']:9.1f} GB/s" if v.get("gbs") else ""))
                if k.startswith("read"):
                    reads.append(v["us"])
        best[p["projection"]] = min(reads)
    c = d["decode_step_cache_warm"]
    a, b = c["36 distinct layers (the bench step)"], c["layer 0 x 36 (weights cache-resident)"]
    v = d.get("hbm_read_step_volume")
    if v:
        rates = {k: x["gbs"] for k, x in v.items() if isinstance(x, dict)}
        best_k = max(rates, key=rates.get)
        out += ["", f"One launch reading the decode step's whole weight volume ({v['bytes']} B) with the same loads:",
                "    " + ", ".join(f"{k} {x['ms']:.4f} ms {x['gbs']:.1f} GB/s" for k, x in v.items()
                               if isinstance(x, dict)),
                f"    best {rates[best_k]:.1f} GB/s ({rates[best_k] / 80:.1f}% of 8 TB/s): the HBM read rate one stream "
                "sustains, the ceiling of a decode step whose launches cost nothing."]
    if d.get("launch_cost"):
        out += ["", "Fixed cost of a launch against its grid (36 launches of a kernel that loads nothing, back to back",
                "in a graph, us per launch):",
                "    " + ", ".join(f"{r['blocks']} x {r['threads']}: {r['us']:.2f}" for r in d["launch_cost"])]
    m = d["moe_t1_shared_in_bank"]
    f1, f0 = m["combine in the shared down GEMV"], m["combine as its own launch"]
    s = sum(best[k] for k in ("qkv", "o", "gate_up", "down"))
    out += ["", "Decode step (36 distinct layers) against the same step on layer 0's weights replayed 36 times",
            f"(50 MB, resident in the last-level cache): {a['ms']:.4f} ms ({a['gbs']:.1f} GB/s) against {b['ms']:.4f} ms",
            f"({b['gbs']:.1f} GB/s): reading the weights from HBM costs {100 * (a['ms'] - b['ms']) / a['ms']:.0f}% "
            "of the step; the rest is per-launch cost.", "",
            "MoE T=1 with the shared expert in the bank (h2048, 128 experts, top-8, I768, W4 gate_up + W8 down,",
            "shared W8 expert of the same I), faster of eager and graph replay per call:",
            f"    combine in the shared down GEMV (default)     {f1['us']:7.2f} us   (eager {f1['eager_us']:.2f}, "
            f"graph {f1['graph_us']:.2f})",
            f"    combine as its own launch (HM_GEMV_COMBINE=0) {f0['us']:7.2f} us   (eager {f0['eager_us']:.2f}, "
            f"graph {f0['graph_us']:.2f})",
            f"    outputs bit-identical: {m['bit_identical']}", "",
            f"Reading: one pass over a decode projection's weights takes at least {min(best.values()):.1f}-"
            f"{max(best.values()):.1f} us per launch in a graph. The per-layer sum of the best read floors,",
            f"{best['qkv']:.2f} + {best['o']:.2f} + {best['gate_up']:.2f} + {best['down']:.2f} = {s:.1f} us, bounds "
            f"a step of one launch per projection at 36 x {s:.1f} = {36 * s:.0f} us;",
            f"the decode step runs at {a['ms'] * 1000 / 36:.1f} us per layer ({a['ms']:.4f} ms)."]
    pw = {r["phase"]: r for r in d.get("power", [])}
    gemm = next((r for k, r in pw.items() if "GEMM" in k), None)
    rnd = next((r for k, r in pw.items() if "random" in k), None)
    if gemm and rnd:
        out += [f"The prefill GEMM draws {gemm['watts']:.0f} W at {gemm['sclk_mhz']} MHz for {gemm['tops']:.0f} TOPS; "
                f"the matrix cores alone, on random operands,",
                f"draw {rnd['watts']:.0f} W at {rnd['sclk_mhz']} MHz for {rnd['tops']:.0f} TOPS: the board's power "
                "management (1400 W) lowers the clock from",
                "2.4 GHz under both, so the GEMM's rate is set by the energy of its arithmetic plus its data movement,",
                "and the matrix-core ceiling on real data is the random-operand rate, not the 5.0 POP/s dense figure."]
    return "\n".join(out)


def profile_sweep(sweep_json):
    d = _last_json(sweep_json)
    out = ["Every GEMM tile and split-K setting on the bench's GEMM shapes, one MI355X.", "",
           "Command (repository root):", PROFILE_SETUP, "  python3 bench.py --tile-sweep > sweep.json",
           "  python3 bench.py --profile sweep sweep.json", "",
           "Per shape: one library call per distinct weight copy (copies exceeding the last-level cache), the",
           "quantization launch included, in a graph; us per call. 'plan' is the library's own choice; a tile",
           "name with /N forces N split-K pieces.", ""]
    for name, r in d.items():
        us = r["us"]
        out.append(f"{name} ({r['copies']} weight copies): best {r['best']} {us[r['best']]} us = {r['tops_best']} TOPS")
        items = [f"{k} {us[k]}" for k in ["plan"] + [k for k in us if k != "plan"]]
        first = [i for i in items if "/" not in i.split()[0]]
        rest = [i for i in items if "/" in i.split()[0]]
        out.append("    " + ", ".join(first))
        for j in range(0, len(rest), 6):
            out.append("    " + ", ".join(rest[j:j + 6]))
    plan_gap = [(n, r["us"]["plan"] / r["us"][r["best"]] - 1) for n, r in d.items()]
    worst = max(plan_gap, key=lambda x: x[1])
    out += ["", f"Reading: the plan is within {100 * worst[1]:.1f}% of the best setting on every shape (worst: {worst[0]})."]
    return "\n".join(out)


def _stats_table(stats_csv, min_pct=0.1):
    rows = list(csv.DictReader(open(stats_csv)))
    tot = sum(float(r["TotalDurationNs"]) for r in rows)
    lines = [f"{'kernel':84} {'calls':>6} {'avg_us':>8} {'min_us':>8} {'max_us':>8} {'pct':>5}"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        pct = 100 * float(r["TotalDurationNs"]) / tot
        if pct < min_pct:
            continue
        lines.append(f"{_kname(r['Name'])[:84]:84} {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:8.2f} "
                     f"{float(r['MinNs']) / 1e3:8.2f} {float(r['MaxNs']) / 1e3:8.2f} {pct:5.1f}")
    lines.append(f"(kernels below {min_pct}% of the total omitted)")
    return lines


def profile_moe(stats_csv, moe_json):
    res = _last_json(moe_json)
    res = res if isinstance(res, list) else res.get("lines", res)
    out = ["MoE 35B-A3B-class expert FFN (h 2048, 128 experts, top-8, I 768, W4 gate_up + W8 down; shared W8",
           "FFN I 2048): kernel statistics, one MI355X.", "",
           "Commands (repository root):", PROFILE_SETUP,
           "  rocprofv3 --kernel-trace --stats --output-format csv -d <out> -o run -- python3 -u bench.py --only moe "
           "> moe.json",
           "  python3 bench.py --profile moe <out>/<host>/<pid>_run_kernel_stats.csv moe.json", "",
           "Workload: rk_npu_hip_moe_run at T=512 and T=1 tokens, steps of both sizes mixed in the table (eager and",
           "graph replays). T=512: device routing (counting sort of the (token, rank) slots), the tokens'",
           "quantization written straight into slot order (one launch, rows through the routing's slot map),",
           "grouped gate_up GEMM + SwiGLU + row max over the ragged expert groups, middle requantization, grouped",
           "down GEMM, combine; the shared expert as a dense FFN. T=1: slot GEMVs (slot = assignment, no routing",
           "launch) for gate_up and down, the shared expert's GEMVs, combine.", ""]
    out += _stats_table(stats_csv)
    out += ["", "bench.py --only moe in the same profiled run:"]
    for r in (res if isinstance(res, list) else [res]):
        out.append(f"    {r['workload']}: {r['value']} {r['unit']} ({r['ms_per_step'] * 1000:.1f} us per step)")
    return "\n".join(out)


def profile_attention(stats_csv, attn_json, pmc1_csv, pmc2_csv):
    res = _last_json(attn_json)
    res = res if isinstance(res, list) else [res]
    out = ["FP16 GQA attention (32 query heads over 8 KV heads, head_dim 128), 36 per-layer KV caches of 4096",
           "rows: kernel statistics and counters, one MI355X.", "",
           "Commands (repository root):", PROFILE_SETUP,
           "  rocprofv3 --kernel-trace --stats --output-format csv -d <out> -o run -- python3 -u bench.py "
           "--only attention > attn.json",
           "  rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_WAVE_CYCLES SQ_WAIT_ANY GRBM_GUI_ACTIVE --output-format csv \\",
           "      -d <pmc1> -o run -- python3 -u bench.py --only attention",
           "  rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS SQ_WAVES GRBM_GUI_ACTIVE "
           "--output-format csv \\",
           "      -d <pmc2> -o run -- python3 -u bench.py --only attention",
           "  python3 bench.py --profile attention <out>/<host>/<pid>_run_kernel_stats.csv attn.json \\",
           "      <pmc1>/<host>/<pid>_run_counter_collection.csv <pmc2>/<host>/<pid>_run_counter_collection.csv", "",
           "Workload (bench.py run_attention): one rk_npu_hip_attention_run per layer cache; decode = 1 query row at",
           "the last position (attn_split_kernel + attn_combine_kernel), prefill = 128 query rows ending at the last",
           "position, causal (attn_mfma_kernel + attn_combine_rows_kernel); eager steps and graph replays both in",
           "the table.", ""]
    out += _stats_table(stats_csv)
    r1, r2 = _counters(pmc1_csv), _counters(pmc2_csv)
    out += ["", "Counters (per-dispatch medians; MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 x 1024);",
            "LDS util = SQ_LDS_IDX_ACTIVE / (GRBM_GUI_ACTIVE / 8 x 256); confl = SQ_LDS_BANK_CONFLICT / "
            "SQ_LDS_IDX_ACTIVE):",
            f"{'kernel':40} {'dur us':>7} {'MFMA':>6} {'WAIT_ANY':>8} {'LDS util':>8} {'confl':>6} {'LDS/wave':>8}"]
    names = sorted({v[1] for v in r1.values() if v[1].startswith("attn_")})
    for name in names:
        k1 = [k for k, v in r1.items() if v[1] == name]
        k2 = [k for k, v in r2.items() if v[1] == name]
        md = lambda disp, ks, c: statistics.median(disp[k][0][c] for k in ks)
        g1, g2 = md(r1, k1, "GRBM_GUI_ACTIVE") / 8, md(r2, k2, "GRBM_GUI_ACTIVE") / 8
        la = md(r2, k2, "SQ_LDS_IDX_ACTIVE")
        out.append(f"{name:40} {statistics.median(r1[k][4] for k in k1):7.2f} "
                   f"{md(r1, k1, 'SQ_VALU_MFMA_BUSY_CYCLES') / (g1 * 1024):6.3f} "
                   f"{md(r1, k1, 'SQ_WAIT_ANY') / md(r1, k1, 'SQ_WAVE_CYCLES'):8.3f} {la / (g2 * 256):8.3f} "
                   f"{(md(r2, k2, 'SQ_LDS_BANK_CONFLICT') / la) if la else 0:6.3f} "
                   f"{md(r2, k2, 'SQ_INSTS_LDS') / md(r2, k2, 'SQ_WAVES'):8.0f}")
    out += ["", "bench.py --only attention in the same profiled run:"]
    for r in res:
        extra = f" ({r['us_per_layer']} us per layer)" if "us_per_layer" in r else ""
        out.append(f"    {r['workload']}: {r['value']} {r['unit']}{extra}")
    return "\n".join(out)


PROFILES = {"roofline": (profile_roofline, 3), "traffic": (profile_traffic, 2),
            "gemm-counters": (profile_gemm_counters, 3), "probes": (profile_probes, 1), "sweep": (profile_sweep, 1),
            "moe": (profile_moe, 2), "attention": (profile_attention, 4)}


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
    ap.add_argument("--roofline-only", nargs="?", const="all", choices=["all", "decode", "prefill", "ffn512", "up128"],
                    help="only the roofline passes of every line (or of one: per-projection decode and prefill "
                         "passes included), no step timing and no CPU baseline: the command to profile")
    ap.add_argument("--tile-sweep", nargs="*", metavar="SHAPE",
                    help="only time every GEMM tile / split-K setting on the bench's GEMM shapes (names "
                         "containing any given word; all by default)")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="no GPU: per-kernel launch statistics of a rocprofv3 kernel-trace CSV")
    ap.add_argument("--summarize-counters", metavar="CSV",
                    help="no GPU: per-kernel counter medians of a rocprofv3 --pmc CSV")
    ap.add_argument("--profile", nargs="+", metavar=("NAME", "INPUT"),
                    help="no GPU: print one file of profiles/ from its commands' outputs (" +
                         ", ".join(PROFILES) + ")")
    args = ap.parse_args()
    if args.profile:
        fn, n = PROFILES[args.profile[0]]
        if len(args.profile) != n + 1:
            ap.error(f"--profile {args.profile[0]} takes {n} inputs")
        print(fn(*args.profile[1:]))
        return
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace))
        return
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters))
        return
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
    if args.roofline_only:
        print(json.dumps(roofline_only(torch, ctx, args.roofline_only)), flush=True)
        return
    if args.tile_sweep is not None:
        print(json.dumps(tile_sweep(torch, ctx, args.tile_sweep)), flush=True)
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
    cpu = not args.no_cpu_baseline
    primary = run_decode(torch, ctx, args.decode_rows, args.steps, args.warmup, cpu, reps=ROOF_REPS)
    secondary = []
    if not args.primary_only:
        m4 = run_decode(torch, ctx, 4, args.steps, args.warmup, cpu, reps=ROOF_REPS)
        secondary.append({"workload": "decode M=4 (MTP/draft verify), same W4A8 set x36",
                          "value": round(m4["value"], 1), "unit": "GB/s", "ms_per_step": round(m4["ms_per_step"], 4),
                          "projections": m4["projections"], "roofline": m4["roofline"],
                          "cpu_baseline": m4.get("cpu_baseline")})
        secondary.append(run_prefill(torch, ctx, 4096, max(4, args.steps // 2), 2, cpu))
        secondary.append(run_ffn512(torch, ctx, max(4, args.steps // 2), 2, want_cpu=cpu))
        up = run_up128(torch, ctx, args.steps, args.warmup, want_cpu=cpu)
        secondary.append(up)
        host = run_host_abi()
        if cpu:
            host[0]["cpu_baseline"] = dict(primary["cpu_baseline"], note="the same work as the primary line's sample")
            host[1]["cpu_baseline"] = dict(up["cpu_baseline"], note="the same work as the M=128 up line's sample")
        secondary.extend(host)
        secondary.extend(run_moe(torch, ctx, max(4, args.steps // 2), 2, want_cpu=cpu))
        attn = run_attention(torch, ctx, max(4, args.steps // 2), want_cpu=cpu)
        secondary.extend(attn)
        if cpu and attn and attn[0].get("cpu_baseline"):
            host[2]["cpu_baseline"] = dict(attn[0]["cpu_baseline"],
                                           note="the resident attention decode line's sample (the same attention)")
    for s in secondary:
        s.pop("kernels", None)
        if "roofline" in s:
            s["roofline"].pop("work_per_launch", None)
    roof = dict(primary["roofline"])
    roof.pop("work_per_launch", None)
    # the whole step's fraction of HBM beside the dominant kernel's
    roof["step_achieved"] = round(primary["value"], 2)
    roof["step_frac"] = round(primary["value"] / HBM_PEAK_GBS, 4)
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
                   "data_flow": "within a layer qkv -> o -> FFN, each launch reading the previous one's output; "
                                "each layer's qkv reads the fixed input",
                   "timing": "faster of eager launches and HIP graph replay of the same step "
                             "(replay checked bit-exact vs eager)", **config_extra},
        "roofline": roof,
        "projections": primary["projections"],
        "cpu_baseline": primary.get("cpu_baseline"),
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
