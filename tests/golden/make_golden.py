#!/usr/bin/env python3
"""Writes the small golden fixtures of tests/golden/ from the C oracle.

The reference ships no golden vectors for this path (its tests compare the
device against its own in-process CPU oracle, src/npu.rs:1533-1566), so the
fixtures pin the oracle's restatement of that CPU semantics on inputs built to
exercise its edge cases: an all-zero row, exact quantization ties (where
round-half-away and round-half-even differ), +-127 saturation from an outlier,
W4 codes at both ends of [-8, 7], SwiGLU arguments beyond the exp clamp, and a
MoE routing with a repeated expert and a zero route weight. Run from the
repository root: python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle  # noqa: E402

F32 = np.float32


def edge_rows(rows: int, k: int, seed: int) -> np.ndarray:
    """rows x k activations: row 0 all zero; row 1 exact ties; row 2 an
    outlier that saturates; the rest N(0,1) rounded to fp16 values."""
    g = np.random.default_rng(seed)
    x = g.standard_normal((rows, k)).astype(np.float16).astype(F32)
    x[0] = 0.0
    # max |x| = 127 gives scale 1, so x = j + 0.5 are exact ties
    x[1] = ((np.arange(k) % 9) - 4).astype(F32) + F32(0.5)
    x[1, 0] = F32(127.0)
    x[2, 3] = F32(-4000.0)
    return x


def w_codes(g, bits, k, n):
    lo, hi = (-8, 8) if bits == 4 else (-127, 128)
    c = g.integers(lo, hi, size=(k, n), dtype=np.int8)
    c[0, :4] = lo
    c[1, :4] = hi - 1
    return c


def main():
    g = np.random.default_rng(0x601D)
    out = {}
    for bits in (8, 4):
        k, n, rows = 96, 80, 6
        codes = w_codes(g, bits, k, n)
        scales = g.uniform(0.001, 0.01, n).astype(F32)
        x = edge_rows(rows, k, 10 + bits)
        y, q, s, acc = oracle.linear(codes, scales, x, intermediates=True)
        out[f"linear_w{bits}"] = dict(codes=codes, scales=scales, x=x, q=q, s=s, acc=acc, y=y)
    # fused gate/up SwiGLU (W4, N % 64 == 0): gate = first N/2 columns
    k, n, rows = 64, 128, 4
    codes = w_codes(g, 4, k, n)
    scales = g.uniform(0.001, 0.01, n).astype(F32)
    x = edge_rows(rows, k, 21)
    x[3] *= F32(300.0)  # gate values far beyond the exp clamp
    out["swiglu_w4"] = dict(codes=codes, scales=scales, x=x, y=oracle.linear_swiglu(codes, scales, x))
    # fused FFN: W4 gate/up -> SwiGLU -> requant -> W8 down
    h, f, rows = 64, 64, 5
    gc, gs = w_codes(g, 4, h, 2 * f), g.uniform(0.001, 0.01, 2 * f).astype(F32)
    dc, ds = w_codes(g, 8, f, h), g.uniform(0.001, 0.01, h).astype(F32)
    x = edge_rows(rows, h, 31)
    y, mid = oracle.ffn(gc, gs, dc, ds, x, with_middle=True)
    out["ffn"] = dict(gu_codes=gc, gu_scales=gs, dn_codes=dc, dn_scales=ds, x=x, mid=mid, y=y)
    # routed MoE with a shared W8 expert
    h, inter, experts, top, rows = 64, 32, 4, 2, 6
    gu = [(w_codes(g, 4, h, 2 * inter), g.uniform(0.001, 0.01, 2 * inter).astype(F32)) for _ in range(experts)]
    dn = [(w_codes(g, 8, inter, h), g.uniform(0.001, 0.01, h).astype(F32)) for _ in range(experts)]
    sh = ((w_codes(g, 8, h, 2 * inter), g.uniform(0.001, 0.01, 2 * inter).astype(F32)),
          (w_codes(g, 8, inter, h), g.uniform(0.001, 0.01, h).astype(F32)))
    x = edge_rows(rows, h, 41)
    logits = g.standard_normal((rows, experts)).astype(F32)
    ids = np.zeros((rows, top), np.int32)
    w = np.zeros((rows, top), F32)
    for r in range(rows):
        ids[r], w[r] = oracle.routes(logits[r], top)
    ids[4, 1] = ids[4, 0]   # repeated expert in one row
    w[5, 1] = F32(0.0)      # skipped route
    y = oracle.moe(gu, dn, x, ids, w, shared=sh)
    moe = dict(x=x, logits=logits, ids=ids, routes=w, y=y,
               sh_gu_codes=sh[0][0], sh_gu_scales=sh[0][1], sh_dn_codes=sh[1][0], sh_dn_scales=sh[1][1])
    for e in range(experts):
        moe[f"gu_codes{e}"], moe[f"gu_scales{e}"] = gu[e]
        moe[f"dn_codes{e}"], moe[f"dn_scales{e}"] = dn[e]
    out["moe"] = moe
    # exp and SwiGLU scalar values across the clamp and special cases
    gv = np.array([0.0, -0.0, 1e-30, -1e-30, 0.5, -0.5, 1.0, -1.0, 10.0, -10.0, 79.9, -79.9, 80.0, -80.0,
                   80.5, -80.5, 88.0, -88.0, 200.0, -200.0, 3.4e38, -3.4e38], F32)
    uv = np.linspace(-3.0, 3.0, gv.size).astype(F32)
    out["scalar"] = dict(exp_in=gv, exp_out=oracle.expf(-gv), g=gv, u=uv, swiglu=oracle.swiglu(gv, uv))
    for name, arrays in out.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrays)
        print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
