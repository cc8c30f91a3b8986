"""Inputs of the reference's own tests, restated as numpy (f32 arithmetic),
plus the seeded synthetic workloads of the benchmark configurations."""
from __future__ import annotations

import numpy as np

F32 = np.float32

# src/npu.rs:1629-1631
REFERENCE_ROWS = [1, 2, 3, 4, 5, 8, 9, 16, 17, 31, 32, 33, 65, 127, 128, 129, 191, 192, 193, 255, 256]


def reference_matrix(bits: int, k: int = 256, n: int = 256):
    """src/npu.rs:1609-1621: codes and scales of quantized_linear_padding_and_swiglu."""
    i = np.arange(k * n, dtype=np.int64)
    mod, off = (16, 8) if bits == 4 else (255, 127)
    codes = (((i * 13 + i // 256 * 7) % mod) - off).astype(np.int8).reshape(k, n)
    scales = (F32(0.002) + (np.arange(n) % 11).astype(F32) * F32(0.0001)).astype(F32)
    return codes, scales


def reference_input(rows: int = 256, k: int = 256):
    """src/npu.rs:1622-1624: ((i*17 + i/256*3) % 127) as f32 / 63 - 1."""
    i = np.arange(rows * k, dtype=np.int64)
    v = ((i * 17 + i // 256 * 3) % 127).astype(F32)
    return (v / F32(63.0) - F32(1.0)).astype(F32).reshape(rows, k)


def narrow_matrix(k: int, n: int):
    """src/npu/narrow_projection.rs:33-38."""
    i = np.arange(k * n, dtype=np.int64)
    codes = (((i * 13 + i // n * 7) % 255) - 127).astype(np.int8).reshape(k, n)
    scales = (F32(0.001) + (np.arange(n) % 11).astype(F32) * F32(0.0001)).astype(F32)
    return codes, scales


def narrow_input(rows: int, k: int):
    """src/npu/narrow_projection.rs:50-52."""
    i = np.arange(rows * k, dtype=np.int64)
    v = ((i * 17 + i // k * 3) % 127).astype(F32)
    return (v / F32(63.0) - F32(1.0)).astype(F32).reshape(rows, k)


def lane_matrix(bits: int, k: int = 513, n: int = 512):
    """src/npu/lane.rs:154-163."""
    i = np.arange(k * n, dtype=np.int64)
    codes = ((i * 7 % 4) - 2).astype(np.int8).reshape(k, n)
    return codes, np.full(n, F32(0.01), F32)


def lane_inputs(rows: int = 128, k: int = 513):
    """src/npu/lane.rs:169-172."""
    i = np.arange(rows * k, dtype=np.int64)
    x0 = (((i % 127).astype(F32) - F32(63.0)) * F32(0.03125)).astype(F32).reshape(rows, k)
    x1 = (x0 * F32(-0.75) + F32(0.01)).astype(F32)
    return x0, x1


# ---- synthetic benchmark workloads (seeded) ------------------------------------

def rng_for(config: int, name: str) -> np.random.Generator:
    """Per-tensor stream: seed 0x5EED0000 + config, stream keyed by the name."""
    key = [ord(c) for c in name]
    return np.random.default_rng([0x5EED0000 + config, *key])


def activations(config: int, name: str, rows: int, k: int, outliers: bool = True) -> np.ndarray:
    """~N(0,1) rows; ceil(0.5% of K) seeded channels scaled x20; rounded to fp16."""
    g = rng_for(config, name)
    x = g.standard_normal((rows, k)).astype(F32)
    if outliers:
        cols = g.choice(k, size=int(np.ceil(0.005 * k)), replace=False)
        x[:, cols] *= F32(20.0)
    return x.astype(np.float16).astype(F32)


def weights(config: int, name: str, bits: int, k: int, n: int):
    g = rng_for(config, name)
    lo, hi = (-8, 8) if bits == 4 else (-127, 128)
    codes = g.integers(lo, hi, size=(k, n), dtype=np.int8)
    scales = g.uniform(0.001, 0.01, size=n).astype(F32)
    return codes, scales
