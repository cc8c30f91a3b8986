"""FP16 grouped-query attention over a device KV cache — the Python mirror of
the reference's src/npu/attention.rs (Attention, FullAttention) and the
attention parts of src/npu.rs (attention_config, AttentionWork,
attention_masked, full_attention), on top of the rk_npu_attention_f16 C ABI.

Arrays cross this layer token-major as in the Rust code (q and output
[rows][query_heads][head_dim], k and v [rows][kv_heads][head_dim], f32) and
are packed head-major fp16 for the C calls (src/npu/attention.rs:240-262,
325-351).
"""
from __future__ import annotations

import ctypes
import math
import threading
from typing import Optional

import numpy as np

from . import _ffi as F
from .npu import NpuError, _Handle, check, ensure


def pack_half(values: np.ndarray) -> np.ndarray:
    """f32 -> fp16 bits, round to nearest even (src/npu/attention.rs:19-44);
    an input that overflows fp16 is rejected, as the reference asserts."""
    half = np.asarray(values, np.float32).astype(np.float16)
    ensure(bool(np.all(np.isfinite(half))), "nonfinite/overflowed FP16 attention input")
    return half.view(np.uint16)


def attention_config(options, query_heads: int, kv_heads: int, dimension: int,
                     softmax_scale: float) -> F.rk_npu_attention_f16_config:
    """src/npu.rs:420-440."""
    cfg = F.rk_npu_attention_f16_config()
    F.lib().rk_npu_attention_f16_config_init(ctypes.byref(cfg))
    cfg.query_heads = query_heads
    cfg.kv_heads = kv_heads
    cfg.head_dim = dimension
    cfg.softmax_scale = softmax_scale
    cfg.max_query_rows = min(options.chunk, 128)
    cfg.max_capacity = -(-options.context // 32) * 32
    cfg.initial_capacity = min(cfg.max_capacity, 128)
    cfg.core_mask = options.npu_mask
    cfg.kv_tile = options.attention_tile
    cfg.flags = F.RK_NPU_ATTENTION_F16_STABLE_SOFTMAX
    return cfg


def _same_geometry(a, b) -> bool:
    return (a.query_heads, a.kv_heads, a.head_dim, a.softmax_scale, a.mask_mode) == (
        b.query_heads, b.kv_heads, b.head_dim, b.softmax_scale, b.mask_mode)


class AttentionWork:
    """src/npu.rs:295-345: the run workspace and its host staging."""

    def __init__(self, backend, config: F.rk_npu_attention_f16_config):
        L = F.lib()
        sizes = F.rk_npu_attention_f16_sizes()
        check(L.rk_npu_attention_f16_query(ctypes.byref(config), config.initial_capacity, config.max_query_rows,
                                           config.initial_capacity, ctypes.byref(sizes)),
              "query native Attention sizes")
        raw = ctypes.c_void_p()
        check(L.rk_npu_attention_f16_prepare(backend.domain, ctypes.byref(config), ctypes.byref(raw)),
              "prepare native Attention")
        self.workspace = _Handle(raw.value, L.rk_npu_attention_f16_workspace_free, "attention workspace",
                                 keep=backend._shared)
        self.config = config
        self.active_core_mask = sizes.active_core_mask


def _run(backend, work: AttentionWork, cache_raw, q_heads: np.ndarray, m: int, position: int,
         half: bool) -> np.ndarray:
    """One rk_npu_attention_f16_run[_half] call on head-major fp16 bits."""
    cfg = work.config
    L = F.lib()
    out = np.empty((cfg.query_heads, m, cfg.head_dim), np.float16 if half else np.float32)
    q_heads = np.ascontiguousarray(q_heads, np.uint16)
    run = L.rk_npu_attention_f16_run_half if half else L.rk_npu_attention_f16_run
    check(run(backend.ctx, work.workspace.raw, cache_raw, q_heads.ctypes.data, m, position,
              out.ctypes.data, None, None), "native GQA run")
    return out


class Attention:
    """src/npu/attention.rs:4-10, 190-352: a causal (or bidirectional) GQA
    KV cache bound to its backend's shared workspace."""

    def __init__(self, backend, cache: _Handle, query_heads: int, kv_heads: int, dimension: int):
        self.backend = backend
        self.cache = cache
        self.query_heads, self.kv_heads, self.dimension = query_heads, kv_heads, dimension
        self._lock = threading.Lock()

    def info(self) -> F.rk_npu_attention_f16_cache_info:
        info = F.rk_npu_attention_f16_cache_info()
        check(F.lib().rk_npu_attention_f16_cache_get_info(self.cache.raw, ctypes.byref(info)), "native KV position")
        return info

    def truncate(self, length: int) -> None:
        ensure(0 <= length <= 2 ** 31 - 1, "invalid native KV prefix length")
        with self._lock:
            check(F.lib().rk_npu_attention_f16_cache_truncate(self.cache.raw, length), "truncate native KV cache")

    def reset(self) -> None:
        with self._lock:
            check(F.lib().rk_npu_attention_f16_cache_load(self.backend.ctx, self.cache.raw, None, None, 0),
                  "reset native KV cache")

    def bytes(self) -> int:
        info = self.info()
        return info.key_bytes + info.value_bytes + info.tail_bytes

    def reserve(self, capacity: int) -> None:
        ensure(capacity <= self.backend.options.context, "native GQA context capacity exceeded")
        with self._lock:
            check(F.lib().rk_npu_attention_f16_cache_reserve(self.backend.ctx, self.cache.raw,
                                                             -(-capacity // 32) * 32), "reserve native KV cache")

    def append(self, k: np.ndarray, v: np.ndarray, rows: int, position: int) -> None:
        """Append projected K/V rows without computing attention."""
        with self._lock:
            self._append(k, v, rows, position)

    def _append(self, k, v, rows, position):
        kh, d = self.kv_heads, self.dimension
        opts = self.backend.options
        ensure(0 < rows <= opts.chunk and position + rows <= opts.context, "native KV append capacity exceeded")
        k = np.asarray(k, np.float32).reshape(-1)
        v = np.asarray(v, np.float32).reshape(-1)
        ensure(k.size == rows * kh * d and v.size == rows * kh * d, "native KV append shape mismatch")
        ensure(self.info().length == position, "native KV cache position mismatch")
        kb = np.ascontiguousarray(pack_half(k.reshape(rows, kh, d)).transpose(1, 0, 2))
        vb = np.ascontiguousarray(pack_half(v.reshape(rows, kh, d)).transpose(1, 0, 2))
        check(F.lib().rk_npu_attention_f16_cache_append(self.backend.ctx, self.cache.raw, kb.ctypes.data,
                                                        vb.ctypes.data, rows), "append native KV")

    def run(self, q: np.ndarray, k: np.ndarray, v: np.ndarray, output: np.ndarray, rows: int,
            position: int) -> None:
        """Append the rows' K/V at `position`, then attend the rows' queries
        (src/npu/attention.rs:299-352); output [rows][query_heads][head_dim]."""
        qh, kh, d = self.query_heads, self.kv_heads, self.dimension
        opts = self.backend.options
        ensure(0 < rows <= opts.chunk and position + rows <= opts.context, "native GQA context capacity exceeded")
        q = np.asarray(q, np.float32).reshape(-1)
        ensure(q.size >= rows * qh * d and output.size >= rows * qh * d and np.size(k) >= rows * kh * d and
               np.size(v) >= rows * kh * d, "attention input/output shape mismatch")
        with self._lock:
            self._append(np.asarray(k, np.float32).reshape(-1)[:rows * kh * d],
                         np.asarray(v, np.float32).reshape(-1)[:rows * kh * d], rows, position)
            work = self.backend._attention
            step = work.config.max_query_rows
            out = output.reshape(-1)
            for offset in range(0, rows, step):
                m = min(step, rows - offset)
                qb = pack_half(q[offset * qh * d:(offset + m) * qh * d].reshape(m, qh, d)).transpose(1, 0, 2)
                res = _run(self.backend, work, self.cache.raw, qb, m, position + offset, False)
                out[offset * qh * d:(offset + m) * qh * d] = res.transpose(1, 0, 2).reshape(-1)


class FullAttention:
    """src/npu/attention.rs:12-17, 45-205: stateless bidirectional attention
    over one complete sequence with its own cache and workspace."""

    def __init__(self, backend, kv: _Handle, work: AttentionWork):
        self.backend, self.kv, self.work = backend, kv, work

    def _load(self, k_bits, v_bits, rows):
        check(F.lib().rk_npu_attention_f16_cache_load(self.backend.ctx, self.kv.raw, k_bits.ctypes.data,
                                                      v_bits.ctypes.data, rows), "load full image KV")

    def _run_full(self, q_bits, k_bits, v_bits, rows, half):
        cfg = self.work.config
        heads, d = cfg.query_heads, cfg.head_dim
        ensure(0 < rows <= cfg.max_capacity,
               f"image Attention rows={rows} exceed prepared buffer capacity={cfg.max_capacity}")
        self._load(np.ascontiguousarray(k_bits.reshape(rows, heads, d).transpose(1, 0, 2)),
                   np.ascontiguousarray(v_bits.reshape(rows, heads, d).transpose(1, 0, 2)), rows)
        out = np.empty((rows, heads, d), np.float16 if half else np.float32)
        step = cfg.max_query_rows
        q_bits = q_bits.reshape(rows, heads, d)
        for offset in range(0, rows, step):
            m = min(step, rows - offset)
            res = _run(self.backend, self.work, self.kv.raw, q_bits[offset:offset + m].transpose(1, 0, 2), m,
                       offset, half)
            out[offset:offset + m] = res.transpose(1, 0, 2)
        return out

    def run_full(self, q, k, v, output, rows: int) -> None:
        cfg = self.work.config
        n = rows * cfg.query_heads * cfg.head_dim
        ensure(all(np.size(a) == n for a in (q, k, v, output)), "full attention tensor shape mismatch")
        res = self._run_full(pack_half(q), pack_half(k), pack_half(v), rows, False)
        output.reshape(-1)[:] = res.reshape(-1)

    def run_full_half(self, q_bits, k_bits, v_bits, output_bits, rows: int) -> None:
        cfg = self.work.config
        n = rows * cfg.query_heads * cfg.head_dim
        ensure(all(np.size(a) == n for a in (q_bits, k_bits, v_bits, output_bits)),
               "full FP16 attention tensor shape mismatch")
        res = self._run_full(np.asarray(q_bits, np.uint16), np.asarray(k_bits, np.uint16),
                             np.asarray(v_bits, np.uint16), rows, True)
        output_bits.reshape(-1)[:] = res.view(np.uint16).reshape(-1)


def create_cache(backend, config) -> _Handle:
    raw = ctypes.c_void_p()
    check(F.lib().rk_npu_attention_f16_cache_create(backend.domain, ctypes.byref(config), ctypes.byref(raw)),
          "create native KV cache")
    return _Handle(raw.value, F.lib().rk_npu_attention_f16_cache_free, "KV cache", keep=backend._shared)


def attention_masked(backend, query_heads: int, kv_heads: int, dimension: int, softmax_scale: float,
                     noncausal: bool) -> Attention:
    """src/npu.rs:706-760."""
    ensure(0 < kv_heads <= 32 and query_heads >= kv_heads and query_heads % kv_heads == 0 and dimension > 0 and
           dimension % 32 == 0 and math.isfinite(softmax_scale) and softmax_scale > 0.0,
           "native GQA requires Hq divisible by Hkv, Hkv within 1..32, D divisible by 32 and a positive softmax scale")
    with backend._lock:
        if backend._attention is None:
            cfg = attention_config(backend.options, query_heads, kv_heads, dimension, softmax_scale)
            if noncausal:
                cfg.mask_mode = F.RK_NPU_ATTENTION_F16_NO_MASK
            backend._attention = AttentionWork(backend, cfg)
        cfg = backend._attention.config
        want = attention_config(backend.options, query_heads, kv_heads, dimension, softmax_scale)
        want.mask_mode = F.RK_NPU_ATTENTION_F16_NO_MASK if noncausal else F.RK_NPU_ATTENTION_F16_CAUSAL
        ensure(_same_geometry(cfg, want), "attention workspace geometry mismatch")
        cache = create_cache(backend, cfg)
    return Attention(backend, cache, query_heads, kv_heads, dimension)


def full_attention(backend, heads: int, dimension: int, rows: int) -> FullAttention:
    """src/npu.rs:662-692."""
    ensure(0 < rows <= (2 ** 31 - 1) // 32 * 32, f"image Attention rows exceed the native integer range: {rows}")
    cfg = attention_config(backend.options, heads, heads, dimension, 1.0 / math.sqrt(dimension))
    cfg.mask_mode = F.RK_NPU_ATTENTION_F16_NO_MASK
    cfg.max_capacity = -(-rows // 32) * 32
    cfg.initial_capacity = cfg.max_capacity
    work = AttentionWork(backend, cfg)
    return FullAttention(backend, create_cache(backend, cfg), work)


def attention_cache_bytes(options, query_heads: int, kv_heads: int, dimension: int, softmax_scale: float) -> int:
    """src/npu.rs:442-466."""
    cfg = attention_config(options, query_heads, kv_heads, dimension, softmax_scale)
    sizes = F.rk_npu_attention_f16_sizes()
    check(F.lib().rk_npu_attention_f16_query(ctypes.byref(cfg), cfg.max_capacity, 1, cfg.max_capacity,
                                             ctypes.byref(sizes)), "query native KV memory")
    return sizes.key_bytes + sizes.value_bytes + sizes.tail_bytes


__all__ = ["Attention", "FullAttention", "AttentionWork", "attention_config", "attention_masked",
           "full_attention", "attention_cache_bytes", "pack_half", "NpuError"]
