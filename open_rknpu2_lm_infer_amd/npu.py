"""Host-side mirror of the reference's quantized-op API over the C ABI.

Mirrors ``src/npu.rs`` (QuantMatrix, Backend, Linear, bucket, padding,
per-(shape, bucket) workspace cache, error reporting), ``src/npu/moe.rs``
(Moe banks and runs), ``src/npu/lane.rs`` (execution lanes: shared weights,
own workspaces) and the router of ``src/model/qwen35/moe.rs:51-67``. It calls
only the rk_npu_* entry points, the same way the Rust layer does through its
bindgen module, so the parity tests read like the reference's own tests.
"""
from __future__ import annotations

import ctypes
import math
import threading
import weakref
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import _ffi as F


class NpuError(RuntimeError):
    """A failed native call (src/npu.rs:187-200) or a rejected argument."""


def check(rc: int, name: str) -> None:
    if rc != 0:
        raise NpuError(f"{name}: {F.strerror(rc)} ({rc})")


def ensure(cond: bool, msg: str) -> None:
    if not cond:
        raise NpuError(msg)


def bucket(rows: int) -> int:
    """src/npu.rs:201-211."""
    ensure(1 <= rows <= 256, "linear batch must be within 1..256")
    if rows <= 128:
        return 1 << (rows - 1).bit_length()
    return (rows + 63) // 64 * 64


@dataclass
class QuantMatrix:
    """src/npu.rs:134-158: codes [K][N] row-major int8, scales [N] f32."""
    bits: int
    k: int
    n: int
    codes: np.ndarray
    scales: np.ndarray

    def validate(self) -> None:
        ensure(self.bits in (4, 8), "linear weights must use 4 or 8 bits")
        ensure(0 < self.k <= 2**31 - 1 and 0 < self.n <= 2**31 - 1, "invalid linear dimensions")
        ensure(np.asarray(self.codes).size == self.k * self.n and np.asarray(self.scales).size == self.n,
               "linear weight shape mismatch")


@dataclass
class ModelOptions:
    """The subset of ModelOptions (src/model.rs:93-113) the op layer reads."""
    chunk: int = 128
    threads: int = 1
    npu_mask: int = 1
    cpu_mask: int = 0
    tune: bool = False
    tune_search: bool = False
    compress_w8a8: bool = False
    context: int = 4096        # KV rows an attention cache may hold
    attention_tile: int = 512  # accepted and ignored (the kernel tiles by itself)


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(ctypes.POINTER(t))


class _Handle:
    """Owning native pointer. `keep` holds whatever must outlive it (the
    context and domain), so finalization order never frees a domain before
    the weights and workspaces allocated in it."""

    def __init__(self, raw, free, name: str, keep=None):
        ensure(bool(raw), f"cannot allocate {name}")
        self.raw = raw
        self._free = free
        self._keep = keep

    def close(self):
        if self.raw:
            self._free(self.raw)
            self.raw = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class _Work:
    w4: Optional[_Handle] = None
    w4_swiglu: Optional[_Handle] = None
    w8: Optional[_Handle] = None
    bytes: int = 0


class _Shared:
    """Context + domain shared by a backend and its execution lanes
    (src/npu.rs:222-283). Holds no strong reference to its lanes."""

    def __init__(self, domain_id: int, device: Optional[str]):
        L = F.lib()
        ensure(0 <= domain_id < F.RK_NPU_IOMMU_DOMAIN_COUNT, "IOMMU domain must be within 0..15")
        self.ctx = _Handle(L.rk_npu_open(device.encode() if device else None), L.rk_npu_close, "GPU context")
        self.domain = _Handle(L.rk_npu_iommu_domain_create(self.ctx.raw, domain_id),
                              L.rk_npu_iommu_domain_free, "allocation domain", keep=self.ctx)
        self.lanes = weakref.WeakSet()
        self.reclaims = 0
        me = weakref.ref(self)

        def reclaim(_cookie):
            # src/npu.rs:234-260: drop idle workspaces; never locks a lane.
            shared = me()
            if shared is not None:
                shared.reclaims += 1
                for lane in list(shared.lanes):
                    lane._idle.clear()

        self._cb = F.RECLAIM_CALLBACK(reclaim)
        L.rk_npu_iommu_domain_set_reclaim(self.domain.raw, ctypes.cast(self._cb, ctypes.c_void_p), None)

    def __del__(self):
        try:
            F.lib().rk_npu_iommu_domain_set_reclaim(self.domain.raw, None, None)
        except Exception:
            pass


class Backend:
    """src/npu.rs:354-905 (Backend) with the fallback (untuned) strategies."""

    def __init__(self, options: Optional[ModelOptions] = None, domain_id: int = 15,
                 device: Optional[str] = None, _shared: Optional[_Shared] = None):
        self.options = options or ModelOptions()
        ensure(1 <= self.options.chunk <= 256, "ubatch-size must be within 1..256")
        self._shared = _shared or _Shared(domain_id, device)
        self._shared.lanes.add(self)
        self.domain_id = domain_id
        self._lock = threading.Lock()
        self.work: Dict[Tuple, _Work] = {}
        self._idle: Dict[Tuple, _Work] = {}
        self.w8_partitions: Dict[Tuple[int, int], int] = {}
        self.fallbacks = set()
        self.loaded_w4 = 0
        self.loaded_w8 = 0
        self.weight_bytes_total = 0
        self.padding_in = np.zeros(0, np.float32)
        self.padding_out = np.zeros(0, np.float32)
        self.keys = set()
        self._attention = None  # the shared attention workspace (src/npu.rs:330, 729-742)

    # -- attention (src/npu.rs:442-466, 662-760; src/npu/attention.rs) ---------
    def attention(self, query_heads: int, kv_heads: int, dimension: int, softmax_scale: float):
        """A causal GQA KV cache on this backend."""
        from . import attention as A
        return A.attention_masked(self, query_heads, kv_heads, dimension, softmax_scale, False)

    def noncausal_gqa(self, query_heads: int, kv_heads: int, dimension: int):
        """Bidirectional GQA (src/npu.rs:694-705)."""
        from . import attention as A
        return A.attention_masked(self, query_heads, kv_heads, dimension, 1.0 / math.sqrt(dimension), True)

    def full_attention(self, heads: int, dimension: int, rows: int):
        from . import attention as A
        return A.full_attention(self, heads, dimension, rows)

    @staticmethod
    def attention_cache_bytes(options, query_heads: int, kv_heads: int, dimension: int, softmax_scale: float) -> int:
        from . import attention as A
        return A.attention_cache_bytes(options, query_heads, kv_heads, dimension, softmax_scale)

    @property
    def domain(self):
        return self._shared.domain.raw

    @property
    def ctx(self):
        return self._shared.ctx.raw

    # -- loading ---------------------------------------------------------------
    def load(self, matrix: QuantMatrix) -> "Linear":
        """src/npu.rs:532-650."""
        matrix.validate()
        L = F.lib()
        codes = np.ascontiguousarray(matrix.codes, np.int8).reshape(-1)
        scales = np.ascontiguousarray(matrix.scales, np.float32).reshape(-1)
        with self._lock:
            if matrix.bits == 4:
                cfg = F.rk_npu_i4_weight_config(matrix.k, matrix.n, 0)
                h = _Handle(L.rk_npu_w4a8_weights_create(self.domain, ctypes.byref(cfg), _ptr(codes, ctypes.c_int8),
                                                         _ptr(scales, ctypes.c_float)),
                            L.rk_npu_w4a8_weights_free, "certified W4 weights", self._shared)
                info = F.rk_npu_w4a8_weight_info()
                check(L.rk_npu_w4a8_weights_query(h.raw, ctypes.byref(info)), "W4 weight query")
                ensure(info.bound_relaxed == 0 and info.multiplier == 1.0, "uncertified W4 weights")
                kt = info.config.k_tile
                nbytes = ctypes.c_uint64()
                check(L.rk_npu_i4_weights_memory_query(ctypes.byref(info.config), ctypes.byref(nbytes)),
                      "W4 weight memory")
                self.weight_bytes_total += nbytes.value + matrix.n * 8
                self.loaded_w4 += 1
                w4, w8 = h, None
            else:
                kt = self._w8_partition(matrix.k, matrix.n)
                cfg = F.rk_npu_matmul_weight_config(matrix.k, matrix.n, kt)
                create = (L.rk_npu_f32i8f32_weights_create_compress if self.options.compress_w8a8
                          else L.rk_npu_f32i8f32_weights_create)
                h = _Handle(create(self.domain, ctypes.byref(cfg), _ptr(codes, ctypes.c_int8),
                                   _ptr(scales, ctypes.c_float)), L.rk_npu_f32i8f32_weights_free, "W8 weights",
                            self._shared)
                req = F.rk_npu_matmul_weight_requirements()
                check(L.rk_npu_f32i8f32_weights_memory_query(ctypes.byref(cfg), ctypes.byref(req)),
                      "W8 weight memory")
                self.weight_bytes_total += req.bytes
                self.loaded_w8 += 1
                w4, w8 = None, h
            key = (matrix.bits, matrix.k, matrix.n, kt)
            self.keys.add(key)
            self._with_work(key, 1)
        return Linear(w4, w8, key, self)

    def _w8_partition(self, k: int, n: int) -> int:
        """src/npu.rs:940-986 without tuning."""
        if (k, n) in self.w8_partitions:
            return self.w8_partitions[(k, n)]
        L = F.lib()
        rows = bucket(self.options.chunk)
        permitted = lambda tile: L.rk_npu_matmul_k_partition_query(rows, k, tile) == 0
        kt = min(k, 4096)
        if not permitted(kt):
            kt = min(k, 2048)
        if not permitted(kt):
            # The GPU reduces all of K in int32; no NPU partition applies.
            kt = k
        self.w8_partitions[(k, n)] = kt
        return kt

    # -- workspaces -----------------------------------------------------------------
    def _w8_strategy(self, key, m) -> F.rk_npu_matmul_strategy:
        """Fallback strategy of src/npu.rs:1060-1077."""
        _, k, n, kt = key
        self.fallbacks.add((key, m))
        s = F.rk_npu_matmul_strategy()
        s.op_kind = F.RK_NPU_MATMUL_F32I8F32_DYNAMIC
        s.M, s.N, s.K, s.k_tile = m, n, k, kt
        cores = bin(self.options.npu_mask).count("1")
        s.n_tile = max(32, min(1024, (n + 31) // 32 // cores * 32))
        s.a_layout = F.RK_NPU_MATMUL_A_LAYOUT_NORMAL
        s.c_layout = F.RK_NPU_MATMUL_C_LAYOUT_NATIVE
        s.wave_count = (k + kt - 1) // kt
        s.n_groups = ((n + 31) // 32 * 32 + s.n_tile - 1) // s.n_tile
        s.npu_core_mask = self.options.npu_mask
        s.cpu_core_mask = self.options.cpu_mask
        s.cpu_threads = self.options.threads
        return s

    def _w4_strategy(self, key, m) -> F.rk_npu_w4a8_strategy_ex:
        """Fallback strategy of src/npu.rs:1180-1193."""
        _, k, n, kt = key
        L = F.lib()
        self.fallbacks.add((key, m))
        s = F.rk_npu_w4a8_strategy_ex()
        L.rk_npu_w4a8_config_init(ctypes.byref(s.base.config), m, n, k)
        L.rk_npu_w4a8_options_init(ctypes.byref(s.execution))
        c = s.base.config
        c.k_tile = kt
        c.m_tile = min(m, 64)
        c.n_tile = min((n + 63) // 64 * 64, 1024)
        c.npu_core_mask = self.options.npu_mask
        c.cpu_threads = self.options.threads
        c.pipeline = F.RK_NPU_W4A8_PIPELINED
        s.base.cpu_core_mask = self.options.cpu_mask
        return s

    def _create_work(self, key, m) -> _Work:
        L = F.lib()
        work = _Work()
        if key[0] == 4:
            s = self._w4_strategy(key, m)
            info = F.rk_npu_w4a8_memory_info_ex()
            check(L.rk_npu_w4a8_memory_query_ex(ctypes.byref(s.base.config), ctypes.byref(s.execution),
                                                ctypes.byref(info)), "W4 memory query")
            work.bytes = info.workspace_bytes
            work.w4 = _Handle(L.rk_npu_w4a8_workspace_create_ex(self.domain, ctypes.byref(s.base.config),
                                                                ctypes.byref(s.execution)),
                              L.rk_npu_w4a8_workspace_free, "W4 workspace", self._shared)
        else:
            s = self._w8_strategy(key, m)
            req = F.rk_npu_matmul_workspace_requirements()
            check(L.rk_npu_matmul_workspace_memory_query(ctypes.byref(s), ctypes.byref(req)), "W8 memory query")
            work.bytes = req.bytes
            work.w8 = _Handle(L.rk_npu_matmul_workspace_create(self.domain, ctypes.byref(s)),
                              L.rk_npu_matmul_workspace_free, "W8 workspace", self._shared)
        return work

    def _with_work(self, key, m) -> _Work:
        wk = (key, m)
        if wk in self.work:
            return self.work[wk]
        work = self._idle.pop(wk, None) or self._create_work(key, m)
        self.work[wk] = work
        return work

    def _with_swiglu_work(self, key, m) -> _Work:
        """src/npu.rs:1284-1334: the fused call uses its own W4 workspace."""
        work = self._with_work(key, m)
        if work.w4_swiglu is None:
            L = F.lib()
            s = self._w4_strategy(key, m)
            s.base.config.cpu_threads = 1 if m == 1 else self.options.threads
            s.execution.reduce_backend = F.RK_NPU_W4A8_REDUCE_CPU
            info = F.rk_npu_w4a8_memory_info_ex()
            check(L.rk_npu_w4a8_memory_query_ex(ctypes.byref(s.base.config), ctypes.byref(s.execution),
                                                ctypes.byref(info)), "W4 SwiGLU memory query")
            work.w4_swiglu = _Handle(L.rk_npu_w4a8_workspace_create_ex(self.domain, ctypes.byref(s.base.config),
                                                                       ctypes.byref(s.execution)),
                                     L.rk_npu_w4a8_workspace_free, "W4 SwiGLU workspace", self._shared)
            work.bytes += info.workspace_bytes
        return work

    def prepare(self, rows: int) -> None:
        m = bucket(rows)
        with self._lock:
            for key in sorted(self.keys):
                self._with_work(key, m)

    def retain_workspaces(self, rows: Sequence[int]) -> None:
        keep = [bucket(r) for r in rows]
        with self._lock:
            self.work = {wk: w for wk, w in self.work.items() if wk[1] in keep}

    def fork_execution(self) -> "Backend":
        """src/npu/lane.rs:86-124: own workspaces, shared context/domain/weights."""
        lane = Backend(self.options, self.domain_id, _shared=self._shared)
        lane.w8_partitions = dict(self.w8_partitions)
        lane.keys = set(self.keys)
        return lane

    def weight_bytes(self) -> int:
        return self.weight_bytes_total

    def domain_memory(self) -> F.rk_npu_domain_memory_stats:
        stats = F.rk_npu_domain_memory_stats()
        check(F.lib().rk_npu_iommu_domain_memory_stats(self.domain, ctypes.byref(stats)), "domain stats")
        return stats

    def stats(self) -> dict:
        mem = self.domain_memory()
        workspace = sum(w.bytes for w in self.work.values()) + (self.padding_in.nbytes + self.padding_out.nbytes)
        return {
            "backend": "hip_matmul", "loaded_w4": self.loaded_w4, "loaded_w8": self.loaded_w8,
            "weight_payload_bytes": self.weight_bytes_total, "workspace_payload_bytes": workspace,
            "linear_padding_bytes": self.padding_in.nbytes + self.padding_out.nbytes,
            "domain_memory": {"live_bytes": mem.live_bytes, "peak_bytes": mem.peak_bytes,
                              "creates": mem.creates, "destroys": mem.destroys},
            "workspace_count": len(self.work),
            "swiglu_workspace_count": sum(1 for w in self.work.values() if w.w4_swiglu is not None),
            "strategy_fallbacks": len(self.fallbacks), "iommu_domain_id": self.domain_id,
        }

    # -- MoE ----------------------------------------------------------------------------
    def load_moe(self, gate: Sequence[QuantMatrix], down: Sequence[QuantMatrix], top: int) -> "Moe":
        return self._load_moe(gate, down, top, None)

    def load_moe_with_shared(self, gate, down, top, shared: Tuple[QuantMatrix, QuantMatrix]) -> "Moe":
        return self._load_moe(gate, down, top, shared)

    def _load_moe(self, gate, down, top, shared) -> "Moe":
        """src/npu/moe.rs:88-219. Routed gate_up must be W4; down may be W4 or W8
        (W8 routed down selects the mixed bank)."""
        ensure(len(gate) > 0 and len(gate) == len(down), "invalid expert bank")
        for m in list(gate) + list(down):
            m.validate()
        ensure(all(g.bits == 4 for g in gate), "grouped MoE requires W4 gate/up weights")
        dn_bits = down[0].bits
        ensure(all(d.bits == dn_bits for d in down), "grouped MoE requires one down precision")
        h, f, e = gate[0].k, gate[0].n // 2, len(gate)
        ensure(all(g.k == h and g.n == 2 * f for g in gate) and all(d.k == f and d.n == h for d in down),
               "incompatible expert matrices")
        keep = []
        experts = (F.rk_npu_moe_w8_expert * (e + (1 if shared else 0)))()
        for i, (g, d) in enumerate(zip(gate, down)):
            arrs = [np.ascontiguousarray(g.codes, np.int8).reshape(-1),
                    np.ascontiguousarray(g.scales, np.float32).reshape(-1),
                    np.ascontiguousarray(d.codes, np.int8).reshape(-1),
                    np.ascontiguousarray(d.scales, np.float32).reshape(-1)]
            keep.append(arrs)
            experts[i] = F.rk_npu_moe_w8_expert(_ptr(arrs[0], ctypes.c_int8), _ptr(arrs[1], ctypes.c_float),
                                                _ptr(arrs[2], ctypes.c_int8), _ptr(arrs[3], ctypes.c_float))
        if shared:
            g, d = shared
            g.validate()
            d.validate()
            ensure(g.bits == 8 and d.bits == 8 and g.k == h and g.n == 2 * f and d.k == f and d.n == h,
                   "joint MoE requires a shared W8 expert with the routed intermediate width")
            arrs = [np.ascontiguousarray(g.codes, np.int8).reshape(-1),
                    np.ascontiguousarray(g.scales, np.float32).reshape(-1),
                    np.ascontiguousarray(d.codes, np.int8).reshape(-1),
                    np.ascontiguousarray(d.scales, np.float32).reshape(-1)]
            keep.append(arrs)
            experts[e] = F.rk_npu_moe_w8_expert(_ptr(arrs[0], ctypes.c_int8), _ptr(arrs[1], ctypes.c_float),
                                                _ptr(arrs[2], ctypes.c_int8), _ptr(arrs[3], ctypes.c_float))
        L = F.lib()
        config = F.rk_npu_moe_w8_config()
        L.rk_npu_moe_w8_config_init(ctypes.byref(config), h, f, e, 1 if shared else 0, top, self.options.chunk)
        config.npu_cores = bin(self.options.npu_mask).count("1")
        config.cpu_threads = self.options.threads
        if dn_bits == 8:
            create, ws_create = L.rk_npu_moe_w4w8_weights_create, L.rk_npu_moe_w4w8_workspace_create
        elif shared:
            create, ws_create = L.rk_npu_moe_w4_weights_create, L.rk_npu_moe_w4_workspace_create
        else:
            create, ws_create = L.rk_npu_moe_quant_weights_create, L.rk_npu_moe_quant_workspace_create
        with self._lock:
            weights = _Handle(create(self.domain, ctypes.byref(config.weights), experts),
                              L.rk_npu_moe_w8_weights_free, "packed MoE expert bank", self._shared)
            workspace = _Handle(ws_create(self.domain, ctypes.byref(config)), L.rk_npu_moe_w8_workspace_free,
                                "grouped MoE workspace", self._shared)
            self.weight_bytes_total += L.rk_npu_moe_w8_weights_device_bytes(weights.raw)
        return Moe(weights, workspace, (h, f, e, top, bool(shared)), self)


class Linear:
    """src/npu.rs:1337-1438."""

    def __init__(self, w4, w8, key, owner: Backend):
        self.w4, self.w8, self.key, self.owner = w4, w8, key, owner

    def k(self) -> int:
        return self.key[1]

    def n(self) -> int:
        return self.key[2]

    def run(self, input: np.ndarray, output: np.ndarray, rows: int, lane: Optional[Backend] = None) -> None:
        self._run(input, output, rows, False, lane)

    def run_swiglu(self, input: np.ndarray, output: np.ndarray, rows: int, lane: Optional[Backend] = None) -> bool:
        if self.w4 is None or self.n() % 64 != 0:
            return False
        self._run(input, output, rows, True, lane)
        return True

    def _run(self, input, output, rows, swiglu, lane):
        m = bucket(rows)
        width = self.n() // 2 if swiglu else self.n()
        inp = np.asarray(input).reshape(-1)
        out = np.asarray(output).reshape(-1)
        ensure(inp.size >= rows * self.k() and out.size >= rows * width, "linear input/output shape mismatch")
        ensure(inp.dtype == np.float32 and out.dtype == np.float32 and inp.flags.c_contiguous
               and out.flags.c_contiguous, "linear buffers must be contiguous f32")
        b = lane or self.owner
        L = F.lib()
        with b._lock:
            work = b._with_swiglu_work(self.key, m) if swiglu else b._with_work(self.key, m)
            if m != rows:
                if b.padding_in.size < m * self.k():
                    b.padding_in = np.zeros(m * self.k(), np.float32)
                if b.padding_out.size < m * width:
                    b.padding_out = np.zeros(m * width, np.float32)
                b.padding_in[:rows * self.k()] = inp[:rows * self.k()]
                b.padding_in[rows * self.k():m * self.k()] = 0.0
                a, c = b.padding_in, b.padding_out
            else:
                a, c = inp, out
            ap, cp = _ptr(a, ctypes.c_float), _ptr(c, ctypes.c_float)
            if self.w4 is not None:
                ws = work.w4_swiglu if swiglu else work.w4
                fn = L.rk_npu_w4a8_run_swiglu_f32 if swiglu else L.rk_npu_w4a8_run_f32
                check(fn(ws.raw, self.w4.raw, ap, cp, None), "W4 SwiGLU run" if swiglu else "W4 run")
            else:
                check(L.rk_npu_f32i8f32_run_dynamic(work.w8.raw, self.w8.raw, ap, cp), "W8 run")
            if m != rows:
                out[:rows * width] = c[:rows * width]


class Moe:
    """src/npu/moe.rs:10-388."""

    def __init__(self, weights: _Handle, workspace: _Handle, key, owner: Backend):
        self.weights, self.workspace, self.key, self.owner = weights, workspace, key, owner

    def max_rows(self) -> int:
        return self.owner.options.chunk

    def weight_bytes(self) -> int:
        return F.lib().rk_npu_moe_w8_weights_device_bytes(self.weights.raw)

    def run(self, input, ids, routes, output, rows: int) -> None:
        h, _, _, top, _ = self.key
        inp = np.asarray(input)
        out = np.asarray(output)
        ids = np.ascontiguousarray(ids, np.int32).reshape(-1)
        routes = np.ascontiguousarray(routes, np.float32).reshape(-1)
        ensure(inp.size == rows * h and out.size == rows * h and ids.size == rows * top
               and routes.size == ids.size, "grouped MoE input shape mismatch")
        ensure(inp.dtype == np.float32 and out.dtype == np.float32 and inp.flags.c_contiguous
               and out.flags.c_contiguous, "MoE buffers must be contiguous f32")
        with self.owner._lock:
            check(F.lib().rk_npu_moe_w8_run_f32(self.workspace.raw, self.weights.raw, rows,
                                                _ptr(inp, ctypes.c_float), _ptr(ids, ctypes.c_int32),
                                                _ptr(routes, ctypes.c_float), _ptr(out, ctypes.c_float), None),
                  "grouped routed FFN")

    def blob_bytes(self) -> int:
        return F.lib().rk_npu_moe_quant_expert_blob_bytes(self.weights.raw)

    def export(self, expert: int) -> bytes:
        ensure(0 <= expert < self.key[2], "expert index out of range")
        n = self.blob_bytes()
        ensure(n > 0, "expert bank has no packed cache representation")
        buf = ctypes.create_string_buffer(n)
        check(F.lib().rk_npu_moe_quant_export_expert(self.weights.raw, expert, buf, n), "export packed expert")
        return buf.raw

    def import_(self, slot: int, data: bytes) -> None:
        ensure(0 <= slot < self.key[2], "expert slot out of range")
        check(F.lib().rk_npu_moe_quant_import_expert(self.weights.raw, slot, data, len(data)),
              "import packed expert")

    def promote(self, slot: int, bank: "Moe", staged: int) -> None:
        check(F.lib().rk_npu_moe_quant_swap_slots(self.weights.raw, slot, bank.weights.raw, staged),
              "promote staged expert")


def routes(logits: Sequence[float], top: int) -> Tuple[List[int], List[float]]:
    """Router of src/model/qwen35/moe.rs:51-67 (caller side, CPU): top-k by
    descending logit (IEEE total order, ties to the lower id), softmax over
    the selected k in f32."""
    x = np.asarray(logits, np.float32).reshape(-1)
    ensure(0 < top <= x.size, "invalid router top-k")
    bits = x.view(np.int32).astype(np.int64)
    key = np.where(bits < 0, bits ^ 0x7FFFFFFF, bits)
    order = sorted(range(x.size), key=lambda i: (-key[i], i))[:top]
    mx = x[order[0]]
    w = [np.float32(math.exp(np.float32(x[i] - mx))) for i in order]
    s = np.float32(0.0)
    for v in w:
        s = np.float32(s + v)
    return [int(i) for i in order], [float(np.float32(v / s)) for v in w]
