"""Device-resident use of the C ABI (rk_npu_hip.h) with torch tensors.

torch provides device memory and streams only; every computation is a
hip_matmul kernel launched through the C ABI on torch's current stream.
"""
from __future__ import annotations

import contextlib
import ctypes
from typing import Dict, List, Optional, Tuple

from . import _ffi as F
from .npu import NpuError, _Handle, _Shared, check, ensure

_DT = {}


def _dtype_code(t) -> int:
    import torch
    if t.dtype == torch.float32:
        return F.RK_NPU_HIP_F32
    if t.dtype == torch.float16:
        return F.RK_NPU_HIP_F16
    raise NpuError(f"unsupported activation dtype {t.dtype}")


def current_stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class DeviceContext:
    """One context + allocation domain; owns weights and workspaces."""

    def __init__(self, domain_id: int = 0, device: Optional[str] = None):
        self.shared = _Shared(domain_id, device)
        self._ws: Dict[Tuple[int, int, int, int], _Handle] = {}

    @property
    def domain(self):
        return self.shared.domain.raw

    def weights(self, bits: int, codes, scales) -> "DeviceWeights":
        """codes: int8 [K][N] cuda tensor, scales: f32 [N] cuda tensor."""
        import torch
        ensure(codes.is_cuda and scales.is_cuda and codes.dtype == torch.int8 and scales.dtype == torch.float32,
               "device weights need cuda int8 codes and f32 scales")
        codes = codes.contiguous()
        scales = scales.contiguous()
        k, n = codes.shape
        L = F.lib()
        torch.cuda.synchronize()
        if bits == 4:
            raw = L.rk_npu_hip_w4a8_weights_create_device(self.domain, ctypes.byref(F.rk_npu_i4_weight_config(k, n, 0)),
                                                          ctypes.c_void_p(codes.data_ptr()),
                                                          ctypes.c_void_p(scales.data_ptr()))
            h = _Handle(raw, L.rk_npu_w4a8_weights_free, "W4 weights", self.shared)
        else:
            raw = L.rk_npu_hip_f32i8f32_weights_create_device(self.domain,
                                                              ctypes.byref(F.rk_npu_matmul_weight_config(k, n, k)),
                                                              ctypes.c_void_p(codes.data_ptr()),
                                                              ctypes.c_void_p(scales.data_ptr()))
            h = _Handle(raw, L.rk_npu_f32i8f32_weights_free, "W8 weights", self.shared)
        return DeviceWeights(h, bits, k, n)

    def weights_from_checkpoint(self, bits: int, k: int, parts) -> "DeviceWeights":
        """Weights from checkpoint storage on the device, fused along N in order.
        parts: (data, scales, fmt) with data a cuda tensor of int32 words
        [n][ceil(k*bits/32)] (fmt RK_NPU_HIP_PACK_QUANTIZED) or int8 codes [n][k]
        (RK_NPU_HIP_INT_QUANTIZED, bits 8) and scales f32 [n]."""
        import torch
        torch.cuda.synchronize()
        arr = (F.rk_npu_hip_checkpoint_part * len(parts))()
        n_total = 0
        keep = []
        for i, (data, scales, fmt) in enumerate(parts):
            ensure(data.is_cuda and scales.is_cuda and scales.dtype == torch.float32, "checkpoint parts must be on the GPU")
            data, scales = data.contiguous(), scales.contiguous()
            keep += [data, scales]
            arr[i] = F.rk_npu_hip_checkpoint_part(data.data_ptr(), scales.data_ptr(), data.shape[0], fmt)
            n_total += data.shape[0]
        L = F.lib()
        raw = L.rk_npu_hip_weights_create_checkpoint(self.domain, bits, k, arr, len(parts))
        free = L.rk_npu_w4a8_weights_free if bits == 4 else L.rk_npu_f32i8f32_weights_free
        h = _Handle(raw, free, f"W{bits} weights from checkpoint storage", self.shared)
        return DeviceWeights(h, bits, k, n_total)

    def workspace(self, bits: int, rows: int, k: int, n: int, cached: bool = True) -> _Handle:
        """The context's workspace for (bits, rows, k, n), created on first use;
        cached=False creates a new one (sized by the plan switches in force,
        e.g. for split-K partials under HM_SPLITS) and does not keep it."""
        key = (bits, rows, k, n)
        if not cached:
            saved = self._ws.pop(key, None)
            try:
                return self.workspace(bits, rows, k, n)
            finally:
                self._ws.pop(key, None)
                if saved is not None:
                    self._ws[key] = saved
        if key not in self._ws:
            L = F.lib()
            if bits == 4:
                cfg = F.rk_npu_w4a8_config()
                opt = F.rk_npu_w4a8_options()
                L.rk_npu_w4a8_config_init(ctypes.byref(cfg), rows, n, k)
                L.rk_npu_w4a8_options_init(ctypes.byref(opt))
                self._ws[key] = _Handle(L.rk_npu_w4a8_workspace_create_ex(self.domain, ctypes.byref(cfg),
                                                                          ctypes.byref(opt)),
                                        L.rk_npu_w4a8_workspace_free, "W4 workspace", self.shared)
            else:
                st = F.rk_npu_matmul_strategy()
                st.op_kind = F.RK_NPU_MATMUL_F32I8F32_DYNAMIC
                st.M, st.N, st.K, st.k_tile = rows, n, k, k
                self._ws[key] = _Handle(L.rk_npu_matmul_workspace_create(self.domain, ctypes.byref(st)),
                                        L.rk_npu_matmul_workspace_free, "W8 workspace", self.shared)
        return self._ws[key]


class DeviceWeights:
    def __init__(self, handle: _Handle, bits: int, k: int, n: int):
        self.handle, self.bits, self.k, self.n = handle, bits, k, n

    def bytes(self) -> int:
        """Algorithmic weight bytes: codes at storage width plus f32 scales."""
        return self.k * self.n * self.bits // 8 + 4 * self.n


def linear(ctx: DeviceContext, w: DeviceWeights, x, out, rows: int, swiglu: bool = False, ws=None, stream=None):
    ws = ws or ctx.workspace(w.bits, rows, w.k, w.n)
    rc = F.lib().rk_npu_hip_linear_run(ws.raw, w.handle.raw, w.bits, ctypes.c_void_p(x.data_ptr()), _dtype_code(x),
                                       ctypes.c_void_p(out.data_ptr()), _dtype_code(out), rows,
                                       F.RK_NPU_HIP_SWIGLU if swiglu else F.RK_NPU_HIP_PLAIN,
                                       stream if stream is not None else current_stream())
    check(rc, "device linear")


def ffn(ctx: DeviceContext, gate_up: DeviceWeights, down: DeviceWeights, x, out, rows: int, gws=None, dws=None,
        stream=None):
    gws = gws or ctx.workspace(gate_up.bits, rows, gate_up.k, gate_up.n)
    dws = dws or ctx.workspace(down.bits, rows, down.k, down.n)
    rc = F.lib().rk_npu_hip_ffn_run(gws.raw, gate_up.handle.raw, gate_up.bits, dws.raw, down.handle.raw, down.bits,
                                    ctypes.c_void_p(x.data_ptr()), _dtype_code(x), ctypes.c_void_p(out.data_ptr()),
                                    _dtype_code(out), rows, stream if stream is not None else current_stream())
    check(rc, "device FFN")


@contextlib.contextmanager
def plan_switch(name: str, value: int):
    """Sets one of the library's plan switches (rk_npu_hip_set_switch, e.g.
    HM_GEMM_VARIANT) for the body of the with-block, then restores it."""
    L = F.lib()
    prev = ctypes.c_int()
    check(L.rk_npu_hip_set_switch(name.encode(), int(value), ctypes.byref(prev)), f"set switch {name}")
    try:
        yield
    finally:
        check(L.rk_npu_hip_set_switch(name.encode(), prev.value, None), f"restore switch {name}")


class KernelProfile:
    """rk_npu_hip_profile_* as a context manager; .stats after exit."""

    def __init__(self, max_launches: int = 65536):
        self.max_launches = max_launches
        self.stats: List[dict] = []

    def __enter__(self):
        check(F.lib().rk_npu_hip_profile_begin(self.max_launches), "profile begin")
        return self

    def __exit__(self, *exc):
        L = F.lib()
        L.rk_npu_hip_profile_end()
        cap = 4096
        arr = (F.rk_npu_hip_kernel_stat * cap)()
        n = ctypes.c_int()
        check(L.rk_npu_hip_profile_read(arr, cap, ctypes.byref(n)), "profile read")
        self.stats = [dict(kind=s.kind, bits=s.bits, epilogue=s.epilogue, rows=s.rows, K=s.K, N=s.N,
                           launches=s.launches, total_ms=s.total_ms, name=s.name.decode())
                      for s in arr[:min(n.value, cap)]]
        return False
