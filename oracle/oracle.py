"""numpy front end of the CPU oracle — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module, and only as the checker or the timed CPU baseline.
Each function forwards to ``librk_oracle.so`` (oracle/rk_oracle.c), whose
header cites the reference file:line every function restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "librk_oracle.so")
_lib = None

_i8p = ctypes.POINTER(ctypes.c_int8)
_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u32p = ctypes.POINTER(ctypes.c_uint32)


def build() -> str:
    """Compile the oracle with its Makefile (gcc only, no GPU)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        L = _lib
        L.orc_bucket.argtypes = [ctypes.c_int]
        L.orc_bucket.restype = ctypes.c_int
        L.orc_quant_dense_row.argtypes = [_f32p, ctypes.c_int, _i8p, _f32p]
        L.orc_quant_moe_row.argtypes = [_f32p, ctypes.c_int, _i8p, _f32p]
        L.orc_gemm_i8.argtypes = [_i8p, _i8p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p]
        L.orc_dequant.argtypes = [ctypes.c_int32, ctypes.c_float, ctypes.c_float]
        L.orc_dequant.restype = ctypes.c_float
        L.orc_linear.argtypes = [_i8p, _f32p, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_int,
                                 _f32p, _i8p, _f32p, _i32p]
        L.orc_expf.argtypes = [ctypes.c_float]
        L.orc_expf.restype = ctypes.c_float
        L.orc_swiglu.argtypes = [ctypes.c_float, ctypes.c_float]
        L.orc_swiglu.restype = ctypes.c_float
        L.orc_linear_swiglu.argtypes = [_i8p, _f32p, ctypes.c_int, ctypes.c_int, _f32p,
                                        ctypes.c_int, _f32p]
        L.orc_ffn.argtypes = [_i8p, _f32p, _i8p, _f32p, ctypes.c_int, ctypes.c_int, _f32p,
                              ctypes.c_int, _f32p, _f32p]
        L.orc_moe.argtypes = [ctypes.POINTER(_i8p), ctypes.POINTER(_f32p),
                              ctypes.POINTER(_i8p), ctypes.POINTER(_f32p),
                              ctypes.c_int, ctypes.c_int, ctypes.c_int,
                              _i8p, _f32p, _i8p, _f32p, ctypes.c_int,
                              _f32p, ctypes.c_int, _i32p, _f32p, ctypes.c_int, _f32p]
        L.orc_routes.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _i32p, _f32p]
        L.orc_routes.restype = ctypes.c_int
        L.orc_unpack_codes.argtypes = [_u32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i8p]
        L.orc_concatenate.argtypes = [ctypes.POINTER(_i8p), ctypes.POINTER(ctypes.c_int),
                                      ctypes.c_int, ctypes.c_int, _i8p]
        L.orc_threads.restype = ctypes.c_int
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def threads() -> int:
    return lib().orc_threads()


def bucket(rows: int) -> int:
    return lib().orc_bucket(rows)


def quant_dense(x: np.ndarray):
    """Per-row dense A8 quantization -> (codes int8 [M][K], scales f32 [M])."""
    x = _c(np.atleast_2d(x), np.float32)
    m, k = x.shape
    q = np.empty((m, k), np.int8)
    s = np.empty(m, np.float32)
    for r in range(m):
        lib().orc_quant_dense_row(_p(x[r], _f32p), k, _p(q[r], _i8p), _p(s[r:], _f32p))
    return q, s


def quant_moe(x: np.ndarray):
    x = _c(np.atleast_2d(x), np.float32)
    m, k = x.shape
    q = np.empty((m, k), np.int8)
    s = np.empty(m, np.float32)
    for r in range(m):
        lib().orc_quant_moe_row(_p(x[r], _f32p), k, _p(q[r], _i8p), _p(s[r:], _f32p))
    return q, s


def gemm_i8(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """int32 acc [M][N] = a [M][K] (int8) x w [K][N] (int8)."""
    a = _c(a, np.int8)
    w = _c(w, np.int8)
    m, k = a.shape
    k2, n = w.shape
    assert k == k2
    acc = np.empty((m, n), np.int32)
    lib().orc_gemm_i8(_p(a, _i8p), _p(w, _i8p), m, k, n, _p(acc, _i32p))
    return acc


def linear(codes: np.ndarray, scales: np.ndarray, x: np.ndarray, intermediates: bool = False):
    """Linear::run oracle: codes [K][N] int8, scales [N], x [rows][K] -> [rows][N]."""
    codes = _c(codes, np.int8)
    scales = _c(scales, np.float32)
    x = _c(np.atleast_2d(x), np.float32)
    k, n = codes.shape
    rows = x.shape[0]
    assert x.shape[1] == k
    out = np.empty((rows, n), np.float32)
    q = np.empty((rows, k), np.int8)
    s = np.empty(rows, np.float32)
    acc = np.empty((rows, n), np.int32)
    lib().orc_linear(_p(codes, _i8p), _p(scales, _f32p), k, n, _p(x, _f32p), rows,
                     _p(out, _f32p), _p(q, _i8p), _p(s, _f32p), _p(acc, _i32p))
    if intermediates:
        return out, q, s, acc
    return out


def expf(x) -> np.ndarray:
    x = np.asarray(x, np.float32)
    f = lib().orc_expf
    return np.array([f(float(v)) for v in x.ravel()], np.float32).reshape(x.shape)


def swiglu(g, u) -> np.ndarray:
    g = np.asarray(g, np.float32)
    u = np.asarray(u, np.float32)
    f = lib().orc_swiglu
    return np.array([f(float(a), float(b)) for a, b in zip(g.ravel(), u.ravel())],
                    np.float32).reshape(g.shape)


def linear_swiglu(codes, scales, x) -> np.ndarray:
    codes = _c(codes, np.int8)
    scales = _c(scales, np.float32)
    x = _c(np.atleast_2d(x), np.float32)
    k, n = codes.shape
    rows = x.shape[0]
    out = np.empty((rows, n // 2), np.float32)
    lib().orc_linear_swiglu(_p(codes, _i8p), _p(scales, _f32p), k, n, _p(x, _f32p), rows,
                            _p(out, _f32p))
    return out


def ffn(gu_codes, gu_scales, dn_codes, dn_scales, x, with_middle: bool = False):
    gu_codes = _c(gu_codes, np.int8)
    dn_codes = _c(dn_codes, np.int8)
    gu_scales = _c(gu_scales, np.float32)
    dn_scales = _c(dn_scales, np.float32)
    x = _c(np.atleast_2d(x), np.float32)
    h, f2 = gu_codes.shape
    f = f2 // 2
    assert dn_codes.shape == (f, h)
    rows = x.shape[0]
    out = np.empty((rows, h), np.float32)
    mid = np.empty((rows, f), np.float32)
    lib().orc_ffn(_p(gu_codes, _i8p), _p(gu_scales, _f32p), _p(dn_codes, _i8p),
                  _p(dn_scales, _f32p), h, f, _p(x, _f32p), rows, _p(out, _f32p),
                  _p(mid, _f32p))
    return (out, mid) if with_middle else out


def moe(gate_up, down, x, ids, routes, shared=None) -> np.ndarray:
    """gate_up / down: lists of (codes, scales) per expert; shared: optional
    ((codes, scales), (codes, scales)); x [rows][h]; ids/routes [rows][top]."""
    gate_up = [(_c(c, np.int8), _c(s, np.float32)) for c, s in gate_up]
    down = [(_c(c, np.int8), _c(s, np.float32)) for c, s in down]
    e = len(gate_up)
    h, i2 = gate_up[0][0].shape
    inter = i2 // 2
    x = _c(np.atleast_2d(x), np.float32)
    ids = _c(ids, np.int32)
    routes = _c(routes, np.float32)
    rows, top = ids.shape
    gu_c = (_i8p * e)(*[_p(c, _i8p) for c, _ in gate_up])
    gu_s = (_f32p * e)(*[_p(s, _f32p) for _, s in gate_up])
    dn_c = (_i8p * e)(*[_p(c, _i8p) for c, _ in down])
    dn_s = (_f32p * e)(*[_p(s, _f32p) for _, s in down])
    out = np.empty((rows, h), np.float32)
    if shared is not None:
        (sgc, sgs), (sdc, sds) = shared
        sgc, sdc = _c(sgc, np.int8), _c(sdc, np.int8)
        sgs, sds = _c(sgs, np.float32), _c(sds, np.float32)
        sh_inter = sgc.shape[1] // 2
        args = (_p(sgc, _i8p), _p(sgs, _f32p), _p(sdc, _i8p), _p(sds, _f32p), sh_inter)
    else:
        args = (None, None, None, None, 0)
    lib().orc_moe(gu_c, gu_s, dn_c, dn_s, e, h, inter, *args, _p(x, _f32p), rows,
                  _p(ids, _i32p), _p(routes, _f32p), top, _p(out, _f32p))
    return out


def routes(logits, top):
    logits = _c(logits, np.float32)
    ids = np.empty(top, np.int32)
    weights = np.empty(top, np.float32)
    rc = lib().orc_routes(_p(logits, _f32p), logits.size, top, _p(ids, _i32p),
                          _p(weights, _f32p))
    if rc != 0:
        raise ValueError("invalid router top-k")
    return ids, weights


def unpack_codes(words: np.ndarray, bits: int, n: int, k: int) -> np.ndarray:
    words = _c(words, np.uint32)
    codes = np.empty((k, n), np.int8)
    lib().orc_unpack_codes(_p(words, _u32p), bits, n, k, _p(codes, _i8p))
    return codes


def concatenate(mats) -> np.ndarray:
    mats = [_c(m, np.int8) for m in mats]
    k = mats[0].shape[0]
    ns = [m.shape[1] for m in mats]
    out = np.empty((k, sum(ns)), np.int8)
    arr = (_i8p * len(mats))(*[_p(m, _i8p) for m in mats])
    nsa = (ctypes.c_int * len(mats))(*ns)
    lib().orc_concatenate(arr, nsa, len(mats), k, _p(out, _i8p))
    return out


def attention(q, k, v, scale: float, position: int, causal: bool) -> np.ndarray:
    """Grouped-query attention over a KV cache, in float64 (numpy; no C
    counterpart). Layouts of src/npu/attention.rs:240-262, 325-351: q
    [query_heads][rows][head_dim], k and v [kv_heads][length][head_dim]
    (fp16 values), query head h reads KV head h // (query_heads // kv_heads);
    row r sits at absolute position ``position + r`` and, with the causal mask,
    sees keys j <= position + r; the softmax subtracts the row max (the
    STABLE_SOFTMAX flag of src/npu.rs:437) and the scores are
    ``scale * (q . k)``. Parity unpinned against the reference: its attention
    is a closed native library (only the call sites are in the repository);
    tests pin this restatement by brute force on tiny inputs and by the
    softmax invariants instead."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    qh, rows, d = q.shape
    kh, length, _ = k.shape
    group = qh // kh
    out = np.empty((qh, rows, d), np.float64)
    for h in range(qh):
        kk, vv = k[h // group], v[h // group]
        s = scale * (q[h] @ kk.T)  # [rows][length]
        if causal:
            limit = position + np.arange(rows)[:, None]
            s = np.where(np.arange(length)[None, :] <= limit, s, -np.inf)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[h] = (p @ vv) / p.sum(axis=1, keepdims=True)
    return out
