"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every fixture bit for bit, and the fixtures satisfy
the closed forms of the reference's CPU semantics (src/npu.rs:1537-1553)
computed here independently with numpy: zero row -> scale 1 and zero codes,
ties rounded half away from zero, +-127 saturation, int32 accumulation as an
exact integer product, dequantization as two single-precision multiplies.
GPU: the HIP path reproduces every fixture bit for bit through the C ABI."""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle
from open_rknpu2_lm_infer_amd import _ffi as F
from open_rknpu2_lm_infer_amd import npu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
F32 = np.float32


def load(name):
    with np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def round_half_away(v):
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


# ---- CPU -----------------------------------------------------------------------

@pytest.mark.parametrize("bits", [8, 4])
def test_linear_fixture_closed_forms(bits):
    d = load(f"linear_w{bits}")
    codes, scales, x, q, s, acc, y = (d[k] for k in ("codes", "scales", "x", "q", "s", "acc", "y"))
    # scale: max|x| / 127 with the FLT_MIN floor, 1 for a zero row
    m = np.abs(x).max(axis=1)
    s_ref = np.where(m == 0, F32(1.0), np.maximum(m / F32(127.0), np.finfo(F32).tiny)).astype(F32)
    assert np.array_equal(s, s_ref)
    assert s[0] == 1.0 and not q[0].any() and not y[0].any()
    # codes: round half away from zero of x * (1/s), clamped to +-127
    inv = (F32(1.0) / s).astype(F32)
    q_ref = np.clip(round_half_away((x * inv[:, None]).astype(F32)), -127, 127).astype(np.int8)
    assert np.array_equal(q, q_ref)
    assert s[1] == 1.0 and x[1, 1] == -2.5 and q[1, 1] == -3  # a tie: away from zero (even gives -2)
    assert q[2].min() == -127                                 # the outlier saturates
    if bits == 4:
        assert codes.min() == -8 and codes.max() == 7
    # int32 accumulation is the exact integer product
    assert np.array_equal(acc, (q.astype(np.int64) @ codes.astype(np.int64)).astype(np.int32))
    # dequantization: (f32(acc) * s) * scale, two rounded multiplies
    y_ref = ((acc.astype(F32) * s[:, None]).astype(F32) * scales[None, :]).astype(F32)
    assert np.array_equal(y, y_ref)


@pytest.mark.parametrize("bits", [8, 4])
def test_oracle_reproduces_linear_fixture(bits):
    d = load(f"linear_w{bits}")
    y, q, s, acc = oracle.linear(d["codes"], d["scales"], d["x"], intermediates=True)
    for got, want in ((y, d["y"]), (q, d["q"]), (s, d["s"]), (acc, d["acc"])):
        assert np.array_equal(got, want)


def test_oracle_reproduces_fused_fixtures():
    d = load("swiglu_w4")
    assert np.array_equal(oracle.linear_swiglu(d["codes"], d["scales"], d["x"]), d["y"])
    lin = oracle.linear(d["codes"], d["scales"], d["x"])
    half = d["codes"].shape[1] // 2
    assert np.array_equal(oracle.swiglu(lin[:, :half], lin[:, half:]), d["y"])  # gate = first N/2
    d = load("ffn")
    y, mid = oracle.ffn(d["gu_codes"], d["gu_scales"], d["dn_codes"], d["dn_scales"], d["x"], with_middle=True)
    assert np.array_equal(y, d["y"]) and np.array_equal(mid, d["mid"])
    assert np.array_equal(oracle.linear(d["dn_codes"], d["dn_scales"], mid), y)  # requant + down
    d = load("scalar")
    assert np.array_equal(oracle.expf(-d["exp_in"]), d["exp_out"])
    assert np.array_equal(oracle.swiglu(d["g"], d["u"]), d["swiglu"])
    g64 = d["g"].astype(np.float64)
    with np.errstate(over="ignore"):  # the formula of native/cpu_kernels/swiglu.cpp:23-26, in double
        ref = g64 / (1.0 + np.exp(-g64)) * d["u"].astype(np.float64)
    fin = np.abs(ref) <= np.finfo(F32).max  # beyond it the f32 product overflows to inf
    ok = np.abs(d["swiglu"] - ref) <= 3e-5 * np.maximum(np.abs(ref), 1.0)  # src/npu.rs:1651-1658
    assert ok[fin].all() and np.isinf(d["swiglu"][~fin]).all()
    assert np.signbit(d["swiglu"][d["g"] < -80]).any()  # gate below the clamp: signed zero


def moe_fixture():
    d = load("moe")
    e = sum(1 for k in d if k.startswith("gu_codes"))
    gu = [(d[f"gu_codes{i}"], d[f"gu_scales{i}"]) for i in range(e)]
    dn = [(d[f"dn_codes{i}"], d[f"dn_scales{i}"]) for i in range(e)]
    sh = ((d["sh_gu_codes"], d["sh_gu_scales"]), (d["sh_dn_codes"], d["sh_dn_scales"]))
    return d, gu, dn, sh


def test_oracle_reproduces_moe_fixture():
    d, gu, dn, sh = moe_fixture()
    assert np.array_equal(oracle.moe(gu, dn, d["x"], d["ids"], d["routes"], shared=sh), d["y"])
    top = d["ids"].shape[1]
    for r in range(4):  # rows 4 and 5 were edited after routing
        ids, w = oracle.routes(d["logits"][r], top)
        assert np.array_equal(ids, d["ids"][r]) and np.array_equal(w, d["routes"][r])


# ---- GPU -----------------------------------------------------------------------

@pytest.fixture(scope="module")
def backend():
    return npu.Backend(npu.ModelOptions(chunk=16))


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [8, 4])
def test_hip_linear_reproduces_fixture(backend, bits):
    d = load(f"linear_w{bits}")
    k, n = d["codes"].shape
    rows = d["x"].shape[0]
    lin = backend.load(npu.QuantMatrix(bits, k, n, d["codes"], d["scales"]))
    out = np.zeros((rows, n), F32)
    print(f"golden linear w{bits}", flush=True)
    lin.run(d["x"], out, rows)
    assert np.array_equal(out, d["y"])


@pytest.mark.gpu
def test_hip_swiglu_reproduces_fixture(backend):
    d = load("swiglu_w4")
    k, n = d["codes"].shape
    rows = d["x"].shape[0]
    lin = backend.load(npu.QuantMatrix(4, k, n, d["codes"], d["scales"]))
    out = np.zeros((rows, n // 2), F32)
    print("golden swiglu", flush=True)
    assert lin.run_swiglu(d["x"], out, rows)
    assert np.array_equal(out, d["y"])


@pytest.mark.gpu
def test_hip_ffn_reproduces_fixture(backend):
    d = load("ffn")
    L = F.lib()
    gc, gs, dc, ds, x = (np.ascontiguousarray(d[k]) for k in ("gu_codes", "gu_scales", "dn_codes", "dn_scales", "x"))
    h, f2 = gc.shape
    f, rows = f2 // 2, x.shape[0]
    p = lambda a, t: a.ctypes.data_as(ctypes.POINTER(t))
    dom, sh = backend.domain, backend._shared
    gw = npu._Handle(L.rk_npu_w4a8_weights_create(dom, ctypes.byref(F.rk_npu_i4_weight_config(h, f2, 0)),
                                                  p(gc, ctypes.c_int8), p(gs, ctypes.c_float)),
                     L.rk_npu_w4a8_weights_free, "gate_up", sh)
    cfg, opt = F.rk_npu_w4a8_config(), F.rk_npu_w4a8_options()
    L.rk_npu_w4a8_config_init(ctypes.byref(cfg), rows, f2, h)
    L.rk_npu_w4a8_options_init(ctypes.byref(opt))
    gws = npu._Handle(L.rk_npu_w4a8_workspace_create_ex(dom, ctypes.byref(cfg), ctypes.byref(opt)),
                      L.rk_npu_w4a8_workspace_free, "gate_up ws", sh)
    dw = npu._Handle(L.rk_npu_f32i8f32_weights_create(dom, ctypes.byref(F.rk_npu_matmul_weight_config(f, h, f)),
                                                      p(dc, ctypes.c_int8), p(ds, ctypes.c_float)),
                     L.rk_npu_f32i8f32_weights_free, "down", sh)
    st = F.rk_npu_matmul_strategy()
    st.M, st.N, st.K, st.k_tile = rows, h, f, f
    dws = npu._Handle(L.rk_npu_matmul_workspace_create(dom, ctypes.byref(st)), L.rk_npu_matmul_workspace_free,
                      "down ws", sh)
    out = np.zeros((rows, h), F32)
    print("golden ffn", flush=True)
    npu.check(L.rk_npu_w4a8_run_ffn_f32(gws.raw, gw.raw, dws.raw, dw.raw, 8, p(x, ctypes.c_float),
                                        p(out, ctypes.c_float), None), "FFN")
    assert np.array_equal(out, d["y"])


@pytest.mark.gpu
def test_hip_moe_reproduces_fixture(backend):
    d, gu, dn, sh = moe_fixture()
    h = d["x"].shape[1]
    rows, top = d["ids"].shape
    gate = [npu.QuantMatrix(4, c.shape[0], c.shape[1], c, s) for c, s in gu]
    down = [npu.QuantMatrix(8, c.shape[0], c.shape[1], c, s) for c, s in dn]
    shared = tuple(npu.QuantMatrix(8, c.shape[0], c.shape[1], c, s) for c, s in sh)
    moe = backend.load_moe_with_shared(gate, down, top, shared)
    out = np.zeros((rows, h), F32)
    print("golden moe", flush=True)
    moe.run(d["x"], d["ids"], d["routes"], out, rows)
    assert np.array_equal(out, d["y"])
