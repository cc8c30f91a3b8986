"""Pins the CPU oracle (no GPU): the reference's known-answer tests, closed
forms, special cases and independent restatements, chosen so that a dropped
term, a wrong rounding rule, a transposed operand or a wrong dequant order fails."""
import math
import struct

import numpy as np
import pytest

from oracle import oracle
from tests import refdata as R

F32 = np.float32


def f32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


def fma_f32(a, b, c):
    """Single-rounding a*b + c in f32, from exact rational arithmetic."""
    from fractions import Fraction
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    f = np.float32(float(exact))
    cands = [np.nextafter(f, F32(-np.inf)), f, np.nextafter(f, F32(np.inf))]
    def key(v):
        d = abs(Fraction(float(v)) - exact)
        odd = int(np.asarray(v, F32).view(np.uint32)) & 1
        return (d, odd)
    return min(cands, key=key)


def test_bucket_closed_form():
    """src/npu.rs:201-211."""
    for rows in range(1, 257):
        expected = 1 << (rows - 1).bit_length() if rows <= 128 else (rows + 63) // 64 * 64
        assert oracle.bucket(rows) == expected
    assert oracle.bucket(1) == 1 and oracle.bucket(4) == 4 and oracle.bucket(5) == 8
    assert oracle.bucket(129) == 192 and oracle.bucket(256) == 256
    assert oracle.bucket(0) == -1 and oracle.bucket(257) == -1


def test_unpack_codes_known_answer():
    """src/model/checkpoint.rs:749-783: words 0x87654321, 0xfedcba98 for [N=2, K=8]."""
    words = np.array([0x87654321, 0xFEDCBA98], np.uint32)
    codes = oracle.unpack_codes(words, 4, 2, 8)
    assert codes.ravel().tolist() == [-7, 0, -6, 1, -5, 2, -4, 3, -3, 4, -2, 5, -1, 6, 0, 7]
    # 8-bit words and a K that is not a multiple of the packing factor
    w8 = np.array([0x04030201, 0x00000005, 0x80FF7F00, 0x00000081], np.uint32)
    c8 = oracle.unpack_codes(w8, 8, 2, 5)
    assert c8[:, 0].tolist() == [1 - 128, 2 - 128, 3 - 128, 4 - 128, 5 - 128]
    assert c8[:, 1].tolist() == [-128, 127 - 128, 255 - 128, 128 - 128, 129 - 128]


def test_routes_known_answer():
    """src/model/qwen35/moe.rs:355-364."""
    ids, w = oracle.routes(np.array([-100.0, 1.0, 3.0, 2.0], F32), 2)
    assert ids.tolist() == [2, 3]
    assert abs(w[0] - 1.0 / (1.0 + math.exp(-1.0))) < 1e-6
    assert abs(float(w.sum()) - 1.0) < 1e-6
    for bad_top, logits in [(1, []), (0, [0.0]), (2, [0.0])]:
        with pytest.raises(ValueError):
            oracle.routes(np.array(logits, F32), bad_top)
    # ties go to the lower id; -0.0 ranks below +0.0 in the total order
    ids, _ = oracle.routes(np.array([1.0, 2.0, 2.0, 0.5], F32), 2)
    assert ids.tolist() == [1, 2]
    ids, _ = oracle.routes(np.array([-0.0, 0.0], F32), 1)
    assert ids.tolist() == [1]


def naive_quant(row, rule):
    """Independent restatement with Python floats rounded to f32 per operation."""
    m = 0.0
    for v in row:
        m = max(m, abs(float(v)))
    if rule == "dense":
        s = 1.0 if m == 0.0 else max(f32(m / 127.0), np.finfo(F32).tiny)
    else:
        s = 1.0 if m == 0.0 else f32(m / 127.0)
    inv = f32(1.0 / s)
    out = []
    for v in row:
        y = f32(float(v) * inv)
        if rule == "dense":
            q = math.floor(abs(y) + 0.5) * (1 if y >= 0 else -1)
        else:
            q = round(y)  # Python rounds half to even
        out.append(max(-127, min(127, int(q))))
    return out, f32(s)


@pytest.mark.parametrize("rule", ["dense", "moe"])
def test_quant_rules_special_rows(rule):
    k = 64
    rows = np.zeros((7, k), F32)
    rows[1, :] = F32(1e-39)
    rows[1, 5] = F32(-3e-39)
    rows[2, :] = (np.arange(k) - 32).astype(F32) + F32(0.5)
    rows[2, 0] = F32(127.0)
    rows[3, :] = F32(-3.0)
    rows[4, :] = F32(0.01)
    rows[4, 9] = F32(250.0)
    rows[5, :] = R.activations(0, "quant-special", 1, k)[0]
    rows[6, :] = F32(-0.0)
    fn = oracle.quant_dense if rule == "dense" else oracle.quant_moe
    q, s = fn(rows)
    for r in range(rows.shape[0]):
        if rule == "moe" and r == 1:
            continue  # below the MoE rule's precondition (max/127 must be a normal float)
        eq, es = naive_quant(rows[r], rule)
        assert q[r].tolist() == eq, f"row {r}"
        assert s[r] == es
    assert s[0] == 1.0 and s[6] == 1.0 and np.all(q[0] == 0)
    if rule == "dense":
        assert s[1] == np.finfo(F32).tiny  # FLT_MIN floor
        assert q[2, 1] == -31 and q[2, 3] == -29 and q[2, 34] == 3  # ties away from zero
    else:
        assert q[2, 1] == -30 and q[2, 3] == -28 and q[2, 34] == 2  # ties to even
    assert np.all(q[3] == -127)
    assert q[4, 9] == 127 and np.all(q[4, :9] == 0)


def test_gemm_brute_force_and_order_independence():
    g = np.random.default_rng(7)
    for (m, k, n) in [(1, 1, 1), (3, 17, 5), (8, 64, 33), (13, 130, 64)]:
        a = g.integers(-127, 128, size=(m, k), dtype=np.int8)
        w = g.integers(-127, 128, size=(k, n), dtype=np.int8)
        acc = oracle.gemm_i8(a, w)
        assert np.array_equal(acc, a.astype(np.int64) @ w.astype(np.int64))
        perm = g.permutation(k)
        assert np.array_equal(oracle.gemm_i8(a[:, perm], w[perm]), acc)
    # extreme magnitudes: K * 127 * 127 stays exact in int32
    k = 2560
    a = np.full((1, k), 127, np.int8)
    w = np.full((k, 3), -127, np.int8)
    assert oracle.gemm_i8(a, w)[0, 0] == -k * 127 * 127


def test_linear_matches_reference_oracle_restatement():
    """src/npu.rs:1533-1557 restated with numpy f32 ops; dequant is
    (f32(acc) * s_row) * s_col (two roundings), not f32(acc) * (s_row * s_col)."""
    codes, scales = R.reference_matrix(8)
    x = R.reference_input(9)
    out, q, s, acc = oracle.linear(codes, scales, x, intermediates=True)
    for r in range(x.shape[0]):
        eq, es = naive_quant(x[r], "dense")
        assert q[r].tolist() == eq and s[r] == es
    assert np.array_equal(acc, q.astype(np.int64) @ codes.astype(np.int64))
    expected = (acc.astype(F32) * s[:, None]).astype(F32) * scales[None, :]
    assert np.array_equal(out, expected.astype(F32))
    other_order = acc.astype(F32) * (s[:, None] * scales[None, :]).astype(F32)
    assert not np.array_equal(out, other_order.astype(F32))


def test_expf_accuracy_and_special_points():
    xs = np.concatenate([np.linspace(-80, 80, 40001, dtype=F32), np.array([0.0, -0.0, 1.0, -1.0], F32)])
    e = oracle.expf(xs)
    ref = np.exp(xs.astype(np.float64))
    rel = np.abs(e.astype(np.float64) / ref - 1.0)
    assert rel.max() < 2.5 * 2.0 ** -23
    assert oracle.expf(np.array([0.0], F32))[0] == 1.0


def test_swiglu_against_reference_formula():
    """Within 3e-5 * max(|e|, 1) of (g/(1+exp(-g)))*u (src/npu.rs:1651-1658);
    g < -80 gives a signed zero; large g gives g * u."""
    g = np.concatenate([np.linspace(-100, 100, 20001, dtype=F32), R.activations(0, "swiglu", 1, 4096)[0] * 3])
    u = np.resize(R.activations(0, "swiglu-u", 1, 4096)[0], g.shape).astype(F32)
    y = oracle.swiglu(g, u).astype(np.float64)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    ref = gd / (1.0 + np.exp(-gd)) * ud
    assert np.all(np.abs(y - ref) <= 3e-5 * np.maximum(np.abs(ref), 1.0))
    z = oracle.swiglu(np.array([-81.0, -1000.0], F32), np.array([2.0, -3.0], F32))
    assert z[0] == 0.0 and math.copysign(1.0, z[0]) == -1.0
    assert z[1] == 0.0 and math.copysign(1.0, z[1]) == 1.0
    big = oracle.swiglu(np.array([90.0], F32), np.array([0.5], F32))
    assert big[0] == F32(45.0)


def test_linear_swiglu_is_split_gate_up():
    codes, scales = R.weights(0, "sw", 4, 96, 128)
    x = R.activations(0, "sw-x", 5, 96)
    y = oracle.linear(codes, scales, x)
    mid = oracle.linear_swiglu(codes, scales, x)
    assert np.array_equal(mid, oracle.swiglu(y[:, :64], y[:, 64:]))


def test_ffn_is_swiglu_then_linear():
    gc, gs = R.weights(0, "ffn-g", 4, 64, 96)
    dc, ds = R.weights(0, "ffn-d", 8, 48, 64)
    x = R.activations(0, "ffn-x", 4, 64)
    out, mid = oracle.ffn(gc, gs, dc, ds, x, with_middle=True)
    assert np.array_equal(mid, oracle.linear_swiglu(gc, gs, x))
    assert np.array_equal(out, oracle.linear(dc, ds, mid))


def test_moe_matches_numpy_restatement():
    h, inter, experts, top, rows = 32, 16, 5, 3, 4
    gate = [R.weights(0, f"mg{e}", 4, h, 2 * inter) for e in range(experts)]
    down = [R.weights(0, f"md{e}", 8, inter, h) for e in range(experts)]
    x = R.activations(0, "mx", rows, h)
    ids = np.array([[0, 1, 2], [4, 4, 0], [3, 2, 1], [1, 0, 4]], np.int32)
    w = np.array([[0.5, 0.3, 0.2], [0.6, 0.4, 0.0], [0.2, 0.2, 0.6], [1.0, -0.5, 0.0]], F32)
    out = oracle.moe(gate, down, x, ids, w)
    qx, sx = oracle.quant_moe(x)
    for r in range(rows):
        s = np.zeros(h, F32)
        for rank in range(top):
            if not (w[r, rank] > 0):
                continue
            gc, gs = gate[ids[r, rank]]
            dc, ds = down[ids[r, rank]]
            acc = qx[r].astype(np.int64) @ gc.astype(np.int64)
            y = (acc.astype(F32) * sx[r]).astype(F32) * gs
            mid = oracle.swiglu(y[:inter], y[inter:])
            qm, sm = oracle.quant_moe(mid[None, :])
            acc2 = qm[0].astype(np.int64) @ dc.astype(np.int64)
            contrib = (acc2.astype(F32) * sm[0]).astype(F32) * ds
            s = np.array([fma_f32(c, w[r, rank], t) for c, t in zip(contrib, s)], F32)
        assert np.array_equal(out[r], s), f"row {r}"


def test_moe_shared_expert_is_added_after_routed_sum():
    h, inter, experts, top = 32, 16, 3, 2
    gate = [R.weights(0, f"sg{e}", 4, h, 2 * inter) for e in range(experts)]
    down = [R.weights(0, f"sd{e}", 4, inter, h) for e in range(experts)]
    sg, sd = R.weights(0, "shg", 8, h, 2 * inter), R.weights(0, "shd", 8, inter, h)
    x = R.activations(0, "sx", 2, h)
    ids = np.array([[0, 2], [1, 1]], np.int32)
    w = np.array([[0.7, 0.3], [0.5, 0.5]], F32)
    routed = oracle.moe(gate, down, x, ids, w)
    both = oracle.moe(gate, down, x, ids, w, shared=(sg, sd))
    alone = oracle.moe([sg], [sd], x, np.zeros((2, 1), np.int32), np.ones((2, 1), F32))
    assert np.array_equal(both, (routed + alone).astype(F32))


def test_concatenate_along_n():
    """src/model/checkpoint.rs:573-604: row k = [A[k] | B[k] | C[k]]."""
    a = np.arange(6, dtype=np.int8).reshape(2, 3)
    b = -np.arange(4, dtype=np.int8).reshape(2, 2)
    c = np.full((2, 1), 9, np.int8)
    out = oracle.concatenate([a, b, c])
    assert out.tolist() == [[0, 1, 2, 0, -1, 9], [3, 4, 5, -2, -3, 9]]
