"""GPU parity of the dense W8A8 / W4A8 linear and the fused SwiGLU against the
oracle, through the C ABI (via the host mirror of src/npu.rs)."""
import ctypes
import threading

import numpy as np
import pytest

from oracle import oracle
from open_rknpu2_lm_infer_amd import _ffi as F
from open_rknpu2_lm_infer_amd import npu
from tests import refdata as R

pytestmark = pytest.mark.gpu


def compare(actual, expected, tol):
    """src/npu.rs:1559-1566: finite and |a-e| <= tol*max(|e|, 1)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert np.all(np.isfinite(a))
    bad = np.abs(a - e) > tol * np.maximum(np.abs(e), 1.0)
    assert not bad.any(), f"{bad.sum()} elements out of tolerance, first at {np.argwhere(bad)[0]}"


@pytest.fixture(scope="module")
def backend():
    return npu.Backend(npu.ModelOptions(chunk=256))


def read_codes(work_handle, bits, rows, k):
    codes = np.zeros((rows, k), np.int8)
    scales = np.zeros(rows, np.float32)
    sums = np.zeros(rows, np.int32)
    rc = F.lib().rk_npu_hip_workspace_codes(work_handle.raw, bits, rows, codes.ctypes.data_as(F.i8p),
                                            scales.ctypes.data_as(F.f32p), sums.ctypes.data_as(F.i32p))
    npu.check(rc, "read codes")
    return codes, scales, sums


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_linear_padding_and_swiglu(backend, bits):
    """Mirror of src/npu.rs:1597-1692 on K = N = 256 over the reference's row list."""
    codes, scales = R.reference_matrix(bits)
    x = R.reference_input()
    reference = oracle.linear(codes, scales, x)
    linear = backend.load(npu.QuantMatrix(bits, 256, 256, codes, scales))
    for rows in R.REFERENCE_ROWS:
        print(f"bits={bits} rows={rows}", flush=True)
        out = np.zeros((rows, 256), np.float32)
        linear.run(x, out, rows)
        compare(out, reference[:rows], 2e-5)
        assert np.array_equal(out, reference[:rows]), "linear output not bit-exact vs oracle"
        if rows == 1:
            assert backend.stats()["linear_padding_bytes"] == 0 or bits == 8
        if bits == 4:
            middle = np.zeros((rows, 128), np.float32)
            assert linear.run_swiglu(x, middle, rows)
            g = reference[:rows, :128].astype(np.float64)
            u = reference[:rows, 128:].astype(np.float64)
            compare(middle, g / (1.0 + np.exp(-g)) * u, 3e-5)
            assert np.array_equal(middle, oracle.linear_swiglu(codes, scales, x[:rows]))
            first = middle.copy()
            ws_bytes = backend.stats()["workspace_payload_bytes"]
            assert linear.run_swiglu(x, middle, rows)
            assert np.array_equal(middle, first)
            assert backend.stats()["workspace_payload_bytes"] == ws_bytes
            linear.run(x, out, rows)
            assert np.array_equal(out, reference[:rows])
        else:
            assert not linear.run_swiglu(x, out, rows)
    backend.retain_workspaces([1, 64])


@pytest.mark.parametrize("bits", [4, 8])
def test_activation_codes_and_int32_bit_exact(bits):
    """The device's int8 codes, row scales and row code sums equal the oracle's;
    with power-of-two scales the int32 accumulators are recovered exactly."""
    k, n, rows = 2560, 1024, 33
    backend = npu.Backend(npu.ModelOptions(chunk=64))
    codes, _ = R.weights(0, "w-exact", bits, k, n)
    x = R.activations(0, "x-exact", rows, k)
    # Row max = 127 * 2^e makes the dynamic scale exactly 2^e.
    for r in range(rows):
        x[r] = x[r] / np.abs(x[r]).max() * np.float32(127.0 * 2.0 ** (r % 5 - 2))
    scales = np.full(n, np.float32(2.0 ** -7), np.float32)
    linear = backend.load(npu.QuantMatrix(bits, k, n, codes, scales))
    out = np.zeros((rows, n), np.float32)
    linear.run(x, out, rows)
    ref, q, s, acc = oracle.linear(codes, scales, x, intermediates=True)
    assert np.array_equal(out, ref)
    work = backend.work[(linear.key, npu.bucket(rows))]
    dq, ds, dsum = read_codes(work.w4 if bits == 4 else work.w8, bits, rows, k)
    assert np.array_equal(dq, q), "activation codes differ"
    assert np.array_equal(ds, s), "row scales differ"
    assert np.array_equal(dsum, q.astype(np.int64).sum(axis=1).astype(np.int32))
    assert np.all(np.abs(acc) < 2**24)
    recovered = out.astype(np.float64) / (s[:, None].astype(np.float64) * 2.0 ** -7)
    assert np.array_equal(recovered, acc.astype(np.float64)), "int32 accumulators differ"


def test_narrow_w8_gdn_gates_match_integer_oracle():
    """Mirror of src/npu/narrow_projection.rs:5-74 (K=2560, N in {32, 64})."""
    backend = npu.Backend(npu.ModelOptions(chunk=32))
    k = 2560
    for n in (32, 64):
        codes, scales = R.narrow_matrix(k, n)
        linear = backend.load(npu.QuantMatrix(8, k, n, codes, scales))
        for rows in (1, 2, 3, 5, 7):
            backend.prepare(rows)
            x = R.narrow_input(rows, k)
            out = np.zeros((rows, n), np.float32)
            linear.run(x, out, rows)
            # the test's own oracle: scale = max/127 (no floor), x * scale.recip()
            for r in range(rows):
                s = np.float32(np.abs(x[r]).max() / np.float32(127.0))
                y = (x[r] * (np.float32(1.0) / s)).astype(np.float64)
                qv = np.clip(np.sign(y) * np.floor(np.abs(y) + 0.5), -127, 127).astype(np.int64)
                acc = qv @ codes.astype(np.int64)
                expected = (acc.astype(np.float32) * s) * scales
                compare(out[r], expected, 2e-6)
            assert np.array_equal(out, oracle.linear(codes, scales, x))


@pytest.mark.parametrize("bits", [4, 8])
def test_independent_execution_lanes_share_weights(bits):
    """Mirror of src/npu/lane.rs:140-240: two lanes with their own workspaces
    over shared weights, concurrent calls bit-exact."""
    primary = npu.Backend(npu.ModelOptions(chunk=128))
    rows, k, n = 128, 513, 512
    codes, scales = R.lane_matrix(bits, k, n)
    linear = primary.load(npu.QuantMatrix(bits, k, n, codes, scales))
    primary.prepare(rows)
    lane = primary.fork_execution()
    lane.prepare(rows)
    assert lane.weight_bytes() == 0
    x0, x1 = R.lane_inputs(rows, k)
    e0 = np.zeros((rows, n), np.float32)
    e1 = np.zeros((rows, n), np.float32)
    linear.run(x0, e0, rows)
    linear.run(x1, e1, rows, lane=lane)
    assert np.array_equal(e0, oracle.linear(codes, scales, x0))
    assert np.array_equal(e1, oracle.linear(codes, scales, x1))
    for _ in range(3):
        o0 = np.zeros_like(e0)
        o1 = np.zeros_like(e1)
        errors = []

        def follower():
            try:
                linear.run(x1, o1, rows, lane=lane)
            except Exception as exc:  # pragma: no cover - reported below
                errors.append(exc)

        t = threading.Thread(target=follower)
        t.start()
        linear.run(x0, o0, rows)
        t.join()
        assert not errors
        assert np.array_equal(o0.view(np.uint32), e0.view(np.uint32))
        assert np.array_equal(o1.view(np.uint32), e1.view(np.uint32))


def test_quant_rule_edge_rows():
    """Zero row (scale 1), FLT_MIN floor, exact half-way ties (away from zero),
    saturation, a single outlier channel."""
    k, n = 64, 64
    backend = npu.Backend(npu.ModelOptions(chunk=8))
    codes, scales = R.weights(0, "edge", 8, k, n)
    linear = backend.load(npu.QuantMatrix(8, k, n, codes, scales))
    x = np.zeros((8, k), np.float32)
    x[1, :] = np.float32(1e-39)                  # max/127 < FLT_MIN -> scale FLT_MIN
    x[1, 3] = np.float32(-2e-39)
    x[2, :] = (np.arange(k) - 32).astype(np.float32) + np.float32(0.5)  # ties after scaling
    x[2, 0] = np.float32(127.0)
    x[3, :] = np.float32(-3.0)                   # saturates at -127
    x[4, :] = np.float32(0.01)
    x[4, 17] = np.float32(200.0)                 # outlier channel
    x[5, ::2] = np.float32(2.5)
    x[5, 1::2] = np.float32(-2.5)
    x[5, 0] = np.float32(127.0 * 2.0)            # scale 2: 2.5/2 = 1.25
    x[6, :] = np.float32(-0.0)
    x[7, :] = np.linspace(-1, 1, k, dtype=np.float32)
    out = np.zeros((8, n), np.float32)
    linear.run(x, out, 8)
    ref, q, s, _ = oracle.linear(codes, scales, x, intermediates=True)
    assert s[0] == 1.0 and s[6] == 1.0 and s[1] == np.finfo(np.float32).tiny
    # -30.5 -> -31 and -28.5 -> -29 (ties away from zero; nearest-even would give -30, -28)
    assert q[2, 1] == -31 and q[2, 3] == -29 and q[2, 34] == 3
    assert np.array_equal(out, ref)
    work = backend.work[(linear.key, 8)]
    dq, ds, _ = read_codes(work.w8, 8, 8, k)
    assert np.array_equal(dq, q) and np.array_equal(ds, s)


def test_workspace_busy_and_bad_arguments():
    backend = npu.Backend(npu.ModelOptions(chunk=8))
    codes, scales = R.weights(0, "bad", 4, 64, 64)
    bad = codes.copy()
    bad[0, 0] = 8  # outside [-8, 7]
    with pytest.raises(npu.NpuError):
        backend.load(npu.QuantMatrix(4, 64, 64, bad, scales))
    with pytest.raises(npu.NpuError):
        backend.load(npu.QuantMatrix(4, 64, 64, codes, -scales))
    with pytest.raises(npu.NpuError):
        npu.bucket(257)
    linear = backend.load(npu.QuantMatrix(4, 64, 64, codes, scales))
    with pytest.raises(npu.NpuError):
        linear.run(np.zeros((2, 63), np.float32), np.zeros((2, 64), np.float32), 2)


def test_allocation_failure_calls_reclaim_then_retries():
    backend = npu.Backend(npu.ModelOptions(chunk=8))
    codes, scales = R.weights(0, "oom", 8, 128, 128)
    L = F.lib()
    before = backend._shared.reclaims
    L.rk_npu_hip_inject_alloc_failures(1)
    linear = backend.load(npu.QuantMatrix(8, 128, 128, codes, scales))
    assert backend._shared.reclaims == before + 1
    L.rk_npu_hip_inject_alloc_failures(2)
    with pytest.raises(npu.NpuError):
        backend.load(npu.QuantMatrix(8, 128, 128, codes, scales))
    L.rk_npu_hip_inject_alloc_failures(0)
    out = np.zeros((1, 128), np.float32)
    x = R.activations(0, "oom-x", 1, 128)
    linear.run(x, out, 1)
    assert np.array_equal(out, oracle.linear(codes, scales, x))


@pytest.mark.parametrize("bits", [4, 8])
def test_host_call_staging_small_and_large(backend, bits):
    """Host-buffer calls below the 8 MiB pinned stage (A and C copied through
    it) and above it (direct pageable copies), each bit-exact against the
    oracle. Rows 1, 256 and 3 run on the workspaces of buckets 1, 256 and 4;
    the 4-row call after the 3-row one reuses the bucket-4 workspace with
    larger A and C, so its pinned stage grows (freed and allocated again)."""
    n = 128
    for rows, k in ((1, 8256), (256, 8256), (3, 8256), (4, 8256)):
        print(f"bits={bits} rows={rows} k={k} a_bytes={rows * k * 4}", flush=True)
        codes, scales = R.weights(7, f"stage{bits}", bits, k, n)
        x = R.activations(7, f"stage-x{rows}", rows, k)
        linear = backend.load(npu.QuantMatrix(bits, k, n, codes, scales))
        out = np.full((rows, n), np.nan, np.float32)
        linear.run(x, out, rows)
        assert np.array_equal(out, oracle.linear(codes, scales, x))
