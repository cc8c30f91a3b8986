"""rk_npu_hip_linear_run_static: the allocation-free linear (scratch in a
library-owned device array) gives the same bits as rk_npu_hip_linear_run with
a workspace, on two calls in a row whose second has fewer rows (the array
keeps the first call's contents), over the GEMV, GEMM and split-K GEMM plans;
rows or shapes beyond the array are rejected before anything is enqueued."""
import ctypes

import numpy as np
import pytest

from oracle import oracle
from open_rknpu2_lm_infer_amd import _ffi as F
from open_rknpu2_lm_infer_amd import device as D
from tests import refdata as R

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    return D.DeviceContext(4)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_static(w, x, out, rows, swiglu):
    return F.lib().rk_npu_hip_linear_run_static(
        w.handle.raw, w.bits, ctypes.c_void_p(x.data_ptr()), D._dtype_code(x), ctypes.c_void_p(out.data_ptr()),
        D._dtype_code(out), rows, F.RK_NPU_HIP_SWIGLU if swiglu else F.RK_NPU_HIP_PLAIN, D.current_stream())


# (bits, K, N, swiglu, first rows, second rows): gate_up at a prefill-sized and
# a decode row count (GEMM then GEMV with a quantization wave), the 9728-long
# down projection at 64 rows (split-K GEMM, partials in the array) then 4
# rows (rows quantized before the GEMV), o at the 256-row limit then 33 rows.
CASES = [(4, 2560, 19456, True, 200, 1),
         (8, 9728, 2560, False, 64, 4),
         (4, 4096, 2560, False, 256, 33),
         (8, 2560, 1024, True, 40, 2)]


@pytest.mark.parametrize("bits,k,n,swiglu,rows1,rows2", CASES)
@pytest.mark.parametrize("fp16", [False, True])
def test_static_linear_matches_workspace_entry(ctx, bits, k, n, swiglu, rows1, rows2, fp16):
    codes, scales = R.weights(21, f"na{bits}-{k}-{n}", bits, k, n)
    w = ctx.weights(bits, dev(codes), dev(scales))
    width = n // 2 if swiglu else n
    for call, rows in enumerate((rows1, rows2)):
        print(f"W{bits} K={k} N={n} swiglu={swiglu} fp16={fp16} call {call}: rows={rows}", flush=True)
        x = R.activations(21, f"na-x{k}-{rows}", rows, k)
        xin = dev(x).half() if fp16 else dev(x)
        ref = torch.full((rows, width), float("nan"), dtype=torch.float32, device="cuda")
        got = torch.full((rows, width), float("nan"), dtype=torch.float32, device="cuda")
        D.linear(ctx, w, xin, ref, rows, swiglu=swiglu)
        rc = run_static(w, xin, got, rows, swiglu)
        assert rc == F.RK_NPU_OK
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"call {call} differs from the workspace entry point"
    # the last call's rows against the oracle as well (small K only: seconds on the CPU)
    if rows <= 4 or k <= 2560:
        want = (oracle.linear_swiglu if swiglu else oracle.linear)(codes, scales, x)
        assert np.array_equal(got.cpu().numpy(), want)


def test_static_linear_rejects_rows_and_shapes_beyond_the_array(ctx):
    k, n = 512, 256
    codes, scales = R.weights(21, "na-small", 8, k, n)
    w = ctx.weights(8, dev(codes), dev(scales))
    x = dev(R.activations(21, "na-xs", 300, k))
    y = torch.zeros(300, n, dtype=torch.float32, device="cuda")
    assert run_static(w, x, y, 0, False) == F.RK_NPU_ERR_PARAM
    assert run_static(w, x, y, F.RK_NPU_HIP_STATIC_MAX_ROWS + 1, False) == F.RK_NPU_ERR_PARAM
    assert run_static(w, x, y, F.RK_NPU_HIP_STATIC_MAX_ROWS, False) == F.RK_NPU_OK
    torch.cuda.synchronize()
    # K = 65536 needs 16 MiB of activation codes at 256 row slots: beyond the array
    kb = 65536
    wb = ctx.weights(8, torch.ones(kb, 64, dtype=torch.int8, device="cuda"),
                     torch.full((64,), 0.01, dtype=torch.float32, device="cuda"))
    xb = torch.zeros(1, kb, dtype=torch.float32, device="cuda")
    yb = torch.full((1, 64), -1.0, dtype=torch.float32, device="cuda")
    assert run_static(wb, xb, yb, 1, False) == F.RK_NPU_ERR_PARAM
    torch.cuda.synchronize()
    assert bool((yb == -1.0).all()), "a rejected call must enqueue nothing"
    # SwiGLU on N % 64 != 0 is unsupported, as for the workspace entry point
    wo = ctx.weights(8, dev(codes[:, :96]), dev(scales[:96]))
    assert run_static(wo, x, y, 1, True) == F.RK_NPU_ERR_UNSUPPORTED
