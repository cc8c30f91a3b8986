"""The opt-in one-launch FFN of one row (ffn_m1_kernel: gate_up blocks publish the
middle row to the down blocks of the same launch through agent-scope
stores and counters): bit-identical to the two-launch FFN and to the oracle,
for every weight-round count of its gate_up blocks (K 2560 / 3072 / 4096:
5 / 6 / 8 rounds), W4 and W8 down, fp16 and f32 rows, forced K-piece counts,
and several calls in a row on the same workspaces with different rows (the
synchronisation words and split-K slots must be clean again after each
launch). The failure report is exercised by forcing the down blocks to give
up at once (HM_FFN_SPIN = -1): the kernel still ends normally, and the
status call and the host-buffer entry report the error exactly once."""
import ctypes

import numpy as np
import pytest

from oracle import oracle
from open_rknpu2_lm_infer_amd import _ffi as F
from open_rknpu2_lm_infer_amd import device as D
from open_rknpu2_lm_infer_amd import npu
from tests import refdata as R

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    return D.DeviceContext(8)


@pytest.fixture(autouse=True)
def one_launch_ffn():
    """The one-launch FFN is opt-in (HM_FFN_FUSED=1): on for these tests."""
    with D.plan_switch("HM_FFN_FUSED", 1):
        yield


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def profiled_names(fn):
    with D.KernelProfile() as prof:
        fn()
        torch.cuda.synchronize()
    return [s["name"] for s in prof.stats]


@pytest.mark.parametrize("h,f", [(2560, 384), (3072, 2240), (4096, 1024)])
@pytest.mark.parametrize("dn_bits", [4, 8])
def test_one_launch_ffn_matches_two_launches_and_oracle(ctx, h, f, dn_bits):
    gc, gs = R.weights(12, f"fz-g{h}", 4, h, 2 * f)
    dc, ds = R.weights(12, f"fz-d{h}-{dn_bits}", dn_bits, f, h)
    gu, dn = ctx.weights(4, dev(gc), dev(gs)), ctx.weights(dn_bits, dev(dc), dev(ds))
    for call in range(3):
        x = R.activations(12, f"fz-x{h}-{call}", 1, h)
        want = oracle.ffn(gc, gs, dc, ds, x)
        for half in (False, True):
            print(f"h={h} f={f} down W{dn_bits} call {call} fp16={half}", flush=True)
            xin = dev(x).half() if half else dev(x)
            y = torch.full((1, h), float("nan"), dtype=torch.float32, device="cuda")
            names = profiled_names(lambda: D.ffn(ctx, gu, dn, xin, y, 1))
            # a tile pair of at most 8 rounds of the 192 weight threads (K <= 3072)
            eligible = h <= 3072
            assert any(n.startswith("ffn_m1") for n in names) == eligible, names
            assert np.array_equal(y.cpu().numpy(), want), f"call {call}"
            with D.plan_switch("HM_FFN_FUSED", 0):
                y2 = torch.full((1, h), float("nan"), dtype=torch.float32, device="cuda")
                names = profiled_names(lambda: D.ffn(ctx, gu, dn, xin, y2, 1))
                assert not any(n.startswith("ffn_m1") for n in names), names
            assert torch.equal(y, y2)


@pytest.mark.parametrize("splits", [1, 2, 3, 5])
def test_one_launch_ffn_forced_piece_counts(ctx, splits):
    """K pieces of the down projection forced (K = 2240: 35 units of 64); the
    down workspace's diagnostics hold the middle row's codes, scale and code
    sum, assembled from the pieces."""
    from tests.test_gpu_linear import read_codes
    h, f = 2560, 2240
    gc, gs = R.weights(12, "fzs-g", 4, h, 2 * f)
    dc, ds = R.weights(12, "fzs-d", 8, f, h)
    gu, dn = ctx.weights(4, dev(gc), dev(gs)), ctx.weights(8, dev(dc), dev(ds))
    dws = ctx.workspace(8, 1, f, h)
    with D.plan_switch("HM_GEMV_SPLITS", splits):
        for call in range(2):
            x = R.activations(12, f"fzs-x{call}", 1, h)
            y = torch.empty(1, h, dtype=torch.float16, device="cuda")
            D.ffn(ctx, gu, dn, dev(x).half(), y, 1, dws=dws)
            torch.cuda.synchronize()
            want, mid = oracle.ffn(gc, gs, dc, ds, x, with_middle=True)
            assert np.array_equal(y.cpu().numpy(), want.astype(np.float16))
            codes, scale, sums = read_codes(dws, 8, 1, f)
            q, qs = oracle.quant_dense(mid)
            assert np.array_equal(codes, q) and np.array_equal(scale, qs)
            assert sums[0] == int(q.astype(np.int64).sum())


def test_one_launch_ffn_failure_is_reported_once(ctx):
    h, f = 2560, 384
    gc, gs = R.weights(12, "fzf-g", 4, h, 2 * f)
    dc, ds = R.weights(12, "fzf-d", 4, f, h)
    gu, dn = ctx.weights(4, dev(gc), dev(gs)), ctx.weights(4, dev(dc), dev(ds))
    gws, dws = ctx.workspace(4, 1, h, 2 * f), ctx.workspace(4, 1, f, h)
    L = F.lib()
    x = R.activations(12, "fzf-x", 1, h)
    y = torch.empty(1, h, dtype=torch.float32, device="cuda")
    assert L.rk_npu_hip_ffn_status(dws.raw, 4) == 0
    with D.plan_switch("HM_FFN_SPIN", -1):
        D.ffn(ctx, gu, dn, dev(x), y, 1, gws=gws, dws=dws)
        assert L.rk_npu_hip_ffn_status(dws.raw, 4) == F.RK_NPU_ERR_DEVICE
    assert L.rk_npu_hip_ffn_status(dws.raw, 4) == 0
    # the launch after a give-up starts from clean synchronisation words
    D.ffn(ctx, gu, dn, dev(x), y, 1, gws=gws, dws=dws)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), oracle.ffn(gc, gs, dc, ds, x))
    assert L.rk_npu_hip_ffn_status(dws.raw, 4) == 0
    # the host-buffer entry (rk_npu_w4a8_run_ffn_f32) reports it itself
    from tests.test_gpu_ffn_moe import FFN
    backend = npu.Backend(npu.ModelOptions(chunk=1))
    hf = FFN(backend, h, f, 1, 4, "fzf-host")
    out = np.zeros((1, h), np.float32)
    with D.plan_switch("HM_FFN_SPIN", -1):
        rc = L.rk_npu_w4a8_run_ffn_f32(hf.gws.raw, hf.gw.raw, hf.dws.raw, hf.dw.raw, 4,
                                       x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                       out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), None)
    assert rc == F.RK_NPU_ERR_DEVICE
    assert np.array_equal(hf.run(x), oracle.ffn(hf.gc, hf.gs, hf.dc, hf.ds, x))


def test_one_launch_ffn_nan_group_matches_two_launches(ctx):
    """A group of 8 middle values that are all NaN (gate columns whose scale
    takes the dequantized product to +-inf, against up columns of zero codes:
    silu(+-inf) * 0): both paths drop that group's maximum from the row max (the
    one-launch producers map a NaN group maximum to 0 before their unsigned
    atomic max, as fmaxf does over the two launches' partial maxima), so the
    outputs are bit-identical, NaNs included."""
    h, f = 2560, 384
    x = R.activations(12, "fzn-x", 1, h)
    gc, gs = R.weights(12, "fzn-g", 4, h, 2 * f)
    gc, gs = gc.copy(), gs.copy()
    # gate columns 0-7: codes of the row's signs (a positive dot product) and
    # a scale that overflows it to +inf; their up columns: zero codes
    gc[:, :8] = np.where(x[0] >= 0, 7, -7).astype(np.int8)[:, None]
    gs[:8] = 3e38
    gc[:, f:f + 8] = 0
    dc, ds = R.weights(12, "fzn-d", 8, f, h)
    mid = oracle.linear_swiglu(gc, gs, x)
    assert np.isnan(mid[0, :8]).all() and np.isfinite(mid[0, 8:]).all()
    gu, dn = ctx.weights(4, dev(gc), dev(gs)), ctx.weights(8, dev(dc), dev(ds))
    y = torch.empty(1, h, dtype=torch.float32, device="cuda")
    names = profiled_names(lambda: D.ffn(ctx, gu, dn, dev(x), y, 1))
    assert any(n.startswith("ffn_m1") for n in names), names
    with D.plan_switch("HM_FFN_FUSED", 0):
        y2 = torch.empty(1, h, dtype=torch.float32, device="cuda")
        D.ffn(ctx, gu, dn, dev(x), y2, 1)
        torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))
    # the finite part of the row sets the down projection's scale in both
    assert np.isfinite(y.cpu().numpy()).any()
