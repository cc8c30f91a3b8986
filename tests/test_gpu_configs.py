"""Oracle parity at the benchmarked shapes themselves (Qwen3-4B and the
35B-A3B-class MoE): each case runs the GPU path at its real size and checks
every row bit for bit against the oracle (the C oracle with OpenMP takes
seconds even for the 4096 x 151936 lm_head).

- W8A8 linear M128 K2560 N9728 with outlier channels, through the reference's
  host-buffer signature rk_npu_f32i8f32_run_dynamic (src/npu.rs:1412-1417)
  and the device entry point.
- Decode M=1 and M=4 W4A8: qkv 2560->6144, o 4096->2560, and the fused
  gate_up 2560->19456 + SwiGLU -> requant -> down 9728->2560 (the split-K
  one-row GEMV and the quantization wave at M=1).
- Prefill M=4096: qkv/o W8A8 (128x128 and 192x256 tiles), gate_up W4A8 +
  SwiGLU -> down W8A8, and the 2560->151936 W8 lm_head (the 256x256 tile
  with its last 128 columns padded), all 4096 rows.
- MoE T=1: hidden 2048, 128 experts, top-8, I=768, W4 gate_up + W8 down, and
  the shared W8 FFN of intermediate 2048."""
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

H, Q, KV, FF, VOCAB = 2560, 4096, 1024, 9728, 151936


@pytest.fixture(scope="module")
def ctx():
    return D.DeviceContext(5)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_w8a8_up_m128_host_abi_and_device():
    codes, scales = R.weights(0, "cfg0-up", 8, H, FF)
    x = R.activations(0, "cfg0-x", 128, H)
    want = oracle.linear(codes, scales, x)
    print("W8A8 M128 K2560 N9728 host ABI", flush=True)
    backend = npu.Backend(npu.ModelOptions(chunk=128))
    lin = backend.load(npu.QuantMatrix(8, H, FF, codes, scales))
    out = np.zeros((128, FF), np.float32)
    lin.run(x, out, 128)
    assert np.array_equal(out, want)
    # the mirror's W8 path runs rk_npu_f32i8f32_run_dynamic on the 128-row bucket
    print("W8A8 M128 device entry, fp16 in and out", flush=True)
    local = D.DeviceContext(6)
    w = local.weights(8, dev(codes), dev(scales))
    y = torch.empty(128, FF, dtype=torch.float16, device="cuda")
    D.linear(local, w, dev(x).half(), y, 128)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), want.astype(np.float16))


@pytest.mark.parametrize("rows", [1, 4])
def test_decode_projection_set_w4a8(ctx, rows):
    for name, k, n in (("qkv", H, Q + 2 * KV), ("o", Q, H)):
        print(f"decode M={rows} {name} {k}x{n} W4", flush=True)
        codes, scales = R.weights(1, f"cfg1-{name}", 4, k, n)
        x = R.activations(1, f"cfg1-x{name}{rows}", rows, k, outliers=False)
        w = ctx.weights(4, dev(codes), dev(scales))
        y = torch.empty(rows, n, dtype=torch.float32, device="cuda")
        D.linear(ctx, w, dev(x).half(), y, rows)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), oracle.linear(codes, scales, x))
    print(f"decode M={rows} FFN gate_up 2560x19456 + SwiGLU -> down 9728x2560 W4", flush=True)
    gc, gs = R.weights(1, "cfg1-gu", 4, H, 2 * FF)
    dc, ds = R.weights(1, "cfg1-dn", 4, FF, H)
    gu, dn = ctx.weights(4, dev(gc), dev(gs)), ctx.weights(4, dev(dc), dev(ds))
    x = R.activations(1, f"cfg1-xffn{rows}", rows, H, outliers=False)
    want = oracle.ffn(gc, gs, dc, ds, x)
    for rep in range(2):  # the split-K slots must be clean for the second call
        y = torch.empty(rows, H, dtype=torch.float32, device="cuda")
        D.ffn(ctx, gu, dn, dev(x).half(), y, rows)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), want), f"call {rep}"
    # the SwiGLU middle alone (rk_npu_w4a8_run_swiglu_f32's output)
    m = torch.empty(rows, FF, dtype=torch.float32, device="cuda")
    D.linear(ctx, gu, dev(x).half(), m, rows, swiglu=True)
    torch.cuda.synchronize()
    assert np.array_equal(m.cpu().numpy(), oracle.linear_swiglu(gc, gs, x))


def test_prefill_m4096_projection_set(ctx):
    rows = 4096
    for name, bits, k, n in (("qkv", 8, H, Q + 2 * KV), ("o", 8, Q, H)):
        print(f"prefill M=4096 {name} {k}x{n} W{bits}", flush=True)
        codes, scales = R.weights(3, f"cfg3-{name}", bits, k, n)
        x = R.activations(3, f"cfg3-x{name}", rows, k)
        w = ctx.weights(bits, dev(codes), dev(scales))
        y = torch.empty(rows, n, dtype=torch.float16, device="cuda")
        D.linear(ctx, w, dev(x).half(), y, rows)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), oracle.linear(codes, scales, x).astype(np.float16))
        del w, y
    print("prefill M=4096 FFN gate_up W4 2560x19456 + SwiGLU -> down W8 9728x2560", flush=True)
    gc, gs = R.weights(3, "cfg3-gu", 4, H, 2 * FF)
    dc, ds = R.weights(3, "cfg3-dn", 8, FF, H)
    gu, dn = ctx.weights(4, dev(gc), dev(gs)), ctx.weights(8, dev(dc), dev(ds))
    x = R.activations(3, "cfg3-xffn", rows, H)
    xd = dev(x).half()
    y = torch.empty(rows, H, dtype=torch.float16, device="cuda")
    D.ffn(ctx, gu, dn, xd, y, rows)
    m = torch.empty(rows, FF, dtype=torch.float16, device="cuda")
    D.linear(ctx, gu, xd, m, rows, swiglu=True)
    torch.cuda.synchronize()
    want, mid = oracle.ffn(gc, gs, dc, ds, x, with_middle=True)
    assert np.array_equal(y.cpu().numpy(), want.astype(np.float16))
    assert np.array_equal(m.cpu().numpy(), mid.astype(np.float16))


def test_prefill_m4096_lm_head(ctx):
    rows = 4096
    print("prefill M=4096 lm_head 2560x151936 W8 (256x256 tile, last tile half padded)", flush=True)
    plan = F.rk_npu_hip_plan()
    npu.check(F.lib().rk_npu_hip_linear_plan(rows, H, VOCAB, 8, ctypes.byref(plan)), "plan")
    assert (plan.kind, plan.block_m, plan.block_n) == (1, 256, 256)
    codes, scales = R.weights(3, "cfg3-head", 8, H, VOCAB)
    x = R.activations(3, "cfg3-xhead", rows, H)
    w = ctx.weights(8, dev(codes), dev(scales))
    y = torch.empty(rows, VOCAB, dtype=torch.float16, device="cuda")
    D.linear(ctx, w, dev(x).half(), y, rows)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    del y, w
    for r0 in range(0, rows, 1024):  # (the oracle's f32 output in slices of 1024 rows: 0.6 GB each)
        assert np.array_equal(got[r0:r0 + 1024], oracle.linear(codes, scales, x[r0:r0 + 1024]).astype(np.float16))


def test_moe_35b_a3b_t1_with_shared_ffn():
    h, inter, experts, top, sh_inter = 2048, 768, 128, 8, 2048
    print("MoE T=1 h2048 E128 top8 I768 W4 gate_up + W8 down", flush=True)
    backend = npu.Backend(npu.ModelOptions(chunk=16))
    gate = [npu.QuantMatrix(4, h, 2 * inter, *R.weights(4, f"cfg4-gu{e}", 4, h, 2 * inter)) for e in range(experts)]
    down = [npu.QuantMatrix(8, inter, h, *R.weights(4, f"cfg4-dn{e}", 8, inter, h)) for e in range(experts)]
    moe = backend.load_moe(gate, down, top)
    g = R.rng_for(4, "cfg4-router")
    x = R.activations(4, "cfg4-x", 1, h, outliers=False)
    ids, w = oracle.routes(g.standard_normal(experts).astype(np.float32), top)
    ids, w = ids[None, :], w[None, :]
    out = np.zeros((1, h), np.float32)
    moe.run(x, ids, w, out, 1)
    want = oracle.moe([(q.codes, q.scales) for q in gate], [(q.codes, q.scales) for q in down], x, ids, w)
    assert np.array_equal(out, want)
    print("MoE T=1 shared W8 FFN 2048->2x2048->2048 (device FFN)", flush=True)
    ctx = D.DeviceContext(7)
    sgc, sgs = R.weights(4, "cfg4-sh-gu", 8, h, 2 * sh_inter)
    sdc, sds = R.weights(4, "cfg4-sh-dn", 8, sh_inter, h)
    sgu, sdn = ctx.weights(8, dev(sgc), dev(sgs)), ctx.weights(8, dev(sdc), dev(sds))
    y = torch.empty(1, h, dtype=torch.float32, device="cuda")
    D.ffn(ctx, sgu, sdn, dev(x), y, 1)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), oracle.ffn(sgc, sgs, sdc, sds, x))
