"""GPU parity of the fused FFN (gate_up -> SwiGLU -> requant -> down) and the
grouped routed MoE FFN against the oracle, through the C ABI."""
import ctypes

import numpy as np
import pytest

from oracle import oracle
from open_rknpu2_lm_infer_amd import _ffi as F
from open_rknpu2_lm_infer_amd import npu
from tests import refdata as R

# imported before the library loads (as in the other device-test modules):
# the device-path test below hands torch tensors to the C ABI
torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _ptr(a, t):
    return a.ctypes.data_as(ctypes.POINTER(t))


class FFN:
    """Gate_up (W4) and down (W4 or W8) weights plus same-M workspaces."""

    def __init__(self, backend, h, f, m, dn_bits, seed_name):
        L = F.lib()
        self.gc, self.gs = R.weights(2, seed_name + "-gu", 4, h, 2 * f)
        self.dc, self.ds = R.weights(2, seed_name + "-dn", dn_bits, f, h)
        self.h, self.f, self.m, self.dn_bits = h, f, m, dn_bits
        dom = backend.domain
        self.gw = npu._Handle(L.rk_npu_w4a8_weights_create(dom, ctypes.byref(F.rk_npu_i4_weight_config(h, 2 * f, 0)),
                                                           _ptr(self.gc.reshape(-1), ctypes.c_int8),
                                                           _ptr(self.gs, ctypes.c_float)),
                              L.rk_npu_w4a8_weights_free, "gate_up", backend._shared)
        cfg = F.rk_npu_w4a8_config()
        opt = F.rk_npu_w4a8_options()
        L.rk_npu_w4a8_config_init(ctypes.byref(cfg), m, 2 * f, h)
        L.rk_npu_w4a8_options_init(ctypes.byref(opt))
        self.gws = npu._Handle(L.rk_npu_w4a8_workspace_create_ex(dom, ctypes.byref(cfg), ctypes.byref(opt)),
                               L.rk_npu_w4a8_workspace_free, "gate_up ws", backend._shared)
        if dn_bits == 4:
            self.dw = npu._Handle(L.rk_npu_w4a8_weights_create(dom, ctypes.byref(F.rk_npu_i4_weight_config(f, h, 0)),
                                                               _ptr(self.dc.reshape(-1), ctypes.c_int8),
                                                               _ptr(self.ds, ctypes.c_float)),
                                  L.rk_npu_w4a8_weights_free, "down", backend._shared)
            L.rk_npu_w4a8_config_init(ctypes.byref(cfg), m, h, f)
            self.dws = npu._Handle(L.rk_npu_w4a8_workspace_create_ex(dom, ctypes.byref(cfg), ctypes.byref(opt)),
                                   L.rk_npu_w4a8_workspace_free, "down ws", backend._shared)
        else:
            self.dw = npu._Handle(L.rk_npu_f32i8f32_weights_create(dom, ctypes.byref(F.rk_npu_matmul_weight_config(f, h, f)),
                                                                   _ptr(self.dc.reshape(-1), ctypes.c_int8),
                                                                   _ptr(self.ds, ctypes.c_float)),
                                  L.rk_npu_f32i8f32_weights_free, "down", backend._shared)
            st = F.rk_npu_matmul_strategy()
            st.M, st.N, st.K, st.k_tile = m, h, f, f
            self.dws = npu._Handle(L.rk_npu_matmul_workspace_create(dom, ctypes.byref(st)),
                                   L.rk_npu_matmul_workspace_free, "down ws", backend._shared)

    def run(self, x):
        out = np.zeros((self.m, self.h), np.float32)
        x = np.ascontiguousarray(x, np.float32)
        npu.check(F.lib().rk_npu_w4a8_run_ffn_f32(self.gws.raw, self.gw.raw, self.dws.raw, self.dw.raw,
                                                  self.dn_bits, _ptr(x, ctypes.c_float), _ptr(out, ctypes.c_float),
                                                  None), "FFN")
        return out


@pytest.mark.parametrize("dn_bits", [4, 8])
@pytest.mark.parametrize("m", [1, 4, 8, 64, 128])
def test_fused_ffn_matches_oracle(dn_bits, m):
    backend = npu.Backend(npu.ModelOptions(chunk=128))
    ffn = FFN(backend, 256, 384, m, dn_bits, f"ffn{m}")
    x = R.activations(2, f"ffn-x{m}", m, 256)
    print(f"ffn dn_bits={dn_bits} m={m}", flush=True)
    out = ffn.run(x)
    ref, mid = oracle.ffn(ffn.gc, ffn.gs, ffn.dc, ffn.ds, x, with_middle=True)
    assert np.array_equal(out, ref)
    # the fused path equals run_swiglu followed by Linear::run on the middle
    g = np.zeros((m, 384), np.float32)
    assert np.array_equal(mid, oracle.linear_swiglu(ffn.gc, ffn.gs, x))


def test_ffn_qwen3_4b_m512_all_rows():
    """Prefill FFN block at its real shape: M=512, H=2560, F=9728, W4 gate_up,
    W8 down; every row against the oracle."""
    backend = npu.Backend(npu.ModelOptions(chunk=256))
    ffn = FFN(backend, 2560, 9728, 512, 8, "ffn512")
    x = R.activations(2, "ffn512-x", 512, 2560)
    out = ffn.run(x)
    ref = oracle.ffn(ffn.gc, ffn.gs, ffn.dc, ffn.ds, x)
    assert np.array_equal(out, ref)
    assert np.all(np.isfinite(out))


def moe_bank(h, inter, experts, dn_bits, tag):
    gate = [npu.QuantMatrix(4, h, 2 * inter, *R.weights(4, f"{tag}-gu{e}", 4, h, 2 * inter)) for e in range(experts)]
    down = [npu.QuantMatrix(dn_bits, inter, h, *R.weights(4, f"{tag}-dn{e}", dn_bits, inter, h)) for e in range(experts)]
    return gate, down


def routed(rows, experts, top, tag):
    g = R.rng_for(4, tag)
    logits = g.standard_normal((rows, experts)).astype(np.float32)
    ids = np.zeros((rows, top), np.int32)
    w = np.zeros((rows, top), np.float32)
    for r in range(rows):
        i, v = oracle.routes(logits[r], top)
        ids[r], w[r] = i, v
    return ids, w


@pytest.mark.parametrize("dn_bits", [4, 8])
@pytest.mark.parametrize("rows", [1, 3, 40])
def test_moe_matches_oracle(dn_bits, rows):
    h, inter, experts, top = 256, 96, 16, 4
    backend = npu.Backend(npu.ModelOptions(chunk=64))
    gate, down = moe_bank(h, inter, experts, dn_bits, f"moe{dn_bits}")
    moe = backend.load_moe(gate, down, top)
    x = R.activations(4, f"moe-x{rows}", rows, h)
    ids, w = routed(rows, experts, top, f"moe-r{rows}")
    if rows >= 3:
        ids[1, 1] = ids[1, 0]      # duplicate expert in one row
        w[2, 3] = np.float32(0.0)  # skipped route
    out = np.zeros((rows, h), np.float32)
    print(f"moe dn_bits={dn_bits} rows={rows}", flush=True)
    moe.run(x, ids, w, out, rows)
    ref = oracle.moe([(g.codes, g.scales) for g in gate], [(d.codes, d.scales) for d in down], x, ids, w)
    assert np.array_equal(out, ref)
    again = np.zeros_like(out)
    moe.run(x, ids, w, again, rows)
    assert np.array_equal(again, out)


@pytest.mark.parametrize("rows,top,qw,fuse", [(5, 2, -1, 1), (1, 2, -1, 1), (1, 8, -1, 1), (1, 8, 1, 1),
                                               (1, 8, -1, 0)])
def test_moe_with_shared_w8_expert(rows, top, qw, fuse):
    """Routed experts plus a shared W8 expert, equal to the oracle. At one
    token the shared expert's down GEMV also runs the combine in its
    epilogue; with a quantization wave forced on (HM_GEMV_QW=1) it cannot,
    nor with HM_GEMV_COMBINE=0, and the combine runs afterwards in place on
    the output. A repeated expert and a skipped (zero) route at one token."""
    from open_rknpu2_lm_infer_amd import device as D
    h, inter, experts = 128, 64, 8
    backend = npu.Backend(npu.ModelOptions(chunk=16))
    gate, down = moe_bank(h, inter, experts, 4, "moesh")
    sg = npu.QuantMatrix(8, h, 2 * inter, *R.weights(4, "sh-gu", 8, h, 2 * inter))
    sd = npu.QuantMatrix(8, inter, h, *R.weights(4, "sh-dn", 8, inter, h))
    moe = backend.load_moe_with_shared(gate, down, top, (sg, sd))
    x = R.activations(4, f"moesh-x{rows}", rows, h)
    ids, w = routed(rows, experts, top, f"moesh-r{rows}-{top}")
    if rows == 1:
        ids[0, 1] = ids[0, 0]  # a repeated expert
        w[0, top - 1] = 0.0    # a skipped route
    out = np.zeros((rows, h), np.float32)
    with D.plan_switch("HM_GEMV_QW", qw), D.plan_switch("HM_GEMV_COMBINE", fuse):
        moe.run(x, ids, w, out, rows)
    ref = oracle.moe([(g.codes, g.scales) for g in gate], [(d.codes, d.scales) for d in down], x, ids, w,
                     shared=((sg.codes, sg.scales), (sd.codes, sd.scales)))
    assert np.array_equal(out, ref)


def test_moe_rejects_out_of_range_ids():
    backend = npu.Backend(npu.ModelOptions(chunk=4))
    gate, down = moe_bank(64, 32, 4, 4, "moebad")
    moe = backend.load_moe(gate, down, 2)
    x = np.zeros((1, 64), np.float32)
    with pytest.raises(npu.NpuError):
        moe.run(x, np.array([[0, 4]], np.int32), np.array([[0.5, 0.5]], np.float32), np.zeros((1, 64), np.float32), 1)


def test_moe_35b_a3b_shape_t512_all_rows():
    """Config-4 shape: hidden 2048, 128 experts, top-8, intermediate 768,
    W4 gate_up + W8 down, T=512 ragged per-expert batches; every token
    against the oracle."""
    h, inter, experts, top, rows = 2048, 768, 128, 8, 512
    backend = npu.Backend(npu.ModelOptions(chunk=256))
    backend.options.chunk = 512  # MoE max_rows (the op layer caps Linear at 256, not MoE)
    gate, down = moe_bank(h, inter, experts, 8, "moe35")
    moe = backend.load_moe(gate, down, top)
    x = R.activations(4, "moe35-x", rows, h)
    ids, w = routed(rows, experts, top, "moe35-r")
    out = np.zeros((rows, h), np.float32)
    moe.run(x, ids, w, out, rows)
    ref = oracle.moe([(g.codes, g.scales) for g in gate], [(d.codes, d.scales) for d in down], x, ids, w)
    assert np.array_equal(out, ref)


def test_moe_blob_export_import_and_slot_swap():
    h, inter, experts, top = 128, 64, 4, 2
    backend = npu.Backend(npu.ModelOptions(chunk=8))
    gate, down = moe_bank(h, inter, experts, 4, "blob")
    moe = backend.load_moe(gate, down, top)
    x = R.activations(4, "blob-x", 3, h)
    ids = np.array([[0, 1], [2, 3], [1, 2]], np.int32)
    w = np.array([[0.5, 0.5], [0.7, 0.3], [0.9, 0.1]], np.float32)
    base = np.zeros((3, h), np.float32)
    moe.run(x, ids, w, base, 3)
    blobs = [moe.export(e) for e in range(experts)]
    assert all(len(b) == moe.blob_bytes() for b in blobs)
    # reversed bank via import into a second bank of the same geometry
    other = backend.load_moe(gate[::-1], down[::-1], top)
    for e in range(experts):
        other.import_(e, blobs[e])
    out = np.zeros_like(base)
    other.run(x, ids, w, out, 3)
    assert np.array_equal(out, base)
    # swap slots 0 and 3 between banks: other now holds gate[::-1][0] = gate[3] at 0
    other.promote(0, moe, 3)
    moe.promote(3, other, 0)  # swap back
    out2 = np.zeros_like(base)
    moe.run(x, ids, w, out2, 3)
    assert np.array_equal(out2, base)
    corrupt = bytearray(blobs[0])
    corrupt[0] ^= 0xFF
    with pytest.raises(npu.NpuError):
        other.import_(0, bytes(corrupt))


def test_resident_moe_equals_paged_composition_on_gpu():
    """The reference's paged path (src/model/experts/paged.rs:590-641, 494-507)
    on the GPU: every nonzero-route assignment as its own row of a top=1 bank
    with route 1.0, then the rank-ordered fma reduction on the host. The
    resident top-8 run must give the same bits, including a repeated expert,
    zero and negative routes."""
    from tests.test_moe_oracle_pin import fma_vec
    h, inter, experts, top, rows = 256, 96, 16, 8, 6
    backend = npu.Backend(npu.ModelOptions(chunk=64))
    gate, down = moe_bank(h, inter, experts, 8, "paged")
    resident = backend.load_moe(gate, down, top)
    single = backend.load_moe(gate, down, 1)
    x = R.activations(4, "paged-x", rows, h)
    ids, w = routed(rows, experts, top, "paged-r")
    ids[1, 3] = ids[1, 0]  # repeated expert
    w[2, 5] = 0.0
    w[3, 1] = -0.25
    out = np.zeros((rows, h), np.float32)
    resident.run(x, ids, w, out, rows)
    jobs = [(r, k) for r in range(rows) for k in range(top) if w[r, k] != 0.0]
    xin = np.stack([x[r] for r, _ in jobs])
    jid = np.array([[ids[r, k]] for r, k in jobs], np.int32)
    contrib = np.zeros((len(jobs), h), np.float32)
    single.run(xin, jid, np.ones((len(jobs), 1), np.float32), contrib, len(jobs))
    by_job = {job: contrib[i] for i, job in enumerate(jobs)}
    want = np.zeros((rows, h), np.float32)
    for r in range(rows):
        s = np.zeros(h, np.float32)
        for k in range(top):
            if w[r, k] > 0.0:
                s = fma_vec(by_job[(r, k)], w[r, k], s)
        want[r] = s
    assert np.array_equal(out, want)


@pytest.mark.parametrize("rows", [1, 3, 20])
def test_moe_device_entry_aligned_unaligned_and_bad_ids(rows):
    """rk_npu_hip_moe_run on device buffers: 1 and 3 rows take the decode-sized
    slot path (an aligned input row is quantized inside the routed gate/up
    blocks, an input off 16-byte alignment by a launch first), 20 rows (80
    assignments) the routed grouped path; all equal the oracle, with a skipped
    (zero) route and a repeated expert. An out-of-range expert id is reported
    by rk_npu_hip_moe_status (once: the report clears), on a live route and on
    a skipped one alike."""
    from open_rknpu2_lm_infer_amd import device as D
    h, inter, experts, top = 256, 96, 6, 4
    gate, down = moe_bank(h, inter, experts, 8, f"moedev{rows}")
    L = F.lib()
    ctx = D.DeviceContext(9)
    arr = (F.rk_npu_moe_w8_expert * experts)()
    for e in range(experts):
        arr[e] = F.rk_npu_moe_w8_expert(gate[e].codes.ctypes.data_as(F.i8p), gate[e].scales.ctypes.data_as(F.f32p),
                                        down[e].codes.ctypes.data_as(F.i8p), down[e].scales.ctypes.data_as(F.f32p))
    cfg = F.rk_npu_moe_w8_config()
    L.rk_npu_moe_w8_config_init(ctypes.byref(cfg), h, inter, experts, 0, top, max(8, rows))
    bank = npu._Handle(L.rk_npu_moe_w4w8_weights_create(ctx.domain, ctypes.byref(cfg.weights), arr),
                       L.rk_npu_moe_w8_weights_free, "MoE bank", ctx.shared)
    work = npu._Handle(L.rk_npu_moe_w4w8_workspace_create(ctx.domain, ctypes.byref(cfg)),
                       L.rk_npu_moe_w8_workspace_free, "MoE workspace", ctx.shared)
    x = R.activations(4, f"moedev-x{rows}", rows, h)
    ids, w = routed(rows, experts, top, f"moedev-r{rows}")
    ids[0, 1] = ids[0, 0]  # a repeated expert
    w[-1, 2] = 0.0         # a skipped route
    ref = oracle.moe([(g.codes, g.scales) for g in gate], [(d.codes, d.scales) for d in down], x, ids, w)
    d_ids = torch.from_numpy(ids).cuda()
    d_w = torch.from_numpy(w).cuda()
    y = torch.empty(rows, h, dtype=torch.float32, device="cuda")
    buf = torch.zeros(rows * h + 4, dtype=torch.float32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for offset in (0, 1):  # 1 float: the input is off 16-byte alignment
        xin = buf[offset:offset + rows * h]
        xin.copy_(torch.from_numpy(x.reshape(-1)))
        y.fill_(float("nan"))
        rc = L.rk_npu_hip_moe_run(work.raw, bank.raw, rows, ctypes.c_void_p(xin.data_ptr()),
                                  ctypes.c_void_p(d_ids.data_ptr()), ctypes.c_void_p(d_w.data_ptr()),
                                  ctypes.c_void_p(y.data_ptr()), stream)
        assert rc == 0
        assert L.rk_npu_hip_moe_status(work.raw) == 0
        assert np.array_equal(y.cpu().numpy(), ref), f"input offset {offset} floats"
    for live in (True, False):  # the bad id on a live route, then on a skipped one
        bad = ids.copy()
        bad[0, 0] = experts  # out of range
        wb = w.copy()
        if not live:
            wb[0, 0] = 0.0
        d_bad = torch.from_numpy(bad).cuda()
        d_wb = torch.from_numpy(wb).cuda()
        rc = L.rk_npu_hip_moe_run(work.raw, bank.raw, rows, ctypes.c_void_p(buf.data_ptr()),
                                  ctypes.c_void_p(d_bad.data_ptr()), ctypes.c_void_p(d_wb.data_ptr()),
                                  ctypes.c_void_p(y.data_ptr()), stream)
        assert rc == 0
        assert L.rk_npu_hip_moe_status(work.raw) == F.RK_NPU_ERR_PARAM, f"live route {live}"
        assert L.rk_npu_hip_moe_status(work.raw) == 0


@pytest.mark.parametrize("flag_order", [(1, 0, 1), (0, 1, 0)])
def test_host_calls_kernel_path_and_copies(flag_order):
    """Host-buffer calls whose input and output each fit 64 KB run on the
    compute queue (a fetch kernel, the work, a copy kernel that publishes C
    and a completion word the CPU polls); HM_HOST_FLAG=0 and larger calls
    copy and wait on the stream. Both paths, alternated on the same
    workspaces (the polled path returns with the stream's last launch still
    ending), give the oracle's result bit for bit: linear W4/W8 at 1 and 3
    rows (small) and 8 rows of K=4096 (128 KB of A: copies either way), the
    fused FFN at M=1, and the MoE at one token and at 40 (output 40 KB,
    inputs at 256-byte aligned stage offsets)."""
    from open_rknpu2_lm_infer_amd import device as D
    backend = npu.Backend(npu.ModelOptions(chunk=64))
    lin = {}
    for bits in (4, 8):
        for rows, k, n in ((1, 2560, 384), (3, 2560, 384), (8, 4096, 256)):
            codes, scales = R.weights(9, f"hostk{bits}-{k}-{n}", bits, k, n)
            lin[(bits, rows)] = (backend.load(npu.QuantMatrix(bits, k, n, codes, scales)), codes, scales, k, n)
    ffn = FFN(backend, 256, 384, 1, 8, "hostk-ffn")
    h, inter, experts, top = 256, 96, 16, 4
    gate, down = moe_bank(h, inter, experts, 8, "hostk-moe")
    moe = backend.load_moe(gate, down, top)
    for flag in flag_order:
        print(f"HM_HOST_FLAG={flag}", flush=True)
        with D.plan_switch("HM_HOST_FLAG", flag):
            for (bits, rows), (linear, codes, scales, k, n) in lin.items():
                x = R.activations(9, f"hostk-x{rows}-{k}-{flag}", rows, k)
                out = np.full((rows, n), np.nan, np.float32)
                linear.run(x, out, rows)
                assert np.array_equal(out, oracle.linear(codes, scales, x)), (bits, rows, flag)
                sw = np.full((rows, n // 2), np.nan, np.float32)
                if linear.run_swiglu(x, sw, rows):  # (W4 weights only)
                    assert np.array_equal(sw, oracle.linear_swiglu(codes, scales, x)), (bits, rows, flag)
            x = R.activations(9, f"hostk-ffn-x{flag}", 1, 256)
            assert np.array_equal(ffn.run(x), oracle.ffn(ffn.gc, ffn.gs, ffn.dc, ffn.ds, x))
            for rows in (1, 40):
                x = R.activations(9, f"hostk-moe-x{rows}-{flag}", rows, h)
                ids, w = routed(rows, experts, top, f"hostk-moe-r{rows}-{flag}")
                out = np.full((rows, h), np.nan, np.float32)
                moe.run(x, ids, w, out, rows)
                ref = oracle.moe([(g.codes, g.scales) for g in gate], [(d.codes, d.scales) for d in down], x, ids, w)
                assert np.array_equal(out, ref), (rows, flag)


def test_host_calls_poll_fallback():
    """With HM_HOST_POLL=0 a kernel-path host call stops polling its
    completion word after the first 256 polls and waits on its stream, then
    reads the word (set by then): the results equal the oracle's bit for bit
    (linear W4 at 1 row, the fused FFN at M=1, the MoE at one token)."""
    from open_rknpu2_lm_infer_amd import device as D
    backend = npu.Backend(npu.ModelOptions(chunk=64))
    codes, scales = R.weights(9, "hostpoll", 4, 2560, 384)
    linear = backend.load(npu.QuantMatrix(4, 2560, 384, codes, scales))
    ffn = FFN(backend, 256, 384, 1, 8, "hostpoll-ffn")
    h, inter, experts, top = 256, 96, 16, 4
    gate, down = moe_bank(h, inter, experts, 8, "hostpoll-moe")
    moe = backend.load_moe(gate, down, top)
    with D.plan_switch("HM_HOST_FLAG", 1), D.plan_switch("HM_HOST_POLL", 0):
        for rep in range(3):
            print(f"HM_HOST_POLL=0 rep {rep}", flush=True)
            x = R.activations(9, f"hostpoll-x{rep}", 1, 2560)
            out = np.full((1, 384), np.nan, np.float32)
            linear.run(x, out, 1)
            assert np.array_equal(out, oracle.linear(codes, scales, x))
            xf = R.activations(9, f"hostpoll-ffn-x{rep}", 1, 256)
            assert np.array_equal(ffn.run(xf), oracle.ffn(ffn.gc, ffn.gs, ffn.dc, ffn.ds, xf))
            xm = R.activations(9, f"hostpoll-moe-x{rep}", 1, h)
            ids, w = routed(1, experts, top, f"hostpoll-moe-r{rep}")
            om = np.full((1, h), np.nan, np.float32)
            moe.run(xm, ids, w, om, 1)
            ref = oracle.moe([(g.codes, g.scales) for g in gate], [(d.codes, d.scales) for d in down], xm, ids, w)
            assert np.array_equal(om, ref)
