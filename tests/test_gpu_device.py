"""Device-resident entry points (rk_npu_hip.h): fp16/fp32 activations in HBM,
results identical to the host-buffer ABI, and HIP-graph replays identical to
eager runs (checked on every replay, with eager work in between)."""
import numpy as np
import pytest

from oracle import oracle
from open_rknpu2_lm_infer_amd import device as D
from open_rknpu2_lm_infer_amd import npu
from tests import refdata as R

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    return D.DeviceContext(3)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows", [1, 3, 8, 40, 300])
def test_device_linear_matches_oracle_f32_and_f16(ctx, bits, rows):
    k, n = 640, 768
    codes, scales = R.weights(5, f"dl{bits}", bits, k, n)
    w = ctx.weights(bits, dev(codes), dev(scales))
    x = R.activations(5, f"dl-x{rows}", rows, k)  # fp16-representable values
    ref = oracle.linear(codes, scales, x)
    y32 = torch.empty(rows, n, dtype=torch.float32, device="cuda")
    D.linear(ctx, w, dev(x), y32, rows)
    torch.cuda.synchronize()
    assert np.array_equal(y32.cpu().numpy(), ref)
    # fp16 activations carry the same values; fp16 output is the f32 result rounded
    y16 = torch.empty(rows, n, dtype=torch.float16, device="cuda")
    D.linear(ctx, w, dev(x).half(), y16, rows)
    torch.cuda.synchronize()
    assert np.array_equal(y16.cpu().numpy(), ref.astype(np.float16))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows", [3, 4])
def test_four_row_gemv_quantized_in_blocks(ctx, bits, rows):
    """HM_GEMV_PREQ=0: the 4-row GEMV quantizes its rows inside every block
    instead of after a quantization launch; plain and SwiGLU outputs, f32 and
    f16 activations, identical to the oracle."""
    k, n = 768, 768
    codes, scales = R.weights(5, f"dlq{bits}", bits, k, n)
    w = ctx.weights(bits, dev(codes), dev(scales))
    x = R.activations(5, f"dlQ-x{rows}", rows, k)
    with D.plan_switch("HM_GEMV_PREQ", 0):
        for xin in (dev(x), dev(x).half()):
            y = torch.empty(rows, n, dtype=torch.float32, device="cuda")
            D.linear(ctx, w, xin, y, rows)
            m = torch.empty(rows, n // 2, dtype=torch.float32, device="cuda")
            D.linear(ctx, w, xin, m, rows, swiglu=True)
            torch.cuda.synchronize()
            assert np.array_equal(y.cpu().numpy(), oracle.linear(codes, scales, x))
            assert np.array_equal(m.cpu().numpy(), oracle.linear_swiglu(codes, scales, x))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("k", [640, 768, 2560, 9728])
def test_gemv_matrix_core_dots(ctx, bits, k):
    """2 to 8 rows: the GEMV's dot products on the matrix cores (K_pad a
    multiple of 128 for W8, 256 for W4; W4 at K = 640 takes the GEMM), rows
    quantized in the block or beforehand (HM_GEMV_PREQ), fp16 and f32 rows,
    plain and SwiGLU, the 512-thread two-window blocks at K = 9728: identical
    to the oracle."""
    n = 256
    codes, scales = R.weights(5, f"gmf{bits}-{k}", bits, k, n)
    w = ctx.weights(bits, dev(codes), dev(scales))
    for rows in (2, 3, 4, 5, 8):
        if rows * k > 60 * 1024:
            continue  # rows too long for the GEMV's LDS: the GEMM runs them
        x = R.activations(5, f"gmf-x{rows}-{k}", rows, k)
        ref, ref_sw = oracle.linear(codes, scales, x), oracle.linear_swiglu(codes, scales, x)
        for preq in (1, 0):
            for xin in (dev(x), dev(x).half()):
                print(f"W{bits} K={k} rows={rows} preq={preq} {xin.dtype}", flush=True)
                with D.plan_switch("HM_GEMV_PREQ", preq):
                    y = torch.empty(rows, n, dtype=torch.float32, device="cuda")
                    D.linear(ctx, w, xin, y, rows)
                    m = torch.empty(rows, n // 2, dtype=torch.float32, device="cuda")
                    D.linear(ctx, w, xin, m, rows, swiglu=True)
                    torch.cuda.synchronize()
                assert np.array_equal(y.cpu().numpy(), ref)
                assert np.array_equal(m.cpu().numpy(), ref_sw)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows,variant,n", [(1100, None, 768), (2100, None, 768), (2100, "0", 768),
                                            (4100, "0", 768), (2100, "0", 640), (300, "0", 896),
                                            (4100, "0", 640), (300, "1", 896), (4100, "1", 640),
                                            (4096, "5", 768), (4100, "5", 640), (300, "5", 896),
                                            (192, "5", 768), (2000, "5", 512)])
def test_device_linear_large_row_tiles(ctx, bits, rows, variant, n):
    """Row counts that select the 128x128 tile, and the 256x256 tile (variant
    0: chosen by the plan for very wide outputs or long K), the 256x128 tile
    (variant 1) and the 192x256 tile (variant 5: its last A load round is
    issued by half of the waves; the plan takes it for M=4096 o and down),
    forced here at small shapes. n = 640 and 896 leave 128 padded columns in
    the last 256-wide tile, as the 2560x151936 lm_head does (plain and SwiGLU
    stores masked at the edge); 4100 and 300 rows end inside a 256-row tile,
    4096, 4100, 300 and 2000 inside a 192-row tile whose rows reach past the
    code buffer's (4096 rows: 22 tiles of 192 cover 4224)."""
    with D.plan_switch("HM_GEMM_VARIANT", -1 if variant is None else int(variant)):
        _large_row_tiles(ctx, bits, rows, n)


def _large_row_tiles(ctx, bits, rows, n):
    k = 640
    codes, scales = R.weights(5, f"dl{bits}-{n}", bits, k, n)
    w = ctx.weights(bits, dev(codes), dev(scales))
    x = R.activations(5, f"dlL-x{rows}", rows, k)
    y = torch.empty(rows, n, dtype=torch.float32, device="cuda")
    D.linear(ctx, w, dev(x), y, rows)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), oracle.linear(codes, scales, x))
    m = torch.empty(rows, n // 2, dtype=torch.float32, device="cuda")
    D.linear(ctx, w, dev(x), m, rows, swiglu=True)
    torch.cuda.synchronize()
    assert np.array_equal(m.cpu().numpy(), oracle.linear_swiglu(codes, scales, x))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_unaligned_output_matches_oracle(ctx, bits, dtype):
    """An output base off 16-byte alignment takes the per-lane store epilogue."""
    rows, k, n = 300, 640, 768
    codes, scales = R.weights(5, f"dl{bits}", bits, k, n)
    w = ctx.weights(bits, dev(codes), dev(scales))
    x = R.activations(5, f"dlU-x{rows}", rows, k)
    t = torch.float16 if dtype == "f16" else torch.float32
    for swiglu, width, ref in ((False, n, oracle.linear(codes, scales, x)),
                               (True, n // 2, oracle.linear_swiglu(codes, scales, x))):
        buf = torch.zeros(rows * width + 1, dtype=t, device="cuda")
        y = buf[1:].view(rows, width)
        D.linear(ctx, w, dev(x), y, rows, swiglu=swiglu)
        torch.cuda.synchronize()
        assert buf[0].item() == 0
        assert np.array_equal(y.cpu().numpy(), ref.astype(np.float16) if dtype == "f16" else ref)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows,n", [(300, 256), (512, 256), (300, 448)])
def test_long_k_split_plan_above_256_rows(ctx, bits, rows, n):
    """Long K (8192) over more than 256 rows: the plan splits K on the 128x128
    tile (pieces summed through int32 partials, then one one-wave block per
    64x64 wave tile for the epilogue); plain fp16 and SwiGLU f32 outputs
    identical to the oracle. 300 rows and 448 columns leave wave tiles
    partly and wholly past the output in both directions."""
    k = 8192
    codes, scales = R.weights(5, f"lks{bits}-{n}", bits, k, n)
    w = ctx.weights(bits, dev(codes), dev(scales))
    x = R.activations(5, f"lks-x{rows}", rows, k)
    y = torch.empty(rows, n, dtype=torch.float16, device="cuda")
    D.linear(ctx, w, dev(x).half(), y, rows)
    m = torch.empty(rows, n // 2, dtype=torch.float32, device="cuda")
    D.linear(ctx, w, dev(x), m, rows, swiglu=True)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), oracle.linear(codes, scales, x).astype(np.float16))
    assert np.array_equal(m.cpu().numpy(), oracle.linear_swiglu(codes, scales, x))


@pytest.mark.parametrize("splits", [2, 3])
def test_split_k_switch_is_bit_exact(ctx, splits):
    """HM_SPLITS: K pieces per tile sum through int32 partials; same result."""
    with D.plan_switch("HM_SPLITS", splits):
        _split_k(splits)


def _split_k(splits):
    local = D.DeviceContext(3)  # workspaces sized under the switch
    rows, k, n = 300, 640, 768
    for bits in (4, 8):
        codes, scales = R.weights(5, f"dl{bits}", bits, k, n)
        w = local.weights(bits, dev(codes), dev(scales))
        x = R.activations(5, f"dlS-x{rows}", rows, k)
        y = torch.empty(rows, n, dtype=torch.float16, device="cuda")
        D.linear(local, w, dev(x).half(), y, rows)
        m = torch.empty(rows, n // 2, dtype=torch.float32, device="cuda")
        D.linear(local, w, dev(x), m, rows, swiglu=True)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), oracle.linear(codes, scales, x).astype(np.float16))
        assert np.array_equal(m.cpu().numpy(), oracle.linear_swiglu(codes, scales, x))


@pytest.mark.parametrize("bits", [4, 8])
def test_gemv_window_configurations_match_oracle(ctx, bits):
    """One- and two-row GEMVs over K values that select every register-window
    configuration of the GEMV launch (3/4/5/6/8 rounds of 256 weight chunks
    per tile group, 512-thread blocks with one 5- or 6-round window, two
    5-round windows, and 8-round windows that ping-pong; a row too long to be
    quantized in the block goes through the quantization launch first), plain
    and SwiGLU, fp16 rows: equal to the oracle."""
    per_k = 2 if bits == 4 else 1  # weight chunks per 64 k per column: W4 4, W8 8 (x2 for SwiGLU)
    ks = [1536, 2048, 2560, 3072, 4096, 5120, 6144, 10240, 16384, 24576]
    for k in ks:
        for swiglu in (False, True):
            n = 256
            codes, scales = R.weights(11, f"dwin{bits}-{k}-{swiglu}", bits, k, n)
            w = ctx.weights(bits, dev(codes), dev(scales))
            for rows in (1, 2):
                print(f"W{bits} K={k} swiglu={swiglu} rows={rows} chunks={k // 64 * 4 * per_k * (2 if swiglu else 1)}",
                      flush=True)
                x = R.activations(11, f"dwin-x{k}-{rows}", rows, k)
                if swiglu:
                    y = torch.empty(rows, n // 2, dtype=torch.float32, device="cuda")
                    D.linear(ctx, w, dev(x).half(), y, rows, swiglu=True)
                    want = oracle.linear_swiglu(codes, scales, x)
                else:
                    y = torch.empty(rows, n, dtype=torch.float32, device="cuda")
                    D.linear(ctx, w, dev(x).half(), y, rows)
                    want = oracle.linear(codes, scales, x)
                torch.cuda.synchronize()
                assert np.array_equal(y.cpu().numpy(), want)


@pytest.mark.parametrize("qw", ["default", "0", "1"])
def test_gemv_quantization_wave_matches_oracle(ctx, qw):
    """One-row GEMVs with K = 2560 (5 rounds of 256 weight chunks per tile
    group: the shapes the block's dedicated quantization wave serves), fp16
    and f32 rows, W4 and W8, plain and SwiGLU: equal to the oracle with the
    wave (default rule or HM_GEMV_QW=1) and without it (HM_GEMV_QW=0); the
    workspace diagnostics hold the row's codes, scale and code sum."""
    with D.plan_switch("HM_GEMV_QW", -1 if qw == "default" else int(qw)):
        _quantization_wave(ctx, qw)


def _quantization_wave(ctx, qw):
    from tests.test_gpu_linear import read_codes
    k = 2560
    for bits, n, swiglu in ((4, 1024, True), (8, 512, False), (4, 4096, False), (8, 1024, True)):
        codes, scales = R.weights(9, f"dqw{bits}-{n}", bits, k, n)
        w = ctx.weights(bits, dev(codes), dev(scales))
        ws = ctx.workspace(bits, 1, k, n)
        for rep, half in enumerate((False, True)):
            print(f"qw={qw} W{bits} n={n} swiglu={swiglu} fp16={half}", flush=True)
            x = R.activations(9, f"dqw-x{rep}", 1, k)
            xin = dev(x).half() if half else dev(x)
            if swiglu:
                y = torch.empty(1, n // 2, dtype=torch.float32, device="cuda")
                D.linear(ctx, w, xin, y, 1, swiglu=True, ws=ws)
                want = oracle.linear_swiglu(codes, scales, x)
            else:
                y = torch.empty(1, n, dtype=torch.float32, device="cuda")
                D.linear(ctx, w, xin, y, 1, ws=ws)
                want = oracle.linear(codes, scales, x)
            torch.cuda.synchronize()
            assert np.array_equal(y.cpu().numpy(), want)
            got, scale, sums = read_codes(ws, bits, 1, k)
            q, qs = oracle.quant_dense(x)
            assert np.array_equal(got, q) and np.array_equal(scale, qs)
            assert sums[0] == int(q.astype(np.int64).sum())


@pytest.mark.parametrize("splits", [1, 2, 3, 4])
def test_gemv_split_k_down_is_bit_exact(ctx, splits):
    """One-row FFN whose down GEMV (K = 2240: 35 units of 64, uneven pieces)
    splits K (HM_GEMV_SPLITS forces the piece count): the pieces' int32 sums
    meet through device-scope atomics and the last piece writes the tile and
    clears the accumulators, so three calls in a row must each equal the
    oracle; the down workspace's diagnostics hold the middle row's codes,
    scale and code sum."""
    with D.plan_switch("HM_GEMV_SPLITS", splits):
        _gemv_split_k_down(ctx, splits)


def _gemv_split_k_down(ctx, splits):
    from tests.test_gpu_linear import read_codes
    h, f = 256, 2240
    for dbits in (4, 8):
        gc, gs = R.weights(7, "dsk-g", 4, h, 2 * f)
        dc, ds = R.weights(7, f"dsk-d{dbits}", dbits, f, h)
        gu = ctx.weights(4, dev(gc), dev(gs))
        dn = ctx.weights(dbits, dev(dc), dev(ds))
        dws = ctx.workspace(dbits, 1, f, h)
        for rep in range(3):
            print(f"splits={splits} down W{dbits} call {rep}", flush=True)
            x = R.activations(7, f"dsk-x{rep}", 1, h)
            y = torch.empty(1, h, dtype=torch.float32, device="cuda")
            D.ffn(ctx, gu, dn, dev(x), y, 1, dws=dws)
            torch.cuda.synchronize()
            want, mid = oracle.ffn(gc, gs, dc, ds, x, with_middle=True)
            assert np.array_equal(y.cpu().numpy(), want)
            codes, scale, sums = read_codes(dws, dbits, 1, f)
            q, qs = oracle.quant_dense(mid)
            assert np.array_equal(codes, q) and np.array_equal(scale, qs)
            assert sums[0] == int(q.astype(np.int64).sum())


@pytest.mark.parametrize("bits", [4, 8])
def test_long_k_split_plan_matches_oracle(ctx, bits):
    """Few tiles over a long K: the plan splits K into pieces (partials, then a
    summing epilogue launch); results equal the oracle's."""
    import ctypes
    from open_rknpu2_lm_infer_amd import _ffi as F
    rows, k, n = 64, 8192, 512
    plan = F.rk_npu_hip_plan()
    assert F.lib().rk_npu_hip_linear_plan(rows, k, n, bits, ctypes.byref(plan)) == 0
    assert plan.kind == 1 and plan.k_splits > 1
    codes, scales = R.weights(5, f"dlK{bits}", bits, k, n)
    w = ctx.weights(bits, dev(codes), dev(scales))
    x = R.activations(5, "dlK-x", rows, k)
    y = torch.empty(rows, n, dtype=torch.float16, device="cuda")
    D.linear(ctx, w, dev(x).half(), y, rows)
    m = torch.empty(rows, n // 2, dtype=torch.float32, device="cuda")
    D.linear(ctx, w, dev(x), m, rows, swiglu=True)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), oracle.linear(codes, scales, x).astype(np.float16))
    assert np.array_equal(m.cpu().numpy(), oracle.linear_swiglu(codes, scales, x))


def _pack_words(codes_kn, bits):
    """compressed-tensors pack-quantized words [n][ceil(k*bits/32)] holding the
    codes [k][n] as code + 2^(bits-1) in consecutive bit fields."""
    k, n = codes_kn.shape
    f = 32 // bits
    cols = -(-k // f)
    u = np.zeros((cols * f, n), np.uint64)
    u[:k] = (codes_kn.astype(np.int64) + (1 << (bits - 1))) & ((1 << bits) - 1)
    u = u.reshape(cols, f, n)
    words = np.zeros((n, cols), np.uint64)
    for i in range(f):
        words |= u[:, i, :].T << np.uint64(i * bits)
    return words.astype(np.uint32)


@pytest.mark.parametrize("case", ["w4_gate_up", "w8_packed_qkv", "w8_int_quantized"])
def test_weights_from_checkpoint_storage(ctx, case):
    """rk_npu_hip_weights_create_checkpoint unpacks / transposes / concatenates
    on the GPU: the words are the reference's format (the oracle's unpack,
    pinned to its known-answer test, recovers the codes), and the weights give
    the same results as weights created from the fused [K][N] codes."""
    from open_rknpu2_lm_infer_amd import _ffi as F
    bits, k, ns, fmt = {"w4_gate_up": (4, 650, (768, 768), F.RK_NPU_HIP_PACK_QUANTIZED),
                        "w8_packed_qkv": (8, 640, (512, 128, 128), F.RK_NPU_HIP_PACK_QUANTIZED),
                        "w8_int_quantized": (8, 648, (384, 256), F.RK_NPU_HIP_INT_QUANTIZED)}[case]
    mats = [R.weights(9, f"ck-{case}-{i}", bits, k, n) for i, n in enumerate(ns)]
    parts = []
    for codes, scales in mats:
        if fmt == F.RK_NPU_HIP_PACK_QUANTIZED:
            words = _pack_words(codes, bits)
            assert np.array_equal(oracle.unpack_codes(words, bits, codes.shape[1], k), codes)
            data = dev(words.view(np.int32))
        else:
            data = dev(np.ascontiguousarray(codes.T))
        parts.append((data, dev(scales), fmt))
    fused_codes = oracle.concatenate([c for c, _ in mats])
    fused_scales = np.concatenate([s_ for _, s_ in mats]).astype(np.float32)
    w_ck = ctx.weights_from_checkpoint(bits, k, parts)
    w_ref = ctx.weights(bits, dev(fused_codes), dev(fused_scales))
    n = fused_codes.shape[1]
    for rows in (3, 300):
        x = R.activations(9, f"ck-x{rows}", rows, k)
        ref = oracle.linear(fused_codes, fused_scales, x)
        for w in (w_ck, w_ref):
            y = torch.empty(rows, n, dtype=torch.float32, device="cuda")
            D.linear(ctx, w, dev(x), y, rows)
            torch.cuda.synchronize()
            assert np.array_equal(y.cpu().numpy(), ref)


def test_weights_from_checkpoint_rejects_bad_input(ctx):
    import ctypes
    from open_rknpu2_lm_infer_amd import _ffi as F
    L = F.lib()
    codes, scales = R.weights(9, "ck-bad", 8, 64, 32)
    data, sc = dev(np.ascontiguousarray(codes.T)), dev(scales)
    arr = (F.rk_npu_hip_checkpoint_part * 1)(F.rk_npu_hip_checkpoint_part(data.data_ptr(), sc.data_ptr(), 32,
                                                                        F.RK_NPU_HIP_INT_QUANTIZED))
    # int-quantized storage exists only for 8-bit weights
    assert not L.rk_npu_hip_weights_create_checkpoint(ctx.domain, 4, 64, arr, 1)
    # a nonpositive scale is rejected (src/model/checkpoint.rs:486-489)
    bad = dev(np.where(np.arange(32) == 5, 0.0, scales).astype(np.float32))
    arr[0].scales = bad.data_ptr()
    assert not L.rk_npu_hip_weights_create_checkpoint(ctx.domain, 8, 64, arr, 1)
    assert not L.rk_npu_hip_weights_create_checkpoint(ctx.domain, 8, 64, arr, 0)
    torch.cuda.synchronize()


@pytest.mark.parametrize("rows", [1, 4, 64])
def test_device_ffn_matches_oracle(ctx, rows):
    h, f = 512, 768
    gc, gs = R.weights(5, "dffn-g", 4, h, 2 * f)
    dc, ds = R.weights(5, "dffn-d", 8, f, h)
    gu = ctx.weights(4, dev(gc), dev(gs))
    dn = ctx.weights(8, dev(dc), dev(ds))
    x = R.activations(5, f"dffn-x{rows}", rows, h)
    y = torch.empty(rows, h, dtype=torch.float32, device="cuda")
    D.ffn(ctx, gu, dn, dev(x), y, rows)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), oracle.ffn(gc, gs, dc, ds, x))


@pytest.mark.parametrize("rows", [1, 4, 96])
def test_graph_replay_matches_eager(ctx, rows):
    h, f = 512, 768
    gc, gs = R.weights(6, "g-g", 4, h, 2 * f)
    dc, ds = R.weights(6, "g-d", 4, f, h)
    qc, qs = R.weights(6, "g-q", 8, h, 384)
    gu = ctx.weights(4, dev(gc), dev(gs))
    dn = ctx.weights(4, dev(dc), dev(ds))
    q = ctx.weights(8, dev(qc), dev(qs))
    x = dev(R.activations(6, f"g-x{rows}", rows, h)).half()
    y1 = torch.empty(rows, h, dtype=torch.float16, device="cuda")
    y2 = torch.empty(rows, 384, dtype=torch.float16, device="cuda")

    def step():
        D.ffn(ctx, gu, dn, x, y1, rows)
        D.linear(ctx, q, x, y2, rows)

    step()
    torch.cuda.synchronize()
    e1, e2 = y1.clone(), y2.clone()
    xf = x.float().cpu().numpy()
    assert np.array_equal(e1.cpu().numpy(), oracle.ffn(gc, gs, dc, ds, xf).astype(np.float16))
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            step()
    torch.cuda.synchronize()
    for _ in range(4):
        y1.zero_()
        y2.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y1, e1) and torch.equal(y2, e2)
        step()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(y1, e1) and torch.equal(y2, e2)
