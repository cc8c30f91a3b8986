"""GPU parity of the FP16 GQA attention (rk_npu_attention_f16_*) against the
float64 oracle (oracle.attention): the reference's call patterns of
src/npu/attention.rs (causal decode/prefill appends, bidirectional GQA, the
full image attention with f32 and fp16 outputs), long contexts split over
many blocks, head dims 64/128/256, the cache bookkeeping (truncate, reset,
reserve, capacity errors) and the device-resident entry points.

Tolerance: the kernel computes in f32 (fp16 inputs, f32 dot products, f32
exp with the hardware exponential, f32 accumulation); the oracle in float64
over the same fp16 inputs. Outputs are convex combinations of value rows, so
the error is bounded by a small multiple of f32 rounding times the value
magnitude. With 16 or more query rows per KV head (head_dim 64/128) the
matrix-core path rounds the softmax weights to fp16 for P V and sums the same
rounded weights, so each weight carries a relative error of at most 2^-11 and
the output moves by at most 2^-11 * max |v_j - out| (random signs make it far
smaller). Both fit max |got - want| <= 2e-3 * max(1, max |want|)."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle
from open_rknpu2_lm_infer_amd import _ffi as F
from open_rknpu2_lm_infer_amd import npu

pytestmark = pytest.mark.gpu

TOL = 2e-3


def close(got, want, tol=TOL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.all(np.isfinite(got))
    scale = max(1.0, float(np.abs(want).max()))
    err = float(np.abs(got - want).max())
    assert err <= tol * scale, f"max error {err:.3g} (scale {scale:.3g})"


def heads_major(a):
    """[rows][heads][d] -> [heads][rows][d]."""
    return np.ascontiguousarray(np.asarray(a).transpose(1, 0, 2))


def run_sequence(att, qh, kh, d, chunks, rng, scale):
    """Appends through Attention.run and checks every call against the oracle."""
    k_all = np.zeros((0, kh, d), np.float16)
    v_all = np.zeros((0, kh, d), np.float16)
    pos = 0
    for rows in chunks:
        print(f"qh={qh} kh={kh} d={d} rows={rows} position={pos}", flush=True)
        q = rng.standard_normal((rows, qh, d)).astype(np.float32)
        k = rng.standard_normal((rows, kh, d)).astype(np.float32)
        v = rng.standard_normal((rows, kh, d)).astype(np.float32)
        out = np.empty((rows, qh, d), np.float32)
        att.run(q, k, v, out, rows, pos)
        k_all = np.concatenate([k_all, k.astype(np.float16)])
        v_all = np.concatenate([v_all, v.astype(np.float16)])
        want = oracle.attention(heads_major(q.astype(np.float16)), heads_major(k_all), heads_major(v_all),
                                float(np.float32(scale)), pos, True)
        close(heads_major(out), want)
        pos += rows
    assert att.info().length == pos
    return k_all, v_all


@pytest.mark.parametrize("d", [128, 64])
def test_causal_gqa_sequence_matches_oracle(d):
    """Prefill chunks, then single-row decode steps and a multi-token step
    (src/npu/attention.rs:299-352), 8 query heads over 2 KV heads. The 37-
    and 128-row chunks give 148 and 512 rows per KV head (8-wave blocks, tiles
    by direct loads over one and several tiles per key split), the 64- and
    17-row chunks 256 and 68 (8- and 4-wave blocks)."""
    be = npu.Backend(npu.ModelOptions(chunk=128, context=1024))
    qh, kh = 8, 2
    scale = d ** -0.5
    att = be.attention(qh, kh, d, scale)
    run_sequence(att, qh, kh, d, (37, 128, 64, 1, 1, 17, 4, 1), np.random.default_rng(3), scale)


def test_long_context_decode_matches_oracle():
    """Qwen3-4B-shaped decode: 32 query heads over 8 KV heads, d = 128, 4000
    cached rows (the keys split over many blocks, partials combined)."""
    be = npu.Backend(npu.ModelOptions(chunk=128, context=4096))
    qh, kh, d = 32, 8, 128
    scale = d ** -0.5
    att = be.attention(qh, kh, d, scale)
    rng = np.random.default_rng(4)
    k_all, v_all = [], []
    for i in range(0, 4000, 125):
        k = rng.standard_normal((125, kh, d)).astype(np.float32)
        v = rng.standard_normal((125, kh, d)).astype(np.float32)
        att.append(k, v, 125, i)
        k_all.append(k.astype(np.float16))
        v_all.append(v.astype(np.float16))
    k_all, v_all = np.concatenate(k_all), np.concatenate(v_all)
    for rows in (1, 4):
        pos = att.info().length
        print(f"decode rows={rows} at {pos}", flush=True)
        q = rng.standard_normal((rows, qh, d)).astype(np.float32)
        k = rng.standard_normal((rows, kh, d)).astype(np.float32)
        v = rng.standard_normal((rows, kh, d)).astype(np.float32)
        out = np.empty((rows, qh, d), np.float32)
        att.run(q, k, v, out, rows, pos)
        k_all = np.concatenate([k_all, k.astype(np.float16)])
        v_all = np.concatenate([v_all, v.astype(np.float16)])
        want = oracle.attention(heads_major(q.astype(np.float16)), heads_major(k_all), heads_major(v_all),
                                float(np.float32(scale)), pos, True)
        close(heads_major(out), want)


@pytest.mark.parametrize("qh,kh,d", [(4, 4, 64), (8, 2, 256), (16, 4, 128)])
def test_bidirectional_gqa_matches_oracle(qh, kh, d):
    """noncausal_gqa (src/npu.rs:694-705): every query row sees every key."""
    be = npu.Backend(npu.ModelOptions(chunk=64, context=512))
    att = be.noncausal_gqa(qh, kh, d)
    rng = np.random.default_rng(5)
    k_all = np.zeros((0, kh, d), np.float16)
    v_all = np.zeros((0, kh, d), np.float16)
    pos = 0
    for rows in (50, 64, 3):
        print(f"bidirectional qh={qh} kh={kh} d={d} rows={rows}", flush=True)
        q = rng.standard_normal((rows, qh, d)).astype(np.float32)
        k = rng.standard_normal((rows, kh, d)).astype(np.float32)
        v = rng.standard_normal((rows, kh, d)).astype(np.float32)
        out = np.empty((rows, qh, d), np.float32)
        att.run(q, k, v, out, rows, pos)
        k_all = np.concatenate([k_all, k.astype(np.float16)])
        v_all = np.concatenate([v_all, v.astype(np.float16)])
        want = oracle.attention(heads_major(q.astype(np.float16)), heads_major(k_all), heads_major(v_all),
                                float(np.float32(d ** -0.5)), pos, False)
        close(heads_major(out), want)
        pos += rows


@pytest.mark.parametrize("causal,d", [(True, 128), (False, 128), (True, 64)])
def test_growing_scores_match_oracle(causal, d):
    """Keys whose magnitude grows along the sequence, so a row's running max
    rises many times over the tiles of one key split (scaled scores up to
    ~50, far past what unshifted fp16 weights hold). 32 query heads over 8
    KV heads with 128 query rows over 2048 keys: the matrix-core path splits
    the keys 8 ways, 4 tiles each (more tiles than its 8-wave blocks' three
    tile buffers), so its deferred rescaling runs inside a split; then a
    1-row decode step over the same cache."""
    be = npu.Backend(npu.ModelOptions(chunk=128, context=2048))
    qh, kh, length = 32, 8, 2048
    scale = d ** -0.5
    att = be.attention(qh, kh, d, scale) if causal else be.noncausal_gqa(qh, kh, d)
    rng = np.random.default_rng(9)
    grow = (0.2 + np.arange(length) / 300.0)[:, None, None]
    k_all = (rng.standard_normal((length, kh, d)) * grow).astype(np.float16)
    v_all = rng.standard_normal((length, kh, d)).astype(np.float16)
    prefix = length - 128
    for i in range(0, prefix, 128):
        att.append(k_all[i:i + 128].astype(np.float32), v_all[i:i + 128].astype(np.float32), 128, i)
    for rows in (128, 1):
        pos = att.info().length
        if rows == 1:
            att.truncate(pos - 1)
            pos -= 1
        print(f"growing scores causal={causal} rows={rows} position={pos}", flush=True)
        q = (rng.standard_normal((rows, qh, d)) * 2.0).astype(np.float32)
        out = np.empty((rows, qh, d), np.float32)
        att.run(q, k_all[pos:pos + rows].astype(np.float32), v_all[pos:pos + rows].astype(np.float32), out, rows, pos)
        want = oracle.attention(heads_major(q.astype(np.float16)), heads_major(k_all[:pos + rows]),
                                heads_major(v_all[:pos + rows]), float(np.float32(scale)), pos, causal)
        close(heads_major(out), want)


@pytest.mark.parametrize("heads,d,rows", [(4, 64, 100), (4, 64, 48), (2, 128, 40)])
def test_full_attention_f32_and_half(heads, d, rows):
    """FullAttention.run_full / run_full_half (src/npu/attention.rs:45-205):
    the fp16 output is the f32 result rounded to nearest. 100 keys take two
    key splits and the combine; 40-48 keys fit one split, where the
    matrix-core kernel writes both outputs itself."""
    be = npu.Backend(npu.ModelOptions(chunk=32, context=512))
    fa = be.full_attention(heads, d, rows)
    rng = np.random.default_rng(6)
    q, k, v = (rng.standard_normal((rows, heads, d)).astype(np.float32) for _ in range(3))
    out = np.empty((rows, heads, d), np.float32)
    fa.run_full(q, k, v, out, rows)
    want = oracle.attention(heads_major(q.astype(np.float16)), heads_major(k.astype(np.float16)),
                            heads_major(v.astype(np.float16)), float(np.float32(d ** -0.5)), 0, False)
    close(heads_major(out), want)
    out_h = np.empty((rows, heads, d), np.uint16)
    fa.run_full_half(q.astype(np.float16).view(np.uint16), k.astype(np.float16).view(np.uint16),
                     v.astype(np.float16).view(np.uint16), out_h, rows)
    assert np.array_equal(out_h.view(np.float16), out.astype(np.float16))


def test_cache_bookkeeping():
    """truncate / reset / reserve / capacity errors (src/npu/attention.rs:190-297)."""
    be = npu.Backend(npu.ModelOptions(chunk=64, context=256))
    qh, kh, d = 4, 2, 64
    scale = d ** -0.5
    att = be.attention(qh, kh, d, scale)
    rng = np.random.default_rng(7)
    k_all, v_all = run_sequence(att, qh, kh, d, (40, 30), rng, scale)
    info0 = att.info()
    cap0, gen0 = info0.capacity, info0.generation
    assert info0.max_capacity == 256  # the context, a multiple of 32
    att.reserve(256)
    assert att.info().capacity == 256 and att.info().length == 70 and att.bytes() == 2 * 2 * 256 * 64 * 2
    # generation: changed by a reallocation, kept by truncate (src/npu.rs:1789)
    gen1 = att.info().generation
    assert (gen1 != gen0) == (cap0 < 256)
    # contents survive the growth: a decode step still matches
    att.truncate(50)
    assert att.info().length == 50 and att.info().generation == gen1
    q = rng.standard_normal((1, qh, d)).astype(np.float32)
    k = rng.standard_normal((1, kh, d)).astype(np.float32)
    v = rng.standard_normal((1, kh, d)).astype(np.float32)
    out = np.empty((1, qh, d), np.float32)
    att.run(q, k, v, out, 1, 50)
    kk = np.concatenate([k_all[:50], k.astype(np.float16)])
    vv = np.concatenate([v_all[:50], v.astype(np.float16)])
    close(heads_major(out), oracle.attention(heads_major(q.astype(np.float16)), heads_major(kk), heads_major(vv),
                                             float(np.float32(scale)), 50, True))
    assert cap0 <= 256
    with pytest.raises(npu.NpuError):
        att.truncate(52)  # longer than held
    with pytest.raises(npu.NpuError):
        att.append(k, v, 1, 7)  # position mismatch
    att.reset()
    assert att.info().length == 0 and att.info().generation != gen1
    with pytest.raises(npu.NpuError):
        att.reserve(512)  # beyond the context
    with pytest.raises(npu.NpuError):
        npu.Backend(npu.ModelOptions()).attention(4, 2, 96, 96 ** -0.5)  # no kernel for head_dim 96


def test_device_entry_points_match_host_path():
    """rk_npu_hip_attention_cache_append / _run on HBM tensors (f32 and fp16
    output) against the oracle."""
    L = F.lib()
    be = npu.Backend(npu.ModelOptions(chunk=16, context=2048))
    qh, kh, d, rows, length = 8, 2, 128, 3, 1500
    cfg = F.rk_npu_attention_f16_config()
    L.rk_npu_attention_f16_config_init(ctypes.byref(cfg))
    cfg.query_heads, cfg.kv_heads, cfg.head_dim = qh, kh, d
    cfg.softmax_scale = d ** -0.5
    cfg.max_query_rows, cfg.max_capacity, cfg.initial_capacity = 16, 2048, 64
    ws, cache = ctypes.c_void_p(), ctypes.c_void_p()
    npu.check(L.rk_npu_attention_f16_prepare(be.domain, ctypes.byref(cfg), ctypes.byref(ws)), "prepare")
    npu.check(L.rk_npu_attention_f16_cache_create(be.domain, ctypes.byref(cfg), ctypes.byref(cache)), "cache")
    try:
        npu.check(L.rk_npu_attention_f16_cache_reserve(be.ctx, cache, 2048), "reserve")
        rng = np.random.default_rng(8)
        k = rng.standard_normal((kh, length, d)).astype(np.float16)
        v = rng.standard_normal((kh, length, d)).astype(np.float16)
        q = rng.standard_normal((qh, rows, d)).astype(np.float16)
        kd, vd, qd = (torch.from_numpy(a.view(np.int16)).cuda() for a in (k, v, q))
        stream = torch.cuda.current_stream().cuda_stream
        half = length // 2  # two appends
        # (the slices stay referenced until the stream is synchronized: the
        # copies read them asynchronously)
        parts = [(kd[:, :half].contiguous(), vd[:, :half].contiguous()),
                 (kd[:, half:].contiguous(), vd[:, half:].contiguous())]
        for kp, vp in parts:
            npu.check(L.rk_npu_hip_attention_cache_append(cache, kp.data_ptr(), vp.data_ptr(), kp.shape[1], stream),
                      "append")
        out32 = torch.empty((qh, rows, d), dtype=torch.float32, device="cuda")
        out16 = torch.empty((qh, rows, d), dtype=torch.float16, device="cuda")
        pos = length - rows
        npu.check(L.rk_npu_hip_attention_run(ws, cache, qd.data_ptr(), rows, pos, out32.data_ptr(), 0, stream), "run")
        npu.check(L.rk_npu_hip_attention_run(ws, cache, qd.data_ptr(), rows, pos, out16.data_ptr(), 1, stream), "run")
        torch.cuda.synchronize()
        want = oracle.attention(q, k, v, float(np.float32(d ** -0.5)), pos, True)
        close(out32.cpu().numpy(), want)
        assert np.array_equal(out16.cpu().numpy(), out32.cpu().numpy().astype(np.float16))
        # past the capacity: rejected before any copy
        big = torch.zeros((kh, 600, d), dtype=torch.float16, device="cuda")
        assert L.rk_npu_hip_attention_cache_append(cache, big.data_ptr(), big.data_ptr(), 600, stream) == \
            F.RK_NPU_ERR_PARAM
    finally:
        L.rk_npu_attention_f16_cache_free(cache)
        L.rk_npu_attention_f16_workspace_free(ws)


@pytest.mark.parametrize("flag_order", [(1, 0, 1), (0, 1, 0)])
def test_host_transfer_paths_agree(flag_order):
    """Host-buffer appends and runs take the kernel path (pinned stage,
    fetch and copy kernels, polled completion word) when the run's q and
    output each fit 64 KB, or copies with waits (HM_HOST_FLAG=0, larger
    runs, appends: a cache stage and stream against 2-D copies). Alternating
    the two on one cache and workspace gives the same bits, and the oracle's
    result within TOL: 1-row decode steps (16 KB output: kernel path), a
    3-row step (48 KB) and a 5-row step (80 KB: copies either way), 32 query
    heads over 8 KV heads, d = 128, after 300 cached rows."""
    from open_rknpu2_lm_infer_amd import device as D
    qh, kh, d = 32, 8, 128
    scale = d ** -0.5
    results = {}
    for order in (flag_order, tuple(1 - f for f in flag_order)):
        be = npu.Backend(npu.ModelOptions(chunk=128, context=1024))
        att = be.attention(qh, kh, d, scale)
        rng = np.random.default_rng(11)
        k_all = np.zeros((0, kh, d), np.float16)
        v_all = np.zeros((0, kh, d), np.float16)
        pos = 0
        outs = []
        for step, rows in enumerate((128, 128, 44, 1, 1, 3, 5, 1)):
            flag = order[step % len(order)]
            print(f"order={order} step={step} rows={rows} HM_HOST_FLAG={flag}", flush=True)
            q = rng.standard_normal((rows, qh, d)).astype(np.float32)
            k = rng.standard_normal((rows, kh, d)).astype(np.float32)
            v = rng.standard_normal((rows, kh, d)).astype(np.float32)
            out = np.full((rows, qh, d), np.nan, np.float32)
            with D.plan_switch("HM_HOST_FLAG", flag):
                att.run(q, k, v, out, rows, pos)
            k_all = np.concatenate([k_all, k.astype(np.float16)])
            v_all = np.concatenate([v_all, v.astype(np.float16)])
            want = oracle.attention(heads_major(q.astype(np.float16)), heads_major(k_all), heads_major(v_all),
                                    float(np.float32(scale)), pos, True)
            close(heads_major(out), want)
            outs.append(out)
            pos += rows
        assert att.info().length == pos
        results[order] = outs
    a, b = results.values()
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


def test_host_poll_fallback_appends_and_runs():
    """HM_HOST_POLL=0: the append and run calls stop polling their
    completion words early and wait on their streams; decode steps after a
    prefill chunk still match the oracle within TOL."""
    from open_rknpu2_lm_infer_amd import device as D
    be = npu.Backend(npu.ModelOptions(chunk=128, context=512))
    qh, kh, d = 32, 8, 128
    scale = d ** -0.5
    att = be.attention(qh, kh, d, scale)
    with D.plan_switch("HM_HOST_POLL", 0):
        run_sequence(att, qh, kh, d, (100, 1, 1, 2), np.random.default_rng(12), scale)
