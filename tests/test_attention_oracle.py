"""CPU checks of the attention oracle and of the device-free attention calls.

The reference binds a closed native attention library, so there are no golden
vectors for this path: the oracle (oracle.attention) is pinned here by brute
force on tiny inputs and by properties the mathematics fixes — one visible key
returns its value row, equal value rows return that row, keys permuted with
their values change nothing without a mask, a zero scale averages the visible
value rows, and the causal mask at the last position equals no mask."""
import ctypes

import numpy as np
import pytest

from oracle import oracle
from open_rknpu2_lm_infer_amd import _ffi as F
from open_rknpu2_lm_infer_amd import npu


def _rand(rng, *shape):
    return rng.standard_normal(shape).astype(np.float16)


def _brute(q, k, v, scale, position, causal):
    qh, rows, d = q.shape
    kh, length, _ = k.shape
    out = np.zeros((qh, rows, d))
    for h in range(qh):
        g = h // (qh // kh)
        for r in range(rows):
            keys = range(min(length, position + r + 1)) if causal else range(length)
            s = [scale * float(np.dot(q[h, r].astype(np.float64), k[g, j].astype(np.float64))) for j in keys]
            mx = max(s)
            w = [np.exp(x - mx) for x in s]
            out[h, r] = sum(wj * v[g, j].astype(np.float64) for wj, j in zip(w, keys)) / sum(w)
    return out


@pytest.mark.parametrize("causal", [True, False])
def test_oracle_matches_brute_force(causal):
    rng = np.random.default_rng(1)
    q, k, v = _rand(rng, 6, 3, 32), _rand(rng, 2, 9, 32), _rand(rng, 2, 9, 32)
    got = oracle.attention(q, k, v, 0.2, 6, causal)
    assert np.allclose(got, _brute(q, k, v, 0.2, 6, causal), rtol=1e-12, atol=1e-12)


def test_oracle_invariants():
    rng = np.random.default_rng(2)
    q, k, v = _rand(rng, 4, 5, 64), _rand(rng, 2, 12, 64), _rand(rng, 2, 12, 64)
    # the first row at position 0 sees key 0 only
    out = oracle.attention(q, k, v, 0.125, 0, True)
    assert np.allclose(out[:, 0], np.repeat(v[:, 0].astype(np.float64), 2, axis=0))
    # equal value rows
    vv = np.repeat(v[:, :1], 12, axis=1)
    out = oracle.attention(q, k, vv, 0.125, 7, False)
    assert np.allclose(out, np.repeat(vv[:, :1].astype(np.float64), 2, axis=0).repeat(5, axis=1))
    # key order does not matter without a mask
    perm = rng.permutation(12)
    a = oracle.attention(q, k, v, 0.125, 0, False)
    b = oracle.attention(q, k[:, perm], v[:, perm], 0.125, 0, False)
    assert np.allclose(a, b, rtol=1e-12, atol=1e-12)
    # zero scale: mean of the visible value rows
    out = oracle.attention(q, k, v, 0.0, 3, True)
    for r in range(5):
        assert np.allclose(out[:, r], np.repeat(v[:, :4 + r].astype(np.float64).mean(axis=1), 2, axis=0))
    # causal rows past the last key see everything, as without a mask
    a = oracle.attention(q[:, :1], k, v, 0.3, 11, True)
    b = oracle.attention(q[:, :1], k, v, 0.3, 0, False)
    assert np.allclose(a, b, rtol=1e-12, atol=1e-12)


def test_config_defaults_and_query():
    L = F.lib()
    cfg = F.rk_npu_attention_f16_config()
    L.rk_npu_attention_f16_config_init(ctypes.byref(cfg))
    assert (cfg.query_heads, cfg.kv_heads, cfg.head_dim) == (32, 8, 128)
    assert cfg.flags == F.RK_NPU_ATTENTION_F16_STABLE_SOFTMAX and cfg.mask_mode == F.RK_NPU_ATTENTION_F16_CAUSAL
    sizes = F.rk_npu_attention_f16_sizes()
    assert L.rk_npu_attention_f16_query(ctypes.byref(cfg), 100, 4, 100, ctypes.byref(sizes)) == 0
    assert sizes.key_bytes == sizes.value_bytes == 8 * 128 * 128 * 2  # capacity rounded up to 128
    # the reference's geometry checks (src/npu.rs:714-728)
    for field, value in (("kv_heads", 0), ("kv_heads", 33), ("query_heads", 12), ("head_dim", 100),
                         ("softmax_scale", 0.0), ("softmax_scale", float("inf")), ("max_query_rows", 0)):
        bad = F.rk_npu_attention_f16_config()
        L.rk_npu_attention_f16_config_init(ctypes.byref(bad))
        setattr(bad, field, value)
        assert L.rk_npu_attention_f16_query(ctypes.byref(bad), 64, 1, 64, ctypes.byref(sizes)) == F.RK_NPU_ERR_PARAM


def test_cache_bytes_mirror_reference_formula():
    """src/npu.rs:442-466: K + V + tail bytes of a max-capacity cache."""
    opts = npu.ModelOptions(chunk=64, context=1000)
    got = npu.Backend.attention_cache_bytes(opts, 16, 4, 64, 0.125)
    assert got == 2 * 4 * 1024 * 64 * 2
