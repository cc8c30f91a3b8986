"""Pins of the MoE oracle (oracle.moe / orc_moe) to what the reference's own
code and the mathematics fix, instead of to a restatement of its formula.

- Composition: the reference's paged expert path runs every assignment with a
  nonzero route as its own top=1 call with route 1.0 (src/model/experts/
  paged.rs:590-641: one row per job, `self.routes.resize(group.len(), 1.)`)
  and then reduces in rank order with a single-rounding fma, skipping routes
  <= 0 (paged.rs:494-507). The resident oracle must equal that composition of
  its own top=1 calls for every row, including repeated experts, zero and
  negative routes.
- The top=1 unit: quant_moe of the token row (its rounding pinned in
  test_oracle.py against an independent restatement), exact int32 products,
  dequant as two f32 multiplies, SwiGLU, quant_moe of the middle row, exact
  products, dequant (MOE_CPU_FUSION_20261023.md:12-13: one requant per
  (token, expert) middle row); an output is contrib * 1.0 + 0.
- Invariants: a row permutation permutes the output; a zero or negative
  route contributes nothing whatever its valid expert id; an expert repeated
  at ranks a < b contributes fma(c, r_b, fma(c, r_a, 0)); the shared expert is
  added after the routed sum (test_oracle.py).
The quant_moe tie rule itself (half to even) rests on the reference's
documents (MOE_CPU_FUSION_20261023.md:13); no reference artefact fixes its
bits, so that part stays restated, not pinned."""
import numpy as np
import pytest

from oracle import oracle
from tests import refdata as R
from tests.test_oracle import fma_f32

F32 = np.float32


def bank(h, inter, experts, tag, down_bits=8):
    gate = [R.weights(6, f"{tag}g{e}", 4, h, 2 * inter) for e in range(experts)]
    down = [R.weights(6, f"{tag}d{e}", down_bits, inter, h) for e in range(experts)]
    return gate, down


def paged_composition(gate, down, x, ids, routes):
    """src/model/experts/paged.rs:494-507 over top=1, route 1.0 calls."""
    rows, top = ids.shape
    h = x.shape[1]
    contributions = {}
    for a in range(rows * top):
        r, rank = divmod(a, top)
        if routes[r, rank] != 0.0:  # paged.rs:594-596: a job per nonzero route
            contributions[a] = oracle.moe(gate, down, x[r:r + 1], ids[r:r + 1, rank:rank + 1],
                                          np.ones((1, 1), F32))[0]
    out = np.zeros((rows, h), F32)
    for r in range(rows):
        s = np.zeros(h, F32)
        for rank in range(top):
            a = r * top + rank
            if routes[r, rank] > 0.0:  # paged.rs:500
                c = contributions[a]
                # fma(c, route, s) in f32, vectorised exactly: the f64 product of two
                # f32 values is exact, and the f64 sum is checked against the
                # single-rounding reference on any element where double rounding
                # could matter
                s = fma_vec(c, routes[r, rank], s)
        out[r] = s
    return out


def fma_vec(c, w, s):
    exact = c.astype(np.float64) * np.float64(w) + s.astype(np.float64)
    out = exact.astype(F32)
    # an f64 sum of two f32 terms can round twice; redo the close calls exactly
    err = np.abs(exact - out.astype(np.float64))
    ulp = np.abs(np.spacing(out)).astype(np.float64)
    for i in np.nonzero(err > 0.49 * ulp)[0]:
        out[i] = fma_f32(c[i], w, s[i])
    return out


def test_fma_vec_matches_single_rounding():
    g = np.random.default_rng(3)
    c = g.standard_normal(2000).astype(F32)
    s = g.standard_normal(2000).astype(F32)
    w = F32(0.37)
    got = fma_vec(c, w, s)
    for i in range(0, 2000, 7):
        assert got[i] == fma_f32(c[i], w, s[i])


def test_resident_moe_equals_paged_top1_composition():
    h, inter, experts, top, rows = 64, 32, 6, 4, 9
    gate, down = bank(h, inter, experts, "pc")
    x = R.activations(6, "pc-x", rows, h)
    g = np.random.default_rng(11)
    ids = np.stack([g.choice(experts, size=top, replace=False) for _ in range(rows)]).astype(np.int32)
    routes = g.dirichlet(np.ones(top), size=rows).astype(F32)
    # edge rows: repeated expert, zero and negative routes, all routes skipped
    ids[1] = [2, 2, 5, 2]
    routes[1] = [0.4, 0.3, 0.0, 0.3]
    routes[2] = [0.5, -0.25, 0.75, 0.0]
    routes[3] = [0.0, 0.0, 0.0, 0.0]
    routes[4] = [-0.0, 0.5, 0.5, 0.0]
    got = oracle.moe(gate, down, x, ids, routes)
    want = paged_composition(gate, down, x, ids, routes)
    assert np.array_equal(got, want)
    assert np.all(got[3] == 0.0)


def test_top1_unit_is_the_expert_ffn_of_pinned_parts():
    h, inter, experts = 48, 40, 3
    gate, down = bank(h, inter, experts, "unit", down_bits=4)
    x = R.activations(6, "unit-x", 5, h)
    x[2] = 0.0  # zero row: scale 1, zero codes
    qx, sx = oracle.quant_moe(x)
    for e in range(experts):
        for r in range(x.shape[0]):
            got = oracle.moe(gate, down, x[r:r + 1], np.array([[e]], np.int32), np.ones((1, 1), F32))[0]
            gc, gs = gate[e]
            dc, ds = down[e]
            y = (oracle.gemm_i8(qx[r:r + 1], gc)[0].astype(F32) * sx[r]).astype(F32) * gs
            mid = oracle.swiglu(y[:inter], y[inter:])
            qm, sm = oracle.quant_moe(mid[None, :])
            contrib = (oracle.gemm_i8(qm, dc)[0].astype(F32) * sm[0]).astype(F32) * ds
            # route 1.0 into a zero sum: contrib * 1 + 0 (which turns -0 into +0)
            assert np.array_equal(got, contrib + F32(0.0)), (e, r)


def test_row_permutation_permutes_the_output():
    h, inter, experts, top, rows = 64, 32, 5, 3, 7
    gate, down = bank(h, inter, experts, "perm")
    x = R.activations(6, "perm-x", rows, h)
    g = np.random.default_rng(5)
    ids = g.integers(0, experts, size=(rows, top)).astype(np.int32)
    routes = g.uniform(-0.2, 1.0, size=(rows, top)).astype(F32)
    base = oracle.moe(gate, down, x, ids, routes)
    p = g.permutation(rows)
    assert np.array_equal(oracle.moe(gate, down, x[p], ids[p], routes[p]), base[p])


@pytest.mark.parametrize("skipped", [0.0, -0.0, -0.5])
def test_skipped_route_contributes_nothing_whatever_its_expert(skipped):
    h, inter, experts, top = 64, 32, 5, 3
    gate, down = bank(h, inter, experts, "skip")
    x = R.activations(6, "skip-x", 2, h)
    ids = np.array([[0, 1, 2], [3, 4, 0]], np.int32)
    routes = np.array([[0.5, skipped, 0.5], [skipped, 0.25, 0.75]], F32)
    base = oracle.moe(gate, down, x, ids, routes)
    for e in range(experts):
        ids2 = ids.copy()
        ids2[0, 1] = e
        ids2[1, 0] = e
        assert np.array_equal(oracle.moe(gate, down, x, ids2, routes), base)


def test_repeated_expert_accumulates_by_nested_fma():
    h, inter, experts = 64, 32, 4
    gate, down = bank(h, inter, experts, "rep")
    x = R.activations(6, "rep-x", 1, h)
    ra, rb = F32(0.3), F32(0.7)
    c = oracle.moe(gate, down, x, np.array([[3]], np.int32), np.ones((1, 1), F32))[0]
    got = oracle.moe(gate, down, x, np.array([[3, 3]], np.int32), np.array([[ra, rb]], F32))[0]
    want = np.array([fma_f32(ci, rb, fma_f32(ci, ra, F32(0.0))) for ci in c], F32)
    assert np.array_equal(got, want)
    # rank order matters only through the fma order
    got_swapped = oracle.moe(gate, down, x, np.array([[3, 3]], np.int32), np.array([[rb, ra]], F32))[0]
    want_swapped = np.array([fma_f32(ci, ra, fma_f32(ci, rb, F32(0.0))) for ci in c], F32)
    assert np.array_equal(got_swapped, want_swapped)
