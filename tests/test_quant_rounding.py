"""The HIP kernels round the dense rule's scaled activations (half away from
zero, src/npu.rs:1544) as trunc(q + copysign(0x1.fffffep-2, q)) after clamping
q to [-127, 127]. This checks that identity against exact half-away-from-zero
rounding for every float32 in [0, 127] (the negative half follows by symmetry
of round-to-nearest-even and truncation), and the reason 0.5 itself would not
do: 0x1.fffffep-2 + 0.5 rounds up to 1."""
import numpy as np

HALF_BELOW = np.float32(0.49999997)


def test_half_below_is_the_float_before_one_half():
    assert HALF_BELOW == np.nextafter(np.float32(0.5), np.float32(0.0))
    # the naive form fails on exactly this input
    assert np.trunc(HALF_BELOW + np.float32(0.5)) == 1.0
    assert np.trunc(HALF_BELOW + HALF_BELOW) == 0.0


def test_truncated_sum_equals_round_half_away_for_every_float_up_to_127():
    top = int(np.float32(127.0).view(np.uint32))
    step = 1 << 25
    bad = 0
    for start in range(0, top + 1, step):
        q = np.arange(start, min(start + step, top + 1), dtype=np.uint32).view(np.float32)
        got = np.trunc(q + HALF_BELOW)                 # float32 add, round to nearest even
        ref = np.floor(q.astype(np.float64) + 0.5)     # exact half away from zero for q >= 0
        bad += int(np.count_nonzero(got != ref))
    assert bad == 0


def test_negative_side_and_ties_sample():
    rng = np.random.default_rng(7)
    q = np.concatenate([np.arange(-127, 128, dtype=np.float32) + np.float32(0.5),
                        rng.uniform(-127, 127, 1 << 20).astype(np.float32),
                        -np.arange(0, 1 << 16, dtype=np.uint32).view(np.float32)])
    q = np.clip(q, -127, 127).astype(np.float32)
    got = np.trunc(q + np.copysign(HALF_BELOW, q).astype(np.float32))
    ref = np.sign(q) * np.floor(np.abs(q.astype(np.float64)) + 0.5)
    assert np.array_equal(got, ref)
