"""A CPU model of the GPU's exact rmsnorm factor (cx_rms_slack,
cx_rms_unsure in cosxamix_amd/csrc/cx_act.h): the bound on the distance
between the workgroup trees' f64 sum of squares and the reference's sum in
order (src/kernels/scalar.rs:47) holds, and wherever the two sums give a
different f32 output the check asks for the sum in order. The trees are
restated in tests/rms_fixtures.py."""
import math

import numpy as np
import pytest

import rms_fixtures as R

U = 2.0 ** -53


def reach_of(x, tot, depth, group):
    """cx_rms_reach with the device's group bound: W' = sum over groups of
    `group` consecutive values (per lane: 8 for the fused prologues, 4 for
    cx_rms_scale) of the group's sum times (n - its first index)."""
    t = x.astype(np.float64) ** 2
    n = x.size
    g = t.reshape(-1, group).sum(axis=1)
    w = float(np.sum(g * (n - group * np.arange(g.size))))
    if not 0 < tot < math.inf:
        return 0, w
    q = min(w / tot, n) if 1e-30 < tot < 1e30 else n
    return int(0.52 * (q + depth)) + 20, w


def risk(v, reach):
    """cx_rms_risk on f64 products v: a product's low 29 mantissa bits
    within reach of 2^28, or 0 < |v| < 2^-126."""
    v = np.asarray(v, np.float64)
    lo = (v.view(np.uint64) & np.uint64(0x1FFFFFFF)).astype(np.int64)
    mid = np.abs(lo - (1 << 28)) <= reach
    tiny = (np.abs(v) < 2.0 ** -126) & (v != 0)
    return bool(np.any(mid | tiny))


def unsure(x, scale, reach):
    return reach > 0 and risk(x.astype(np.float64) * scale, reach)


def _vectors():
    rng = np.random.default_rng(11)
    for n in (896, 2048, 4096):
        for i in range(40):
            kind = i % 4
            if kind == 0:
                x = rng.normal(0, 1, n)
            elif kind == 1:  # a residual stream: small values, a few large
                x = rng.normal(0, 0.02, n)
                x[rng.integers(0, n, 4)] *= 300
            elif kind == 2:  # wide dynamic range
                x = rng.normal(0, 1, n) * np.exp(rng.normal(0, 4, n))
            else:  # values on a coarse grid: many ties in the adds
                x = rng.integers(-64, 64, n) / 8.0
            yield x.astype(np.float32)
        for seed in range(4):
            yield R.splitting_vector(n, seed)[0]


@pytest.mark.parametrize("tree", ["tree8", "tree4"])
def test_the_bound_holds_and_the_check_catches_every_split(tree):
    split = 0
    for x in _vectors():
        n = x.size
        s_seq, s_tree = R.seq_sum(x), R.TREES[tree](x)
        group = 8 if tree == "tree8" else 4
        depth = (n + 2047) // 2048 * 8 + 16 if tree == "tree8" else (n + 1023) // 1024 * 4 + 16
        reach, w = reach_of(x, s_tree, depth, group)
        # the sums' distance is within the bound the reach is made from
        assert abs(s_seq - s_tree) <= U * (w + depth * s_tree) * 1.000001, (n, s_seq, s_tree)
        sc_t, sc_s = R.factor(s_tree, n, 1e-6), R.factor(s_seq, n, 1e-6)
        differs = not np.array_equal(np.float32(x.astype(np.float64) * sc_t),
                                     np.float32(x.astype(np.float64) * sc_s))
        split += differs
        if differs:
            assert unsure(x, sc_t, reach), n
    assert split >= 12  # the constructed vectors, at least


def test_the_check_reads_midpoints_and_tiny_values():
    """The bit test on known products: exactly on an f32 rounding midpoint
    (1 + 2^-24, halfway between 1 and the next f32), a few f64 ulps either
    side, far from it, an f32 value itself, zero and an f32 subnormal."""
    mid = np.array([1.0 + 2.0 ** -24]).view(np.uint64)
    def at(d):
        return (mid.astype(np.int64) + d).astype(np.uint64).view(np.float64)
    assert risk(at(0), 8) and risk(at(5), 8) and risk(at(-5), 8)
    assert not risk(at(9), 8) and not risk(at(-9), 8) and not risk(at(1 << 20), 8)
    assert not risk([1.0, 3.0, -2.5], 8) and not risk([0.0, -0.0], 8)
    assert risk([1e-39], 8) and risk([-3e-40], 8)
    # a midpoint below a power of two (the f32 below 2 and 2 itself)
    assert risk([2.0 - 2.0 ** -24], 8)
