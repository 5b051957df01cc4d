"""The softmax sum's binade scan (seq_sum_scan, cosxamix_amd/csrc/cx_ops.hip),
modelled on the CPU with numpy float32 and checked bit for bit against the
reference's sequential sum (`tot += e`, src/ops.rs:1221-1225).

The model follows the kernel step by step: the first `head` terms added one
by one, then windows of 256 positions in which the terms, rounded to the
running sum's unit u = 2^(E-23), are prefix-summed as integers; the first
position whose sum reaches 2^(E+1), or whose x / u is exactly halfway (or
not finite), is added as one f32 add and the next window starts after it.
The GPU kernel itself is checked against the oracle in
tests/test_gpu_kernels.py (test_decode_attention_sum_edge_cases and the
attention path tests); this file pins the algorithm, including the cases a
seeded GPU run meets rarely (ties, subnormal starts, long runs in one
binade).
"""
import numpy as np
import pytest

F = np.float32


def _binade(s):
    e = int((np.array([s], F).view(np.uint32)[0] >> 23) & 0xFF)
    return max(e, 1) - 127


def scan_sum(x, tot=0.0, head=256):
    x = np.asarray(x, F)
    n, tot = len(x), F(tot)
    p = min(n, head)
    for i in range(p):
        tot = F(tot + x[i])
    if p >= n:
        return tot
    E = _binade(tot)
    A = F(np.ldexp(tot, 23 - E))
    while True:
        w = x[p:p + 256]
        with np.errstate(over="ignore", invalid="ignore"):
            q = np.ldexp(w, 23 - E).astype(F)
            r = np.rint(q)
            half = ~(np.abs(q - r) < 0.5)
        P = np.cumsum(r, dtype=F)
        H = F(F(16777216.0) - A)
        ev = np.nonzero(half | (P >= H))[0]
        at = int(ev[0]) if len(ev) else 256
        room = n - p
        stop = min(at, room)
        if stop:
            A = F(A + P[stop - 1])
        if at >= room:
            return F(np.ldexp(A, E - 23))
        s = F(F(np.ldexp(A, E - 23)) + x[p + at])
        p += at + 1
        if not np.isfinite(s):
            for i in range(p, n):
                s = F(s + x[i])
            return s
        if p >= n:
            return s
        E = _binade(s)
        A = F(np.ldexp(s, 23 - E))


def seq_sum(x, tot=0.0):
    tot = F(tot)
    for v in np.asarray(x, F):
        tot = F(tot + v)
    return tot


def _exps(rng, n, mode):
    z = rng.normal(0, 1, n)
    if mode == "sink":
        z[0] = 10
    elif mode == "bimodal":
        z = np.where(rng.random(n) < 0.5, -30, 0) + rng.normal(0, 1, n)
    elif mode == "ties":
        z = np.floor(rng.normal(0, 4, n))
    elif mode == "tiny":
        z = -100 * rng.random(n)
    elif mode == "wide":
        z = rng.normal(0, 40, n)
    s = z.astype(F)
    return np.exp((s - s.max()).astype(F)).astype(F)


def _same(a, b):
    return (np.isnan(a) and np.isnan(b)) or np.array([a], F).view(np.uint32)[0] == np.array(
        [b], F).view(np.uint32)[0]


@pytest.mark.parametrize("mode", ["normal", "sink", "bimodal", "ties", "tiny", "wide"])
def test_scan_sum_equals_sequential_sum(mode):
    rng = np.random.default_rng(["normal", "sink", "bimodal", "ties", "tiny", "wide"].index(mode))
    for n in (1, 5, 63, 255, 256, 257, 300, 548, 1000, 2047, 4096, 8448):
        for head in (256, 64, 0):
            x = _exps(rng, n, mode)
            assert _same(scan_sum(x, 0.0, head), seq_sum(x)), (mode, n, head)
            # from a nonzero start (the kernel's later stages and calls)
            t0 = seq_sum(x[: n // 3])
            assert _same(scan_sum(x[n // 3:], t0, 0), seq_sum(x)), (mode, n, "split")


def test_scan_sum_binade_edges_and_nan():
    # every term 1: the sum lands exactly on each power of two
    x = np.ones(5000, F)
    assert scan_sum(x, 0.0, 0) == F(5000)
    # halfway terms (x / u = k + 1/2 for the running sum's unit u) from odd
    # and even multiples of u: the tie goes to the even sum, which
    # round-half-even of x / u alone gets wrong from an odd one
    for base in (F(1.0), F(3.0), F(1024.0), F(2.0 ** -130)):
        u = F(np.ldexp(F(1.0), _binade(base) - 23))
        for start in (base, F(base + u)):
            for pattern in ((1.5, 0.5, 0.5), (0.5, 1.5), (2.5,)):
                x = np.resize(np.array([u * k for k in pattern], F), 700)
                assert _same(scan_sum(x, start, 0), seq_sum(x, start)), (base, start, pattern)
    # subnormal terms from a zero start, then a jump past 2^-125
    x = np.full(600, np.ldexp(F(1.0), -149), F)
    x[400] = F(1e-30)
    assert _same(scan_sum(x, 0.0, 0), seq_sum(x))
    # a NaN term: NaN from it on
    x = np.ones(900, F)
    x[700] = np.nan
    assert np.isnan(scan_sum(x, 0.0, 0)) and np.isnan(seq_sum(x))
