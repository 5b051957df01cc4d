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


def _passes(a, target, mode):
    return a >= target if mode == "reach" else a > target


def scan(x, tot=0.0, head=256, mode="sum", target=0.0):
    """The kernel's seq_scan: (sum, at). mode "sum" (at = n), or "exceed" /
    "reach": at = the first position whose running sum is > / >= target and
    the sum ends there, else at = n and the sum is the whole one (a NaN sum
    ends a search at once)."""
    x = np.asarray(x, F)
    n, tot, target = len(x), F(tot), F(target)
    find = mode != "sum"

    def serial(t, p):
        for i in range(p, n):
            if find and np.isnan(t):
                break
            t = F(t + x[i])
            if find and _passes(t, target, mode):
                return t, i
        return t, n

    p = 0
    if head and n:
        p = min(n, head)
        t0 = tot
        for i in range(p):
            tot = F(tot + x[i])
        if find and (_passes(tot, target, mode) or np.isnan(tot)):
            t = t0
            for j in range(p):
                t = F(t + x[j])
                if _passes(t, target, mode):
                    return t, j
            return t, n
    if p >= n:
        return tot, n
    if not tot < np.inf:
        return serial(tot, p)
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
            if find:  # the running sums before the first event, exact
                sums = np.ldexp(F(A) + P, E - 23).astype(F)
                g = np.nonzero(_passes(sums, target, mode))[0]
                pa = int(g[0]) if len(g) else 256
                if pa < stop:
                    return F(sums[pa]), p + pa
        if stop:
            A = F(A + P[stop - 1])
        if at >= room:
            return F(np.ldexp(A, E - 23)), n
        s = F(F(np.ldexp(A, E - 23)) + x[p + at])
        if find and _passes(s, target, mode):
            return s, p + at
        p += at + 1
        if not s < np.inf:
            return serial(s, p)
        if p >= n:
            return s, n
        E = _binade(s)
        A = F(np.ldexp(s, 23 - E))


def scan_sum(x, tot=0.0, head=256):
    return scan(x, tot, head)[0]


def seq_sum(x, tot=0.0):
    tot = F(tot)
    for v in np.asarray(x, F):
        tot = F(tot + v)
    return tot


def seq_find(x, tot, target, mode):
    """The reference's running-sum search: the first i whose sum passes."""
    tot, target = F(tot), F(target)
    for i, v in enumerate(np.asarray(x, F)):
        tot = F(tot + v)
        if _passes(tot, target, mode):
            return tot, i
    return tot, len(x)


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


def _probs(rng, n, mode):
    e = _exps(rng, n, mode)
    return (e * F(F(1.0) / seq_sum(e))).astype(F)


@pytest.mark.parametrize("mode", ["normal", "sink", "bimodal", "ties", "tiny", "wide"])
@pytest.mark.parametrize("search", ["exceed", "reach"])
def test_scan_search_equals_sequential_search(mode, search):
    # the sampler's running sums: probabilities in index order (the draw
    # with top_p >= 1) and in descending order (the nucleus cut and the
    # draw inside it), against targets between, on and past the sums
    rng = np.random.default_rng(10 + ["normal", "sink", "bimodal", "ties", "tiny", "wide"].index(mode))
    for n in (1, 7, 255, 256, 257, 700, 2048, 5000):
        for order in ("index", "descending"):
            x = _probs(rng, n, mode)
            if order == "descending":
                x = -np.sort(-x)
            run = np.cumsum(x, dtype=F)  # numpy's float32 cumsum adds in order
            targets = [F(rng.random()), F(0.9), F(0.0), F(-1.0), F(2.0), run[n // 2], run[-1],
                       run[min(n - 1, 300)], np.nextafter(run[n // 3], F(0)), F(np.inf), F(np.nan)]
            for target in targets:
                for head in (256, 0):
                    got = scan(x, 0.0, head, search, target)
                    want = seq_find(x, 0.0, target, search)
                    assert got[1] == want[1] and _same(got[0], want[0]), (mode, n, order, target,
                                                                          head, got, want)
            # continued from a partial sum, as the nucleus's second search is
            k = n // 4
            t0 = seq_sum(x[:k])
            for target in (F(0.9), run[-1], F(rng.random())):
                got = scan(x[k:], t0, 256, search, target)
                want = seq_find(x[k:], t0, target, search)
                assert got[1] == want[1] and _same(got[0], want[0]), (mode, n, target, "cont")


def test_scan_search_on_the_sums_and_nan():
    # a target equal to a running sum: "reach" stops there, "exceed" at the
    # first larger sum; equal terms make long runs of distinct sums
    x = np.full(3000, F(1.0 / 3000), F)
    run = np.cumsum(x, dtype=F)
    for j in (0, 1, 255, 256, 257, 1000, 2047, 2999):
        for head in (256, 0):
            assert scan(x, 0.0, head, "reach", run[j])[1] == seq_find(x, 0.0, run[j], "reach")[1] == j
            want = seq_find(x, 0.0, run[j], "exceed")
            assert scan(x, 0.0, head, "exceed", run[j]) [1] == want[1] > j
    # zero terms: sums that repeat
    x = np.zeros(1000, F)
    x[::7] = F(1e-3)
    for target in (F(0.0), F(1e-3), F(0.05)):
        for search in ("exceed", "reach"):
            for head in (256, 0):
                got, want = scan(x, 0.0, head, search, target), seq_find(x, 0.0, target, search)
                assert got[1] == want[1] and _same(got[0], want[0]), (target, search, head)
    # a NaN term: a crossing before it is found, none after it
    x = np.full(900, F(1e-3), F)
    x[600] = np.nan
    for head in (256, 0):
        assert scan(x, 0.0, head, "exceed", F(0.3))[1] == seq_find(x, 0.0, F(0.3), "exceed")[1]
        got = scan(x, 0.0, head, "exceed", F(0.7))
        assert got[1] == 900 and np.isnan(got[0])
    x[100] = np.nan  # inside the head
    got = scan(x, 0.0, 256, "reach", F(0.05))
    assert got == seq_find(x, 0.0, F(0.05), "reach")
    got = scan(x, 0.0, 256, "reach", F(0.5))
    assert got[1] == 900 and np.isnan(got[0])


# ---------------------------------------------------------------------------
# The sampler's workgroup version (stage_scan_mw, cosxamix_amd/csrc/
# cx_sample.hip): stages of SEG positions; stage 0 (the head) and a sum that
# is not finite go to scan() whole; otherwise up to 16 windows of 256 are
# summed in parallel in units of the binade of the running sum where they
# start, the totals combined in order, and the first window with an event
# (a tie or a term that is not finite, the running sum reaching 2^(E+1), or
# for a search a window-end sum that passes the target) runs through scan()
# alone; the windows after it start again in the new binade.
SEG, WIN = 4096, 256


def _window_total(w, k):
    q = np.ldexp(w.astype(np.float64), k)  # x / u exact in f64
    r = np.rint(q)
    bad = bool(np.any(~(np.abs(q - r) < 0.5)))
    return r.sum(), bad  # exact integers (or inf/NaN with `bad` set)


def stage_scan(v, tot, head, mode, target):
    find = mode != "sum"
    m, nw = len(v), (len(v) + WIN - 1) // WIN
    s, w0 = F(tot), 0
    while w0 < nw:
        if (head and w0 == 0) or not np.isfinite(s):
            t, at = scan(v[WIN * w0:], s, head and w0 == 0, mode, target)
            return t, (WIN * w0 + at if at < m - WIN * w0 else m)
        E = _binade(s)
        k = 23 - E
        A0 = float(np.ldexp(np.float64(s), k))
        cnt = min(nw - w0, SEG // WIN)
        run, j = A0, cnt
        for i in range(cnt):
            N, bad = _window_total(v[WIN * (w0 + i): WIN * (w0 + i + 1)], k)
            end = run + N
            if bad or end >= 2.0 ** 24 or (find and _passes(F(np.ldexp(end, -k)), target, mode)):
                j = i
                break
            run = end
        s = F(np.ldexp(run, -k))
        if j == cnt:
            w0 += cnt
            continue
        lo = WIN * (w0 + j)
        t, at = scan(v[lo: lo + WIN], s, 0, mode, target)
        if find and at < len(v[lo: lo + WIN]):
            return t, lo + at
        s, w0 = t, w0 + j + 1
    return s, m


def chain(x, tot=0.0, mode="sum", target=0.0):
    x = np.asarray(x, F)
    s = F(tot)
    for b in range(0, len(x), SEG):
        s, at = stage_scan(x[b: b + SEG], s, b == 0, mode, F(target))
        if at < len(x[b: b + SEG]):
            return s, b + at
    return s, len(x)


@pytest.mark.parametrize("mode", ["normal", "sink", "bimodal", "ties", "tiny", "wide"])
def test_workgroup_stage_scan_equals_sequential(mode):
    rng = np.random.default_rng(40 + ["normal", "sink", "bimodal", "ties", "tiny", "wide"].index(mode))
    for n in (1, 300, 4096, 4097, 9000, 20000):
        x = _exps(rng, n, mode)
        assert _same(chain(x)[0], seq_sum(x)), (mode, n)
        p = (x * F(F(1.0) / seq_sum(x))).astype(F)
        for order in ("index", "descending"):
            y = -np.sort(-p) if order == "descending" else p
            run = np.cumsum(y, dtype=F)
            for target in (F(rng.random()), F(0.9), run[n // 2], run[min(n - 1, 5000)],
                           np.nextafter(run[n // 3], F(0)), F(2.0), F(np.nan)):
                for search in ("exceed", "reach"):
                    got, want = chain(y, 0.0, search, target), seq_find(y, 0.0, target, search)
                    assert got[1] == want[1] and _same(got[0], want[0]), (mode, n, order, target,
                                                                          search, got, want)


def test_workgroup_stage_scan_events_inside_a_stage():
    # every term 1 from 4096: the sum crosses 2^13 and 2^14 inside stages;
    # halfway terms after the head; a NaN in the third stage
    x = np.ones(20000, F)
    assert chain(x)[0] == seq_sum(x)
    u = F(np.ldexp(F(1.0), _binade(F(4096.0)) - 23))
    y = np.ones(12000, F)
    y[5000:5100] = u * F(0.5)
    y[7001] = u * F(1.5)
    assert _same(chain(y)[0], seq_sum(y))
    y[9000] = np.nan
    assert np.isnan(chain(y)[0]) and np.isnan(seq_sum(y))
    run = np.cumsum(y[:8999], dtype=F)
    # (the halfway terms at 5000.. leave the sum where it is: ties to even)
    for j in (4096, 4097, 5050, 7001, 8191, 8192, 8998):
        for search in ("reach", "exceed"):
            got, want = chain(y, 0.0, search, run[j]), seq_find(y, 0.0, run[j], search)
            assert got[1] == want[1] and _same(got[0], want[0]), (j, search)
