"""Vectors on which the workgroup trees' f64 sum of squares and the
reference's sum in order (src/kernels/scalar.rs:47) give rmsnorm outputs
that differ in an f32: the cases the GPU's exactness check
(cx_rms_slack / cx_rms_seq_sum) exists for. Built on the CPU from the
trees' definitions; shared by the GPU tests, not a test module."""
import math

import numpy as np


def seq_sum(x):
    """The reference's f64 sum of squares, in order from 0."""
    s = 0.0
    for v in np.asarray(x, np.float32).tolist():
        s += v * v
    return s


def _pairwise(v):
    """A wave's xor butterfly over 64 lane sums (cx_wave_sum_d): the
    balanced pairwise tree in lane order."""
    v = np.asarray(v, np.float64)
    while v.size > 1:
        v = v[0::2] + v[1::2]
    return float(v[0])


def _waves(lanes):
    """256 lane sums: each wave's tree, then ((w0 + w1) + w2) + w3."""
    w = [_pairwise(lanes[64 * i:64 * (i + 1)]) for i in range(4)]
    return ((w[0] + w[1]) + w[2]) + w[3]


def tree8_sum(x):
    """The fused GEMV prologues' tree (k_gemv, k_gemv_row_norm, k_gemv_glu,
    k_gemv_row_glu, k_gemv32): lane l sums x[8l + 2048j + e]^2 over j then
    e, in order from 0; then the waves."""
    t = np.asarray(x, np.float32).astype(np.float64) ** 2
    n = t.size
    lanes = np.zeros(256)
    for j in range(0, n, 2048):
        for e in range(8):
            idx = j + 8 * np.arange(256) + e
            ok = idx < n
            lanes[ok] = lanes[ok] + t[idx[ok]]
    return _waves(lanes)


def tree4_sum(x):
    """cx_rms_scale's tree (k_rmsnorm, k_norm_quant, k_norm_rows,
    k_norm_quant_gemm): lane l sums x[4l + 1024j + e]^2 over j then e."""
    t = np.asarray(x, np.float32).astype(np.float64) ** 2
    n = t.size
    lanes = np.zeros(256)
    for j in range(0, n, 1024):
        for e in range(4):
            idx = j + 4 * np.arange(256) + e
            ok = idx < n
            lanes[ok] = lanes[ok] + t[idx[ok]]
    return _waves(lanes)


TREES = {"tree8": tree8_sum, "tree4": tree4_sum}


def factor(s, n, eps):
    """1 / sqrt(sum / n + eps) in f64 (src/kernels/scalar.rs:48)."""
    return 1.0 / math.sqrt(s / n + float(np.float32(eps)))


def f32_of(a, scale):
    """(a as f64 * scale) as f32."""
    return np.float32(float(np.float32(a)) * scale)


def splitting_vector(n, seed, trees=("tree8", "tree4"), eps=1e-6, j=None, tries=3000):
    """x (float32[n], N(0, 1)) whose element j -- the largest magnitude of
    its 32-value sub-block, so that it is the sub-block's amax and a change
    of its f32 changes the quantized activation's scale -- normalizes to
    one f32 with the sum in order and to another with each named tree's
    sum. Two more elements of that sub-block are tuned for it: a coarse one
    that brings the sum near the value that puts x_j * scale on an f32
    rounding midpoint, and a fine one of ~2^-8 whose f32 steps move the
    sum by a few of its ulps. Returns (x, j)."""
    rng = np.random.default_rng(seed)
    j = n - 1 if j is None else j
    sb = j // 32 * 32
    c, f = sb + (j - sb + 1) % 32, sb + (j - sb + 2) % 32
    e32 = float(np.float32(eps))
    for attempt in range(64):
        x = rng.normal(0, 1, n).astype(np.float32)
        x[j] = np.float32(4.5 + rng.random())
        x[f] = np.float32(2.0 ** -8)
        xj = float(x[j])
        s0 = seq_sum(x)
        y = xj * factor(s0, n, eps)
        lo = np.float32(y)
        hi = np.nextafter(lo, np.float32(np.inf) if y > float(lo) else np.float32(-np.inf))
        mid = (float(lo) + float(hi)) / 2
        target = n * ((xj / mid) ** 2 - e32)
        need = float(x[c]) ** 2 + (target - s0)  # x_c^2 that puts the sum on target
        if not 0.01 < need < 16.0:
            continue
        x[c] = np.float32(math.sqrt(need))
        s1 = seq_sum(x)
        fine = float(x[f]) ** 2 + (target - s1)
        if fine <= 0:
            continue
        base = np.float32(math.sqrt(fine))
        up, down = base, base
        for step in range(tries):
            if step % 2 == 0:
                v, up = up, np.nextafter(up, np.float32(np.inf))
            else:
                down = np.nextafter(down, np.float32(-np.inf))
                v = down
            x[f] = v
            want = f32_of(xj, factor(seq_sum(x), n, eps))
            if all(f32_of(xj, factor(TREES[t](x), n, eps)) != want for t in trees):
                assert np.argmax(np.abs(x[sb:sb + 32])) == j - sb
                return x.copy(), j
    raise RuntimeError("no splitting vector found")
