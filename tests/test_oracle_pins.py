"""Closed-form pins for the oracle functions that the reference's own
compiled kernels and known answers leave open: the RoPE rotation direction,
the attention scale, Azar's seeds and Box-Muller normals, the Q6_K byte
layout and the bytes of the k-quant quantizers (CPU only).

Every expected value here comes from outside the oracle: float64
mathematics, the published FNV-1a test vectors, the byte table the
reference documents for Q6_K (src/kernels/scalar.rs:276-291), or integer
block designs whose bytes follow from the format alone. Each check is chosen
so that a plausible slip (a flipped sign, a dropped scale, swapped outputs,
a permuted group, a misplaced bit) fails it; tests/test_oracle_mutants.py
compiles such slips into copies of the oracle and shows that they do.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

M64 = (1 << 64) - 1
FNV_PRIME = 0x100000001B3
TAU32 = np.float32(6.283185307179586)  # std::f32::consts::TAU


# ------------------------------------------------------------------ RoPE
@pytest.mark.parametrize("base", [10000.0, 1e6])
@pytest.mark.parametrize("pos", [1, 2, 7, 100])
def test_rope_one_hot_rotation_direction(base, pos):
    """src/ops.rs:1185-1189: value i turns against i + d/2 by +angle:
    [1,0,0,0] -> [cos, 0, sin, 0] and [0,0,1,0] -> [-sin, 0, cos, 0]."""
    hd = 4
    c, s = O.rope_tables(hd, base, pos + 1)
    c0, s0 = float(c[pos * 2]), float(s[pos * 2])
    c1, s1 = float(c[pos * 2 + 1]), float(s[pos * 2 + 1])
    # pair 0 turns by pos radians (its frequency is base^0 = 1), pair 1 by
    # pos / sqrt(base)
    assert abs(c0 - math.cos(pos)) < 2e-7 and abs(s0 - math.sin(pos)) < 2e-7
    a1 = pos / math.sqrt(base)
    assert abs(c1 - math.cos(a1)) < 2e-7 and abs(s1 - math.sin(a1)) < 2e-7
    cases = {(1, 0, 0, 0): (c0, 0, s0, 0), (0, 0, 1, 0): (-s0, 0, c0, 0),
             (0, 1, 0, 0): (0, c1, 0, s1), (0, 0, 0, 1): (0, -s1, 0, c1)}
    for x, want in cases.items():
        got = O.rope(np.array(x, np.float32), 1, 1, hd, c, s, pos)
        assert got.tolist() == [np.float32(w) for w in want], (x, got, want)


def test_rope_matches_the_float64_rotation():
    heads, hd, tokens, pos, base = 3, 8, 2, 5, 10000.0
    c, s = O.rope_tables(hd, base, 16)
    x = np.random.default_rng(3).normal(0, 1, tokens * heads * hd).astype(np.float32)
    got = O.rope(x, tokens, heads, hd, c, s, pos).reshape(tokens, heads, hd)
    half = hd // 2
    for t in range(tokens):
        ang = (pos + t) * base ** (-2.0 * np.arange(half) / hd)
        for h in range(heads):
            a = x.reshape(tokens, heads, hd)[t, h, :half].astype(np.float64)
            b = x.reshape(tokens, heads, hd)[t, h, half:].astype(np.float64)
            want = np.concatenate([a * np.cos(ang) - b * np.sin(ang),
                                   a * np.sin(ang) + b * np.cos(ang)])
            assert np.allclose(got[t, h], want, atol=2e-6), (t, h)


# ------------------------------------------------------------- attention
def _attention64(q, k, v, tokens, total, heads, kvh, hd):
    q = q.astype(np.float64).reshape(tokens, heads, hd)
    k = k.astype(np.float64).reshape(total, kvh, hd)
    v = v.astype(np.float64).reshape(total, kvh, hd)
    out = np.zeros((tokens, heads, hd))
    for t in range(tokens):
        vis = total - tokens + t + 1
        for h in range(heads):
            g = h // (heads // kvh)
            sc = k[:vis, g] @ q[t, h] / math.sqrt(hd)
            p = np.exp(sc - sc.max())
            out[t, h] = (p / p.sum()) @ v[:vis, g]
    return out.ravel()


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("tokens,total", [(1, 2), (1, 3), (2, 3)])
def test_attention_matches_scaled_softmax_closed_form(hd, tokens, total):
    """src/ops.rs:1287: score = q.k * (1/sqrt(head_dim)); causal softmax over
    the visible positions; out = sum_p prob_p v_p. The q.k values are O(10)
    so that any other scale changes the weights."""
    heads, kvh = 4, 2
    rng = np.random.default_rng(hd + 7 * total + tokens)
    q = rng.normal(0, 1, tokens * heads * hd).astype(np.float32)
    k = rng.normal(0, 1, total * kvh * hd).astype(np.float32)
    v = rng.normal(0, 1, total * kvh * hd).astype(np.float32)
    got = O.attention(q, k, v, tokens, total, heads, kvh, hd)
    want = _attention64(q, k, v, tokens, total, heads, kvh, hd)
    assert np.allclose(got, want, rtol=1e-5, atol=2e-6)


# ------------------------------------------------------ Azar / semilla_de
def test_seed_of_is_fnv1a_then_row_then_model():
    """src/daiss.rs:364-379. The name hash is FNV-1a 64 (published vectors:
    "" -> cbf29ce484222325, "a" -> af63dc4c8601ec8c, "foobar" ->
    85944171f73967e8); then the row is xored in and multiplied by the FNV
    prime, and the model seed rotated left by 17 is xored last."""
    for name, h in (("", 0xCBF29CE484222325), ("a", 0xAF63DC4C8601EC8C),
                    ("foobar", 0x85944171F73967E8)):
        assert O.seed_of(0, name, 0) == (h * FNV_PRIME) & M64
    h = 0xAF63DC4C8601EC8C
    assert O.seed_of(0, "a", 5) == ((h ^ 5) * FNV_PRIME) & M64
    model = 0x8000000000000003
    rot = ((model << 17) | (model >> 47)) & M64
    assert O.seed_of(model, "a", 5) == (((h ^ 5) * FNV_PRIME) & M64) ^ rot


def _xorshift(seed):
    s = seed or 0x9E3779B97F4A7C15
    while True:
        s ^= s >> 12
        s ^= (s << 25) & M64
        s ^= s >> 27
        yield (s * 0x2545F4914F6CDD1D) & M64


@pytest.mark.parametrize("model,name,row", [(0, "blk.0.attn_q.weight", 3), (42, "token_embd.weight", 0),
                                            (7, "output.weight", 151935)])
def test_normals_are_box_muller_on_the_exact_uniforms(model, name, row):
    """src/daiss.rs:344-356: u = ((next >> 40) + 1) / 2^24 (exact in f32);
    r = sigma sqrt(-2 ln u1); a = TAU * u2 (an f32 product);
    (z0, z1) = (r cos a, r sin a). Checked in float64 to a few f32 ulps."""
    sigma = np.float32(0.02)
    width = 64
    got = O.daiss_row(model, name, row, float(sigma), width)
    g = _xorshift(O.seed_of(model, name, row))
    for i in range(0, width, 2):
        u1 = ((next(g) >> 40) + 1) / 16777216.0
        u2 = ((next(g) >> 40) + 1) / 16777216.0
        a = float(TAU32 * np.float32(u2))
        r = float(sigma) * math.sqrt(-2.0 * math.log(u1))
        for z, want in ((got[i], r * math.cos(a)), (got[i + 1], r * math.sin(a))):
            assert abs(float(z) - want) <= 5e-7 * abs(want) + 1e-12, (i, z, want)


# ------------------------------------------------------------------ Q6_K
Q6_SCALES = np.array([1, -2, 3, -4, 5, -6, 7, -8, 9, -10, 11, -12, 13, -14, 15, -16], np.int8)


def _q6_index_ql(byte, high):
    """The table of src/kernels/scalar.rs:283-291: in half h (ql bytes
    64h..64h+63) group 0 is the low nibble of the first 32 bytes, 1 the low
    nibble of the next 32, 2 and 3 their high nibbles."""
    h, r = divmod(byte, 64)
    return 128 * h + 32 * ((r // 32) + (2 if high else 0)) + r % 32


def _q6_index_qh(byte, pair):
    """qh bytes 32h..32h+31 of half h: bit pair p holds group p's two high bits."""
    h, i = divmod(byte, 32)
    return 128 * h + 32 * pair + i


def _q6_one_hot_blocks():
    blocks, qs = [], []
    for byte in range(128):
        for high in (0, 1):
            b = np.zeros(210, np.uint8)
            b[byte] = 0x10 if high else 0x01
            q = np.zeros(256, np.int32)
            q[_q6_index_ql(byte, high)] = 1
            blocks.append(b)
            qs.append(q)
    for byte in range(64):
        for pair in range(4):
            b = np.zeros(210, np.uint8)
            b[128 + byte] = 1 << (2 * pair)
            q = np.zeros(256, np.int32)
            q[_q6_index_qh(byte, pair)] = 16
            blocks.append(b)
            qs.append(q)
    # every value at 63 (all bits set)
    b = np.zeros(210, np.uint8)
    b[:192] = 0xFF
    blocks.append(b)
    qs.append(np.full(256, 63, np.int32))
    for b in blocks:
        b[192:208] = Q6_SCALES.view(np.uint8)
        b[208:210] = (0x00, 0x38)  # d = f16 0.5
    return np.stack(blocks), np.stack(qs)


def test_q6k_one_hot_bytes_dequantize_and_unpack_per_the_table():
    blocks, qs = _q6_one_hot_blocks()
    n = len(blocks)
    y = O.dequantize(O.Q6_K, blocks.ravel(), n * 256).reshape(n, 256)
    sc = np.repeat(Q6_SCALES.astype(np.float32), 16)
    want = (np.float32(0.5) * sc)[None, :] * (qs - 32).astype(np.float32)
    assert np.array_equal(y, want)
    q, esc, _ = O.unpack_i8(O.Q6_K, blocks.ravel(), n * 256)
    assert np.array_equal(q.reshape(n, 256), (qs - 32).astype(np.int8))
    assert np.array_equal(esc.reshape(n, 16), np.tile(np.float32(0.5) * Q6_SCALES.astype(np.float32), (n, 1)))


def test_q6k_one_hot_bytes_row_dot_per_the_table():
    """The row dot sum_s xe[s] (d sc[s]) (E_s - 32 xs[s]), E_s = sum x q over
    raw q in [0, 63] (src/kernels/scalar.rs:294-324), in float64."""
    blocks, qs = _q6_one_hot_blocks()
    rng = np.random.default_rng(6)
    xq = rng.integers(-127, 128, 256).astype(np.int8)
    xe = rng.uniform(0.001, 0.02, 16).astype(np.float32)
    xs = xq.reshape(16, 16).astype(np.float32).sum(1).astype(np.float32)
    sc = 0.5 * Q6_SCALES.astype(np.float64)
    for b, q in zip(blocks, qs):
        e = (xq.astype(np.int64) * q).reshape(16, 16).sum(1)
        terms = xe.astype(np.float64) * sc * (e - 32.0 * xs)
        got = O.dot_row(O.Q6_K, b, xq, xe, xs)
        assert abs(got - terms.sum()) <= 1e-5 * np.abs(terms).sum(), (got, terms.sum())


# ------------------------------------------------------- the quantizers
def _f16(v):
    return int(np.float16(v).view(np.uint16))


def _pack_k4_scales(le, lm):
    """Six-bit scale/min codes j = 0..7 into 12 bytes, the layout that
    src/quant.rs:108-117 reads: j < 4 in the low six bits of bytes j and
    j + 4; j >= 4 as nibbles of byte j + 4, their top two bits in the top
    bits of bytes j - 4 (scale) and j (min)."""
    q = [0] * 12
    for j in range(8):
        if j < 4:
            q[j] |= le[j]
            q[j + 4] |= lm[j]
        else:
            q[j + 4] |= (le[j] & 15) | ((lm[j] & 15) << 4)
            q[j - 4] |= (le[j] >> 4) << 6
            q[j] |= (lm[j] >> 4) << 6
    return q


def _grid_32(rng, nmax, max_level=None):
    """A 256-value block of 8 sub-blocks of 32 on an exact grid:
    x = 2^-12 le_j (l - c_j), l in [0, top] with 0 and top present, so the
    least-squares fit of each sub-block is exact (scale 2^-12 le_j, min
    2^-12 le_j c_j). One sub-block has le = 63 and one le c = 63, so the block
    scales are exactly d = dmin = 2^-12 and the codes are le_j and le_j c_j."""
    top = nmax if max_level is None else max_level
    le = rng.integers(1, 64, 8)
    c = np.array([rng.integers(0, min(top, 63 // v) + 1) for v in le])
    j0, j1 = rng.choice(8, 2, replace=False)
    le[j0], c[j0] = 63, rng.integers(0, 2)
    pairs = [(p, q) for p, q in ((63, 1), (21, 3), (9, 7), (7, 9), (3, 21)) if q <= top]
    le[j1], c[j1] = pairs[rng.integers(len(pairs))]
    lv = rng.integers(0, top + 1, (8, 32))
    for j in range(8):
        a, b = rng.choice(32, 2, replace=False)
        lv[j, a], lv[j, b] = 0, top
    x = (np.float32(2.0 ** -12) * (le[:, None] * (lv - c[:, None])).astype(np.float32)).ravel()
    return x, le, le * c, lv


def _q4k_bytes(le, lm, lv):
    out = [*divmod(_f16(2.0 ** -12), 256)[::-1], *divmod(_f16(2.0 ** -12), 256)[::-1]]
    out += _pack_k4_scales(le, lm)
    for p in range(4):
        out += [int(a) | (int(b) << 4) for a, b in zip(lv[2 * p], lv[2 * p + 1])]
    return np.array(out, np.uint8)


def _q5k_bytes(le, lm, lv):
    out = [*divmod(_f16(2.0 ** -12), 256)[::-1], *divmod(_f16(2.0 ** -12), 256)[::-1]]
    out += _pack_k4_scales(le, lm)
    qh = [0] * 32
    for p in range(4):
        for i in range(32):
            qh[i] |= ((int(lv[2 * p, i]) >> 4) << (2 * p)) | ((int(lv[2 * p + 1, i]) >> 4) << (2 * p + 1))
    out += qh
    for p in range(4):
        out += [(int(a) & 15) | ((int(b) & 15) << 4) for a, b in zip(lv[2 * p], lv[2 * p + 1])]
    return np.array(out, np.uint8)


@pytest.mark.parametrize("t,nmax,pack", [(O.Q4_K, 15, _q4k_bytes), (O.Q5_K, 31, _q5k_bytes)])
def test_q4k_q5k_quantizer_bytes_on_an_exact_grid(t, nmax, pack):
    """src/quant_kquants.rs:295-399 on grid blocks: the expected bytes are
    the designed codes, and they dequantize back to x exactly."""
    rng = np.random.default_rng(nmax)
    for _ in range(24):
        x, le, lm, lv = _grid_32(rng, nmax)
        want = pack(le, lm, lv)
        assert np.array_equal(O.dequantize(t, want, 256), x)  # the layout, independently
        got = O.quantize_blocks(t, x)
        assert np.array_equal(got, want), (np.nonzero(got != want)[0], le, lm)


def test_q4k_search_starts_one_level_below_nmax():
    """Q4_K's search (src/quant_kquants.rs:352-359: from -1.0 in steps of 0.1)
    tries (nmax - 1) / range first: sub-blocks whose levels span 0..14 fit
    exactly there and keep their codes; a search starting elsewhere cannot
    reach that fit."""
    rng = np.random.default_rng(14)
    for _ in range(24):
        x, le, lm, lv = _grid_32(rng, 15, max_level=14)
        want = _q4k_bytes(le, lm, lv)
        assert np.array_equal(O.dequantize(O.Q4_K, want, 256), x)
        assert np.array_equal(O.quantize_blocks(O.Q4_K, x), want)


@pytest.mark.parametrize("t,nmax", [(O.Q4_K, 15), (O.Q5_K, 31)])
def test_q4k_q5k_quantizer_zero_mins(t, nmax):
    """Sub-blocks of one power-of-two scale and no offset: every code is 63,
    dmin is 0 and d is f16(1 / (63 / s)), the block step of
    src/quant_kquants.rs:321-326."""
    rng = np.random.default_rng(100 + nmax)
    s = np.float32(2.0 ** -9)
    lv = rng.integers(0, nmax + 1, (8, 32))
    lv[:, 0], lv[:, 1] = 0, nmax
    x = (s * lv.astype(np.float32)).ravel()
    got = O.quantize_blocks(t, x)
    d = _f16(np.float32(1.0) / (np.float32(63.0) / s))
    assert int(got[0]) | (int(got[1]) << 8) == d and got[2] == 0 and got[3] == 0
    want = (_q4k_bytes if t == O.Q4_K else _q5k_bytes)([63] * 8, [0] * 8, lv)
    assert np.array_equal(got[4:], want[4:])


def _q3k_bytes(d_f, e, L):
    hmask, qs, packed = [0] * 32, [0] * 64, [0] * 12
    for j in range(16):
        u = int(e[j]) + 32
        if j < 8:
            packed[j] |= u & 15
        else:
            packed[j - 8] |= (u & 15) << 4
        packed[8 + j % 4] |= (u >> 4) << (2 * (j // 4))
    for idx in range(256):
        v = int(L[idx // 16, idx % 16])
        half, rnd, place = idx // 128, (idx % 128) // 32, idx % 32
        qs[half * 32 + place] |= (v & 3) << (2 * rnd)
        if v & 4:
            hmask[place] |= 1 << (half * 4 + rnd)
    return np.array(hmask + qs + packed + [_f16(d_f) & 255, _f16(d_f) >> 8], np.uint8)


@pytest.mark.parametrize("sign", [1, -1])
def test_q3k_quantizer_bytes_on_an_exact_grid(sign):
    """src/quant_kquants.rs:29-228 on grid blocks: sub-block j holds
    x = d e_j lam, lam in [-4, 3] with -4 present (so its largest magnitude
    fixes the scale exactly), d = -sign 2^-10, e_j in [-32, 31] with
    e = -32 in one sub-block (the block's largest scale, sign sign).
    The codes are u = e + 32 and l = lam + 4, and the block dequantizes to x."""
    rng = np.random.default_rng(3 + sign)
    d_f = -sign * 2.0 ** -10
    for _ in range(24):
        e = rng.integers(-31, 32, 16)
        j_big, j_zero = rng.choice(16, 2, replace=False)
        e[j_big] = -32
        lam = rng.integers(-4, 4, (16, 16))
        for j in range(16):
            lam[j, rng.integers(16)] = -4
        e[j_zero] = 0  # an all-zero sub-block: scale 0, l = 4
        lam[e == 0] = 0
        x = (np.float32(d_f) * (e[:, None] * lam).astype(np.float32)).ravel()
        want = _q3k_bytes(d_f, e, lam + 4)
        assert np.array_equal(O.dequantize(O.Q3_K, want, 256), x)
        got = O.quantize_blocks(O.Q3_K, x)
        assert np.array_equal(got, want), (np.nonzero(got != want)[0], e)


def _q2k_bytes(le, lm, lv):
    qs = [0] * 64
    for idx in range(256):
        half, rnd = idx // 128, (idx % 128) // 32
        qs[half * 32 + idx % 32] |= int(lv[idx // 16, idx % 16]) << (2 * rnd)
    d = _f16(2.0 ** -12)
    return np.array([int(a) | (int(b) << 4) for a, b in zip(le, lm)] + qs +
                    [d & 255, d >> 8, d & 255, d >> 8], np.uint8)


def test_q2k_quantizer_bytes_on_an_exact_grid():
    """src/quant_kquants.rs:99-157, 231-291 on grid blocks: sub-block j holds
    x = 2^-12 le_j (l - c_j), l in [0, 3] with 0 and 3 present; one
    sub-block has le = 15 and one le c = 15, so d = dmin = 2^-12 and the
    4-bit codes are le_j and le_j c_j."""
    rng = np.random.default_rng(2)
    for _ in range(24):
        le = rng.integers(1, 16, 16)
        c = np.array([rng.integers(0, min(3, 15 // v) + 1) for v in le])
        j0, j1 = rng.choice(16, 2, replace=False)
        le[j0], c[j0] = 15, rng.integers(0, 2)
        le[j1], c[j1] = ((15, 1), (5, 3))[rng.integers(2)]
        lv = rng.integers(0, 4, (16, 16))
        for j in range(16):
            a, b = rng.choice(16, 2, replace=False)
            lv[j, a], lv[j, b] = 0, 3
        x = (np.float32(2.0 ** -12) * (le[:, None] * (lv - c[:, None])).astype(np.float32)).ravel()
        want = _q2k_bytes(le, le * c, lv)
        assert np.array_equal(O.dequantize(O.Q2_K, want, 256), x)
        got = O.quantize_blocks(O.Q2_K, x)
        assert np.array_equal(got, want), (np.nonzero(got != want)[0], le, c)


# ------------------------------------------- the k-quant search on any block
# src/quant_kquants.rs:236-243, 353-359, 375-381: the search's parameters
# (sub-block size, nmax, first step, step, steps, absolute error)
SEARCH = {O.Q2_K: (16, 3, -0.5, 0.1, 15, True),
          O.Q4_K: (32, 15, -1.0, 0.1, 20, False),
          O.Q5_K: (32, 31, -0.5, 0.1, 15, False)}


def _round_away(v):
    """f32::round (half away from zero) of float32 values, exactly."""
    v = np.asarray(v, np.float64)
    return np.where(v >= 0, np.floor(v + 0.5), np.ceil(v - 0.5))


def _search_float64(x, w, nmax, first, step, steps, absolute):
    """The documented search (cuantos_qkx, src/quant_kquants.rs:99-157) on
    the sub-block x with weights w, its fits and errors in float64: start
    from the plain rounding at nmax / (max - min) with scale 1/iscale and
    min = min(0, min x); then for k = 0..steps form the codes at
    (first + step k + nmax) / (max - min) from the best min so far, fit the
    weighted least-squares scale and min (the min held at 0 when it would be
    positive), and keep the fit if its weighted error is lower. Only the
    codes are formed with f32 roundings, as the search forms them. Returns
    (codes, scale, min)."""
    f = np.float32
    mx = x.max()
    mn = min(f(0), x.min())
    err = (lambda r: np.abs(r)) if absolute else (lambda r: r * r)
    xd, wd = x.astype(np.float64), w.astype(np.float64)

    def codes(isc, m):
        return np.clip(_round_away(f(isc) * (x - f(m)).astype(f)), 0, nmax)

    isc = f(f(nmax) / f(mx - mn))
    a = codes(isc, mn)
    s, m = float(f(1) / isc), float(mn)
    best = float(np.sum(wd * err(s * a + m - xd)))
    sw, sx = wd.sum(), (wd * xd).sum()
    for k in range(steps + 1):
        isc = f(f(f(first) + f(step) * f(k)) + f(nmax)) / f(mx - f(m))
        c = codes(isc, m)
        if np.all(c == c[0]):  # no fit: the search skips it (D = 0)
            continue
        sl, sl2, sxl = (wd * c).sum(), (wd * c * c).sum(), (wd * c * xd).sum()
        dd = sw * sl2 - sl * sl
        cs, cm = (sw * sxl - sx * sl) / dd, (sl2 * sx - sl * sxl) / dd
        if cm > 0:
            cs, cm = sxl / sl2, 0.0
        e = float(np.sum(wd * err(cs * c + cm - xd)))
        if e < best:
            a, s, m, best = c, cs, cm, e
    return a, s, m


@pytest.mark.parametrize("t", [O.Q2_K, O.Q4_K, O.Q5_K], ids=["Q2_K", "Q4_K", "Q5_K"])
def test_kquant_search_on_random_blocks(t):
    """On random N(0, 0.02) blocks (the fixtures' weights, some widened),
    each sub-block's codes, scale and min from the oracle's search equal the
    documented search run in float64 with the reference's weights and error:
    |v| and absolute error for Q2_K (src/quant_kquants.rs:236-249), media +
    |v| (media the block's RMS) and squared error for Q4_K/Q5_K (301-305),
    the steps of 353-359 and 375-381. Where an f32 near-tie takes the
    search down another path the two may differ, but the oracle's result
    must then not be worse: its float64 error under the reference's weights
    is at most the documented search's (within 1e-6). A wrong weighting,
    error or step count gives worse fits."""
    sub, nmax, first, step, steps, absolute = SEARCH[t]
    err = (lambda r: np.abs(r)) if absolute else (lambda r: r * r)
    rng = np.random.default_rng(t)
    off, worse, total = [], [], 0
    for blk in range(150):
        x = (rng.normal(0, 0.02, 256) * (1 + 4 * (blk % 3 == 0) * rng.random(256))).astype(np.float32)
        scales, neg_mins, l = O.kquant_search(t, x)
        media = math.sqrt(float(np.sum(x.astype(np.float64) ** 2)) / 256)
        for j in range(256 // sub):
            xs = x[j * sub:(j + 1) * sub]
            xd = xs.astype(np.float64)
            w = np.abs(xd) + (0.0 if t == O.Q2_K else media)
            a, s, m = _search_float64(xs, w, nmax, first, step, steps, absolute)
            got, gs, gm = l[j * sub:(j + 1) * sub], float(scales[j]), -float(neg_mins[j])
            total += 1
            if (np.array_equal(a, got) and abs(gs - s) <= 1e-4 * abs(s)
                    and abs(gm - m) <= 1e-4 * float(np.abs(xs).max())):
                continue
            off.append((blk, j))
            e_doc = float(np.sum(w * err(s * a + m - xd)))
            e_got = float(np.sum(w * err(gs * got + gm - xd)))
            if e_got > e_doc * (1 + 1e-6):
                worse.append((blk, j, e_got / e_doc - 1))
    assert total == 150 * 256 // sub
    assert not worse, (len(worse), worse[:8])
    assert len(off) <= total // 200, (len(off), total, off[:8])


def test_q3k_search_scale_is_the_fit_of_its_codes():
    """cuantos_q3 (src/quant_kquants.rs:29-84): the returned scale is the
    x^2-weighted least-squares scale of the final codes (value - 4), and the
    refinement never leaves the codes worse than the first rounding at
    -nmax / (the value of largest magnitude)."""
    rng = np.random.default_rng(33)
    f = np.float32
    for blk in range(100):
        x = rng.normal(0, 0.02, 256).astype(np.float32)
        scales, _, l = O.kquant_search(O.Q3_K, x)
        for j in range(16):
            xs = x[j * 16:(j + 1) * 16]
            xd = xs.astype(np.float64)
            w = xd * xd
            li = l[j * 16:(j + 1) * 16].astype(np.float64) - 4
            assert np.all((li >= -4) & (li <= 3))
            fit = np.sum(w * xd * li) / np.sum(w * li * li)
            assert abs(float(scales[j]) - fit) <= 1e-4 * abs(fit), (blk, j)
            big = xs[np.argmax(np.abs(xs))]
            l0 = np.clip(_round_away(f(f(-4) / big) * xs), -4, 3)

            def e(c):
                return np.sum(w * xd * xd) - np.sum(w * xd * c) ** 2 / np.sum(w * c * c)
            assert e(li) <= e(l0) * (1 + 1e-9) + 1e-30, (blk, j)
