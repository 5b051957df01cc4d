"""Pins the CPU oracle's format code: f16, dequantize, unpack, quantizers,
the activation quantizer and the row dots (CPU only).

Each check is a known answer from the reference's own tests, an exhaustive
comparison against an independent implementation (numpy / the CPU's F16C),
a closed form, or the reference's own compiled kernels (golden vectors)."""
import math

import numpy as np
import pytest

from oracle import oracle as O

KQ = (O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K)


# ------------------------------------------------------------------ f16
def test_f16_known_answers():  # src/quant.rs:813-826
    assert O.f16_to_f32(0x0000) == 0.0 and math.copysign(1, O.f16_to_f32(0x8000)) < 0
    assert O.f16_to_f32(0x3C00) == 1.0 and O.f16_to_f32(0xBC00) == -1.0
    assert O.f16_to_f32(0x4000) == 2.0 and O.f16_to_f32(0x7BFF) == 65504.0
    assert math.isinf(O.f16_to_f32(0x7C00)) and math.isnan(O.f16_to_f32(0x7E00))
    assert O.f16_to_f32(0x0001) == 2.0 ** -24
    assert O.f16_to_f32(0x03FF) == 1023.0 * 2.0 ** -24


def test_f16_to_f32_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(v)) for v in h], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_trip_known_answers():  # src/quant.rs:938-971
    for v in [0.0, -0.0, 1.0, -1.0, 0.5, 2.0, 65504.0, -65504.0, 6.1035156e-5, 5.9604645e-8,
              1.0 / 1024.0]:
        back = np.float32(O.f16_to_f32(O.f32_to_f16(v)))
        assert back.view(np.uint32) == np.float32(v).view(np.uint32), v
    assert math.isinf(O.f16_to_f32(O.f32_to_f16(1e30)))
    assert math.isinf(O.f16_to_f32(O.f32_to_f16(-1e30)))
    assert math.isnan(O.f16_to_f32(O.f32_to_f16(float("nan"))))
    mid = (O.f16_to_f32(0x3C00) + O.f16_to_f32(0x3C01)) / 2.0
    assert O.f32_to_f16(mid) == 0x3C00  # ties to even


def test_f32_to_f16_matches_numpy_round_to_nearest_even():
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32)
    # bias towards the f16 range, subnormals and ties
    bits[:50_000] = (bits[:50_000] & 0x807FFFFF) | (rng.integers(96, 145, 50_000).astype(np.uint32) << 23)
    bits[50_000:60_000] &= 0x8000E000 | (0xFF << 23)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    # [2^-38, 2^-32) is the wrapped-shift region (next test); everything else
    # is IEEE round-to-nearest-even with saturation to inf
    wrap = (np.abs(x) >= 2.0 ** -38) & (np.abs(x) < 2.0 ** -32)
    x = x[~wrap]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, want)


def test_f32_to_f16_wrapped_shift_region():
    """src/quant.rs:716-722 shifts a u32 by sh+13 = 32..37 bits for
    |x| in [2^-38, 2^-32); a Rust release build masks the amount to 5 bits.
    Restated from that rule: man >> (n & 31), rest/half masked likewise."""
    def rust_release(v):
        b = int(np.float32(v).view(np.uint32))
        sign, mag = (b >> 16) & 0x8000, b & 0x7FFFFFFF
        sh = -14 - ((mag >> 23) - 127)
        if sh > 24:
            return sign
        man = (mag & 0x7FFFFF) | 0x800000
        val = man >> ((sh + 13) & 31)
        rest = man & ((1 << ((sh + 13) & 31)) - 1)
        half = 1 << ((sh + 12) & 31)
        return (sign | (val + (rest > half or (rest == half and val & 1)))) & 0xFFFF
    for v in [2.0 ** -38, 3e-12, -5.8e-11, 2.0 ** -33, 1.9e-10, -2.3e-10]:
        assert O.f32_to_f16(v) == rust_release(v), v
    assert O.f32_to_f16(0.0) == 0 and O.f32_to_f16(1e-30) == 0


# -------------------------------------------------------- dequant / unpack
def test_q8_0_by_hand():  # src/quant.rs:830-839
    b = np.zeros(34, np.uint8)
    b[0], b[1] = 0x00, 0x3C
    b[2], b[3] = 5, np.uint8(253)
    y = O.dequantize(O.Q8_0, b, 32)
    assert y[0] == 5.0 and y[1] == -3.0


@pytest.mark.parametrize("t,sub", [(O.Q8_0, 32), (O.Q5_0, 32), (O.Q2_K, 16), (O.Q3_K, 16),
                                   (O.Q4_K, 32), (O.Q5_K, 32), (O.Q6_K, 16)])
def test_unpack_reconstructs_dequantize_exactly(t, sub):  # src/quant.rs:892-928
    n = 3
    data = ((np.arange(n * O.BYTES_PER_BLOCK[t]) * 97 + 13) % 251).astype(np.uint8)
    vals = n * O.VALUES_PER_BLOCK[t]
    want = O.dequantize(t, data, vals)
    q, esc, off = O.unpack_i8(t, data, vals)
    rec = (np.repeat(esc, sub) * q.astype(np.float32) + np.repeat(off, sub)).astype(np.float32)
    ok = np.isfinite(want)
    # f32 equality as the reference's assert_eq! (-0.0 == 0.0)
    assert np.array_equal(rec[ok], want[ok])
    assert np.array_equal(np.isnan(rec), np.isnan(want))


# ------------------------------------------------------------- quantizers
def _normals(n, sigma, seed=7):
    out = np.empty(n, np.float32)
    for r in range(0, n, 2048):
        out[r:r + 2048] = O.daiss_row(seed, "normals", r // 2048, sigma, min(2048, n - r))
    return out


def _round_trip(t, x):
    b = O.quantize_blocks(t, x)
    assert b.size == O.row_bytes(t, x.size)
    return O.dequantize(t, b, x.size)


def _rmse(a, b):
    return float(np.sqrt(np.mean((a.astype(np.float64) - b) ** 2)))


def test_quantizer_error_is_the_formats():  # src/quant_kquants.rs:427-437
    x = _normals(256 * 64, 0.02)
    e = {t: _rmse(x, _round_trip(t, x)) / 0.02 for t in KQ}
    assert e[O.Q4_K] < e[O.Q3_K] < e[O.Q2_K]
    assert e[O.Q5_K] < e[O.Q4_K] / 1.6
    assert e[O.Q4_K] < 0.09 and e[O.Q3_K] < 0.2 and e[O.Q2_K] < 0.42


@pytest.mark.parametrize("t", KQ)
def test_quantizer_zeros_round_trip(t):  # src/quant_kquants.rs:440-451
    z = np.zeros(256, np.float32)
    assert np.array_equal(_round_trip(t, z), z)
    x = _normals(256, 0.5)
    x[32:64] = 0
    y = _round_trip(t, x)
    assert _rmse(x, y) < 0.3 and np.isfinite(y).all()


@pytest.mark.parametrize("t", KQ)
def test_quantizer_uneven_scales_and_one_sign(t):  # src/quant_kquants.rs:456-477
    x = _normals(256, 0.001)
    x[:16] *= 1000
    y = _round_trip(t, x)
    assert _rmse(x[:16], y[:16]) < 0.5 and np.isfinite(y).all()
    pos = np.abs(_normals(256, 0.1))
    assert _rmse(pos, _round_trip(t, pos)) < 0.05
    assert _rmse(-pos, _round_trip(t, -pos)) < 0.05


@pytest.mark.parametrize("t,sub", [(O.Q2_K, 16), (O.Q3_K, 16), (O.Q4_K, 32), (O.Q5_K, 32)])
def test_quantizer_keeps_each_sub_block_scale(t, sub):  # src/quant_kquants.rs:482-503
    n = 256 // sub
    x = np.zeros(256, np.float32)
    for j in range(n):
        amp = np.float32(0.1 * (1.0 + j / n))
        x[j * sub:(j + 1) * sub] = np.where(np.arange(sub) % 2 == 0, amp, -amp)
    y = _round_trip(t, x)
    for j in range(n):
        assert _rmse(x[j * sub:(j + 1) * sub], y[j * sub:(j + 1) * sub]) < 0.06


def test_daiss_sigma_after_quantization():  # src/daiss.rs:719-720
    for t in (O.Q2_K, O.Q3_K, O.Q4_K):
        w = O.daiss_matrix(7, "blk.1.ffn_up.weight", 64, 768, 0.02, t)
        y = O.dequantize(t, w.ravel(), 64 * 768)
        assert abs(float(np.sqrt(np.mean(y.astype(np.float64) ** 2))) - 0.02) < 0.005


# --------------------------------------------------------------- the RNG
def test_azar_seed_and_streams():  # src/daiss.rs:750-765
    a = O.daiss_row(1, "t", 0, 1.0, 64)
    assert np.array_equal(a, O.daiss_row(1, "t", 0, 1.0, 64))
    assert not np.array_equal(a, O.daiss_row(2, "t", 0, 1.0, 64))
    assert not np.array_equal(a, O.daiss_row(1, "t", 1, 1.0, 64))


def test_seed_of_is_fnv1a_then_row_then_rotated_seed():  # src/daiss.rs:364-379
    def fnv(name, row, model):
        h = 0xcbf29ce484222325
        for b in name.encode():
            h = ((h ^ b) * 0x100000001B3) & (2 ** 64 - 1)
        h = ((h ^ row) * 0x100000001B3) & (2 ** 64 - 1)
        rot = ((model << 17) | (model >> 47)) & (2 ** 64 - 1)
        return h ^ rot
    for name, row, seed in [("token_embd.weight", 0, 42), ("blk.3.ffn_down.weight", 917, 7),
                            ("", 5, 0)]:
        assert O.seed_of(seed, name, row) == fnv(name, row, seed)


def test_normals_have_the_stated_deviation():  # src/daiss.rs:771-786
    v = O.daiss_row(1234, "sigma", 0, 0.02, 20000).astype(np.float64)
    assert abs(v.mean()) < 0.001 and abs(v.std() - 0.02) < 0.001


# ---------------------------------------------------- activation quantizer
def _round_half_away(v):
    v = v.astype(np.float64)
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


@pytest.mark.parametrize("sub", [16, 32])
def test_quantize_act_closed_form(sub):  # src/ops.rs:178-198, 472-483
    rng = np.random.default_rng(sub)
    x = rng.normal(0, 1, 4096).astype(np.float32)
    x[64:96] = 0.0                      # a zero sub-block
    x[200:232] *= 1e-30                 # tiny, subnormal products
    x[300] = 1e30
    q, e, s = O.quantize_act(x, sub)
    xb = x.reshape(-1, sub)
    amax = np.abs(xb).max(1)
    want_e = np.where(amax > 0, amax / np.float32(127), 0).astype(np.float32)
    assert np.array_equal(e.view(np.uint32), want_e.view(np.uint32))
    inv = np.where(amax > 0, np.float32(127) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    want_q = _round_half_away((xb * inv[:, None]).astype(np.float32)).astype(np.int64)
    assert np.array_equal(q.reshape(-1, sub).astype(np.int64), want_q)
    assert np.array_equal(s, q.reshape(-1, sub).astype(np.int64).sum(1).astype(np.float32))


def test_quantize_act_invariants():  # src/ops.rs:1431-1457
    x = np.sin(np.arange(64, dtype=np.float32) * np.float32(0.21)) * 3
    q, e, _ = O.quantize_act(x, 32)
    assert (q != -128).all()
    rec = q.astype(np.float32) * np.repeat(e, 32)
    assert (np.abs(rec - x) <= np.repeat(e, 32) * 0.51).all()
    q, e, s = O.quantize_act(np.zeros(64, np.float32), 32)
    assert np.isfinite(e).all() and (q == 0).all() and (s == 0).all()


# ---------------------------------------------------------------- row dots
def _golden_cases(golden):
    for t in KQ:
        for k in (2048, 11008):
            n = f"{O.NAMES[t]}_{k}"
            for an in ("normal", "extreme"):
                refs = {key.split("_ref_")[1]: golden[key] for key in golden.files
                        if key.startswith(f"{n}_{an}_ref_")}
                yield t, k, golden[f"{n}_w"], [golden[f"{n}_{an}_{s}"] for s in ("xq", "xe", "xs")], refs


def test_golden_reference_kernels_agree_with_each_other(golden):
    for t, k, w, (xq, xe, xs), refs in _golden_cases(golden):
        vals = list(refs.values())
        for v in vals[1:]:
            assert np.allclose(v, vals[0], rtol=1e-6, atol=0), (O.NAMES[t], k)


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def test_scalar_dots_match_the_reference_kernels(golden):
    """Against the reference's own compiled kernels. Bars: the reference's
    scalar-vs-vectorized |a-b|/max(|b|,1) < 1e-5 at the width it states it
    for, k=2048 (src/kernels/mod.rs:809-900); and relative L2 <= 1e-5 over
    the rows (the GEMV bar) at every width. At k=11008 two float orders of
    the reference itself differ by up to 1.5e-5 on a cancelling row."""
    for t, k, w, (xq, xe, xs), refs in _golden_cases(golden):
        got = np.array([O.dot_row(t, row, xq, xe, xs) for row in w], np.float32)
        for name, want in refs.items():
            assert rel_l2(got, want) <= 1e-5, (O.NAMES[t], k, name)
            if k == 2048:
                err = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want), 1.0)
                assert err.max() < 1e-5, (O.NAMES[t], k, name, err.max())


@pytest.mark.parametrize("t", KQ + (O.Q6_K,))
def test_subsums_are_the_brute_force_integer_sums(t):
    sub = O.SUB[t]
    rng = np.random.default_rng(t)
    nb = 4
    w = rng.integers(0, 256, nb * O.BYTES_PER_BLOCK[t], dtype=np.uint8)
    xq = rng.integers(-127, 128, nb * 256).astype(np.int8)
    q, _, _ = O.unpack_i8(t, w, nb * 256)
    bias = {O.Q3_K: 4, O.Q6_K: 32}.get(t, 0)  # the scalar kernels' unsigned form
    want = ((q.astype(np.int64) + bias) * xq).reshape(-1, sub).sum(1)
    assert np.array_equal(O.subsums(t, w, xq).astype(np.int64), want)


@pytest.mark.parametrize("t", KQ + (O.Q6_K,))
def test_dot_equals_dequantize_times_activation(t):  # q2k.rs:325-340, q5k.rs:195-213
    sub = O.SUB[t]
    for seed in (3, 5, 7, 11, 13):
        x = O.daiss_row(seed, "act", 0, 1.0, 2048)
        xq, xe, xs = O.quantize_act(x, sub)
        if t == O.Q6_K:
            rng = np.random.default_rng(seed)
            w = rng.integers(0, 256, 8 * 210, dtype=np.uint8)
            w[208::210], w[209::210] = 0x00, 0x24  # finite d
        else:
            w = O.daiss_matrix(seed, "w", 1, 2048, 0.02, t)[0]
        deq = O.dequantize(t, w, 2048).astype(np.float64)
        want = float(deq @ (xq.astype(np.float64) * np.repeat(xe, sub)))
        got = O.dot_row(t, w, xq, xe, xs)
        assert abs(got - want) <= 1e-3 * max(abs(want), 1.0)


def test_live_reference_kernels_on_random_rows():
    r = O.load_ref()
    if r is None:
        pytest.skip("oracle/_ref not built (no /root/reference here)")
    for t, kernels in O.ref_kernels(r).items():
        for seed in (3, 5, 7, 11, 13):
            w = O.daiss_matrix(seed, "live", 3, 4096, 0.02, t)
            xq, xe, xs = O.quantize_act(O.daiss_row(seed, "x", 0, 1.0, 4096), O.SUB[t])
            for row in w:
                s = O.dot_row(t, row, xq, xe, xs)
                for name, fn in kernels:
                    v = fn(O._p(np.ascontiguousarray(row), O._u8p), O._p(xq, O._i8p),
                           O._p(xe, O._f32p), O._p(xs, O._f32p), 16)
                    assert abs(v - s) / max(abs(s), 1.0) < 1e-5, (name, seed)
