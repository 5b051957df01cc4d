"""GPU parity of the kernels (MI355X), through the C ABI.

Bars (written per test): activation quantization, the GEMV's integer
sub-block sums, RoPE and the k-quant quantizer are bit-exact; GEMV outputs
are within relative L2 1e-5 of the reference (its compiled kernels via the
golden vectors, and the oracle's scalar restatement), plus the reference's
per-row bar |a-b|/max(|b|,1) < 1e-5 at k=2048."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu
KQ = (O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K)
F16_AT = {O.Q2_K: (80, 82), O.Q3_K: (108,), O.Q4_K: (0, 2), O.Q5_K: (0, 2), O.Q6_K: (208,)}


@pytest.fixture(scope="module")
def cx(dev):
    from cosxamix_amd import kernels, ops
    return ops, kernels


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def random_rows(t, rows, k, seed):
    """Random bytes with finite f16 scales (any bit pattern of the quants)."""
    rng = np.random.default_rng(seed)
    bpb = O.BYTES_PER_BLOCK[t]
    w = rng.integers(0, 256, (rows, k // 256 * bpb), dtype=np.uint8)
    for b in range(k // 256):
        for off in F16_AT[t]:
            h = rng.integers(0x1000, 0x3000, rows)
            w[:, b * bpb + off] = h & 0xFF
            w[:, b * bpb + off + 1] = h >> 8
    return w


# ------------------------------------------------ activation quantization
@pytest.mark.parametrize("sub", [16, 32])
def test_quantize_act_bit_exact(cx, dev, sub):
    ops, _ = cx
    rng = np.random.default_rng(sub)
    x = rng.normal(0, 1, (3, 11008)).astype(np.float32)
    x[0, :64] = 0.0
    x[1, 100:140] *= 1e-30
    x[1, 500] = 3e38
    x[2, 7], x[2, 300], x[2, 301] = np.nan, np.inf, -np.inf
    x[2, 1000:1032] = np.float32(2.5) * np.sign(rng.normal(size=32))  # exact .5 ties
    # subnormal sub-blocks: 127 / amax overflows to inf, so v * inv is +-inf
    # (Rust's `as i32` saturates, `as i8` keeps the low byte) or 0 * inf = NaN
    x[0, 2048:2080] = np.float32(1e-40) * np.sign(rng.normal(size=32))
    x[1, 4096:4128] = 0.0
    x[1, 4097] = np.float32(-1e-42)
    xq, xe, xs = (a.cpu().numpy() for a in ops.cuantizar_i8_en(T(x, dev), sub))
    for r in range(3):
        q, e, s = O.quantize_act(x[r], sub)
        assert np.array_equal(xq[r], q), r
        assert np.array_equal(xe[r].view(np.uint32), e.view(np.uint32)), r
        assert np.array_equal(xs[r].view(np.uint32), s.view(np.uint32)), r


# --------------------------------------------------------------- the GEMV
@pytest.mark.parametrize("t", KQ + (O.Q6_K,))
@pytest.mark.parametrize("k", [2048, 11008])
def test_gemv_integer_subsums_bit_exact(cx, dev, t, k):
    ops, _ = cx
    n = 37
    w = random_rows(t, n, k, seed=t * 7 + k)
    xq = np.random.default_rng(k).integers(-127, 128, k).astype(np.int8)
    ns = k // O.SUB[t]
    xe = np.ones(ns, np.float32)
    xs = np.zeros(ns, np.float32)
    got = ops.gemv_subsums(t, T(w, dev), n, k, T(xq, dev), T(xe, dev), T(xs, dev)).cpu().numpy()
    for r in range(n):
        assert np.array_equal(got[r], O.subsums(t, w[r], xq)), (O.NAMES[t], k, r)


def _golden_cases(golden):
    for t in KQ:
        for k in (2048, 11008):
            n = f"{O.NAMES[t]}_{k}"
            for an in ("normal", "extreme"):
                refs = {key.split("_ref_")[1]: golden[key] for key in golden.files
                        if key.startswith(f"{n}_{an}_ref_")}
                yield t, k, golden[f"{n}_w"], [golden[f"{n}_{an}_{s}"] for s in ("xq", "xe", "xs")], refs


def test_gemv_matches_the_reference_kernels(cx, dev, golden):
    ops, _ = cx
    for t, k, w, (xq, xe, xs), refs in _golden_cases(golden):
        y = ops.gemv(t, T(w, dev), w.shape[0], k, T(xq, dev), T(xe, dev), T(xs, dev)).cpu().numpy()
        for name, want in refs.items():
            assert rel_l2(y, want) <= 1e-5, (O.NAMES[t], k, name, rel_l2(y, want))
            if k == 2048:
                err = np.abs(y.astype(np.float64) - want) / np.maximum(np.abs(want), 1.0)
                assert err.max() < 1e-5, (O.NAMES[t], k, name, err.max())


def test_kernel_contract_on_host_arrays(cx, golden):
    """cx_dot_q*k_i8: the reference's `Kernel` ABI, host pointers in, f32 out."""
    _, kernels = cx
    for t, k, w, (xq, xe, xs), refs in _golden_cases(golden):
        got = np.array([kernels.dot_qk_i8(t, row, xq, xe, xs) for row in w], np.float32)
        for name, want in refs.items():
            assert rel_l2(got, want) <= 1e-5, (O.NAMES[t], k, name)
    with pytest.raises(ValueError):
        kernels.dot_q4k_i8(w[0], xq[:100], xe, xs)


@pytest.mark.parametrize("t", KQ + (O.Q6_K,))
def test_gemv_matches_oracle_random_bytes(cx, dev, t):
    ops, _ = cx
    for k in (2048, 4096, 11008, 14336):
        n = 300
        w = random_rows(t, n, k, seed=k + t)
        x = np.random.default_rng(t).normal(0, 1, k).astype(np.float32)
        xq, xe, xs = O.quantize_act(x, O.SUB[t])
        y = ops.gemv(t, T(w, dev), n, k, T(xq, dev), T(xe, dev), T(xs, dev)).cpu().numpy()
        want = np.array([O.dot_row(t, w[r], xq, xe, xs) for r in range(n)], np.float32)
        assert rel_l2(y, want) <= 1e-5, (O.NAMES[t], k, rel_l2(y, want))


@pytest.mark.parametrize("t", (O.Q4_K, O.Q5_K))
def test_row_kernels_bit_exact(cx, dev, t):
    """The plain Q4_K/Q5_K row kernels: k = 2048 and 4096 (a row's lanes hold
    half super-blocks), 17 to 64 super-blocks (a wave a row: the down
    projections at 43 and 56): every output bit-identical to the scalar
    spec's row sum (orc_dot_*), with row counts that leave a partial last
    tile."""
    ops, _ = cx
    for k, n in ((2048, 45), (4096, 300), (4352, 37), (11008, 300), (14336, 61), (16384, 9)):
        w = random_rows(t, n, k, seed=3 * k + t)
        x = np.random.default_rng(k - t).normal(0, 1, k).astype(np.float32)
        xq, xe, xs = O.quantize_act(x, O.SUB[t])
        y = ops.gemv(t, T(w, dev), n, k, T(xq, dev), T(xe, dev), T(xs, dev)).cpu().numpy()
        want = np.array([O.dot_row(t, w[r], xq, xe, xs) for r in range(n)], np.float32)
        bad = np.nonzero(y.view(np.uint32) != want.view(np.uint32))[0]
        assert bad.size == 0, (O.NAMES[t], k, bad[:5], y[bad[:3]], want[bad[:3]])


# BASELINE config 2 shapes (rows x cols) for every type; config 1 is Q4_K gate
SHAPES = [(2048, 2048), (256, 2048), (11008, 2048), (2048, 11008)]


@pytest.mark.parametrize("t", KQ)
def test_config2_sweep_matches_oracle(cx, dev, t):
    ops, _ = cx
    for n, k in SHAPES:
        w = O.daiss_matrix(5, f"sweep.{n}x{k}", n, k, 0.02, t)
        x = O.daiss_row(9, "sweep.x", 0, 1.0, k)
        xq, xe, xs = O.quantize_act(x, O.SUB[t])
        want = O.matmul_fused(t, x[None, :], w, n, threads=16)[0]
        y = torch.empty(n, dtype=torch.float32, device=dev)
        ops.matmul_auto((1, k, n), T(x, dev), T(w, dev), t, y)
        y = y.cpu().numpy()
        assert rel_l2(y, want) <= 1e-5, (O.NAMES[t], n, k, rel_l2(y, want))
        y2 = ops.gemv(t, T(w, dev), n, k, T(xq, dev), T(xe, dev), T(xs, dev)).cpu().numpy()
        assert np.array_equal(y.view(np.uint32), y2.view(np.uint32)), "in-kernel quantization"


def test_matmul_auto_rows_equal_single_rows(cx, dev):  # src/ops.rs:1364-1393
    ops, _ = cx
    k, n, m = 2048, 300, 5
    w = O.daiss_matrix(3, "rows", n, k, 0.02, O.Q4_K)
    lhs = np.stack([O.daiss_row(3, "lhs", f, 1.0, k) for f in range(m)])
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    ops.matmul_auto((m, k, n), T(lhs, dev), T(w, dev), O.Q4_K, dst)
    for f in range(m):
        one = torch.empty(n, dtype=torch.float32, device=dev)
        ops.matmul_auto((1, k, n), T(lhs[f], dev), T(w, dev), O.Q4_K, one)
        assert torch.equal(dst[f], one)
    with pytest.raises(ValueError):
        ops.matmul_auto((m, k, n), T(lhs, dev), T(w, dev), O.Q4_K, one)


@pytest.mark.parametrize("t,n,k,ms", [
    (O.Q4_K, 11008, 2048, (8, 32, 40, 70, 512)),  # BASELINE config 4, first matrix
    (O.Q4_K, 2048, 11008, (8, 32, 512)),           # config 4, second matrix (43 blocks)
    (O.Q5_K, 1000, 4096, (3, 16, 17, 64, 100, 200)),  # ragged n, partial tiles
    (O.Q4_K, 2048, 2048, (2, 12, 16)),             # few rows: one 16-row tile, mostly padding
    # the 16-value sub-block formats (two masked MFMAs a 32-value group)
    (O.Q6_K, 2048, 11008, (2, 17, 64)),             # Q*_K_M down projections
    (O.Q6_K, 1000, 2048, (5, 130)),
    (O.Q3_K, 2100, 2048, (3, 33)),
    (O.Q2_K, 777, 4096, (16, 70)),
])
def test_batched_mfma_bit_identical_to_rows_and_oracle(cx, dev, t, n, k, ms):
    """matmul_auto with m > 1 (int8 MFMA path) against the single-row GEMV
    (bit-identical: same integer sums, same f32 terms in scalar order) and,
    on sampled outputs, against the oracle's scalar row dot (src/ops.rs:1364-1393:
    a row of a batch equals the row alone)."""
    ops, _ = cx
    w = random_rows(t, n, k, n + k)
    wd = T(w, dev)
    rng = np.random.default_rng(k)
    for m in ms:
        lhs = rng.normal(0, 1, (m, k)).astype(np.float32)
        lhs[0, :32] = 0.0  # an all-zero sub-block
        dst = torch.empty((m, n), dtype=torch.float32, device=dev)
        ops.matmul_auto((m, k, n), T(lhs, dev), wd, t, dst)
        xq, xe, xs = ops.cuantizar_i8_en(T(lhs, dev), O.SUB[t])
        got = dst.cpu().numpy()
        for a in range(m):
            y = ops.gemv(t, wd, n, k, xq[a].contiguous(), xe[a].contiguous(), xs[a].contiguous())
            assert np.array_equal(got[a].view(np.uint32), y.cpu().numpy().view(np.uint32)), (m, a)
        q, e, s = (v.cpu().numpy() for v in (xq, xe, xs))
        for a, r in ((0, 0), (m - 1, n - 1), (m // 2, n // 3)):
            want = O.dot_row(t, w[r], q[a], e[a], s[a])
            assert np.float32(want).view(np.uint32) == got[a, r].view(np.uint32), (m, a, r)


def test_multi_1row_bit_identical_to_single_calls(cx, dev):  # src/ops.rs:1614-1670
    ops, _ = cx
    k = 2048
    mats = [(O.daiss_matrix(1, "q", 2048, k, 0.02, O.Q4_K), O.Q4_K),
            (O.daiss_matrix(1, "k", 256, k, 0.02, O.Q4_K), O.Q4_K),
            (random_rows(O.Q6_K, 256, k, 4), O.Q6_K),
            (O.daiss_matrix(1, "g", 512, k, 0.02, O.Q3_K), O.Q3_K)]
    x = T(O.daiss_row(2, "x", 0, 1.0, k), dev)
    outs = [torch.empty(w.shape[0], dtype=torch.float32, device=dev) for w, _ in mats]
    ops.matmul_varias_una_fila(x, [(T(w, dev), t) for w, t in mats], outs)
    for (w, t), o in zip(mats, outs):
        one = torch.empty(w.shape[0], dtype=torch.float32, device=dev)
        ops.matmul_auto((1, k, w.shape[0]), x, T(w, dev), t, one)
        assert torch.equal(o, one), O.NAMES[t]


# ------------------------------------------------------------ quantizers
@pytest.mark.parametrize("t", KQ)
def test_gpu_quantizer_bit_exact(cx, dev, t):
    """cx_quantize_blocks gives the oracle quantizer's bytes for the same f32."""
    ops, _ = cx
    rows = [O.daiss_row(7, "qz", r, 0.02, 2048) for r in range(16)]
    z = np.zeros(2048, np.float32)
    z[256:512] = np.abs(O.daiss_row(1, "pos", 0, 0.1, 256))
    z[512:768] = -np.abs(O.daiss_row(1, "neg", 0, 0.1, 256))
    z[768:784] = 50.0
    z[1024:1280] = O.daiss_row(2, "big", 0, 30.0, 256)
    rows.append(z)
    x = np.concatenate(rows).astype(np.float32)
    got = ops.cuantizar_bloques(t, T(x, dev)).cpu().numpy()
    want = O.quantize_blocks(t, x)
    assert np.array_equal(got, want), (O.NAMES[t], int((got != want).sum()))


# --------------------------------------------------------- per-token ops
def test_rmsnorm_matches_oracle(cx, dev):
    ops, _ = cx
    x = np.random.default_rng(1).normal(0, 3, (4, 2048)).astype(np.float32)
    w = np.random.default_rng(2).normal(1, 0.1, 2048).astype(np.float32)
    out = torch.empty((4, 2048), dtype=torch.float32, device=dev)
    ops.rmsnorm(out, T(x, dev), T(w, dev), 1e-6)
    out = out.cpu().numpy()
    for r in range(4):
        want = O.rmsnorm(x[r], w, 1e-6)
        assert np.max(np.abs(out[r] - want) / np.maximum(np.abs(want), 1e-30)) < 1e-6
    z = torch.zeros(8, dtype=torch.float32, device=dev)
    o = torch.full((8,), 9.9, device=dev)
    ops.rmsnorm(o, z, torch.ones(8, device=dev), 1e-6)  # scalar.rs:370-376
    assert torch.isfinite(o).all()


def test_rope_bit_exact_and_tables(cx, dev):
    ops, _ = cx
    hd, heads, toks = 128, 16, 3
    c, s = ops.frecuencias_rope(hd, 1e6, 64)
    oc, os_ = O.rope_tables(hd, 1e6, 64)
    assert np.array_equal(c, oc) and np.array_equal(s, os_)
    x = np.random.default_rng(3).normal(0, 1, toks * heads * hd).astype(np.float32)
    xt = T(x, dev)
    ops.rope(xt, (toks, heads, hd), T(c, dev), T(s, dev), 17)
    want = O.rope(x, toks, heads, hd, oc, os_, 17)
    assert np.array_equal(xt.cpu().numpy().view(np.uint32), want.view(np.uint32))
    with pytest.raises(ValueError):
        ops.rope(xt, (toks, heads, hd), T(c, dev), T(s, dev), 62)


def test_softmax_silu_argmax(cx, dev):
    ops, _ = cx
    x = np.random.default_rng(4).normal(0, 10, (3, 1000)).astype(np.float32)
    xt = T(x, dev)
    ops.softmax(xt, 1000)
    got = xt.cpu().numpy()
    assert np.allclose(got, O.softmax(x, 1000), rtol=1e-5, atol=1e-9)
    assert np.allclose(got.sum(1), 1.0, atol=1e-5)
    inf = T(np.full(10, -np.inf, np.float32), dev)
    ops.softmax(inf, 10)
    assert torch.allclose(inf, torch.full((10,), 0.1, device=dev))  # ops.rs:1214-1219
    g = np.random.default_rng(5).normal(0, 4, 11008).astype(np.float32)
    o = torch.empty(11008, dtype=torch.float32, device=dev)
    ops.silu(o, T(g, dev))
    assert np.allclose(o.cpu().numpy(), O.silu(g), rtol=2e-6, atol=1e-12)
    # argmax: first index of the max (src/sampler.rs:159-165), NaN at 0 wins
    for v in ([0.1, 3.0, 2.0, 3.0], [-5.0, -1.0, -3.0], [1.0], [np.nan, 5.0, 1.0],
              [1.0, np.nan, 7.0, 7.0], [-np.inf, -np.inf]):
        a = np.array(v, np.float32)
        assert ops.argmax(T(a, dev)) == O.argmax(a), v
    big = np.random.default_rng(6).normal(0, 1, 151936).astype(np.float32)
    big[100] = big[151935] = 50.0
    assert ops.argmax(T(big, dev)) == 100


@pytest.mark.parametrize("heads,kvh,hd", [(16, 2, 128), (32, 8, 128), (4, 2, 64), (28, 4, 128),
                                          (8, 8, 64), (32, 2, 128)])
def test_decode_attention_paths(cx, dev, heads, kvh, hd):
    """The model's decode attention: order-exact mode bit-identical to the
    oracle (src/ops.rs:1258-1325) at any length, for 1, 2, 4, 7, 8 and 16
    query heads per KV group, on either side of the softmax-V kernel's
    limits (768/769: the sum one add a position, then by binade scan;
    2048/2049: 128-position stages, then 256); split-K mode within f32
    rounding."""
    ops, _ = cx
    for total in (1, 2, 37, 63, 64, 65, 100, 150, 255, 256, 257, 640, 768, 769, 1000, 2048, 2049,
                  4096, 4097, 8300):
        rng = np.random.default_rng(total + heads)
        q = rng.normal(0, 1, heads * hd).astype(np.float32)
        k = rng.normal(0, 1, total * kvh * hd).astype(np.float32)
        v = rng.normal(0, 1, total * kvh * hd).astype(np.float32)
        want = O.attention(q, k, v, 1, total, heads, kvh, hd)
        for mode in (1, 2):
            out = torch.empty(heads * hd, dtype=torch.float32, device=dev)
            ops.atencion_decode(T(q, dev), T(k, dev), T(v, dev), (total, heads, kvh, hd), out, mode)
            got = out.cpu().numpy()
            if mode == 1:
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (total, mode)
            else:
                assert np.allclose(got, want, rtol=1e-5, atol=1e-6), (
                    total, float(np.max(np.abs(got - want))))


@pytest.mark.parametrize("heads,kvh", [(16, 2), (32, 8)])
def test_decode_attention_long_path_limits(cx, dev, heads, kvh):
    """Order-exact decode attention on either side of the long one-token
    path's limits: 4096/4097 (the scores from k_att_qk from 4097 on), 6145
    (three stages of the softmax sum's 2048 positions and one more),
    11520/11521 (the last cache the long path holds in LDS, then
    k_att_sv); bit-identical to the oracle."""
    ops, _ = cx
    hd = 128
    for total in (4096, 4097, 6145, 11520, 11521):
        rng = np.random.default_rng(total + 3 * heads)
        q = rng.normal(0, 1, heads * hd).astype(np.float32)
        k = rng.normal(0, 1, total * kvh * hd).astype(np.float32)
        v = rng.normal(0, 1, total * kvh * hd).astype(np.float32)
        want = O.attention(q, k, v, 1, total, heads, kvh, hd)
        out = torch.empty(heads * hd, dtype=torch.float32, device=dev)
        ops.atencion_decode(T(q, dev), T(k, dev), T(v, dev), (total, heads, kvh, hd), out, 1)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)), total


@pytest.mark.parametrize("heads,kvh", [(16, 2), (32, 8)])
def test_decode_attention_sum_edge_cases(cx, dev, heads, kvh):
    """Order-exact decode attention on scores that stress the sum of exps:
    a wide spread (most exps subnormal or zero, the sum starting far below
    1 and jumping binades), equal keys (every exp 1, the sum landing on
    each power of two exactly), a peaked first position, and a NaN key row
    (that KV group's outputs NaN, the others bit-identical)."""
    ops, _ = cx
    hd = 128
    for total in (1, 63, 64, 65, 300, 548, 2047, 8300):
        rng = np.random.default_rng(7 * total + heads)
        base_q = rng.normal(0, 1, heads * hd).astype(np.float32)
        k = rng.normal(0, 1, total * kvh * hd).astype(np.float32)
        v = rng.normal(0, 1, total * kvh * hd).astype(np.float32)
        cases = {"spread": (base_q * 40, k), "equal": (base_q, np.tile(k[:kvh * hd], total)),
                 "peak": (base_q, k.copy())}
        cases["peak"][1][:kvh * hd] = np.repeat(base_q.reshape(kvh, -1, hd)[:, 0], 1, 0).ravel() * 6
        if total > 2:
            kn = k.copy()
            kn[(total // 2) * kvh * hd] = np.nan  # KV group 0 at the middle position
            cases["nan"] = (base_q, kn)
        for name, (q, kk) in cases.items():
            q = np.ascontiguousarray(q, np.float32)
            kk = np.ascontiguousarray(kk, np.float32)
            want = O.attention(q, kk, v, 1, total, heads, kvh, hd)
            out = torch.empty(heads * hd, dtype=torch.float32, device=dev)
            ops.atencion_decode(T(q, dev), T(kk, dev), T(v, dev), (total, heads, kvh, hd), out, 1)
            got = out.cpu().numpy()
            nan = np.isnan(want)
            assert np.array_equal(np.isnan(got), nan), (total, name)
            if name == "nan":
                assert nan[: heads // kvh * hd].all() and not nan[heads // kvh * hd:].any()
            assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), (total, name)


def test_attention_matches_oracle_and_properties(cx, dev):
    ops, _ = cx
    heads, kvh, hd = 16, 2, 128
    for tokens, total in [(1, 1), (1, 300), (5, 40), (1, 700)]:
        rng = np.random.default_rng(total)
        q = rng.normal(0, 1, tokens * heads * hd).astype(np.float32)
        k = rng.normal(0, 1, total * kvh * hd).astype(np.float32)
        v = rng.normal(0, 1, total * kvh * hd).astype(np.float32)
        out = torch.empty(tokens * heads * hd, dtype=torch.float32, device=dev)
        ops.atencion(T(q, dev), T(k, dev), T(v, dev), (tokens, total, heads, kvh, hd), out)
        want = O.attention(q, k, v, tokens, total, heads, kvh, hd)
        assert np.allclose(out.cpu().numpy(), want, rtol=1e-5, atol=1e-6), (tokens, total)
    with pytest.raises(ValueError):
        ops.atencion(T(q, dev), T(k, dev), T(v, dev), (tokens, total, heads, 3, hd), out)
