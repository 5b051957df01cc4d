"""Pins the oracle's per-token ops and operators on the CPU: known answers
and properties from the reference's own tests, and closed forms."""
import numpy as np
import pytest

from oracle import oracle as O


def test_dot_known_answers():  # src/kernels/scalar.rs:331-344
    f = lambda a, b: O.lib.orc_dot_f32(O._p(np.array(a, np.float32), O._f32p),  # noqa: E731
                                       O._p(np.array(b, np.float32), O._f32p), len(a))
    assert f([1, 2, 3], [4, 5, 6]) == 32.0
    assert f([1, -2], [3, 4]) == -5.0


def test_rmsnorm_known_answers():  # src/kernels/scalar.rs:346-376
    s = O.rmsnorm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 1e-6)
    assert abs(np.sqrt(np.mean(s ** 2)) - 1) < 1e-4
    p = np.array([2, 3, 4, 5], np.float32)
    assert np.allclose(O.rmsnorm(np.ones(4, np.float32), p, 1e-6), p, atol=1e-4)
    assert np.isfinite(O.rmsnorm(np.zeros(8, np.float32), np.ones(8, np.float32), 1e-6)).all()
    x = np.random.default_rng(0).normal(0, 2, 2048).astype(np.float32)
    want = (x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)).astype(np.float32)
    assert np.allclose(O.rmsnorm(x, np.ones(2048, np.float32), 1e-6), want, rtol=1e-6)


def test_silu_closed_form():
    x = np.linspace(-20, 20, 1001, dtype=np.float32)
    assert np.allclose(O.silu(x), x / (1 + np.exp(-x.astype(np.float64))), rtol=1e-6, atol=1e-30)


def test_argmax_ties_take_the_first():  # src/sampler.rs:159-165
    assert O.argmax(np.array([0.1, 3.0, 2.0, 3.0], np.float32)) == 1
    assert O.argmax(np.array([-5.0, -1.0, -3.0], np.float32)) == 1
    assert O.argmax(np.array([1.0], np.float32)) == 0
    assert O.argmax(np.array([np.nan, 2.0], np.float32)) == 0
    assert O.argmax(np.array([1.0, np.nan, 2.0], np.float32)) == 2


def test_softmax_invariants():  # src/ops.rs:1763-1797
    x = np.random.default_rng(1).normal(0, 30, (4, 500)).astype(np.float32)
    p = O.softmax(x, 500)
    assert np.allclose(p.sum(1), 1, atol=1e-5) and (p >= 0).all()
    assert np.array_equal(np.argmax(p, 1), np.argmax(x, 1))
    big = O.softmax(np.array([90.0, 0.0], np.float32), 2)
    assert np.isfinite(big).all()
    assert np.allclose(O.softmax(np.full(4, -np.inf, np.float32), 4), 0.25)
    with pytest.raises(ValueError):
        O.softmax(np.zeros(5, np.float32), 2)


def test_rope_identity_at_zero_and_norm_preserving():  # src/ops.rs:1806-1845
    heads, dim, tokens = 2, 8, 3
    c, s = O.rope_tables(dim, 10000.0, 16)
    orig = np.sin(np.arange(tokens * heads * dim, dtype=np.float32) * np.float32(0.37))
    x0 = O.rope(orig[: heads * dim], 1, heads, dim, c, s, 0)
    assert np.allclose(x0, orig[: heads * dim], atol=1e-6)
    x = O.rope(orig, tokens, heads, dim, c, s, 5)
    half = dim // 2
    for t in range(tokens):
        for h in range(heads):
            b = t * heads * dim + h * dim
            before = orig[b:b + half] ** 2 + orig[b + half:b + dim] ** 2
            after = x[b:b + half] ** 2 + x[b + half:b + dim] ** 2
            assert np.allclose(before, after, atol=1e-5)
    assert np.abs(x - orig).max() > 1e-3
    with pytest.raises(ValueError):
        O.rope(orig, tokens, heads, dim, c, s, 14)
    # the tables: closed form f32 powf frequency, f64 angle
    j, p = 3, 11
    freq = np.float32(1.0) / np.float32(np.float32(10000.0) ** np.float32(2 * j / dim))
    assert abs(c[p * half + j] - np.float32(np.cos(p * np.float64(freq)))) <= 1e-7


def test_attention_properties():  # src/ops.rs:1959-2062
    heads, kvh, dim = 4, 2, 8
    wq, wkv = heads * dim, kvh * dim
    q = np.sin(np.arange(wq, dtype=np.float32) * np.float32(0.3))
    k = np.cos(np.arange(wkv, dtype=np.float32) * np.float32(0.7))
    v = np.arange(wkv, dtype=np.float32)
    out = O.attention(q, k, v, 1, 1, heads, kvh, dim)
    for h in range(heads):
        g = h // (heads // kvh)
        assert np.allclose(out[h * dim:(h + 1) * dim], v[g * dim:(g + 1) * dim], atol=1e-5)
    total, tokens = 6, 3
    k = np.sin(np.arange(total * wkv, dtype=np.float32) * np.float32(0.21))
    v = np.cos(np.arange(total * wkv, dtype=np.float32) * np.float32(0.13))
    q = np.sin(np.arange(tokens * wq, dtype=np.float32) * np.float32(0.37))
    out = O.attention(q, k, v, tokens, total, heads, kvh, dim)
    for h in range(heads):
        g = h // (heads // kvh)
        for d in range(dim):
            col = v.reshape(total, wkv)[:, g * dim + d]
            o = out.reshape(tokens, wq)[:, h * dim + d]
            assert (o >= col.min() - 1e-5).all() and (o <= col.max() + 1e-5).all()
    v2 = v.copy().reshape(total, wkv)
    v2[-1] += 100
    out2 = O.attention(q, k, v2.ravel(), tokens, total, heads, kvh, dim)
    assert np.allclose(out[: (tokens - 1) * wq], out2[: (tokens - 1) * wq], atol=1e-5)
    assert np.abs(out[(tokens - 1) * wq:] - out2[(tokens - 1) * wq:]).max() > 1e-3


def test_matmul_one_row_equals_a_batch():  # src/ops.rs:1364-1393
    k, n = 512, 96
    w = O.daiss_matrix(4, "w", n, k, 0.02, O.Q4_K)
    lhs = np.stack([O.daiss_row(4, "x", f, 1.0, k) for f in range(4)])
    batch = O.matmul_fused(O.Q4_K, lhs, w, n, threads=4)
    for f in range(4):
        assert np.array_equal(batch[f], O.matmul_fused(O.Q4_K, lhs[f], w, n)[0])


def test_multi_1row_bit_identical_to_separate_calls():  # src/ops.rs:1614-1670
    k = 512
    mats = [(O.daiss_matrix(1, "q", 96, k, 0.02, O.Q4_K), O.Q4_K, 96),
            (O.daiss_matrix(1, "k", 32, k, 0.02, O.Q3_K), O.Q3_K, 32),
            (O.daiss_matrix(1, "v", 40, k, 0.02, O.Q5_K), O.Q5_K, 40)]
    x = O.daiss_row(2, "x", 0, 1.0, k)
    outs = O.matmul_multi_1row(x, mats, threads=4)
    for (w, t, n), o in zip(mats, outs):
        assert np.array_equal(o, O.matmul_fused(t, x, w, n)[0])


def test_tiny_model_is_deterministic_and_cache_consistent():
    """The oracle forward on a tiny daiss-shaped model: forward(p) twice gives
    the same logits, and forward(p) == forward(p[:k]) then forward(p[k:])."""
    cfg = dict(layers=2, dim=256, heads=4, kv_heads=2, ffn=512, vocab=300, ctx=64, eps=1e-6,
               rope_base=10000.0)
    tensors, types = {"token_embd.weight": O.daiss_row(1, "e", 0, 0.02, 300 * 256)}, {}
    tensors["output_norm.weight"] = np.ones(256, np.float32)
    tensors["output.weight"] = O.daiss_matrix(1, "output.weight", 300, 256, 0.02, O.Q4_K)
    types["output.weight"] = O.Q4_K
    for i in range(2):
        p = f"blk.{i}."
        for n in ("attn_norm.weight", "ffn_norm.weight"):
            tensors[p + n] = np.ones(256, np.float32)
        for n, d in (("attn_q.bias", 256), ("attn_k.bias", 128), ("attn_v.bias", 128)):
            tensors[p + n] = np.zeros(d, np.float32)
        for n, rows, width in (("attn_q", 256, 256), ("attn_k", 128, 256), ("attn_v", 128, 256),
                               ("attn_output", 256, 256), ("ffn_gate", 512, 256),
                               ("ffn_up", 512, 256), ("ffn_down", 256, 512)):
            tensors[p + n + ".weight"] = O.daiss_matrix(1, p + n, rows, width, 0.02, O.Q4_K)
            types[p + n + ".weight"] = O.Q4_K
    m = O.Model(cfg, tensors, types, threads=4)
    p = np.array([5, 17, 200, 3, 99, 42], np.uint32)
    a = m.forward(p, m.new_cache(32))
    assert np.array_equal(a, m.forward(p, m.new_cache(32)))
    c = m.new_cache(32)
    m.forward(p[:4], c)
    b = m.forward(p[4:], c)
    assert np.allclose(a, b, atol=1e-6)
    # token by token gives the same bits (every step is a function of its
    # own row; the last layer's shortcut for the last row changes nothing)
    c = m.new_cache(32)
    for tok in p:
        one = m.forward(np.array([tok], np.uint32), c)
    assert np.array_equal(a.view(np.uint32), one.view(np.uint32))
    toks = m.generate(p, 5, m.new_cache(32))
    assert len(toks) == 5 and (toks < 300).all()


F16_AT = {O.Q2_K: (80, 82), O.Q3_K: (108,), O.Q4_K: (0, 2), O.Q5_K: (0, 2), O.Q6_K: (208,)}


@pytest.mark.parametrize("t", [O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K, O.Q6_K])
def test_fused_matmul_equals_the_per_row_kernels(t):
    """orc_matmul_fused runs the scalar kernels restructured (rows prepared
    once, four activation rows as four chains): bit-identical to the
    per-row kernel for every (row, activation) pair, at any row count."""
    rng = np.random.default_rng(t)
    for k, n in ((256, 33), (2048, 40), (4352, 9)):
        bpb = O.BYTES_PER_BLOCK[t]
        w = rng.integers(0, 256, (n, k // 256 * bpb), dtype=np.uint8)
        for b in range(k // 256):
            for off in F16_AT[t]:
                h = rng.integers(0x1000, 0x3000, n)
                w[:, b * bpb + off], w[:, b * bpb + off + 1] = h & 0xFF, h >> 8
        for m in (1, 3, 4, 9):
            lhs = rng.normal(0, 1, (m, k)).astype(np.float32)
            got = O.matmul_fused(t, lhs, w, n, threads=3)
            for f in range(m):
                xq, xe, xs = O.quantize_act(lhs[f], O.SUB[t])
                want = np.array([O.dot_row(t, w[r], xq, xe, xs) for r in range(n)], np.float32)
                assert np.array_equal(got[f].view(np.uint32), want.view(np.uint32)), (k, m, f)
