"""Q8_0 and Q5_0 on the GPU (MI355X): the formats of models whose width is
not a multiple of 256 (src/gguf.rs:80-82; daiss-0.5b, src/daiss.rs:91-102),
which the reference multiplies by its buffer path (ops::matmul_i8_directo,
src/ops.rs:310-414; matmul_varias_una_fila, 968-993).

Bars: the integer block sums and every GEMV output are bit-exact against
the oracle's restatement of that path (the same f32 operations in the same
order); the Q8_0 quantizer's bytes are the oracle's; models built from these
formats decode token for token with the oracle and their logits are equal."""
import numpy as np
import pytest
import torch

from gguf_fixtures import gguf_bytes, mirror, mixed_model, oracle_of, q5_0_bytes
from oracle import oracle as O

pytestmark = pytest.mark.gpu
B32 = (O.Q8_0, O.Q5_0)


@pytest.fixture(scope="module")
def ops(dev):
    from cosxamix_amd import ops
    return ops


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def rows_of(t, n, k, seed):
    if t == O.Q5_0:
        return q5_0_bytes(n, k, seed)
    x = np.random.default_rng(seed).normal(0, 0.02, n * k).astype(np.float32)
    return O.quantize_blocks(O.Q8_0, x).reshape(n, -1)


@pytest.mark.parametrize("t", B32, ids=["Q8_0", "Q5_0"])
@pytest.mark.parametrize("n,k", [(1, 32), (17, 160), (896, 896), (4864, 896), (896, 4864),
                                 (300, 2048)])
def test_gemv_bit_exact_with_the_buffer_path(ops, dev, t, n, k):
    w = rows_of(t, n, k, n + k)
    x = np.random.default_rng(k).normal(0, 1, k).astype(np.float32)
    xq, xe, xs = ops.cuantizar_i8_en(T(x, dev), 32)
    y = ops.gemv(t, T(w, dev), n, k, xq, xe, xs).cpu().numpy()
    want = O.matmul_direct(t, x, w, n, threads=8)[0]
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", B32, ids=["Q8_0", "Q5_0"])
def test_block_sums_are_exact(ops, dev, t):
    n, k = 40, 896
    w = rows_of(t, n, k, 7)
    x = np.random.default_rng(3).normal(0, 1, k).astype(np.float32)
    xq, xe, xs = ops.cuantizar_i8_en(T(x, dev), 32)
    got = ops.gemv_subsums(t, T(w, dev), n, k, xq, xe, xs).cpu().numpy()
    q, _, _ = O.unpack_i8(t, w, n * k)
    want = (q.reshape(n, k // 32, 32).astype(np.int64) *
            xq.cpu().numpy().reshape(1, k // 32, 32).astype(np.int64)).sum(-1)
    assert np.array_equal(got, want)


def test_q8_0_quantizer_bytes_are_the_oracles(ops, dev):
    x = np.random.default_rng(1).normal(0, 0.5, 32 * 999).astype(np.float32)
    x[:32] = 0.0  # an all-zero block: d = 0
    x[32:64] *= 1e6
    got = ops.cuantizar_bloques(O.Q8_0, T(x, dev)).cpu().numpy()
    assert np.array_equal(got, O.quantize_blocks(O.Q8_0, x))


@pytest.mark.parametrize("t", B32, ids=["Q8_0", "Q5_0"])
def test_matmul_auto_rows_and_multi(ops, dev, t):
    """Several rows equal one row at a time (src/ops.rs:1364-1393) and the
    oracle; one pass over several matrices equals separate calls bit for
    bit (src/ops.rs:1614-1670), mixing in the k-quants."""
    k, n, m = 512, 96, 5
    w = rows_of(t, n, k, 2)
    lhs = np.random.default_rng(2).normal(0, 1, (m, k)).astype(np.float32)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    ops.matmul_auto((m, k, n), T(lhs, dev), T(w, dev), t, dst)
    want = O.matmul_direct(t, lhs, w, n)
    assert np.array_equal(dst.cpu().numpy(), want)
    mats = [(T(w, dev), t), (T(O.daiss_matrix(1, "q", 70, k, 0.02, O.Q4_K), dev), O.Q4_K),
            (T(rows_of(O.Q5_0 if t == O.Q8_0 else O.Q8_0, 33, k, 4), dev),
             O.Q5_0 if t == O.Q8_0 else O.Q8_0)]
    outs = [torch.empty(m_.shape[0], dtype=torch.float32, device=dev) for m_, _ in mats]
    x = T(lhs[0], dev)
    ops.matmul_varias_una_fila(x, mats, outs)
    for (wm, tm), o in zip(mats, outs):
        one = torch.empty(wm.shape[0], dtype=torch.float32, device=dev)
        ops.matmul_auto((1, k, wm.shape[0]), x, wm, tm, one)
        assert torch.equal(o, one), tm


@pytest.mark.parametrize("t", B32, ids=["Q8_0", "Q5_0"])
@pytest.mark.parametrize("m,n,k", [(2, 64, 896), (17, 100, 896), (64, 4864, 896),
                                   (130, 896, 4864), (33, 257, 2048)])
def test_mfma_contraction_bit_exact(ops, dev, t, m, n, k):
    """Several rows (the batched prefill's shape) on the int8 MFMA
    contraction: every output equals the buffer path's, ragged tiles
    included."""
    w = rows_of(t, n, k, m + n)
    lhs = np.random.default_rng(m * n).normal(0, 1, (m, k)).astype(np.float32)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    ops.matmul_auto((m, k, n), T(lhs, dev), T(w, dev), t, dst)
    want = O.matmul_direct(t, lhs, w, n, threads=8)
    assert np.array_equal(dst.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_q8_0_daiss_model_matches_the_oracle(dev):
    """A daiss model written in Q8_0, the reference writer's type
    (src/daiss.rs:206-220), at daiss-0.5b's widths (dim 896, 14/2 heads of
    64, ffn 4864): logits and greedy tokens equal to the oracle's."""
    from cosxamix_amd import forward as F
    cfg = F.Config(2, 896, 14, 2, 4864, 640, 256)
    m = F.Modelo(cfg, tipo=O.Q8_0, semilla=21)
    ref = mirror(m)
    prompt = np.random.default_rng(5).integers(0, 640, 24).astype(np.uint32)
    lg, top = m.forward(prompt, m.nueva_cache(128))
    want = ref.forward(prompt, ref.new_cache(128))
    assert np.array_equal(lg, want) and top == O.argmax(want)
    got = m.generar(prompt, 24, m.nueva_cache(256))
    assert np.array_equal(got, ref.generate(prompt, 24, ref.new_cache(256)))
    # the batched prefill (MFMA) equals token-by-token decoding, bit for bit
    c1, c2 = m.nueva_cache(128), m.nueva_cache(128)
    l1, _ = m.forward(prompt, c1)
    for tok in prompt:
        l2, _ = m.forward([tok], c2)
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))


MIXED_05B = {"attn_q": O.Q5_0, "attn_k": O.Q5_0, "attn_v": O.Q8_0, "attn_output": O.Q5_0,
             "ffn_gate": O.Q5_0, "ffn_up": O.Q8_0, "ffn_down": O.Q6_K}


@pytest.mark.parametrize("over,varied", [(MIXED_05B, False),
                                         (dict(MIXED_05B, ffn_up=O.Q5_0, ffn_down=O.Q8_0), False),
                                         (MIXED_05B, True),
                                         (dict(MIXED_05B, ffn_up=O.Q5_0, ffn_down=O.Q8_0), True)],
                         ids=["q4_k_m", "q5_0-gate-up", "q4_k_m-varied", "q5_0-gate-up-varied"])
def test_qwen_0_5b_style_mixed_file_matches_the_oracle(dev, tmp_path, over, varied):
    """The layout of real Qwen2.5-0.5B Q4_K_M files: Q5_0/Q8_0 matrices of
    width 896, a k-quant ffn_down (width 4864 = 19 blocks of 256), a Q8_0
    token_embd tied to the lm_head. The second file's gate and up are both
    Q5_0 (one fused gate/up/SwiGLU launch) and its ffn_down Q8_0. `varied`:
    every norm ~ N(1, 0.1), q/k/v biases ~ N(0, 0.3) in both layers (the
    32-value block kernels' fused rmsnorm and bias epilogues)."""
    from cosxamix_amd import forward as F
    shape = dict(dim=896, heads=14, kv_heads=2, ffn=4864)
    data, host, types = mixed_model(seed=8, override=over, shape=shape, embd=O.Q8_0,
                                    varied=varied)
    path = tmp_path / "qwen05.gguf"
    path.write_bytes(data)
    m = F.Modelo.abrir(path)
    assert (m.cfg.dim, m.cfg.ffn) == (896, 4864)
    ref = oracle_of(host, types, shape=shape)
    prompt = np.array([3, 600, 17, 99, 5, 250, 41], np.uint32)
    gc, oc = m.nueva_cache(64), ref.new_cache(64)
    lg, _ = m.forward(prompt, gc)
    want = ref.forward(prompt, oc)
    assert np.array_equal(lg, want)
    for _ in range(5):  # teacher-forced single steps
        t = np.array([O.argmax(want)], np.uint32)
        lg, _ = m.forward(t, gc)
        want = ref.forward(t, oc)
        assert np.array_equal(lg, want)
    g = m.generar(prompt, 12, m.nueva_cache(64))
    assert np.array_equal(g, ref.generate(prompt, 12, ref.new_cache(64)))
