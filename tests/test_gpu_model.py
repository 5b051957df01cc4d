"""GPU parity of the decode loop (Modelo::forward / generar) against the
oracle's forward (src/forward.rs:375-559) on the same weights.

Bars: logits max-abs <= 1e-3 (north star) at every step and greedy token
sequences identical; for caches up to 4096 tokens (the order-exact decode
attention) the logits must be bit-identical to the oracle's. Cache
semantics as src/forward.rs:98-127.

Why bit-identical and not a tolerance: in a deep random-init model one
ulp of difference upstream can flip an i8 rounding of a later activation
quantization, and the next RMSNorm of the small residual stream turns that
flip into a 1e-2 logit change. So the GPU path computes every f32 in the
reference's order (GEMV row sums, softmax sums, attention accumulation,
glibc's expf) and matches it bit for bit."""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def mirror(model, threads=16):
    """The GPU model's tensors copied to the host, as an oracle Model."""
    tensors, types = {}, {}
    for i, (name, t, dims, nb) in enumerate(model.tensores()):
        tensors[name] = model.tensor(i)
        types[name] = t
    c = model.cfg
    cfg = dict(layers=c.capas, dim=c.dim, heads=c.cabezas, kv_heads=c.cabezas_kv, ffn=c.ffn,
               vocab=c.vocab, ctx=c.contexto, eps=c.eps, rope_base=c.rope)
    return O.Model(cfg, tensors, types, threads=threads)


@pytest.fixture(scope="module")
def F(dev):
    from cosxamix_amd import forward
    return forward


CASES = [
    # (name, config, linear type, down type)
    ("mini-q4k", dict(capas=3, dim=256, cabezas=4, cabezas_kv=2, ffn=768, vocab=1000,
                      contexto=300, rope=10000.0), O.Q4_K, O.Q4_K),
    ("3b-heads-q4k", dict(capas=2, dim=2048, cabezas=16, cabezas_kv=2, ffn=11008, vocab=3000,
                          contexto=200, rope=1e6), O.Q4_K, O.Q4_K),
    ("8b-heads-q4k-q5kdown", dict(capas=1, dim=4096, cabezas=32, cabezas_kv=8, ffn=14336,
                                  vocab=2000, contexto=200, rope=5e5), O.Q4_K, O.Q5_K),
    ("mini-q2k", dict(capas=2, dim=512, cabezas=8, cabezas_kv=2, ffn=1536, vocab=1500,
                      contexto=200, rope=10000.0), O.Q2_K, O.Q3_K),
    # gate/up/SwiGLU in one launch, quantizing for a down of 16-value sub-blocks
    ("mini-q5k-q3kdown", dict(capas=2, dim=512, cabezas=8, cabezas_kv=2, ffn=1536, vocab=1500,
                              contexto=200, rope=10000.0), O.Q5_K, O.Q3_K),
    ("mini-q4k-q2kdown", dict(capas=2, dim=768, cabezas=6, cabezas_kv=2, ffn=2304, vocab=900,
                              contexto=200, rope=10000.0), O.Q4_K, O.Q2_K),
    # k = 2048: the row-layout gate/up/SwiGLU launch for Q5_K, quantizing for
    # a down of 16-value sub-blocks
    ("2048-q5k-q3kdown", dict(capas=1, dim=2048, cabezas=16, cabezas_kv=2, ffn=1024, vocab=1000,
                              contexto=200, rope=1e6), O.Q5_K, O.Q3_K),
]


@pytest.mark.parametrize("name,cfg,t,tdown", CASES, ids=[c[0] for c in CASES])
def test_forward_logits_and_greedy_tokens_match_oracle(F, name, cfg, t, tdown):
    c = F.Config(eps=1e-6, **cfg)
    m = F.Modelo(c, tipo=t, semilla=42, tipo_down=tdown, tipo_salida=t)
    ref = mirror(m)
    rng = np.random.default_rng(len(name))
    prompt = rng.integers(0, c.vocab, 24).astype(np.uint32)

    cache = m.nueva_cache(120)
    rc = ref.new_cache(120)
    lg, am = m.forward(prompt, cache)
    want = ref.forward(prompt, rc)
    assert np.max(np.abs(lg - want)) <= 1e-3, (name, float(np.max(np.abs(lg - want))))
    assert np.array_equal(lg.view(np.uint32), want.view(np.uint32)), name
    assert am == O.argmax(lg)
    assert cache.largo() == rc.len == 24

    # teacher-forced steps: feed the oracle's token to both, compare logits
    tok = O.argmax(want)
    for step in range(8):
        lg, _ = m.forward([tok], cache)
        want = ref.forward([tok], rc)
        assert np.array_equal(lg.view(np.uint32), want.view(np.uint32)), (name, step)
        tok = O.argmax(want)

    # greedy generation from scratch: identical sequences
    cache2 = m.nueva_cache(120)
    rc2 = ref.new_cache(120)
    got = m.generar(prompt, 24, cache2)
    exp = ref.generate(prompt, 24, rc2)
    assert np.array_equal(got, exp), (name, got, exp)
    assert cache2.largo() == rc2.len == 48


VARIED = [
    # (name, config, linear type, down type, prompt length); k = 2048: the
    # row kernels' fused rmsnorm (q/k/v, gate/up/SwiGLU); k = 4096: the LDS
    # gate/up/SwiGLU kernel; a 300-token prompt: two prefill chunks of the
    # MFMA contraction's fused rmsnorm; 896: the 32-value block kernels
    ("2048-q4k", dict(capas=2, dim=2048, cabezas=16, cabezas_kv=2, ffn=11008, vocab=3000,
                      contexto=200, rope=1e6), O.Q4_K, O.Q4_K, 24),
    ("4096-q4k-q5kdown", dict(capas=2, dim=4096, cabezas=32, cabezas_kv=8, ffn=14336,
                              vocab=2000, contexto=200, rope=5e5), O.Q4_K, O.Q5_K, 24),
    ("2048-q5k-q3kdown-300", dict(capas=2, dim=2048, cabezas=16, cabezas_kv=2, ffn=1024,
                                  vocab=1000, contexto=400, rope=1e6), O.Q5_K, O.Q3_K, 300),
    ("512-q2k-q3kdown", dict(capas=2, dim=512, cabezas=8, cabezas_kv=2, ffn=1536, vocab=1500,
                             contexto=200, rope=10000.0), O.Q2_K, O.Q3_K, 24),
    ("896-q8_0", dict(capas=2, dim=896, cabezas=14, cabezas_kv=2, ffn=4864, vocab=640,
                      contexto=200), O.Q8_0, O.Q8_0, 40),
]


@pytest.mark.parametrize("name,cfg,t,tdown,plen", VARIED, ids=[c[0] for c in VARIED])
def test_varied_norms_and_biases_match_oracle(F, name, cfg, t, tdown, plen):
    """Every norm weight ~ N(1, 0.1) (attn_norm, ffn_norm and output_norm,
    each its own draw) and q/k/v biases ~ N(0, 0.3) in every layer, as in
    real files (src/forward.rs:422-436, 472-474, 495-498): the fused norm
    prologues must multiply by the right weight, and the epilogues add the
    right bias. Prefill logits, teacher-forced steps and greedy tokens are
    bit-identical to the oracle's."""
    from gguf_fixtures import vary_norms_and_biases
    c = F.Config(eps=1e-6, **cfg)
    m = F.Modelo(c, tipo=t, semilla=17, tipo_down=tdown, tipo_salida=t)
    names = vary_norms_and_biases(m, seed=len(name))
    assert len(names) == 5 * c.capas + 1
    ref = mirror(m)
    prompt = np.random.default_rng(plen).integers(0, c.vocab, plen).astype(np.uint32)
    cache, rc = m.nueva_cache(plen + 40), ref.new_cache(plen + 40)
    lg, _ = m.forward(prompt, cache)
    want = ref.forward(prompt, rc)
    assert np.array_equal(lg.view(np.uint32), want.view(np.uint32)), name
    tok = O.argmax(want)
    for step in range(4):
        lg, _ = m.forward([tok], cache)
        want = ref.forward([tok], rc)
        assert np.array_equal(lg.view(np.uint32), want.view(np.uint32)), (name, step)
        tok = O.argmax(want)
    got = m.generar(prompt, 16, m.nueva_cache(plen + 40))
    exp = ref.generate(prompt, 16, ref.new_cache(plen + 40))
    assert np.array_equal(got, exp), (name, got, exp)


def test_long_cache_attention_path_bit_identical_to_oracle(F):
    """Caches above 4096 tokens stream the scores through LDS instead of
    holding them (cx_attn.hip); the arithmetic order is still the
    reference's, so logits stay bit-identical: a 4200-token cache, a
    150-token prefill and 24 teacher-forced steps, then greedy tokens."""
    c = F.Config(capas=1, dim=2048, cabezas=16, cabezas_kv=2, ffn=2048, vocab=800,
                 contexto=5000, rope=1e6)
    m = F.Modelo(c, semilla=5)
    ref = mirror(m)
    prompt = np.random.default_rng(2).integers(0, 800, 150).astype(np.uint32)
    cache, rc = m.nueva_cache(4200), ref.new_cache(4200)
    lg, _ = m.forward(prompt, cache)
    want = ref.forward(prompt, rc)
    for step in range(24):
        assert np.array_equal(lg.view(np.uint32), want.view(np.uint32)), step
        tok = O.argmax(want)
        lg, _ = m.forward([tok], cache)
        want = ref.forward([tok], rc)
    got = m.generar(prompt, 12, m.nueva_cache(4200))
    exp = ref.generate(prompt, 12, ref.new_cache(4200))
    assert np.array_equal(got, exp)


def test_cache_truncate_and_prefix_reuse(F):  # src/forward.rs:98-127
    c = F.Config(capas=2, dim=256, cabezas=4, cabezas_kv=2, ffn=768, vocab=500, contexto=128)
    m = F.Modelo(c, semilla=3)
    p = np.arange(20, dtype=np.uint32) * 7 % 500
    a = m.nueva_cache(64)
    la, _ = m.forward(p, a)
    a.truncar(12)
    assert a.largo() == 12
    lb, _ = m.forward(p[12:], a)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    a.limpiar()
    lc, _ = m.forward(p, a)
    assert np.array_equal(la.view(np.uint32), lc.view(np.uint32))
    with pytest.raises(Exception):
        m.forward(np.arange(60, dtype=np.uint32), a)  # past the cache
    with pytest.raises(Exception):
        m.forward([500], a)  # not in the vocabulary


def test_generate_stops_at_eos(F):  # src/forward.rs:544-557
    c = F.Config(capas=1, dim=256, cabezas=4, cabezas_kv=2, ffn=768, vocab=500, contexto=128)
    m = F.Modelo(c, semilla=9)
    p = np.array([1, 2, 3, 4], np.uint32)
    full = m.generar(p, 10, m.nueva_cache(64))
    eos = int(full[3])
    first = int(np.nonzero(full == eos)[0][0])
    cache = m.nueva_cache(64)
    cut = m.generar(p, 10, cache, fin=eos)
    assert np.array_equal(cut, full[:first])
    assert cache.largo() == len(p) + first


def test_generator_matches_oracle_rows(F):
    """GPU daiss rows vs the host restatement: the xorshift stream is exact;
    the normals use the device's logf/cosf/sinf, so allow an ulp or two."""
    c = F.Config(capas=1, dim=256, cabezas=4, cabezas_kv=2, ffn=768, vocab=300, contexto=64)
    m = F.Modelo(c, semilla=11)
    names = [t[0] for t in m.tensores()]
    emb = m.tensor(names.index("token_embd.weight")).reshape(300, 256)
    for r in (0, 1, 299):
        want = O.daiss_row(11, "token_embd.weight", r, 0.02, 256)
        assert np.allclose(emb[r], want, rtol=4e-6, atol=1e-9)
    i = names.index("blk.0.ffn_gate.weight")
    q = m.tensor(i)
    want = O.daiss_matrix(11, "blk.0.ffn_gate.weight", 768, 256, 0.02, O.Q4_K)
    same = np.mean(np.all(q == want, axis=1))
    assert same > 0.95, same
    norm = m.tensor(names.index("blk.0.attn_norm.weight"))
    bias = m.tensor(names.index("blk.0.attn_q.bias"))
    assert (norm == 1.0).all() and (bias == 0.0).all()


def test_lm_head_argmax_ties_and_nan(F):
    """The decode step's argmax runs in the lm_head's epilogue (each row tile
    writes its largest logit and row, one launch reduces the pairs): the
    reference's argmax (src/sampler.rs:129-137) over the whole vocabulary,
    the first index among equal maxima, a NaN never winning. The row with
    the largest logit is copied into rows 70 and 2800 (other tiles of the
    lm_head's 8-row tiles), and row 3's first block scale is set to NaN (f16
    0x7E00); logits bit-identical to the oracle's and the token its argmax,
    in the decode step and after a prefill."""
    from cosxamix_amd import _lib as L
    from gguf_fixtures import write_tensor
    c = F.Config(capas=1, dim=2048, cabezas=16, cabezas_kv=2, ffn=1024, vocab=3000, contexto=64)
    m = F.Modelo(c, tipo=L.Q4_K, semilla=77, tipo_salida=L.Q4_K)
    try:
        io = [x[0] for x in m.tensores()].index("output.weight")
        W = m.tensor(io)
        rb = W.shape[1]
        lg, am = m.forward(np.array([5], np.uint32), m.nueva_cache(8))
        j = int(np.argmax(lg))
        assert am == j
        for r in (70, 2800):
            write_tensor(m, io, W[j], byte_offset=r * rb)
        row3 = W[3].copy()
        row3[0:2] = (0x00, 0x7E)
        write_tensor(m, io, row3, byte_offset=3 * rb)
        ref = mirror(m)
        for prompt in ([5], [5, 9], [9]):
            lg, am = m.forward(np.array(prompt, np.uint32), m.nueva_cache(8))
            want = ref.forward(np.array(prompt, np.uint32), ref.new_cache(8))
            assert np.isnan(lg[3]) and np.isnan(want[3])  # (NaN payloads may differ)
            fin = np.arange(c.vocab) != 3
            assert np.array_equal(lg[fin].view(np.uint32), want[fin].view(np.uint32)), prompt
            top = np.nanmax(want)
            assert am == O.argmax(want) == int(np.nonzero(want == top)[0][0]), (prompt, am)
        # the tie itself, for the prompt the copies were made from
        lg, am = m.forward(np.array([5], np.uint32), m.nueva_cache(8))
        assert lg[70] == lg[2800] == lg[j] and am == min(j, 70)
    finally:
        m.close()
