"""The batched prefill on the GPU (MI355X): Modelo::forward over several
tokens (src/forward.rs:375-505) runs one pass per layer over chunks of
tokens (the int8 MFMA contraction for Q4_K/Q5_K, the GEMV row by row for
other types, the decode attention kernels with one query per grid slice).
It must give what feeding the same tokens one at a time gives, bit for bit:
the logits of the last token, and through the KV cache every later step.
Both attention paths are covered (scores held in LDS for caches up to
4096 tokens, streamed above), prompts longer than one chunk, a prefill that
starts at a nonzero cache length, and a model whose matrices take the
row-by-row fallback."""
import numpy as np
import pytest

from gguf_fixtures import mirror, mixed_model, oracle_of
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def F(dev):
    from cosxamix_amd import forward
    return forward


def tokens(n, vocab, seed):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.uint32)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def check_model(F, m, cap, n_prompt, n_more, seed):
    """forward(prompt) vs one token at a time, then a second multi-token
    forward at a nonzero length, then greedy steps from both caches."""
    V = m.cfg.vocab
    prompt, more = tokens(n_prompt, V, seed), tokens(n_more, V, seed + 1)
    a, b = m.nueva_cache(cap), m.nueva_cache(cap)
    la, ta = m.forward(prompt, a)
    for t in prompt:
        lb, tb = m.forward(np.array([t], np.uint32), b)
    assert same_bits(la, lb) and ta == tb
    assert a.largo() == b.largo() == n_prompt
    la, ta = m.forward(more, a)
    for t in more:
        lb, tb = m.forward(np.array([t], np.uint32), b)
    assert same_bits(la, lb) and ta == tb
    for _ in range(4):  # the caches hold the same keys and values
        la, ta = m.forward(np.array([ta], np.uint32), a)
        lb, tb = m.forward(np.array([tb], np.uint32), b)
        assert same_bits(la, lb) and ta == tb
    return prompt


@pytest.mark.parametrize("cap", [512, 4160], ids=["lds-scores", "streamed-scores"])
def test_prefill_equals_token_by_token_daiss(F, cap):
    # Q5_K attention and gate/up (contraction), Q3_K ffn_down (row by row),
    # Q4_K lm_head; 300 tokens = two chunks
    cfg = F.Config(2, 256, 4, 2, 512, 640, 4608)
    m = F.Modelo(cfg, tipo=O.Q5_K, semilla=21, tipo_down=O.Q3_K, tipo_salida=O.Q4_K)
    check_model(F, m, cap, 300, 37, seed=3)


def test_prefill_equals_token_by_token_mixed_gguf(F, tmp_path):
    # Q3_K..Q6_K per tensor, quantized tied embedding, biases in layer 0 only;
    # against the oracle too
    data, host, types = mixed_model(seed=8, ctx=1024)
    p = tmp_path / "mixed.gguf"
    p.write_bytes(data)
    m = F.Modelo.abrir(p)
    prompt = check_model(F, m, 600, 270, 20, seed=4)
    ref = oracle_of(host, types, ctx=1024)
    c = m.nueva_cache(600)
    lg, _ = m.forward(prompt, c)
    assert same_bits(lg, ref.forward(prompt, ref.new_cache(600)))


def test_generate_after_prefill_matches_oracle(F):
    # cx_generate prefills the prompt, then decodes; the oracle runs the
    # reference's token loop (src/forward.rs:533-559)
    cfg = F.Config(2, 256, 4, 2, 512, 640, 1024)
    m = F.Modelo(cfg, tipo=O.Q4_K, semilla=5)
    prompt = tokens(257, cfg.vocab, 9)  # one chunk and one token
    got = m.generar(prompt, 16, m.nueva_cache(512))
    ref = mirror(m)
    want = ref.generate(prompt, 16, ref.new_cache(512))
    assert np.array_equal(got, want)
