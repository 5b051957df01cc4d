"""BASELINE.json's configurations 3, 4 and 5 at their own workloads, through
the HIP path against the oracle (GPU).

- Config 3: the daiss-3b model (36 layers, every linear Q4_K, vocab 151936),
  the bench's seeded 512-token prompt, bit-identical logits after the
  prefill and at teacher-forced steps, and the 128 greedy tokens identical.
- Config 4: both Q4_K matrices (11008 x 2048 and 2048 x 11008, N(0, 0.02)
  quantized by the quantizer) times 8, 32 and 512 seeded N(0, 1) rows through
  matmul_auto (int8 MFMA for m > 1), every output bit-identical to the
  reference's per-row matmul (ops::matmul_i8_fusionado, src/ops.rs:435-522)
  as the oracle restates it.
- Config 5: the Llama-3-8B shape (32/8 heads of 128, SwiGLU 14336, vocab
  128256, rope 5e5; Q4_K linears, Q5_K ffn_down, Q4_K lm_head) at 2 of its
  32 layers, an 8192-token seeded prefix prefilled through cx_forward (the
  chunked prefill and the streamed-score attention past 4096 positions at
  32/8 heads), then bit-identical teacher-forced logits and 16 identical
  greedy tokens; and the whole model (all 32 layers, the bench's weights)
  after a 4200-token prefix (positions past 4096), bit-identical logits at
  4 teacher-forced steps and 12 identical greedy tokens.
Bars: bit-identical logits (so max-abs 0 <= the north star's 1e-3) and
identical greedy tokens; matmul outputs bit-identical."""
import sys
import time

import numpy as np
import pytest
import torch

from bench import prompt_tokens
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


def note(*a):
    """A progress line (seen with pytest -s: these tests run for minutes)."""
    print(f"[{time.strftime('%H:%M:%S')}]", *a, file=sys.stderr, flush=True)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.timeout(600)
def test_config3_prompt_512_and_128_greedy_tokens(F):
    m = F.Modelo(F.DAISS_3B, semilla=42)
    ref = mirror(m)
    note("config 3: model on the host")
    prompt = prompt_tokens(512, F.DAISS_3B.vocab)
    cache, rc = m.nueva_cache(512 + 129), ref.new_cache(512 + 129)
    lg, _ = m.forward(prompt, cache)
    want = ref.forward(prompt, rc)
    note("config 3: prompt forwarded")
    assert same_bits(lg, want)
    for step in range(3):  # teacher-forced: the oracle's token to both
        tok = O.argmax(want)
        lg, am = m.forward([tok], cache)
        want = ref.forward([tok], rc)
        assert same_bits(lg, want), step
        assert am == O.argmax(want)
    got = m.generar(prompt, 128, m.nueva_cache(512 + 129))
    exp = ref.generate(prompt, 128, ref.new_cache(512 + 129))
    note("config 3: 128 tokens generated")
    assert len(got) == 128 and np.array_equal(got, exp), np.nonzero(got != exp)[0][:5]
    m.close()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("n,k", [(11008, 2048), (2048, 11008)])
def test_config4_every_output_equals_the_per_row_matmul(dev, n, k):
    from cosxamix_amd import ops
    w = O.daiss_matrix(42, f"config4.{n}x{k}", n, k, 0.02, O.Q4_K)
    wd = torch.from_numpy(w).to(dev)
    for m in (8, 32, 512):
        x = np.random.default_rng(m * 7 + n).normal(0, 1, (m, k)).astype(np.float32)
        dst = torch.empty((m, n), dtype=torch.float32, device=dev)
        ops.matmul_auto((m, k, n), torch.from_numpy(x).to(dev), wd, O.Q4_K, dst)
        want = O.matmul_fused(O.Q4_K, x, w, n, threads=16)
        note(f"config 4: {n}x{k} m={m}")
        got = dst.cpu().numpy()
        assert same_bits(got, want), (m, np.argwhere(got.view(np.uint32) != want.view(np.uint32))[:5])


@pytest.mark.timeout(900)
def test_config5_8192_prefix_two_layers(F):
    c = F.Config(capas=2, dim=4096, cabezas=32, cabezas_kv=8, ffn=14336, vocab=128256,
                 contexto=8192 + 64, eps=1e-5, rope=500_000.0)
    m = F.Modelo(c, tipo=O.Q4_K, semilla=8, tipo_down=O.Q5_K, tipo_salida=O.Q4_K)
    ref = mirror(m)
    note("config 5: model on the host")
    prefix = prompt_tokens(8192, c.vocab, seed=5)
    cache, rc = m.nueva_cache(8192 + 40), ref.new_cache(8192 + 40)
    lg, _ = m.forward(prefix, cache)
    note("config 5: prefix prefilled on the GPU")
    want = ref.forward(prefix, rc)
    note("config 5: prefix forwarded by the oracle")
    assert same_bits(lg, want)
    for step in range(16):
        tok = O.argmax(want)
        lg, _ = m.forward([tok], cache)
        want = ref.forward([tok], rc)
        assert same_bits(lg, want), step
    tok = np.array([O.argmax(want)], np.uint32)
    got = m.generar(tok, 16, cache)
    exp = ref.generate(tok, 16, rc)
    assert np.array_equal(got, exp), (got, exp)
    assert cache.largo() == rc.len == 8192 + 16 + 17
    note("config 5: steps and tokens equal")
    m.close()


@pytest.mark.timeout(900)
def test_config5_full_depth(F):
    """The bench's config-5 model itself, all 32 layers (its weights:
    semilla 8): a 4200-token prefix (the chunked prefill, then decode
    attention past 4096 positions), 4 teacher-forced steps and 12 greedy
    tokens, each side continuing on its own cache."""
    c = F.LLAMA3_8B
    m = F.Modelo(c, tipo=O.Q4_K, semilla=8, tipo_down=O.Q5_K, tipo_salida=O.Q4_K)
    ref = mirror(m)
    note("config 5 full depth: model on the host")
    n0 = 4200
    prefix = prompt_tokens(n0, c.vocab, seed=5)
    cap = n0 + 40
    cache, rc = m.nueva_cache(cap), ref.new_cache(cap)
    lg, _ = m.forward(prefix, cache)
    want = ref.forward(prefix, rc)
    note("config 5 full depth: prefix forwarded by both")
    assert same_bits(lg, want)
    for step in range(4):  # teacher-forced: the oracle's token to both
        tok = O.argmax(want)
        lg, am = m.forward([tok], cache)
        want = ref.forward([tok], rc)
        assert same_bits(lg, want), step
        assert am == O.argmax(want)
    got, exp = [], []
    tg = te = O.argmax(want)
    for _ in range(12):  # greedy, each side from its own logits
        got.append(tg)
        exp.append(te)
        lg, tg = m.forward([tg], cache)
        want = ref.forward([te], rc)
        te = O.argmax(want)
    got.append(tg)
    exp.append(te)
    note("config 5 full depth: tokens generated")
    assert got == exp, (got, exp)
    assert same_bits(lg, want)
    assert cache.largo() == rc.len == n0 + 4 + 12
    m.close()
