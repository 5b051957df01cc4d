"""The GPU sampler (cx_sample: sampler::Muestreador::elegir,
src/sampler.rs:61-152) against the oracle's, token for token and generator
state for generator state; then Modelo::generar with a sampler
(src/forward.rs:533-559) against the oracle's loop."""
import numpy as np
import pytest
import torch

from gguf_fixtures import mirror
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def S(dev):
    from cosxamix_amd import sampler
    return sampler


def logits_of(kind, n, seed):
    rng = np.random.default_rng(seed)
    if kind == "normal":
        return rng.normal(0, 3, n).astype(np.float32)
    if kind == "peaked":
        x = rng.normal(0, 1, n).astype(np.float32)
        x[rng.integers(0, n, 5)] += 12.0
        return x
    if kind == "flat":  # every probability equal: the full order, ties by index
        return np.ones(n, np.float32)
    if kind == "steps":  # many exact ties at several levels
        return (rng.integers(0, 6, n) * 0.5).astype(np.float32)
    if kind == "soft":  # nearly flat and untied: the random-init model's logits
        return rng.normal(0, 0.3, n).astype(np.float32)
    raise ValueError(kind)


CASES = [
    ("normal", 151936, 0.8, 0.9), ("normal", 151936, 1.0, 1.0), ("normal", 151936, 1.5, 0.5),
    ("peaked", 151936, 0.7, 0.95), ("normal", 3000, 1.0, 0.0), ("flat", 5000, 1.0, 0.9),
    ("steps", 4000, 1.0, 0.7), ("normal", 1, 1.0, 0.9), ("normal", 7, 2.0, 1.0),
    ("peaked", 128256, 0.6, 1.0), ("flat", 151936, 0.8, 0.9), ("soft", 151936, 0.8, 0.9),
    ("soft", 151936, 1.0, 0.999), ("steps", 100000, 1.0, 0.95),
]


@pytest.mark.parametrize("kind,n,temp,top_p", CASES,
                         ids=[f"{k}-{n}-t{t}-p{p}" for k, n, t, p in CASES])
def test_sampler_matches_oracle(S, dev, kind, n, temp, top_p):
    lg = logits_of(kind, n, n + int(temp * 10))
    d = torch.from_numpy(lg).to(dev)
    g = S.Muestreador(1234 + n, temp, top_p)
    o = O.Sampler(1234 + n, temp, top_p)
    draws = 12 if n > 100000 else 30
    got = [g.elegir(d) for _ in range(draws)]
    want = [o.choose(lg) for _ in range(draws)]
    assert got == want
    assert g.estado == o.state


def test_a_nan_top_p_keeps_the_candidates(S, dev):
    """top_p NaN (f32::clamp keeps it): the candidates' mass is not below it,
    so the nucleus is the 1024 most probable tokens, whole
    (src/sampler.rs:96-114)."""
    lg = logits_of("soft", 20000, 3)
    d = torch.from_numpy(lg).to(dev)
    g = S.Muestreador(77, 1.0, float("nan"))
    o = O.Sampler(77, 1.0, float("nan"))
    got = [g.elegir(d) for _ in range(20)]
    assert got == [o.choose(lg) for _ in range(20)]
    order = np.lexsort((np.arange(lg.size), -lg))  # descending logit, then index
    assert set(got) <= set(order[:1024].tolist())


def test_greedy_and_empty(S, dev):
    g = S.Muestreador.voraz()
    assert g.elegir(torch.tensor([0.1, 3.0, 2.0, 3.0], device=dev)) == 1
    assert g.estado == 0x9E3779B97F4A7C15  # no draw
    assert S.Muestreador(5, 1.0, 1.0).elegir(torch.empty(0, device=dev)) == 0


def test_the_nucleus_cuts_the_tail(S, dev):  # src/sampler.rs:171-179
    lg = torch.zeros(5000, device=dev)
    lg[42] = 10.0
    g = S.Muestreador(7, 1.0, 0.5)
    assert all(g.elegir(lg) == 42 for _ in range(50))


def test_generate_with_sampler_matches_oracle(S, dev):
    from cosxamix_amd import forward as F
    cfg = F.Config(2, 256, 4, 2, 512, 640, 512)
    m = F.Modelo(cfg, tipo=O.Q4_K, semilla=3)
    ref = mirror(m)
    prompt = np.random.default_rng(1).integers(0, 640, 40).astype(np.uint32)
    for temp, top_p, seed in ((0.8, 0.9, 77), (1.3, 1.0, 5), (0.5, 0.3, 0)):
        g = S.Muestreador(seed, temp, top_p)
        o = O.Sampler(seed, temp, top_p)
        got = m.generar(prompt, 24, m.nueva_cache(256), muestreador=g)
        want = O.generate_sampled(ref, prompt, 24, o, ref.new_cache(256))
        assert np.array_equal(got, want), (temp, top_p)
        assert g.estado == o.state  # the draws the reference makes, no more
        # the same sampler continues its sequence in a second generation
        got2 = m.generar(prompt[:10], 8, m.nueva_cache(256), muestreador=g)
        want2 = O.generate_sampled(ref, prompt[:10], 8, o, ref.new_cache(256))
        assert np.array_equal(got2, want2)
        assert g.estado == o.state


def test_generate_with_sampler_stops_at_the_end_token(S, dev):
    from cosxamix_amd import forward as F
    cfg = F.Config(2, 256, 4, 2, 512, 640, 512)
    m = F.Modelo(cfg, tipo=O.Q4_K, semilla=3)
    ref = mirror(m)
    prompt = np.random.default_rng(2).integers(0, 640, 12).astype(np.uint32)
    full = O.generate_sampled(ref, prompt, 30, O.Sampler(9, 1.0, 1.0), ref.new_cache(256))
    eos = int(full[7])
    first = int(np.argmax(full == eos))
    g, o = S.Muestreador(9, 1.0, 1.0), O.Sampler(9, 1.0, 1.0)
    got = m.generar(prompt, 30, m.nueva_cache(256), fin=eos, muestreador=g)
    want = O.generate_sampled(ref, prompt, 30, o, ref.new_cache(256), eos=eos)
    assert np.array_equal(got, want) and len(got) == first
    assert g.estado == o.state  # the end token's draw counted
