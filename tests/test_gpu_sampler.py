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


def first_u(seed):
    """u of the sampler's first draw (Azar::siguiente, src/daiss.rs:330-337;
    uniforme, src/sampler.rs:55-58)."""
    M = 2**64 - 1
    x = (seed & M) or 0x9E3779B97F4A7C15
    x ^= x >> 12
    x ^= (x << 25) & M
    x ^= x >> 27
    return np.float32(((x * 0x2545F4914F6CDD1D) & M) >> 40) / np.float32(16777216.0)


def test_targets_on_exact_running_sums(S, dev):
    """The three running-sum searches with targets equal to a running sum,
    past the first 256 positions and the first 2048-position stage of the
    GPU's sums: the draw over the index order (the first sum > u), the
    nucleus cut (the first sum >= top_p enters) and the draw inside the
    nucleus (the first sum > u * total). Each case is chosen so that a search
    stopping one position early or late, or using the other inequality,
    returns another token; the expected tokens come from the running sums
    here and are checked against the oracle too."""
    n = 151936
    lg = logits_of("soft", n, 5)
    p = O.softmax(lg, n)  # temperature 1: z = logit
    run = np.cumsum(p, dtype=np.float32)  # in order, one f32 add a position
    order = np.lexsort((np.arange(n), -p))  # descending, ties by index
    rund = np.cumsum(p[order], dtype=np.float32)
    d = torch.from_numpy(lg).to(dev)
    us = [(s, first_u(s)) for s in range(1, 60000)]

    def first_above(r, t, last):
        i = int(np.searchsorted(r[:last + 1], t, side="right"))
        return min(i, last)

    def check(seed, top_p, want):
        assert O.Sampler(seed, 1.0, top_p).choose(lg) == want, (seed, top_p)
        assert S.Muestreador(seed, 1.0, top_p).elegir(d) == want, (seed, top_p)

    # 1. top_p = 1: u equals run[i]; the token is i + 1 (i with >=)
    hits = [(s, int(np.searchsorted(run, u))) for s, u in us]
    hits = [(s, i) for s, i in hits if 2048 < i < n - 1 and run[i] == us[s - 1][1]]
    assert len(hits) >= 2
    for s, i in hits[:3]:
        assert run[i + 1] > run[i]
        check(s, 1.0, i + 1)
    # 2. top_p = rund[j]: the nucleus is order[0..j] (j in the candidates, and
    # past them); u close enough to 1 that the draw takes its last token, and
    # would take order[j + 1] from a nucleus one longer
    for j in (700, 1500, 5000):
        top_p = float(rund[j])
        found = 0
        for s, u in us:
            want = first_above(rund, np.float32(u * rund[j]), j)
            late = first_above(rund, np.float32(u * rund[j + 1]), j + 1)
            if want == j and late == j + 1:
                check(s, top_p, int(order[j]))
                found += 1
                if found == 2:
                    break
        assert found == 2, j
    # 3. the draw inside a nucleus of 100,001 tokens: u * total equals rund[i]
    J = 100000
    top_p = float(rund[J])
    found = 0
    for s, u in us:
        t = np.float32(u * rund[J])
        i = int(np.searchsorted(rund[:J + 1], t))
        if 2048 < i < J and rund[i] == t:
            assert rund[i + 1] > t
            check(s, top_p, int(order[i + 1]))
            found += 1
            if found == 3:
                break
    assert found == 3
