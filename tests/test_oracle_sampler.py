"""The oracle's sampler (sampler::Muestreador, src/sampler.rs:27-152) on the
CPU: the reference's own sampler tests (src/sampler.rs:154-240) and closed
forms of its arithmetic."""
import numpy as np
import pytest


@pytest.fixture(scope="module")
def O():
    from oracle import oracle
    return oracle


def azar_u(state: int):
    """Azar::siguiente (src/daiss.rs:330-337) and the uniform of
    src/sampler.rs:55-58, in Python integers: (next state, u)."""
    M = 2**64 - 1
    x = state
    x ^= x >> 12
    x ^= (x << 25) & M
    x ^= x >> 27
    r = (x * 0x2545F4914F6CDD1D) & M
    return x, np.float32(r >> 40) / np.float32(16777216.0)


def test_greedy_is_the_max(O):  # src/sampler.rs:158-164
    s = O.Sampler(0, 0.0, 1.0)
    assert s.choose([0.1, 3.0, 2.0, 3.0]) == 1
    assert s.choose([-5.0, -1.0, -3.0]) == 1
    assert s.choose([1.0]) == 0
    assert s.state == 0x9E3779B97F4A7C15  # no draw when greedy
    assert O.Sampler(5, 1.0, 1.0).choose([]) == 0  # empty logits


def test_the_nucleus_cuts_the_tail(O):  # src/sampler.rs:171-179
    lg = np.zeros(5000, np.float32)
    lg[42] = 10.0
    s = O.Sampler(7, 1.0, 0.5)
    assert all(s.choose(lg) == 42 for _ in range(200))


def test_frequencies_follow_the_probabilities(O):  # src/sampler.rs:185-201
    lg = np.log(np.array([0.5, 0.3, 0.2], np.float32))
    s = O.Sampler(12345, 1.0, 1.0)
    n = 30_000
    counts = np.bincount([s.choose(lg) for _ in range(n)], minlength=3)
    for i, want in enumerate([0.5, 0.3, 0.2]):
        assert abs(counts[i] / n - want) < 0.015, (i, counts)


def test_a_flat_distribution_takes_the_full_order(O):  # src/sampler.rs:205-219
    lg = np.ones(5000, np.float32)
    s = O.Sampler(3, 1.0, 0.9)
    seen = {s.choose(lg) for _ in range(3000)}
    assert len(seen) > 1024, len(seen)


def test_the_seed_decides(O):  # src/sampler.rs:222-239
    lg = np.sin(np.arange(300, dtype=np.float32) * np.float32(0.07))
    a = O.Sampler(99, 0.8, 0.9)
    b = O.Sampler(99, 0.8, 0.9)
    assert [a.choose(lg) for _ in range(50)] == [b.choose(lg) for _ in range(50)]
    c = O.Sampler(100, 0.8, 0.9)
    assert [c.choose(lg) for _ in range(50)] != [a.choose(lg) for _ in range(50)]


def test_one_draw_per_choice_and_its_uniform(O):
    """One Azar draw per call with temperature; with top_p = 1 the token is
    the first index whose sequential running sum of the softmax exceeds u
    (src/sampler.rs:79-81, 139-152)."""
    rng = np.random.default_rng(4)
    lg = rng.normal(0, 2, 700).astype(np.float32)
    s = O.Sampler(2024, 0.7, 1.0)
    st = s.state
    for _ in range(20):
        st, u = azar_u(st)
        z = lg * np.float32(1.0 / np.float32(0.7))
        p = z.copy()
        O.lib.orc_softmax(O._p(p, O._f32p), p.size, p.size)
        run = np.cumsum(p, dtype=np.float32)  # add.accumulate: sequential
        want = int(np.argmax(run > u)) if (run > u).any() else p.size - 1
        assert s.choose(lg) == want
        assert s.state == st


def test_top_p_prefix_of_the_descending_order(O):
    """top_p < 1: the shortest prefix of the descending order whose running
    sum reaches top_p, then the running sum against u * total; ties by index."""
    lg = np.array([2.0, 1.0, 2.0, 0.5, 1.0, -1.0], np.float32)
    s = O.Sampler(11, 1.0, 0.6)
    st = s.state
    p = lg.copy()
    O.lib.orc_softmax(O._p(p, O._f32p), p.size, p.size)
    order = sorted(range(p.size), key=lambda i: (-p[i], i))
    acc, cut = np.float32(0), len(order)
    for i, t in enumerate(order):
        acc = np.float32(acc + p[t])
        if acc >= np.float32(0.6):
            cut = i + 1
            break
    total = np.float32(0)
    for t in order[:cut]:
        total = np.float32(total + p[t])
    for _ in range(30):
        st, u = azar_u(st)
        target, run, want = np.float32(u * total), np.float32(0), order[cut - 1]
        for t in order[:cut]:
            run = np.float32(run + p[t])
            if run > target:
                want = t
                break
        assert s.choose(lg) == want
