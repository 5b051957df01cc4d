"""The boundary's contracts beyond the arithmetic (GPU, through the C ABI):

- the level-1 kernel contract is reentrant and thread-safe like the
  reference's pure `type Kernel` (src/kernels/q2k.rs:153), which rayon calls
  from many threads at once (src/ops.rs:487-500);
- level-2 operators on several host threads do not share scratch;
- Cache::prefijo / Cache::bytes (src/forward.rs:117-136) and the session
  prefix borrowing of MotorPropio (src/engine_own.rs:227-245);
- Modelo::generar's stopping rules (src/forward.rs:544-557): the stop token
  is neither returned nor forwarded, al_token stops at once, and the cache
  holds the prompt plus the forwarded tokens; a cache smaller than
  n + max_new is fine when generation stops first;
- a model freed before its caches.
Bars: bit-identical results (same kernels, same inputs) and the oracle's
tokens and logits."""
import concurrent.futures as cf
import ctypes as C
import threading

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def F(dev):
    from cosxamix_amd import forward
    return forward


def _golden_rows(golden, t, k):
    n = f"{O.NAMES[t]}_{k}"
    refs = {key: golden[key] for key in golden.files if key.startswith(f"{n}_normal_ref_")}
    return golden[f"{n}_w"], [golden[f"{n}_normal_{s}"] for s in ("xq", "xe", "xs")], refs


def test_kernel_contract_is_thread_safe(dev, golden):
    """8 host threads call cx_dot_q4k_i8 and cx_dot_q3k_i8 at once on
    different golden rows (3 rounds each, started together): every result is
    the bits the same call gives alone, and the rows stay within the
    reference kernels' bar."""
    from cosxamix_amd import kernels
    cases = []
    for t in (O.Q4_K, O.Q3_K):
        for k in (2048, 11008):
            w, (xq, xe, xs), refs = _golden_rows(golden, t, k)
            alone = np.array([kernels.dot_qk_i8(t, r, xq, xe, xs) for r in w], np.float32)
            for want in refs.values():
                err = np.linalg.norm(alone - want) / np.linalg.norm(want)
                assert err <= 1e-5, (O.NAMES[t], k, err)
            cases.append((t, w, xq, xe, xs, alone))
    start = threading.Barrier(8)

    def work(tid):
        start.wait()
        bad = []
        for rnd in range(3):
            for ci, (t, w, xq, xe, xs, alone) in enumerate(cases):
                rows = range((tid + rnd) % 8, len(w), 8)  # a different slice per thread and round
                for r in rows:
                    got = np.float32(kernels.dot_qk_i8(t, w[r], xq, xe, xs))
                    if got.view(np.uint32) != alone[r].view(np.uint32):
                        bad.append((tid, rnd, ci, r, float(got), float(alone[r])))
        return bad

    with cf.ThreadPoolExecutor(8) as ex:
        bad = [b for f in [ex.submit(work, i) for i in range(8)] for b in f.result()]
    assert not bad, bad[:10]


def test_operators_on_several_threads_do_not_share_scratch(dev):
    """cx_matmul_auto quantizes its rows into per-thread scratch: 4 threads,
    each on its own stream, give the bits of the same calls made alone."""
    from cosxamix_amd import ops
    n, k = 1024, 2048
    w = torch.from_numpy(O.daiss_matrix(3, "w", n, k, 0.02, O.Q4_K)).to(dev)
    xs = [torch.randn(m, k, generator=torch.Generator().manual_seed(m), dtype=torch.float32).to(dev)
          for m in (1, 3, 8, 32)]
    def mm(x):
        y = torch.empty(x.shape[0], n, dtype=torch.float32, device=dev)
        ops.matmul_auto((x.shape[0], k, n), x, w, O.Q4_K, y)
        return y

    alone = [mm(x).cpu() for x in xs]
    torch.cuda.synchronize()
    start = threading.Barrier(4)

    def work(i):
        s = torch.cuda.Stream(device=dev)
        start.wait()
        with torch.cuda.stream(s):
            outs = [mm(xs[i]) for _ in range(20)]
        s.synchronize()
        return [o.cpu() for o in outs]

    with cf.ThreadPoolExecutor(4) as ex:
        res = [f.result() for f in [ex.submit(work, i) for i in range(4)]]
    for i in range(4):
        for o in res[i]:
            assert torch.equal(o.view(torch.int32), alone[i].view(torch.int32)), i


def test_a_thread_that_exits_with_work_queued_hands_its_scratch_on_in_order(dev):
    """Thread A queues 12 cx_matmul_auto calls on its own stream and ends
    without waiting for them; thread B then takes A's context (and scratch)
    from the pool and queues 12 calls on another stream, the first of them
    growing the scratch. B's first use waits, on the device, for A's queued
    work: every output of both threads is the bits of the same call alone."""
    from cosxamix_amd import ops
    n, k = 4096, 2048
    w = torch.from_numpy(O.daiss_matrix(5, "w", n, k, 0.02, O.Q4_K)).to(dev)
    xa = [torch.randn(64, k, generator=torch.Generator().manual_seed(100 + i)).to(dev)
          for i in range(12)]
    xb = [torch.randn(256 if i == 0 else 48, k, generator=torch.Generator().manual_seed(200 + i)).to(dev)
          for i in range(12)]

    def mm(x, y=None):
        y = torch.empty(x.shape[0], n, device=dev) if y is None else y
        ops.matmul_auto((x.shape[0], k, n), x, w, O.Q4_K, y)
        return y

    alone_a = [mm(x).cpu() for x in xa]
    alone_b = [mm(x).cpu() for x in xb]
    torch.cuda.synchronize()
    outs = {}

    def run(name, xs):
        s = torch.cuda.Stream(device=dev)
        with torch.cuda.stream(s):
            ys = [torch.full((x.shape[0], n), float("nan"), device=dev) for x in xs]
            for x, y in zip(xs, ys):
                mm(x, y)
        outs[name] = (s, ys)  # no synchronization before the thread ends

    ta = threading.Thread(target=run, args=("a", xa))
    ta.start()
    ta.join()
    tb = threading.Thread(target=run, args=("b", xb))
    tb.start()
    tb.join()
    for name, alone in (("a", alone_a), ("b", alone_b)):
        s, ys = outs[name]
        s.synchronize()
        for i, (y, want) in enumerate(zip(ys, alone)):
            assert torch.equal(y.cpu().view(torch.int32), want.view(torch.int32)), (name, i)


SMALL = dict(capas=2, dim=256, cabezas=4, cabezas_kv=2, ffn=768, vocab=500, contexto=128)


def test_cache_prefix_and_bytes(F):
    """Cache::prefijo then a forward of the rest equals the forward on the
    original cache, bit for bit (the prefix borrowing of
    src/engine_own.rs:227-245); Cache::bytes counts len tokens of K and V."""
    c = F.Config(**SMALL)
    m = F.Modelo(c, semilla=4)
    per_tok = 2 * c.capas * c.dim_kv() * 4
    p = (np.arange(30, dtype=np.uint32) * 13 + 5) % c.vocab
    a = m.nueva_cache(64)
    assert a.bytes() == 0
    la, _ = m.forward(p, a)
    assert a.bytes() == 30 * per_tok
    b = a.prefijo(18)
    assert b.largo() == 18 and b.bytes() == 18 * per_tok
    lb, _ = m.forward(p[18:], b)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    # the source is unchanged, and keeps decoding as before
    assert a.largo() == 30
    tok = int(np.argmax(la))
    l1, _ = m.forward([tok], a)
    l2, _ = m.forward([tok], b)
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))
    # n past the length copies what there is; a smaller capacity works too
    d = a.prefijo(1000, capacidad=40)
    assert d.largo() == 31
    e = a.prefijo(10, capacidad=12)
    le, _ = m.forward(p[10:12], e)
    ref = a.prefijo(10)
    lr, _ = m.forward(p[10:12], ref)
    assert np.array_equal(le.view(np.uint32), lr.view(np.uint32))
    with pytest.raises(Exception):
        a.prefijo(20, capacidad=10)  # 20 tokens do not fit
    # engine_own: borrow, then truncate to the common prefix
    f = a.prefijo(25)
    f.truncar(9)
    lf, _ = m.forward(p[9:], f)
    assert np.array_equal(la.view(np.uint32), lf.view(np.uint32))


def _oracle_greedy(m, prompt, max_new):
    from test_gpu_model import mirror
    ref = mirror(m)
    return ref.generate(prompt, max_new, ref.new_cache(len(prompt) + max_new + 1))


def test_generate_early_stop_with_a_small_cache(F):
    """The stop token ends generation unforwarded; a cache smaller than
    n + max_new works when generation stops first; the tokens are the
    oracle's."""
    c = F.Config(**SMALL)
    m = F.Modelo(c, semilla=9)
    p = np.array([1, 2, 3, 4, 5], np.uint32)
    exp = _oracle_greedy(m, p, 12)
    eos = int(exp[5])
    first = int(np.nonzero(exp == eos)[0][0])
    cache = m.nueva_cache(len(p) + first)  # room for the forwards before the stop only
    got = m.generar(p, 100, cache, fin=eos)
    assert np.array_equal(got, exp[:first]), (got, exp)
    assert cache.largo() == len(p) + first
    # the same run continues on the cache: forward the next token
    full = m.generar(p, 12, m.nueva_cache(64))
    assert np.array_equal(full, exp)
    # a cache that fills before any stop: an error that carries the tokens
    # made so far (three forwarded, the fourth made with no room for it)
    from cosxamix_amd import _lib as L
    small = m.nueva_cache(len(p) + 3)
    with pytest.raises(L.CacheLlena, match="full") as err:
        m.generar(p, 12, small)
    assert np.array_equal(err.value.tokens, exp[:4]) and small.largo() == len(p) + 3
    # step times: one per step that forwarded a returned token, none for the
    # steps run ahead past the stop
    cache = m.nueva_cache(64)
    got, ms = m.generar(p, 100, cache, fin=eos, tiempos=True)
    assert np.array_equal(got, exp[:first]) and len(ms) == first == cache.largo() - len(p)
    assert np.all(ms > 0), ms


def test_generate_callback_and_stop_list(F):
    """al_token sees every token in order and stops at once on False (that
    token is returned, not forwarded); `fines` holds several stop tokens."""
    c = F.Config(**SMALL)
    m = F.Modelo(c, semilla=12)
    p = np.array([7, 8, 9], np.uint32)
    exp = m.generar(p, 16, m.nueva_cache(64))
    seen = []

    def al_token(t):
        seen.append(t)
        return len(seen) < 4

    cache = m.nueva_cache(64)
    got = m.generar(p, 16, cache, al_token=al_token)
    assert np.array_equal(got, exp[:4]) and seen == list(exp[:4])
    assert cache.largo() == len(p) + 3
    # every token accepted: the whole run, as without a callback
    cache = m.nueva_cache(64)
    got = m.generar(p, 16, cache, al_token=lambda t: True)
    assert np.array_equal(got, exp) and cache.largo() == len(p) + 16
    # two stop tokens: whichever comes first
    a, b = int(exp[9]), int(exp[6])
    cut = min(int(np.nonzero(exp == a)[0][0]), int(np.nonzero(exp == b)[0][0]))
    cache = m.nueva_cache(64)
    got = m.generar(p, 16, cache, fines=[a, b])
    assert np.array_equal(got, exp[:cut]) and cache.largo() == len(p) + cut
    # an exception in the callback stops generation and is raised
    with pytest.raises(KeyError):
        m.generar(p, 16, m.nueva_cache(64), al_token=lambda t: {}[t])


def test_sampled_stream_equals_sampled_generate(F):
    from cosxamix_amd import sampler
    c = F.Config(**SMALL)
    m = F.Modelo(c, semilla=13)
    p = np.array([3, 1, 4, 1, 5], np.uint32)
    a = m.generar(p, 20, m.nueva_cache(64), muestreador=sampler.Muestreador(7, 0.9, 0.8))
    s = sampler.Muestreador(7, 0.9, 0.8)
    b = m.generar(p, 20, m.nueva_cache(64), muestreador=s, al_token=lambda t: True)
    assert np.array_equal(a, b)


def test_model_freed_before_its_cache(dev):
    """cx_model_free with a live cache defers the release to the last
    cx_cache_free; the cache stays usable until then."""
    from cosxamix_amd import _lib as L
    lib = L.load()
    cfg = L.CxConfig(1, 256, 4, 2, 768, 300, 64, 1e-6, 10000.0)
    mh, ch = C.c_void_p(), C.c_void_p()
    L.check(lib.cx_model_create_daiss(C.byref(cfg), L.Q4_K, L.Q4_K, L.Q4_K, 5, C.byref(mh)), "model")
    L.check(lib.cx_cache_new(mh, 32, C.byref(ch)), "cache")
    lib.cx_model_free(mh)
    toks = np.array([1, 2, 3], np.uint32)
    am = C.c_uint32()
    L.check(lib.cx_forward(mh, ch, toks.ctypes.data_as(L._u32p), 3, None, C.byref(am)), "forward")
    c2 = C.c_void_p()
    assert lib.cx_cache_new(mh, 32, C.byref(c2)) != 0  # no new cache on a freed model
    lib.cx_cache_free(ch)  # releases the model too


def test_stream_read_probe(dev):
    """cx_stream_read (the bench's read-peak probe) reads the whole buffer:
    its fold reaches the sink only for the data that makes it 0x9E3779B9."""
    import ctypes as C
    from cosxamix_amd import _lib as L
    lib = L.load()
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    for nbytes in (16, 4096, 5 << 20, (5 << 20) + 48):
        buf = torch.zeros(nbytes // 4, dtype=torch.int32, device=dev)
        L.check(lib.cx_stream_read(C.c_void_p(buf.data_ptr()), nbytes, C.c_void_p(sink.data_ptr()), s), "read")
        torch.cuda.synchronize()
        assert int(sink.item()) == 0
        # one word anywhere -- the last one -- set to the value the fold stores
        buf[-1] = torch.tensor(0x9E3779B9, dtype=torch.int64).to(torch.int32)
        L.check(lib.cx_stream_read(C.c_void_p(buf.data_ptr()), nbytes, C.c_void_p(sink.data_ptr()), s), "read")
        torch.cuda.synchronize()
        assert int(sink.item()) & 0xFFFFFFFF == 0x9E3779B9, nbytes
        sink.zero_()
    assert lib.cx_stream_read(C.c_void_p(buf.data_ptr() + 4), 32, C.c_void_p(sink.data_ptr()), s) == -1
