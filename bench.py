#!/usr/bin/env python3
"""Benchmark of the MI355X decode path (one GPU).

Headline: batch-1 greedy decode of a Qwen2.5-3B-shape
model (daiss-3b, src/daiss.rs:103-114) with every linear in Q4_K, f32
embeddings/norms/biases and an f32 KV cache; a seeded 512-token uniform
prompt is prefilled (not timed), W warm-up tokens are decoded, then exactly
K decode steps are timed with HIP events recorded between the captured
per-token graphs on the model's stream. value = K / (time of the K steps).

Roofline: the dominant kernel, the Q4_K GEMV, at BASELINE config 1
(11008 x 2048, the ffn_gate shape): launched back to back inside a captured
HIP graph on torch's stream, rotating over the model's 36 distinct ffn_gate
matrices (456 MB, so the 256 MB Infinity Cache cannot serve repeats);
achieved = 12,727,808 algorithmic bytes / average launch duration.

CPU baseline: the same 3B model's weights copied to the host and decoded by
the oracle forward whose Q4_K row kernel is the reference's own compiled
`cosxamix_q4k_completo` (oracle/_ref), threaded like ops.rs (32-row tasks)
over the host's cores; same 512-token prompt, then a few timed decode tokens.

Batched (the "batched" object): Q4_K 11008 x 2048 and
2048 x 11008 times m = 8, 32, 512 activation rows through cx_matmul_auto
(int8 MFMA), against the reference's per-row CPU matmul.

Q8_0 (the "decode_0_5b_q8_0" object): daiss-0.5b, whose 896-wide matrices
only the 32-value block formats can hold, written in Q8_0 and decoded by the
same loop.

Usage: python bench.py [--gpus 1] [--steps 128] [--warmup 8] [--no-cpu]
       python bench.py --batched-only
       python bench.py --trace-summary gpurun_out/.../kernel_trace.csv
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s (3B-shape Q4_K, bs=1); k-quant GEMV achieved HBM GB/s"
HBM_PEAK_GBPS = 8000.0
CONFIG1_BYTES = 12_727_808  # W 12,681,216 + xq 2048 + xe/xs 2*64*4 + y 11008*4


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def prompt_tokens(n: int, vocab: int, seed: int = 1234):
    """A seeded uniform prompt: xorshift64* (src/daiss.rs:333-341) mod vocab."""
    import numpy as np
    s = seed or 0x9E3779B97F4A7C15
    out = np.empty(n, np.uint32)
    M = (1 << 64) - 1
    for i in range(n):
        s ^= s >> 12
        s ^= (s << 25) & M
        s ^= s >> 27
        out[i] = ((s * 0x2545F4914F6CDD1D) & M) % vocab
    return out


def cpu_info():
    """The host CPU as the reference sizes its pool (num_cpus::get_physical,
    src/main.rs:578-595): (model name, ISA flags that matter to the
    reference's kernels, logical CPUs this process may use, physical cores
    among them)."""
    name, flags, cpus = "unknown", [], {}
    cur = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in list(f) + [""]:
                if not line.strip():
                    if "processor" in cur:
                        cpus[int(cur["processor"])] = cur
                    cur = {}
                    continue
                k, _, v = line.partition(":")
                cur[k.strip()] = v.strip()
    except OSError:
        pass
    try:
        allowed = sorted(os.sched_getaffinity(0))
    except AttributeError:
        allowed = sorted(cpus) or list(range(os.cpu_count() or 1))
    if cpus:
        first = cpus.get(allowed[0], next(iter(cpus.values())))
        name = first.get("model name", name)
        have = set(first.get("flags", "").split())
        flags = [f for f in ("avx2", "fma", "f16c", "avx512f", "avx512bw", "avx512vl",
                             "avx512_vnni", "avx_vnni") if f in have]
        cores = {(cpus[c].get("physical id"), cpus[c].get("core id")) for c in allowed if c in cpus}
        physical = len(cores) if all(k != (None, None) for k in cores) else len(allowed)
    else:
        physical = len(allowed)
    return name, flags, len(allowed), physical


def decode_bench(F, L, steps, warmup, prompt_len):
    import numpy as np
    cfg = F.DAISS_3B
    t0 = time.perf_counter()
    m = F.Modelo(cfg, tipo=L.Q4_K, semilla=42)
    log(f"[bench] 3B model generated in HBM in {time.perf_counter() - t0:.1f}s "
        f"({m.bytes_por_token() / 1e9:.3f} GB of weights per token)")
    prompt = prompt_tokens(prompt_len, cfg.vocab)
    cache = m.nueva_cache(prompt_len + warmup + steps + 1)
    t0 = time.perf_counter()
    toks, ms = m.generar(prompt, warmup + steps, cache, tiempos=True)
    wall = time.perf_counter() - t0
    timed = [float(v) for v in ms[warmup:warmup + steps]]
    total_ms = sum(timed)
    log(f"[bench] prefill+decode wall {wall:.2f}s; {steps} timed steps: {total_ms:.2f} ms, "
        f"median {statistics.median(timed) * 1000:.1f} us/token")
    return m, prompt, toks, timed, total_ms


def config5_bench(F, L, steps=256, warmup=8, prefix=8192):
    """the Llama-3-8B shape (qwen2 architecture, zero
    biases), Q4_K linears, Q5_K ffn_down, Q4_K lm_head; an 8192-token seeded
    random prefix prefilled into the f32 KV cache, then `steps` greedy
    tokens, timed per step with HIP events after `warmup` untimed ones."""
    import numpy as np
    cfg = F.LLAMA3_8B
    t0 = time.perf_counter()
    m = F.Modelo(cfg, tipo=L.Q4_K, semilla=8, tipo_down=L.Q5_K, tipo_salida=L.Q4_K)
    gen_s = time.perf_counter() - t0
    prompt = prompt_tokens(prefix, cfg.vocab, seed=5)
    cache = m.nueva_cache(prefix + warmup + steps + 1)
    t0 = time.perf_counter()
    first = int(m.forward(prompt, cache, logits=False)[1])  # the prefix's next token
    prefill_s = time.perf_counter() - t0
    toks, ms = m.generar(np.array([first], np.uint32), warmup + steps, cache, tiempos=True)
    timed = [float(v) for v in ms[warmup:warmup + steps]]
    total = sum(timed) * 1e-3
    w = m.bytes_por_token()
    ctx_mid = prefix + 1 + warmup + steps // 2
    kv = 2 * cfg.capas * cfg.dim_kv() * 4 * ctx_mid
    out = {"workload": "BASELINE config 5: Llama-3-8B-shape daiss model (32 layers, hidden 4096, "
                       "32/8 heads x 128, SwiGLU 14336, vocab 128256, rope 5e5), Q4_K linears, "
                       "Q5_K ffn_down, Q4_K lm_head, f32 KV cache (order-exact attention), "
                       f"{prefix}-token seeded random prefix, greedy decode",
           "prefix_tokens": prefix, "decode_tokens": steps, "warmup": warmup,
           "tok_per_s": round(steps / total, 2),
           "median_us_per_token": round(statistics.median(timed) * 1000, 2),
           "weight_bytes_per_token": w, "kv_bytes_per_token_mid": kv,
           "effective_GBps": round((w + kv) / (total / steps) / 1e9, 1),
           "hbm_frac": round((w + kv) / (total / steps) / 1e9 / HBM_PEAK_GBPS, 4),
           "prefill_s": round(prefill_s, 3), "prefill_tok_per_s": round(prefix / prefill_s, 1),
           "model_generation_s": round(gen_s, 2)}
    log(f"[bench] config 5: prefill {prefix} tokens {prefill_s:.2f}s; {steps} tokens at "
        f"{out['tok_per_s']} tok/s ({out['median_us_per_token']} us median), "
        f"{out['effective_GBps']} GB/s effective")
    m.close()
    return out


def attention_bench(calls):
    """cx_attention_decode (the model's order-exact decode kernels) on seeded
    q, K and V: the 3B shape at 548 cached positions and config 5's at 8448.
    Wall time a call (the operator synchronizes: the position state lives in
    shared scratch); kernel times come from a profiler's trace."""
    import torch
    from cosxamix_amd import ops
    out = {}
    g = torch.Generator(device="cuda").manual_seed(3)
    for name, total, heads, kvh, hd in (("3b", 548, 16, 2, 128), ("config5", 8448, 32, 8, 128)):
        q = torch.randn(heads * hd, device="cuda", generator=g)
        k = torch.randn(total * kvh * hd, device="cuda", generator=g)
        v = torch.randn(total * kvh * hd, device="cuda", generator=g)
        o = torch.empty(heads * hd, device="cuda")
        for _ in range(3):
            ops.atencion_decode(q, k, v, (total, heads, kvh, hd), o)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(calls):
            ops.atencion_decode(q, k, v, (total, heads, kvh, hd), o)
        torch.cuda.synchronize()
        out[name] = {"positions": total, "heads": heads, "kv_heads": kvh, "head_dim": hd,
                     "us_per_call": round((time.perf_counter() - t0) / calls * 1e6, 2)}
    return out


def small_model_bench(F, L, steps=128, warmup=8, prompt_len=512):
    """daiss-0.5b (src/daiss.rs:91-102: dim 896, 24 layers, 14/2 heads of
    64, SwiGLU 4864) written in Q8_0, the reference writer's type: every
    matrix is 896 or 4864 values wide and runs the Q8_0 GEMV. Same loop as
    the headline: 512-token prompt, `warmup` untimed tokens, `steps` timed."""
    cfg = F.DAISS_0_5B
    m = F.Modelo(cfg, tipo=L.Q8_0, semilla=42)
    prompt = prompt_tokens(prompt_len, cfg.vocab)
    cache = m.nueva_cache(prompt_len + warmup + steps + 1)
    toks, ms = m.generar(prompt, warmup + steps, cache, tiempos=True)
    timed = [float(v) for v in ms[warmup:warmup + steps]]
    total = sum(timed) * 1e-3
    w = m.bytes_por_token()
    kv = 2 * cfg.capas * cfg.dim_kv() * 4 * (prompt_len + warmup + steps // 2)
    out = {"workload": "daiss-0.5b (24 layers, hidden 896, 14/2 heads x 64, SwiGLU 4864, vocab "
                       "151936), every matrix Q8_0 (896- and 4864-wide rows), f32 KV cache, "
                       "512-token seeded prompt, greedy decode",
           "decode_tokens": steps, "tok_per_s": round(steps / total, 2),
           "median_us_per_token": round(statistics.median(timed) * 1000, 2),
           "weight_bytes_per_token": w,
           "effective_GBps": round((w + kv) / (total / steps) / 1e9, 1),
           "first_tokens": [int(t) for t in toks[:8]]}
    log(f"[bench] daiss-0.5b Q8_0: {out['tok_per_s']} tok/s ({out['median_us_per_token']} us "
        f"median), {out['effective_GBps']} GB/s effective")
    out["prefill"] = prefill_bench(m, prompt)
    m.close()
    return out


def sampled_bench(m, prompt, steps=64, warmup=8, temp=0.8, top_p=0.9):
    """The same token loop with Muestreador(42, temp, top_p) drawing on the
    GPU inside the captured step: median per-token time."""
    from cosxamix_amd import sampler
    cache = m.nueva_cache(len(prompt) + warmup + steps + 1)
    toks, ms = m.generar(prompt, warmup + steps, cache, tiempos=True,
                         muestreador=sampler.Muestreador(42, temp, top_p))
    timed = [float(v) for v in ms[warmup:warmup + steps]]
    med = statistics.median(timed)
    out = {"temperature": temp, "top_p": top_p, "median_us_per_token": round(med * 1000, 2),
           "tok_per_s": round(1000.0 / med, 2), "first_tokens": [int(t) for t in toks[:8]]}
    log(f"[bench] sampled decode (t={temp}, top_p={top_p}): {out['median_us_per_token']} us/token")
    return out


def prefill_bench(m, prompt, reps=5):
    """Modelo::forward of the whole prompt on an empty cache (the batched
    prefill): the median wall time of `reps` calls after one warm-up call,
    each ending with the last token's logits on the host."""
    cache = m.nueva_cache(len(prompt) + 1)
    m.forward(prompt, cache)  # allocates the prefill buffers
    times = []
    for _ in range(reps):
        cache.truncar(0)
        t0 = time.perf_counter()
        m.forward(prompt, cache)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    out = {"prompt_tokens": len(prompt), "median_ms": round(med * 1e3, 3),
           "tok_per_s": round(len(prompt) / med, 1), "reps": reps}
    log(f"[bench] prefill of {len(prompt)} tokens: {med * 1e3:.2f} ms ({out['tok_per_s']} tok/s)")
    return out


def gemv_roofline(F, L, m, iters=360, reps=5):
    import torch
    from cosxamix_amd import ops
    lib = L.load()
    names = [t[0] for t in m.tensores()]
    gates = [m.tensor_ptr(i) for i, n in enumerate(names) if n.endswith("ffn_gate.weight")]
    n, k = 11008, 2048
    gen = torch.Generator(device="cuda").manual_seed(2048)
    x = torch.randn(k, generator=gen, device="cuda", dtype=torch.float32)
    xq, xe, xs = ops.cuantizar_i8_en(x, 32)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    import ctypes as C

    def launch(i):
        rc = lib.cx_gemv(L.Q4_K, C.c_void_p(gates[i % len(gates)]), n, k, C.c_void_p(xq.data_ptr()),
                         C.c_void_p(xe.data_ptr()), C.c_void_p(xs.data_ptr()),
                         C.c_void_p(y.data_ptr()), C.c_void_p(torch.cuda.current_stream().cuda_stream))
        L.check(rc, "gemv")

    for i in range(8):
        launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            launch(i)
    g.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) * 1e-3 / iters)
    avg = statistics.median(per)
    gbps = CONFIG1_BYTES / avg / 1e9
    log(f"[bench] config-1 Q4_K GEMV: {avg * 1e6:.2f} us/launch over {len(gates)} rotating "
        f"matrices -> {gbps:.0f} GB/s ({gbps / HBM_PEAK_GBPS:.1%} of 8 TB/s)")
    return avg, gbps, len(gates)


def gemv_sustained(iters=30, reps=5, n=151936, k=2048, copies=3):
    """The config-1 GEMV's kernel (cx_gemv, Q4_K, k = 2048) at the lm_head
    shape, 151936 x 2048 (175 MB a launch), where the launch boundary and
    the first bytes' latency are a few percent of the launch: the rate the
    kernel streams weights at. Three rotating matrices of random bytes with
    finite f16 scales (525 MB, past the 256 MB Infinity Cache; the rate does
    not depend on the values), in a captured graph, HIP events around it."""
    import ctypes as C
    import torch
    from cosxamix_amd import _lib as L, ops
    lib = L.load()
    rb = ops.row_bytes(L.Q4_K, k)
    mats = []
    for i in range(copies):
        w = torch.randint(0, 256, (n * rb,), dtype=torch.uint8, device="cuda")
        v = w.view(n * k // 256, 144)
        v[:, 1] = 0x2C  # d = f16 0x2Cxx, dmin = 0x24xx: finite
        v[:, 3] = 0x24
        mats.append(w)
    x = torch.randn(k, device="cuda")
    xq, xe, xs = ops.cuantizar_i8_en(x, 32)
    y = torch.empty(n, device="cuda")

    def launch(i):
        w = mats[i % copies]
        L.check(lib.cx_gemv(L.Q4_K, C.c_void_p(w.data_ptr()), n, k, C.c_void_p(xq.data_ptr()),
                            C.c_void_p(xe.data_ptr()), C.c_void_p(xs.data_ptr()),
                            C.c_void_p(y.data_ptr()),
                            C.c_void_p(torch.cuda.current_stream().cuda_stream)), "gemv")

    for i in range(copies):
        launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            launch(i)
    g.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) * 1e-3 / iters)
    avg = statistics.median(per)
    nbytes = n * rb + k + 2 * (k // 32) * 4 + n * 4
    gbps = nbytes / avg / 1e9
    log(f"[bench] the same GEMV at {n}x{k}: {avg * 1e6:.2f} us/launch -> {gbps:.0f} GB/s "
        f"({gbps / HBM_PEAK_GBPS:.1%} of 8 TB/s)")
    del mats
    torch.cuda.empty_cache()
    return {"shape": f"{n}x{k} (the lm_head shape)", "achieved": round(gbps, 1),
            "frac": round(gbps / HBM_PEAK_GBPS, 4), "us_per_launch": round(avg * 1e6, 2),
            "bytes_per_launch": nbytes, "rotating_matrices": copies}


PROBE_COPY_BYTES = 64 << 20


def read_peak(L, m, iters=360, reps=5):
    """Measured read rates for the roofline (cx_stream_read: 16-byte loads
    over a grid, no arithmetic after them), each a captured graph of
    launches timed with HIP events, median of `reps`:
    - 4 buffers of 256 MB in turn (1 GB, past the 256 MB Infinity Cache):
      the read peak this chip reaches from HBM;
    - the model's 36 ffn_gate matrices in turn, 12,681,216 B a launch, the
      config-1 GEMV's own bytes: what a launch of that size can read with
      nothing else to do (the launch boundary and the first bytes' latency
      included);
    - a 64 MiB device-to-device copy (torch), 128 MiB moved."""
    import ctypes as C
    import torch
    lib = L.load()
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = lambda: C.c_void_p(torch.cuda.current_stream().cuda_stream)

    def timed(bufs, nbytes, n_launch):
        def launch(i):
            L.check(lib.cx_stream_read(C.c_void_p(bufs[i % len(bufs)]), nbytes,
                                       C.c_void_p(sink.data_ptr()), stream()), "stream_read")
        for i in range(len(bufs)):
            launch(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n_launch):
                launch(i)
        g.replay()
        torch.cuda.synchronize()
        per = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            g.replay()
            e1.record()
            torch.cuda.synchronize()
            per.append(e0.elapsed_time(e1) * 1e-3 / n_launch)
        return statistics.median(per)

    big = [torch.empty(256 << 20, dtype=torch.uint8, device="cuda").random_(0, 255) for _ in range(4)]
    t_big = timed([b.data_ptr() for b in big], 256 << 20, 40)
    del big
    names = [t[0] for t in m.tensores()]
    gates = [m.tensor_ptr(i) for i, n in enumerate(names) if n.endswith("ffn_gate.weight")]
    wbytes = 11008 * 2048 // 256 * 144
    t_gate = timed(gates, wbytes, iters)
    src = torch.empty(PROBE_COPY_BYTES, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    per = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            dst.copy_(src)
        e1.record()
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) * 1e-3 / 10)
    t_copy = statistics.median(per)
    del src, dst
    torch.cuda.empty_cache()
    out = {"read_GBps": round((256 << 20) / t_big / 1e9, 1),
           "read_12_7MB_GBps": round(wbytes / t_gate / 1e9, 1),
           "read_12_7MB_us": round(t_gate * 1e6, 3),
           "copy_64MiB_GBps": round(2 * PROBE_COPY_BYTES / t_copy / 1e9, 1)}
    log(f"[bench] measured reads: {out['read_GBps']} GB/s over 1 GB; {out['read_12_7MB_GBps']} "
        f"GB/s ({out['read_12_7MB_us']} us) a 12.7 MB launch over the 36 ffn_gate matrices; "
        f"64 MiB copy {out['copy_64MiB_GBps']} GB/s (read + write)")
    return out


def gemv_probe():
    """The workload the PMC passes count: config-1 Q4_K GEMVs over 36
    rotating matrices (random bytes with finite f16 scales: traffic does not
    depend on values), then a 64 MiB device-to-device copy whose HBM bytes
    are known (64 MiB read + 64 MiB written): the calibration kernel."""
    import ctypes as C
    import torch
    from cosxamix_amd import _lib as L, ops
    lib = L.load()
    n, k = 11008, 2048
    rb = ops.row_bytes(L.Q4_K, k)
    mats = []
    for i in range(36):
        w = torch.randint(0, 256, (n * rb,), dtype=torch.uint8, device="cuda")
        v = w.view(n * k // 256, 144)
        v[:, 1] = 0x2C  # d = f16 0x2Cxx, dmin = 0x24xx: finite
        v[:, 3] = 0x24
        mats.append(w)
    x = torch.randn(k, device="cuda")
    xq, xe, xs = ops.cuantizar_i8_en(x, 32)
    y = torch.empty(n, device="cuda")
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    for _ in range(3):
        for w in mats:
            L.check(lib.cx_gemv(L.Q4_K, C.c_void_p(w.data_ptr()), n, k, C.c_void_p(xq.data_ptr()),
                                C.c_void_p(xe.data_ptr()), C.c_void_p(xs.data_ptr()),
                                C.c_void_p(y.data_ptr()), s), "gemv")
    src = torch.empty(PROBE_COPY_BYTES, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def _pmc_per_dispatch(csv_dir, counter):
    """Mean counter value (KiB) per dispatch of the GEMV and of the copy."""
    import csv
    import glob
    vals = {"gemv": [], "copy": []}
    for path in glob.glob(os.path.join(csv_dir, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            for r in csv.DictReader(f):
                if r.get("Counter_Name") != counter:
                    continue
                name = r.get("Kernel_Name", "")
                key = "gemv" if "k_gemv" in name else ("copy" if "opy" in name else None)
                if key:
                    vals[key].append(float(r["Counter_Value"]))
    if not vals["gemv"] or not vals["copy"]:
        return None
    # the copy runs 3 times: its first dispatch may include page-table warm-up
    return statistics.median(vals["gemv"]), statistics.median(vals["copy"])


def gemv_traffic():
    """HBM bytes per config-1 GEMV from two rocprofv3 --pmc passes over
    `bench.py --gemv-probe` (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch),
    each scaled by what the same counter reads for the 64 MiB copy. Returns
    (bytes, detail) or (None, reason)."""
    import shutil
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3")
    if not prof:
        return None, "rocprofv3 not found"
    out = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="cx_pmc_", dir="/tmp")
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "pmc", "--",
               sys.executable, os.path.abspath(__file__), "--gemv-probe"]
        try:
            r = subprocess.run(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"),
                               capture_output=True, text=True, timeout=180)
        except subprocess.TimeoutExpired:
            return None, f"rocprofv3 --pmc {counter} timed out"
        got = _pmc_per_dispatch(d, counter)
        shutil.rmtree(d, ignore_errors=True)
        if got is None:
            return None, f"rocprofv3 --pmc {counter}: no counter rows (rc {r.returncode})"
        out[counter] = got
    fetch_g, fetch_c = out["FETCH_SIZE"]
    write_g, write_c = out["WRITE_SIZE"]
    f_scale, w_scale = PROBE_COPY_BYTES / fetch_c, PROBE_COPY_BYTES / write_c
    traffic = fetch_g * f_scale + write_g * w_scale
    log(f"[bench] PMC: gemv FETCH {fetch_g:.0f} KiB, WRITE {write_g:.0f} KiB per dispatch; "
        f"64 MiB copy reads {fetch_c:.0f} KiB, writes {write_c:.0f} KiB -> scales "
        f"{f_scale:.3f} / {w_scale:.3f}; traffic {traffic / 1e6:.3f} MB per GEMV")
    return traffic, {"fetch_kib": round(fetch_g, 1), "write_kib": round(write_g, 1),
                     "copy_fetch_kib": round(fetch_c, 1), "copy_write_kib": round(write_c, 1),
                     "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4)}


# the GPU box's CPU share: pools are sized to it whatever the host reports
BOX_CPU_SHARE = 16


def cpu_baseline(F, L, m, prompt, gpu_tokens, gpu_step1, decode_tokens=16, decode_tokens_1t=4):
    """The reference's CPU decode of the same model: the 3B weights copied to
    the host; the prompt prefilled by the oracle (not timed); then decode
    tokens timed with the Q4_K row kernel the reference runs on x86 (its own
    compiled cosxamix_q4k_completo, oracle/_ref) over all physical cores, as
    the reference's pool is sized (src/main.rs:578-595), and again on one
    thread. The per-token ops around the row kernel (rmsnorm, rope,
    attention, SwiGLU, argmax, the 32-row task loop) are the oracle's C
    restatement of the reference's.

    Parity with the reference as it runs by default on x86 (its asm Q4_K
    row kernel, which sums in AVX2 lane order, not the scalar spec's order
    that the GPU and the oracle follow bit for bit): the CPU tokens against
    the GPU's `gpu_tokens` (the same prompt, greedy), and the first decode
    step's logits against the GPU's `gpu_step1`."""
    import numpy as np
    from oracle import oracle as O
    ref = O.load_ref()
    kind = "reference" if ref is not None else "port"
    name, flags, logical, physical = cpu_info()
    threads = max(1, min(physical, BOX_CPU_SHARE))
    t0 = time.perf_counter()
    tensors, types = {}, {}
    for i, (nm, t, _, _) in enumerate(m.tensores()):
        tensors[nm] = m.tensor(i)
        types[nm] = t
    c = m.cfg
    cfg = dict(layers=c.capas, dim=c.dim, heads=c.cabezas, kv_heads=c.cabezas_kv, ffn=c.ffn,
               vocab=c.vocab, ctx=c.contexto, eps=c.eps, rope_base=c.rope)
    model = O.Model(cfg, tensors, types, threads=threads)
    kern = O.ref_row_kernel(ref, O.Q4_K) if ref is not None else None
    log(f"[bench] cpu baseline: weights on host in {time.perf_counter() - t0:.1f}s; {name}, "
        f"{physical} physical cores of {logical} CPUs, {threads} threads; flags {flags}; row "
        f"kernel {'cosxamix_q4k_completo' if ref else 'oracle scalar'}")
    cache = model.new_cache(len(prompt) + decode_tokens + decode_tokens_1t + 1)
    t0 = time.perf_counter()
    lg = model.forward(prompt, cache)
    pre = time.perf_counter() - t0
    model.set_q4k_kernel(kern)
    tok = O.argmax(lg)
    toks, first = [tok], []

    def decode(n):
        per = []
        nonlocal tok
        for _ in range(n):
            t1 = time.perf_counter()
            lg = model.forward(np.array([tok], np.uint32), cache)
            per.append(time.perf_counter() - t1)
            if not first:
                first.append(lg)
            tok = O.argmax(lg)
            toks.append(tok)
        return statistics.median(per)

    med = decode(decode_tokens)
    model.set_threads(1)
    med1 = decode(decode_tokens_1t)
    log(f"[bench] cpu baseline: prefill {len(prompt)} tokens {pre:.1f}s (oracle kernels); decode "
        f"median {med * 1e3:.1f} ms/token on {threads} threads ({1 / med:.2f} tok/s), "
        f"{med1 * 1e3:.1f} ms/token on 1 ({1 / med1:.2f} tok/s)")
    n = min(len(toks), len(gpu_tokens))
    same = 0
    while same < n and int(toks[same]) == int(gpu_tokens[same]):
        same += 1
    dev = float(np.max(np.abs(first[0] - gpu_step1)))
    log(f"[bench] cpu baseline ({'asm' if ref else 'scalar'} Q4_K row kernel) against the GPU: "
        f"first {same} of {n} greedy tokens equal, first decode step logits max-abs {dev:.3g}")
    return {"value": round(1.0 / med, 3), "unit": "tok/s", "cores": threads, "kind": kind,
            "tokens_compared": n, "tokens_equal": same,
            "first_step_logits_max_abs": round(dev, 6),
            "value_1_thread": round(1.0 / med1, 3), "cpu": name, "isa_flags": flags,
            "physical_cores": physical, "logical_cpus": logical,
            "sample": (f"same 3B Q4_K weights on the host; {len(prompt)}-token prompt prefilled "
                       f"(untimed), then the median of {decode_tokens} decode tokens on {threads} "
                       f"threads (all physical cores, at most the box's share of "
                       f"{BOX_CPU_SHARE}) and of {decode_tokens_1t} on 1 thread. Row kernel: the "
                       f"reference's compiled cosxamix_q4k_completo (AVX2 asm); the per-token ops "
                       f"(rmsnorm, rope, attention, SwiGLU, argmax) are the oracle's C "
                       f"restatement of the reference's, in 32-row tasks as src/ops.rs")}


CONFIG4_MS = (8, 32, 512)


def batched_bench(L, m, with_cpu, calls=20, reps=5):
    """the model's layer-0 Q4_K ffn_gate (11008 x 2048) and
    ffn_down (2048 x 11008) times m = 8, 32, 512 seeded N(0, 1) activation
    rows through cx_matmul_auto (activation quantization + the int8 MFMA
    contraction), timed as a captured graph of `calls` calls on torch's
    stream. The CPU side is the reference's per-row path: its compiled Q4_K
    row kernel (cosxamix_q4k_completo) in the oracle's 32-row task loop."""
    import ctypes as C
    import numpy as np
    import torch
    from oracle import oracle as O
    lib = L.load()
    names = [t[0] for t in m.tensores()]
    mats = []
    for suffix in ("blk.0.ffn_gate.weight", "blk.0.ffn_down.weight"):
        i = names.index(suffix)
        _, t, (k, n), _ = m.tensores()[i]
        assert t == L.Q4_K
        mats.append((suffix, i, n, k))
    ref = O.load_ref() if with_cpu else None
    threads = max(1, min(cpu_info()[3], BOX_CPU_SHARE))
    stream = lambda: C.c_void_p(torch.cuda.current_stream().cuda_stream)
    cases = []
    for name, i, n, k in mats:
        wp = m.tensor_ptr(i)
        host_w = m.tensor(i) if with_cpu else None
        for rows in sorted(CONFIG4_MS, reverse=True):  # the largest first sizes the scratch
            gen = torch.Generator(device="cuda").manual_seed(rows * 7 + n)
            x = torch.randn(rows, k, generator=gen, device="cuda", dtype=torch.float32)
            y = torch.empty(rows, n, device="cuda", dtype=torch.float32)

            def call():
                L.check(lib.cx_matmul_auto(rows, k, n, C.c_void_p(x.data_ptr()), C.c_void_p(wp),
                                           L.Q4_K, C.c_void_p(y.data_ptr()), stream()), "matmul_auto")

            for _ in range(3):
                call()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(calls):
                    call()
            g.replay()
            torch.cuda.synchronize()
            per = []
            for _ in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                g.replay()
                e1.record()
                torch.cuda.synchronize()
                per.append(e0.elapsed_time(e1) * 1e-3 / calls)
            sec = statistics.median(per)
            case = {"matrix": f"{n}x{k}", "m": rows, "us": round(sec * 1e6, 2),
                    "int_TOPs": round(2.0 * rows * n * k / sec / 1e12, 2),
                    "us_per_row": round(sec * 1e6 / rows, 3)}
            if with_cpu:
                xh = x.cpu().numpy()
                kern = O.ref_row_kernel(ref, O.Q4_K) if ref is not None else None
                runs = []
                for _ in range(3):
                    t0 = time.perf_counter()
                    want = O.matmul_fused(O.Q4_K, xh, host_w, n, threads=threads, kernel=kern)
                    runs.append(time.perf_counter() - t0)
                cpu = statistics.median(runs)
                got = y.cpu().numpy().astype(np.float64)
                err = float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))
                case.update({"cpu_ms": round(cpu * 1e3, 2), "speedup_vs_cpu": round(cpu / sec, 1),
                             "rel_l2_vs_cpu": float(f"{err:.3g}")})
            log(f"[bench] config 4 {name} m={rows}: {case}")
            cases.append(case)
            del g
    return {"workload": "BASELINE config 4: layer-0 Q4_K ffn_gate (11008x2048) and ffn_down "
                        "(2048x11008) of the daiss-3b model x m seeded N(0,1) f32 rows; "
                        "cx_matmul_auto = activation quantization + int8 MFMA contraction, "
                        f"median of {reps} replays of a captured graph of {calls} calls",
            "cases": cases,
            "cpu": None if not with_cpu else
            (f"reference per-row path: {'cosxamix_q4k_completo' if ref is not None else 'oracle scalar'}"
             f" row kernel, 32-row tasks over {threads} threads, median of 3 runs")}


def trace_summary(path):
    """Per (kernel, grid) dispatch statistics from a rocprofv3 kernel trace."""
    import csv
    rows = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            key = (r.get("Kernel_Name", "?")[:90], r.get("Grid_Size_X", r.get("Grid_Size", "?")),
                   r.get("Workgroup_Size_X", r.get("Workgroup_Size", "?")))
            d = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            rows.setdefault(key, []).append(d)
    print(f"{'kernel':90s} {'grid':>9s} {'wg':>4s} {'calls':>6s} {'avg_us':>9s} {'med_us':>9s}")
    for (k, g, w), ds in sorted(rows.items(), key=lambda kv: -sum(kv[1])):
        print(f"{k:90s} {g:>9s} {w:>4s} {len(ds):6d} {sum(ds) / len(ds) / 1e3:9.2f} "
              f"{statistics.median(ds) / 1e3:9.2f}")


def token_summary(path, ntok=8):
    """Per decode token from a rocprofv3 kernel trace of a decode run: the
    kernels between consecutive lm_head launches (the largest GEMV grid),
    averaged over the last `ntok` tokens that ran no batched prefill kernel
    (a run that also times the prompt's prefill ends with those)."""
    import collections
    import csv
    import re
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            g = int(r.get("Grid_Size_X", r.get("Grid_Size"))) // int(
                r.get("Workgroup_Size_X", r.get("Workgroup_Size")))
            rows.append((r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"]), g))
    rows.sort(key=lambda r: r[1])
    lm_grid = max(r[3] for r in rows if "k_gemv" in r[0])
    lm = [i for i, r in enumerate(rows) if r[3] == lm_grid and "k_gemv" in r[0]]
    pairs = [(a, b) for a, b in zip(lm[:-1], lm[1:])
             if not any("k_gemm" in r[0] or "k_quantize_gemm" in r[0] for r in rows[a + 1:b])]
    per = collections.defaultdict(list)
    spans = []
    for a, b in pairs[-ntok:]:
        seg = rows[a + 1:b + 1]
        spans.append(seg[-1][2] - rows[a][2])
        for r in seg:
            m = re.search(r"(k_[a-z_0-9]+(<[^>]*>)?)", r[0])
            per[(m.group(1) if m else r[0][:40], r[3])].append(r[2] - r[1])
    busy = sum(sum(v) for v in per.values()) / ntok
    print(f"{ntok} tokens: span {statistics.mean(spans) / 1e3:.1f} us per token on the GPU, "
          f"kernel time {busy / 1e3:.1f} us")
    print("| kernel | workgroups | calls/token | avg µs | µs/token |")
    print("|---|---:|---:|---:|---:|")
    for (k, g), v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        print(f"| {k} | {g} | {len(v) // ntok} | {statistics.mean(v) / 1e3:.2f} | "
              f"{sum(v) / 1e3 / ntok:.1f} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-traffic", action="store_true")
    ap.add_argument("--gemv-probe", action="store_true")
    ap.add_argument("--batched-only", action="store_true",
                    help="only the config-4 batched contraction (GPU side), e.g. under rocprofv3")
    ap.add_argument("--trace-summary")
    ap.add_argument("--per-token", type=int, default=0,
                    help="with --trace-summary: the per-token breakdown of the last N decode tokens")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the headline decode (e.g. under rocprofv3)")
    ap.add_argument("--sampled-only", action="store_true",
                    help="only the temperature/top-p decode of the 3B model")
    ap.add_argument("--config5-only", action="store_true",
                    help="only BASELINE config 5 (8B shape, 8K context)")
    ap.add_argument("--no-config5", action="store_true")
    ap.add_argument("--attention-only", action="store_true",
                    help="the decode attention operator alone at the 3B shape (548 positions) "
                         "and config 5's (8448 positions, 32/8 heads): for kernel profiles")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the config-1 GEMV roofline loop (e.g. under rocprofv3)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the 3B model's batched prefill of --prompt tokens")
    ap.add_argument("--small-only", action="store_true",
                    help="only the daiss-0.5b Q8_0 decode (the 32-value block GEMV)")
    a = ap.parse_args()
    if a.trace_summary:
        if a.per_token:
            token_summary(a.trace_summary, a.per_token)
        else:
            trace_summary(a.trace_summary)
        return 0
    if a.gemv_probe:
        gemv_probe()
        return 0
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the decode loop of "
              "the reference is single-device); run with --gpus 1", file=sys.stderr)
        return 2
    import torch
    assert torch.cuda.is_available(), "bench.py needs the GPU"
    torch.cuda.set_device(0)
    from cosxamix_amd import _lib as L
    from cosxamix_amd import forward as F

    if a.attention_only:
        print(json.dumps(attention_bench(a.steps)), flush=True)
        return 0
    if a.config5_only:  # --steps above 128 (the default) up to 256, the full run's count
        print(json.dumps(config5_bench(F, L, steps=min(a.steps, 256), warmup=a.warmup)),
              flush=True)
        return 0
    if a.sampled_only:
        m = F.Modelo(F.DAISS_3B, tipo=L.Q4_K, semilla=42)
        print(json.dumps(sampled_bench(m, prompt_tokens(a.prompt, F.DAISS_3B.vocab), a.steps,
                                       a.warmup)), flush=True)
        m.close()
        return 0
    if a.small_only:
        print(json.dumps(small_model_bench(F, L, a.steps, a.warmup, a.prompt)), flush=True)
        return 0
    if a.prefill_only:
        m = F.Modelo(F.DAISS_3B, tipo=L.Q4_K, semilla=42)
        print(json.dumps(prefill_bench(m, prompt_tokens(a.prompt, F.DAISS_3B.vocab))), flush=True)
        m.close()
        return 0
    if a.roofline_only:
        m = F.Modelo(F.DAISS_3B, tipo=L.Q4_K, semilla=42)
        avg, gbps, ncopies = gemv_roofline(F, L, m)
        peak = read_peak(L, m)
        m.close()
        sus = gemv_sustained()
        print(json.dumps({"us_per_launch": round(avg * 1e6, 3), "GBps": round(gbps, 1),
                          "frac": round(gbps / HBM_PEAK_GBPS, 4), "rotating_matrices": ncopies,
                          "measured": peak, "frac_of_measured_peak": round(gbps / peak["read_GBps"], 4),
                          "frac_of_read_at_this_size": round(gbps / peak["read_12_7MB_GBps"], 4),
                          "sustained": sus}), flush=True)
        return 0
    if a.batched_only:
        m = F.Modelo(F.DAISS_3B, tipo=L.Q4_K, semilla=42)
        print(json.dumps(batched_bench(L, m, False)), flush=True)
        return 0
    m, prompt, toks, timed, total_ms = decode_bench(F, L, a.steps, a.warmup, a.prompt)
    tok_s = a.steps / (total_ms * 1e-3)
    if a.decode_only:
        print(json.dumps({"decode_tok_per_s": round(tok_s, 2),
                          "median_us_per_token": round(statistics.median(timed) * 1000, 2)}),
              flush=True)
        m.close()
        return 0
    per_tok_bytes = m.bytes_por_token()
    kv_bytes = 2 * F.DAISS_3B.capas * F.DAISS_3B.dim_kv() * 4 * (a.prompt + a.warmup + a.steps // 2)
    prefill = prefill_bench(m, prompt)
    sampled = sampled_bench(m, prompt)
    avg, gbps, ncopies = gemv_roofline(F, L, m)
    measured = read_peak(L, m)
    sustained = gemv_sustained()
    traffic, tdetail = (None, "skipped (--no-traffic)") if a.no_traffic else gemv_traffic()
    cpu = None
    if not a.no_cpu:
        # the GPU's logits at the first decode step, for the parity note
        c1 = m.nueva_cache(len(prompt) + 2)
        m.forward(prompt, c1, logits=False)
        step1, _ = m.forward([int(toks[0])], c1)
        c1.close()
        cpu = cpu_baseline(F, L, m, prompt, toks, step1)
    batched = batched_bench(L, m, not a.no_cpu)
    m.close()
    config5 = None if a.no_config5 else config5_bench(F, L)
    small = small_model_bench(F, L)
    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(total_ms / a.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic",
        "config": {"workload": "greedy decode, Qwen2.5-3B-shape daiss model (36 layers, hidden "
                               "2048, 16/2 heads x 128, SwiGLU 11008, vocab 151936), all "
                               "linears Q4_K, f32 KV cache, random-init weights",
                   "prompt_tokens": a.prompt, "decode_tokens": a.steps, "batch": 1},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     "traffic": None if traffic is None else int(traffic),
                     "traffic_source": tdetail,
                     "kernel": "k_gemv_row<Q4_K> config 1 (11008x2048, 48-row tiles of 12 waves)",
                     "us_per_launch": round(avg * 1e6, 3), "bytes_per_launch": CONFIG1_BYTES,
                     "rotating_matrices": ncopies,
                     # measured on this box: the read peak (1 GB), the read rate of a
                     # launch of the GEMV's own 12.7 MB with nothing else to do, a copy
                     "measured_peak": measured,
                     "frac_of_measured_peak": round(gbps / measured["read_GBps"], 4),
                     "frac_of_read_at_this_size": round(gbps / measured["read_12_7MB_GBps"], 4),
                     # the same kernel where the launch's fixed cost is amortized
                     "sustained": sustained},
        "cpu_baseline": cpu,
        "decode": {"median_us_per_token": round(statistics.median(timed) * 1000, 2),
                   "weight_bytes_per_token": per_tok_bytes,
                   "effective_GBps": round((per_tok_bytes + kv_bytes) / (total_ms * 1e-3 / a.steps) / 1e9, 1),
                   # the whole step's bytes (weights + KV read) over its time, against 8 TB/s
                   "hbm_frac": round((per_tok_bytes + kv_bytes) / (total_ms * 1e-3 / a.steps) / 1e9
                                     / HBM_PEAK_GBPS, 4),
                   "first_tokens": [int(t) for t in toks[:8]]},
        "batched": batched,
        "prefill": prefill,
        "sampled_decode": sampled,
        "config5": config5,
        "decode_0_5b_q8_0": small,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
