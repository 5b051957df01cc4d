"""GGUF test models written byte by byte (the layout of src/gguf.rs:119-342,
independent of the library's writer), their oracle counterparts, and the
host mirror of a GPU model. Shared by the GPU model tests; not a test
module."""
import struct

import numpy as np

from oracle import oracle as O


MINI = dict(layers=2, dim=256, heads=4, kv_heads=2, ffn=512, vocab=640, ctx=128, eps=1e-6,
            rope_base=1_000_000.0)


def gguf_bytes(meta, tensors):
    """meta: [(key, type, value)] with type 4 (u32), 6 (f32), 8 (string);
    tensors: [(name, dims, ggml type, bytes)]. Data 32-byte aligned."""
    def text(s):
        b = s.encode()
        return struct.pack("<Q", len(b)) + b
    out = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta))
    for k, t, v in meta:
        out += text(k) + struct.pack("<I", t)
        out += struct.pack("<I", v) if t == 4 else struct.pack("<f", v) if t == 6 else text(v)
    off, offs = 0, []
    for name, dims, t, data in tensors:
        out += text(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", t, off)
        offs.append(off)
        off = (off + len(data) + 31) // 32 * 32
    out += b"\0" * ((32 - len(out) % 32) % 32)
    base = len(out)
    for (name, dims, t, data), o in zip(tensors, offs):
        out += b"\0" * (base + o - len(out)) + bytes(data)
    return out


def q6k_bytes(rows, width, seed):
    """Q6_K rows with any quants and small finite scales (the reference has
    no Q6_K quantizer)."""
    rng = np.random.default_rng(seed)
    nb = width // 256
    b = rng.integers(0, 256, (rows * nb, 210), dtype=np.uint8)
    b[:, 192:208] = rng.integers(-20, 20, (rows * nb, 16), dtype=np.int8).view(np.uint8)
    h = rng.integers(0x0C00, 0x1400, rows * nb)
    b[:, 208], b[:, 209] = h & 0xFF, h >> 8
    return b.reshape(rows, -1)


def q5_0_bytes(rows, width, seed):
    """Q5_0 rows with any quants and small finite scales (the reference has
    no Q5_0 quantizer)."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (rows * width // 32, 22), dtype=np.uint8)
    h = rng.integers(0x1000, 0x1800, rows * width // 32)
    b[:, 0], b[:, 1] = h & 0xFF, h >> 8
    return b.reshape(rows, -1)


def mixed_model(seed=5, override=None, ctx=None, shape=None, embd=None, varied=False):
    """A 2-layer qwen2 GGUF: per-tensor types (k-quants by default,
    overridable), a token_embd (Q4_K by default) tied to the lm_head, q/k/v
    biases in layer 0 only and unit norms; with `varied`, every norm
    (output_norm too) ~ N(1, 0.1) and q/k/v biases ~ N(0, 0.3) in every
    layer, each tensor its own draw. `shape` overrides MINI's dims. Returns
    (file bytes, host tensors by name, types by name)."""
    c = dict(MINI, ctx=ctx or MINI["ctx"], **(shape or {}))
    D, I, V = c["dim"], c["ffn"], c["vocab"]
    kvd = c["kv_heads"] * D // c["heads"]
    rng = np.random.default_rng(seed)
    host, types, gg = {}, {}, []

    def quant(name, t, rows, width, sigma):
        if t == O.Q6_K:
            b = q6k_bytes(rows, width, seed + len(host))
        elif t == O.Q5_0:
            b = q5_0_bytes(rows, width, seed + len(host))
        else:
            b = O.daiss_matrix(seed, name, rows, width, sigma, t)
        host[name], types[name] = b, t
        gg.append((name, [width, rows], t, b.tobytes()))

    def vec(name, n, ones=False):
        if varied:
            v = rng.normal(1.0, 0.1, n) if ones else rng.normal(0, 0.3, n)
        else:
            v = np.ones(n) if ones else rng.normal(0, 0.02, n)
        v = v.astype(np.float32)
        host[name], types[name] = v, O.F32
        gg.append((name, [n], O.F32, v.tobytes()))

    quant("token_embd.weight", embd or O.Q4_K, V, D, 1.0)
    mats = {"attn_q": O.Q4_K, "attn_k": O.Q5_K, "attn_v": O.Q6_K, "attn_output": O.Q3_K,
            "ffn_gate": O.Q4_K, "ffn_up": O.Q5_K, "ffn_down": O.Q6_K}
    mats.update(override or {})
    for i in range(c["layers"]):
        p = f"blk.{i}."
        vec(p + "attn_norm.weight", D, ones=True)
        quant(p + "attn_q.weight", mats["attn_q"], D, D, 0.02)
        quant(p + "attn_k.weight", mats["attn_k"], kvd, D, 0.02)
        quant(p + "attn_v.weight", mats["attn_v"], kvd, D, 0.02)
        if i == 0 or varied:  # biases in layer 0 only, unless varied
            vec(p + "attn_q.bias", D)
            vec(p + "attn_k.bias", kvd)
            vec(p + "attn_v.bias", kvd)
        quant(p + "attn_output.weight", mats["attn_output"], D, D, 0.02)
        vec(p + "ffn_norm.weight", D, ones=True)
        quant(p + "ffn_gate.weight", mats["ffn_gate"], I, D, 0.02)
        quant(p + "ffn_up.weight", mats["ffn_up"], I, D, 0.02)
        quant(p + "ffn_down.weight", mats["ffn_down"], D, I, 0.02)
    vec("output_norm.weight", D, ones=True)
    meta = [("general.architecture", 8, "qwen2"), ("qwen2.block_count", 4, c["layers"]),
            ("qwen2.context_length", 4, c["ctx"]), ("qwen2.embedding_length", 4, D),
            ("qwen2.attention.head_count", 4, c["heads"]),
            ("qwen2.attention.head_count_kv", 4, c["kv_heads"]),
            ("qwen2.attention.layer_norm_rms_epsilon", 6, c["eps"]),
            ("qwen2.rope.freq_base", 6, c["rope_base"])]
    return gguf_bytes(meta, gg), host, types


def oracle_of(host, types, ctx=None, shape=None):
    """The oracle forward of the mixed model: embedding dequantized to f32,
    the tied lm_head as token_embd's bytes, zero biases where absent."""
    c = dict(MINI, ctx=ctx or MINI["ctx"], **(shape or {}))
    D, kvd = c["dim"], c["kv_heads"] * c["dim"] // c["heads"]
    t = dict(host)
    ty = dict(types)
    emb, et = host["token_embd.weight"], types["token_embd.weight"]
    t["token_embd.weight"] = O.dequantize(et, emb.reshape(-1), c["vocab"] * D)
    t["output.weight"], ty["output.weight"] = emb, et
    for i in range(c["layers"]):
        for b, n in (("attn_q.bias", D), ("attn_k.bias", kvd), ("attn_v.bias", kvd)):
            t.setdefault(f"blk.{i}.{b}", np.zeros(n, np.float32))
    return O.Model(c, t, ty, threads=8)


def vary_norms_and_biases(model, seed, norm_sigma=0.1, bias_sigma=0.3):
    """Writes into a GPU model's own device tensors: every `*_norm.weight`
    (output_norm included) ~ N(1, norm_sigma) and every `.bias` ~ N(0,
    bias_sigma), each tensor its own draw (an F32 cx_dequantize is a device
    copy). Returns the names it wrote. A daiss model has unit norms and zero
    biases by definition (src/daiss.rs:396-407); real files do not."""
    import ctypes as C
    import torch
    from cosxamix_amd import _lib as L
    lib = L.load()
    rng = np.random.default_rng(seed)
    done = []
    for i, (name, t, dims, nb) in enumerate(model.tensores()):
        if t != O.F32 or not (name.endswith("_norm.weight") or name.endswith(".bias")):
            continue
        n = nb // 4
        v = rng.normal(1.0, norm_sigma, n) if name.endswith("_norm.weight") else rng.normal(0, bias_sigma, n)
        src = torch.from_numpy(v.astype(np.float32)).cuda()
        L.check(lib.cx_dequantize(O.F32, C.c_void_p(src.data_ptr()), n,
                                  C.c_void_p(model.tensor_ptr(i)),
                                  C.c_void_p(torch.cuda.current_stream().cuda_stream)),
                "vary_norms_and_biases")
        torch.cuda.synchronize()
        assert np.array_equal(model.tensor(i), v.astype(np.float32)), name
        done.append(name)
    return done


def write_tensor(model, idx, data, byte_offset=0):
    """Writes `data` (any dtype, a whole number of 4-byte words) into a GPU
    model's tensor `idx` at `byte_offset`, on the device (an F32
    cx_dequantize is a device copy)."""
    import ctypes as C
    import torch
    from cosxamix_amd import _lib as L
    lib = L.load()
    raw = np.ascontiguousarray(data).view(np.uint8).ravel()
    assert raw.size % 4 == 0 and byte_offset % 4 == 0
    assert byte_offset + raw.size <= model.tensores()[idx][3]
    src = torch.from_numpy(raw.view(np.float32).copy()).cuda()
    L.check(lib.cx_dequantize(O.F32, C.c_void_p(src.data_ptr()), raw.size // 4,
                              C.c_void_p(model.tensor_ptr(idx) + byte_offset),
                              C.c_void_p(torch.cuda.current_stream().cuda_stream)),
            "write_tensor")
    torch.cuda.synchronize()


def mirror(model, threads=16):
    """A GPU model's tensors copied to the host, as an oracle Model."""
    tensors, types = {}, {}
    for i, (name, t, dims, nb) in enumerate(model.tensores()):
        tensors[name] = model.tensor(i)
        types[name] = t
    c = model.cfg
    cfg = dict(layers=c.capas, dim=c.dim, heads=c.cabezas, kv_heads=c.cabezas_kv, ffn=c.ffn,
               vocab=c.vocab, ctx=c.contexto, eps=c.eps, rope_base=c.rope)
    return O.Model(cfg, tensors, types, threads=threads)
