"""GGUF models on the GPU (MI355X): Modelo::abrir (src/forward.rs:187-266)
through cx_model_open.

- A daiss model written with cx_model_save_gguf and opened again gives
  the same tensors and bit-identical logits and greedy tokens.
- A mixed-format file written here (an independent writer of the GGUF layout,
  src/gguf.rs:119-342) opens and matches the oracle forward bit for bit:
  per-tensor k-quant types as real Q*_K_M files have, a quantized token_embd
  dequantized per token, the lm_head tied to it (no output.weight,
  src/forward.rs:218-227), and biases present in one layer and absent in the
  other.
- Files the path cannot run are refused with an error, not a crash."""
import struct

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def F(dev):
    from cosxamix_amd import forward
    return forward


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


def mixed_model(seed=5, override=None):
    c = MINI
    D, I, V = c["dim"], c["ffn"], c["vocab"]
    kvd = c["kv_heads"] * D // c["heads"]
    rng = np.random.default_rng(seed)
    host, types, gg = {}, {}, []

    def quant(name, t, rows, width, sigma):
        if t == O.Q6_K:
            b = q6k_bytes(rows, width, seed + len(host))
        else:
            b = O.daiss_matrix(seed, name, rows, width, sigma, t)
        host[name], types[name] = b, t
        gg.append((name, [width, rows], t, b.tobytes()))

    def vec(name, n, ones=False):
        v = np.ones(n, np.float32) if ones else rng.normal(0, 0.02, n).astype(np.float32)
        host[name], types[name] = v, O.F32
        gg.append((name, [n], O.F32, v.tobytes()))

    quant("token_embd.weight", O.Q4_K, V, D, 1.0)
    mats = {"attn_q": O.Q4_K, "attn_k": O.Q5_K, "attn_v": O.Q6_K, "attn_output": O.Q3_K,
            "ffn_gate": O.Q4_K, "ffn_up": O.Q5_K, "ffn_down": O.Q6_K}
    mats.update(override or {})
    for i in range(c["layers"]):
        p = f"blk.{i}."
        vec(p + "attn_norm.weight", D, ones=True)
        quant(p + "attn_q.weight", mats["attn_q"], D, D, 0.02)
        quant(p + "attn_k.weight", mats["attn_k"], kvd, D, 0.02)
        quant(p + "attn_v.weight", mats["attn_v"], kvd, D, 0.02)
        if i == 0:  # biases in layer 0 only
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


def oracle_of(host, types):
    """The oracle forward of the mixed model: embedding dequantized to f32,
    the tied lm_head as token_embd's bytes, zero biases where absent."""
    c = dict(MINI)
    D, kvd = c["dim"], c["kv_heads"] * c["dim"] // c["heads"]
    t = dict(host)
    ty = dict(types)
    emb = host["token_embd.weight"]
    t["token_embd.weight"] = O.dequantize(O.Q4_K, emb.reshape(-1), c["vocab"] * D)
    t["output.weight"], ty["output.weight"] = emb, O.Q4_K
    for i in range(c["layers"]):
        for b, n in (("attn_q.bias", D), ("attn_k.bias", kvd), ("attn_v.bias", kvd)):
            t.setdefault(f"blk.{i}.{b}", np.zeros(n, np.float32))
    return O.Model(c, t, ty, threads=8)


def test_daiss_model_round_trips_through_gguf(F, tmp_path):
    cfg = F.Config(2, 256, 4, 2, 512, 640, 128)
    a = F.Modelo(cfg, tipo=O.Q4_K, semilla=11, tipo_down=O.Q5_K, tipo_salida=O.Q3_K)
    path = tmp_path / "daiss.gguf"
    a.guardar(path)
    from cosxamix_amd import gguf
    g = gguf.Gguf.abrir(path)
    assert g.meta_entero("qwen2.block_count") == 2 and g.meta_texto("general.architecture") == "qwen2"
    assert g.tensor("blk.1.ffn_down.weight").dims == [512, 256]
    assert g.tensor("blk.0.attn_q.bias").dims == [256]
    b = F.Modelo.abrir(path)
    # eps and the RoPE base travel as f32, as the reference writes them
    assert b.cfg == F.Config(*[np.float32(v).item() if isinstance(v, float) else v
                               for v in vars(cfg).values()])
    ta, tb = a.tensores(), b.tensores()
    assert [x[:3] for x in ta] == [x[:3] for x in tb]
    for i in (0, 2, len(ta) - 1):
        assert np.array_equal(a.tensor(i).view(np.uint8), b.tensor(i).view(np.uint8))
    prompt = np.array([5, 17, 600, 3, 42], np.uint32)
    ca, cb = a.nueva_cache(64), b.nueva_cache(64)
    la, _ = a.forward(prompt, ca)
    lb, _ = b.forward(prompt, cb)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    assert np.array_equal(a.generar(prompt, 12, a.nueva_cache(64)),
                          b.generar(prompt, 12, b.nueva_cache(64)))


def test_mixed_format_file_matches_the_oracle(F, tmp_path):
    data, host, types = mixed_model()
    path = tmp_path / "mixed.gguf"
    path.write_bytes(data)
    m = F.Modelo.abrir(path)
    assert (m.cfg.ffn, m.cfg.vocab) == (MINI["ffn"], MINI["vocab"])
    names = [t[0] for t in m.tensores()]
    assert "output.weight" not in names and "blk.1.attn_q.bias" not in names
    ref = oracle_of(host, types)
    prompt = np.array([3, 600, 17, 99, 5, 250], np.uint32)
    gc, oc = m.nueva_cache(64), ref.new_cache(64)
    lg, top = m.forward(prompt, gc)
    want = ref.forward(prompt, oc)
    assert np.array_equal(lg, want)  # equal as floats (+0 where a bias is absent)
    assert top == O.argmax(want)
    for _ in range(6):  # teacher-forced single steps
        t = np.array([O.argmax(want)], np.uint32)
        lg, _ = m.forward(t, gc)
        want = ref.forward(t, oc)
        assert np.array_equal(lg, want)
    g = m.generar(prompt, 10, m.nueva_cache(64))
    w = ref.generate(prompt, 10, ref.new_cache(64))
    assert np.array_equal(g, w)


def test_files_the_path_cannot_run_are_refused(F, tmp_path):
    data, host, types = mixed_model(seed=9)
    # a missing tensor
    cut = data.replace(b"blk.1.ffn_up.weight", b"blk.1.ffn_XX.weight")
    p = tmp_path / "missing.gguf"
    p.write_bytes(cut)
    with pytest.raises(ValueError, match="ffn_up"):
        F.Modelo.abrir(p)
    # a matrix in a type the GEMV does not read (Q8_0)
    data, _, _ = mixed_model(seed=9, override={"attn_output": O.Q8_0})
    p2 = tmp_path / "q8.gguf"
    p2.write_bytes(data)
    with pytest.raises(ValueError, match="attn_output"):
        F.Modelo.abrir(p2)
    # a matrix of the wrong shape: ffn_up declared with one row less
    data, host, _ = mixed_model(seed=9)
    name = b"blk.0.ffn_up.weight"
    i = data.index(name) + len(name) + 4 + 8  # n_dims, then the width: the rows
    bad = data[:i] + struct.pack("<Q", MINI["ffn"] - 1) + data[i + 8:]
    p3 = tmp_path / "shape.gguf"
    p3.write_bytes(bad)
    with pytest.raises(ValueError, match="ffn_up"):
        F.Modelo.abrir(p3)
    with pytest.raises(ValueError):
        F.Modelo.abrir(tmp_path / "does-not-exist.gguf")
