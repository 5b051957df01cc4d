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

from gguf_fixtures import MINI, gguf_bytes, mixed_model, oracle_of
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def F(dev):
    from cosxamix_amd import forward
    return forward



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


@pytest.mark.parametrize("varied", [False, True], ids=["unit-norms", "varied-norms-biases"])
def test_mixed_format_file_matches_the_oracle(F, tmp_path, varied):
    """varied: every norm ~ N(1, 0.1) and q/k/v biases in both layers."""
    data, host, types = mixed_model(varied=varied)
    path = tmp_path / "mixed.gguf"
    path.write_bytes(data)
    m = F.Modelo.abrir(path)
    assert (m.cfg.ffn, m.cfg.vocab) == (MINI["ffn"], MINI["vocab"])
    names = [t[0] for t in m.tensores()]
    assert "output.weight" not in names and ("blk.1.attn_q.bias" in names) == varied
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
    # a matrix in a type the reference cannot unpack either (Q4_0): the Q8_0
    # file with the type id changed, its 34-byte blocks read as 18-byte ones
    data, _, _ = mixed_model(seed=9, override={"attn_output": O.Q8_0})
    name = b"blk.0.attn_output.weight"
    i = data.index(name) + len(name) + 4 + 16  # n_dims, two dims: the type
    assert struct.unpack("<I", data[i:i + 4])[0] == O.Q8_0
    p2 = tmp_path / "q4_0.gguf"
    p2.write_bytes(data[:i] + struct.pack("<I", 2) + data[i + 4:])
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
