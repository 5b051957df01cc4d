"""GGUF reading on the host (no GPU): the library's parser against the
reference's own GGUF tests (src/gguf.rs:448-630). The test file below is
the byte layout of the reference's `gguf_de_prueba` (src/gguf.rs:454-506),
rebuilt here as data; the expected values are the reference test's
assertions."""
import struct

import numpy as np
import pytest


@pytest.fixture(scope="module")
def G():
    from cosxamix_amd import gguf
    return gguf


def text(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def fixture_file(alignment=None) -> bytes:
    """src/gguf.rs:454-506: 2 tensors, 4 metadata entries (a string, a u32,
    an f32, a list of strings), padding to 32, then 4096 bytes of 0xAB.
    With `alignment`, a fifth entry general.alignment (u32) and that padding."""
    nm = 4 + (alignment is not None)
    b = b"GGUF" + struct.pack("<IQQ", 3, 2, nm)
    b += text("general.architecture") + struct.pack("<I", 8) + text("qwen2")
    b += text("qwen2.block_count") + struct.pack("<II", 4, 24)
    b += text("qwen2.rope.freq_base") + struct.pack("<I", 6) + struct.pack("<f", 1_000_000.0)
    b += text("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, 2) + text("hola") + text("chau")
    if alignment is not None:
        b += text("general.alignment") + struct.pack("<II", 4, alignment)
    b += text("norm.weight") + struct.pack("<IQIQ", 1, 8, 0, 0)
    b += text("blk.0.attn_q.weight") + struct.pack("<IQQIQ", 2, 64, 2, 8, 32)
    al = alignment or 32
    b += b"\0" * ((al - len(b) % al) % al)
    return b + b"\xAB" * 4096


def write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return p


def test_reads_header_metadata_and_tensors(G, tmp_path):  # src/gguf.rs:514-545
    g = G.Gguf.abrir(write(tmp_path, "ok.gguf", fixture_file()))
    assert g.version == 3
    assert g.meta_texto("general.architecture") == "qwen2"
    assert g.meta_entero("qwen2.block_count") == 24
    assert g.meta_decimal("qwen2.rope.freq_base") == 1_000_000.0
    # the list was read whole, not skipped
    assert g.meta_tipo("tokenizer.ggml.tokens") == (9, 2)
    assert g.meta_texto("tokenizer.ggml.tokens", 1) == "chau"
    assert len(g.tensores) == 2
    q = g.tensor("blk.0.attn_q.weight")
    assert q.dims == [64, 2]
    assert q.tipo == 8  # Q8_0
    assert q.elementos() == 128
    assert q.bytes() == 136  # 4 blocks of 34 bytes
    assert g.tensor("no.such.tensor") is None
    assert g.meta_entero("missing.key") is None
    # decimal reads an integer too (Valor::decimal, src/gguf.rs:157-163)
    assert g.meta_decimal("qwen2.block_count") == 24.0


def test_respects_the_declared_alignment(G, tmp_path):  # src/gguf.rs:551-561
    base = fixture_file()
    g = G.Gguf.abrir(write(tmp_path, "align.gguf", base))
    assert g.inicio_datos % 32 == 0 and g.inicio_datos >= 1
    # a file that declares another alignment starts its data there
    g64 = G.Gguf.abrir(write(tmp_path, "align64.gguf", fixture_file(alignment=64)))
    assert g64.alineacion == 64 and g64.inicio_datos % 64 == 0
    header_end = len(fixture_file(alignment=64)) - 4096
    assert g64.inicio_datos == header_end


def test_rejects_what_is_not_gguf(G, tmp_path):  # src/gguf.rs:563-568
    with pytest.raises(ValueError):
        G.Gguf.abrir(write(tmp_path, "no.bin", b"esto no es un modelo"))


def test_a_truncated_file_is_an_error(G, tmp_path):  # src/gguf.rs:570-580
    with pytest.raises(ValueError):
        G.Gguf.abrir(write(tmp_path, "short.gguf", fixture_file()[:40]))


def test_bad_versions_dims_and_types_are_errors(G, tmp_path):  # src/gguf.rs:283-307
    f = bytearray(fixture_file())
    f[4:8] = struct.pack("<I", 1)
    with pytest.raises(ValueError):
        G.Gguf.abrir(write(tmp_path, "v1.gguf", bytes(f)))
    g = fixture_file()
    i = g.index(text("norm.weight")) + len(text("norm.weight"))
    bad_dims = g[:i] + struct.pack("<I", 5) + g[i + 4:]
    with pytest.raises(ValueError):
        G.Gguf.abrir(write(tmp_path, "dims.gguf", bad_dims))
    j = i + 4 + 8  # after n_dims and the one dim: the type
    bad_type = g[:j] + struct.pack("<I", 5) + g[j + 4:]  # 5 is not a GGML type
    with pytest.raises(ValueError):
        G.Gguf.abrir(write(tmp_path, "type.gguf", bad_type))


def test_block_sizes_are_the_formats(G):  # src/gguf.rs:583-608
    for t, vals, nbytes in [(0, 1, 4), (1, 1, 2), (2, 32, 18), (6, 32, 22), (8, 32, 34),
                            (10, 256, 84), (11, 256, 110), (12, 256, 144), (13, 256, 176),
                            (14, 256, 210)]:
        assert G.GEOMETRIA[t] == (vals, nbytes)


def test_tensor_bytes_match_the_file_and_respect_bounds(G, tmp_path):  # src/gguf.rs:610-640
    data = fixture_file()
    p = write(tmp_path, "map.gguf", data)
    g = G.Gguf.abrir(p)
    for t in g.tensores:
        got = g.datos_de(t)
        start = g.inicio_datos + t.offset
        assert np.array_equal(got, np.frombuffer(data[start:start + t.bytes()], np.uint8))
    # a tensor asking past the end of the file: an error, not a read
    far = G.InfoTensor(g.tensores[0].nombre, [1 << 40], g.tensores[0].tipo, 0)
    with pytest.raises(ValueError, match="the file has"):
        g.datos_de(far)
    # and an absurd offset, the other road to the same place
    off = G.InfoTensor(g.tensores[0].nombre, [8], 0, (1 << 64) - 16)
    with pytest.raises(ValueError):
        g.datos_de(off)
