"""The C-ABI library without a GPU: it loads, exports every symbol
include/cosxamix_hip.h declares, and its host-only entry points (geometry,
RoPE tables, argument validation) behave. No kernel is launched here."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cosxamix_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cx_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from cosxamix_amd import _lib
    _lib.load()
    return _lib


def test_library_exports_every_declared_symbol(L):
    names = declared()
    assert len(names) >= 30
    out = subprocess.run(["nm", "-D", "--defined-only", L.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s(cx_\w+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    # the ctypes binding covers the same set
    assert set(L.SIGNATURES) == set(names)


def test_library_is_gfx950_code(L):
    """The embedded code object of our own build targets gfx950, and only it."""
    data = open(L.LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-f]+)", data))
    assert targets == {b"gfx950"}, targets


def test_geometry_matches_the_reference(L):  # src/gguf.rs:83-111, quant.rs:213-219
    lib = L.load()
    for t, bpb in O.BYTES_PER_BLOCK.items():
        k = 4096
        assert lib.cx_row_bytes(t, k) == k // O.VALUES_PER_BLOCK[t] * bpb
        assert lib.cx_sub_block(t) == O.SUB.get(t, 0)
    assert lib.cx_row_bytes(O.Q4_K, 1000) == 0
    assert lib.cx_row_bytes(99, 256) == 0


def test_rope_tables_bit_identical_to_oracle(L):  # src/ops.rs:1108-1129
    lib = L.load()
    for hd, base, ctx in [(128, 1e6, 700), (64, 10000.0, 2048), (128, 500000.0, 300)]:
        c = np.zeros(ctx * hd // 2, np.float32)
        s = np.zeros_like(c)
        assert lib.cx_rope_tables(hd, base, ctx, c.ctypes.data_as(L._f32p),
                                  s.ctypes.data_as(L._f32p)) == 0
        oc, os_ = O.rope_tables(hd, base, ctx)
        assert np.array_equal(c.view(np.uint32), oc.view(np.uint32))
        assert np.array_equal(s.view(np.uint32), os_.view(np.uint32))


def test_argument_errors_are_reported_not_crashed(L):
    lib = L.load()
    p = C.c_void_p(1)  # never dereferenced: validation fails first
    assert lib.cx_matmul_auto(1, 1000, 4, p, p, O.Q4_K, p, None) == -1
    assert "256" in L.last_error()
    assert lib.cx_matmul_auto(1, 2048, 4, p, p, O.F32, p, None) == -1
    assert lib.cx_quantize_act(p, 1, 100, 24, p, p, p, None) == -1
    assert lib.cx_softmax(p, 10, 3, None) == -1
    assert lib.cx_attention(p, p, p, 2, 1, 4, 2, 8, p, None) == -1
    assert lib.cx_rope(p, 3, 2, 8, p, p, 16, 14, None) == -1
    assert lib.cx_rope(p, 1, 1, 3, p, p, 16, 0, None) == -1
    cfg = L.CxConfig(1, 100, 4, 2, 768, 10, 64, 1e-6, 1e4)
    h = C.c_void_p()
    assert lib.cx_model_create_daiss(C.byref(cfg), O.Q4_K, O.Q4_K, O.Q4_K, 1, C.byref(h)) == -1
    assert "head_dim" in L.last_error()
    # daiss-0.5b's dim of 896 is 3.5 blocks of 256: k-quants refused (Q8_0 is its type)
    cfg = L.CxConfig(1, 896, 14, 2, 4864, 10, 64, 1e-6, 1e4)
    assert lib.cx_model_create_daiss(C.byref(cfg), O.Q4_K, O.Q4_K, O.Q4_K, 1, C.byref(h)) == -1
    assert "whole blocks" in L.last_error()
    assert lib.cx_model_create_daiss(C.byref(cfg), O.Q6_K, O.Q6_K, O.Q6_K, 1, C.byref(h)) == -1
    assert "quantizers" in L.last_error()
    assert lib.cx_matmul_auto(1, 100, 4, p, p, O.Q8_0, p, None) == -1
    assert "32" in L.last_error()


def test_noalloc_checks_arguments_before_sizing_its_scratch(L):
    """cx_matmul_auto_noalloc refuses a type with no quantized path (Q4_0,
    an unknown id) or a ragged row with CX_EINVAL before it sizes its
    scratch (which divides by the type's sub-block)."""
    lib = L.load()
    p = C.c_void_p(1)  # never dereferenced: validation fails first
    for t in (2, 15, 99):  # Q4_0, Q8_K, not a type
        assert lib.cx_matmul_auto_noalloc(4, 256, 8, p, p, t, p, None) == L.CX_EINVAL, t
        assert "no quantized path" in L.last_error()
    assert lib.cx_matmul_auto_noalloc(4, 1000, 8, p, p, O.Q4_K, p, None) == L.CX_EINVAL
    assert "256" in L.last_error()
    assert lib.cx_matmul_auto_noalloc(4, 256, 8, None, p, O.Q4_K, p, None) == L.CX_EINVAL
    assert "null" in L.last_error()
