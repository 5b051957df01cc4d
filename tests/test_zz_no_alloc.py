"""cx_matmul_auto_noalloc (the allocation-free variant of cx_matmul_auto)
through the C ABI: bit-identical to cx_matmul_auto on two calls in a row,
the second smaller (the shared device array keeps the first call's bytes),
for the MFMA contraction (m > 1), the GEMV (m = 1), the 32-value block
types and F32; a call needing more than the array is refused."""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _call(lib, fn, m, k, n, x, w, t, y):
    from cosxamix_amd import _lib as L
    rc = fn(m, k, n, C.c_void_p(x.data_ptr()), C.c_void_p(w.data_ptr()), t,
            C.c_void_p(y.data_ptr()), C.c_void_p(torch.cuda.current_stream().cuda_stream))
    L.check(rc, "matmul")


CASES = [  # (type, k, n, (first m, second m))
    (O.Q4_K, 2048, 1024, (64, 8)),
    (O.Q5_K, 4096, 512, (33, 1)),
    (O.Q3_K, 2048, 768, (17, 5)),
    (O.Q8_0, 896, 640, (40, 3)),
    (O.Q6_K, 1024, 300, (1, 1)),
]


@pytest.mark.parametrize("t,k,n,ms", CASES, ids=[O.NAMES.get(c[0], "Q8_0") + f"-{c[3]}" for c in CASES])
def test_noalloc_equals_matmul_auto(dev, t, k, n, ms):
    from cosxamix_amd import _lib as L
    lib = L.load()
    if t == O.Q6_K:  # no quantizer for Q6_K: random quants, a finite f16 d per block
        wb = np.random.default_rng(6).integers(0, 256, (n, k // 256, 210), dtype=np.uint8)
        wb[:, :, 208], wb[:, :, 209] = 0x00, 0x20
        w = torch.from_numpy(wb.reshape(n, -1)).to(dev)
    else:
        w = torch.from_numpy(O.daiss_matrix(21, "w", n, k, 0.02, t)).to(dev)
    for m in ms:
        x = torch.randn(m, k, generator=torch.Generator().manual_seed(m + k), dtype=torch.float32).to(dev)
        want = torch.empty(m, n, device=dev)
        got = torch.full((m, n), float("nan"), device=dev)
        _call(lib, lib.cx_matmul_auto, m, k, n, x, w, t, want)
        _call(lib, lib.cx_matmul_auto_noalloc, m, k, n, x, w, t, got)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (t, m)


def test_noalloc_f32_and_the_size_limit(dev):
    from cosxamix_amd import _lib as L
    lib = L.load()
    k, n = 256, 96
    w = torch.randn(n, k, generator=torch.Generator().manual_seed(1)).to(dev)
    for m in (7, 2):
        x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(dev)
        want, got = torch.empty(m, n, device=dev), torch.empty(m, n, device=dev)
        _call(lib, lib.cx_matmul_auto, m, k, n, x, w, O.F32, want)
        _call(lib, lib.cx_matmul_auto_noalloc, m, k, n, x, w, O.F32, got)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    # 4096 rows of 14336 values need ~88 MB of scratch: refused, nothing
    # launched (the pointers are checked for null, never dereferenced)
    p = C.c_void_p(1)
    big = lib.cx_matmul_auto_noalloc(4096, 14336, 16, p, p, O.Q4_K, p, None)
    assert big == L.CX_EINVAL and b"past its" in lib.cx_last_error()
    # a type with no quantized path (Q4_0) is refused before the scratch is
    # sized; the next call works as before
    assert lib.cx_matmul_auto_noalloc(4, 256, 8, p, p, 2, p, None) == L.CX_EINVAL
    assert b"no quantized path" in lib.cx_last_error()
    x = torch.randn(3, k, generator=torch.Generator().manual_seed(9)).to(dev)
    want, got = torch.empty(3, n, device=dev), torch.empty(3, n, device=dev)
    _call(lib, lib.cx_matmul_auto, 3, k, n, x, w, O.F32, want)
    _call(lib, lib.cx_matmul_auto_noalloc, 3, k, n, x, w, O.F32, got)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
