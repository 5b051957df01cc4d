"""GPU parity of the format operators (MI355X), through the C ABI:
quant::descuantizar / descuantizar_filas / desempaquetar_i8 bit-exact with the
oracle (src/quant.rs:124-468), and matmul_auto's F32/F16 branch (ops::matmul,
src/ops.rs:87-156) within f32 rounding (relative L2 <= 1e-5) of a float64
product."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

ALL = (O.F32, O.F16, O.Q8_0, O.Q5_0, O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K, O.Q6_K)
QUANT = ALL[2:]
# byte offsets of the f16 scales inside a block (kept finite)
F16_AT = {O.Q8_0: (0,), O.Q5_0: (0,), O.Q2_K: (80, 82), O.Q3_K: (108,), O.Q4_K: (0, 2),
          O.Q5_K: (0, 2), O.Q6_K: (208,)}
VPB = {O.F32: 1, O.F16: 1, O.Q8_0: 32, O.Q5_0: 32}


@pytest.fixture(scope="module")
def ops(dev):
    from cosxamix_amd import ops
    return ops


def T(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def random_bytes(t, n, seed):
    """n values of type t: random quants, finite f16 scales (any bit pattern
    of the rest), finite F16/F32 values."""
    rng = np.random.default_rng(seed)
    if t == O.F32:
        return rng.normal(0, 3, n).astype(np.float32).view(np.uint8)
    if t == O.F16:
        h = rng.integers(0, 0x7C00, n, dtype=np.uint16) | (rng.integers(0, 2, n, dtype=np.uint16) << 15)
        return h.view(np.uint8)
    bpb, vpb = O.BYTES_PER_BLOCK[t], VPB.get(t, 256)
    nb = n // vpb
    b = rng.integers(0, 256, (nb, bpb), dtype=np.uint8)
    for off in F16_AT[t]:
        h = rng.integers(0x0400, 0x3C00, nb) | (rng.integers(0, 2, nb) << 15)
        b[:, off] = h & 0xFF
        b[:, off + 1] = h >> 8
    return b.reshape(-1)


@pytest.mark.parametrize("t", ALL)
def test_dequantize_bit_exact(ops, dev, t):  # src/quant.rs:124-162, 501-679
    n = 4096 + (8 if t in (O.F32, O.F16) else 0) + (3 if t == O.F16 else 0)
    b = random_bytes(t, n, seed=t + 1)
    got = ops.descuantizar(t, T(b, dev), n).cpu().numpy()
    want = O.dequantize(t, b, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), O.NAMES.get(t, t)


def test_dequantize_q8_0_hand_kat(ops, dev):  # src/quant.rs:830-839: d = 1, q = -16..15
    q = np.arange(-16, 16, dtype=np.int8)
    blk = np.concatenate([np.array([0x00, 0x3C], np.uint8), q.view(np.uint8)])
    got = ops.descuantizar(O.Q8_0, T(blk, dev), 32).cpu().numpy()
    assert np.array_equal(got, q.astype(np.float32))


def test_dequantize_rejects_partial_blocks(ops, dev):
    b = T(random_bytes(O.Q4_K, 256, 3), dev)
    with pytest.raises(ValueError):
        ops.descuantizar(O.Q4_K, b, 100)


@pytest.mark.parametrize("t", (O.F16, O.Q8_0, O.Q4_K, O.Q6_K, O.Q3_K))
def test_dequantize_rows_bit_exact(ops, dev, t):  # src/quant.rs:172-205
    width, rows = 512, 9
    b = random_bytes(t, width * rows, seed=40 + t)
    pick = [3, 0, 8, 8, 5]
    got = ops.descuantizar_filas(t, T(b, dev), width, pick).cpu().numpy()
    rb = O.row_bytes(t, width)
    for i, r in enumerate(pick):
        want = O.dequantize(t, b[r * rb:(r + 1) * rb], width)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), (t, r)
    with pytest.raises(ValueError):  # a row past the data is an error (src/quant.rs:194-197)
        ops.descuantizar_filas(t, T(b, dev), width, [rows])


@pytest.mark.parametrize("t", QUANT)
def test_unpack_bit_exact_and_reconstructs_dequantize(ops, dev, t):  # src/quant.rs:238-468, 892-928
    n = 4096
    b = random_bytes(t, n, seed=70 + t)
    q, esc, off, sub = ops.desempaquetar_i8(t, T(b, dev), n)
    q, esc, off = (v.cpu().numpy() for v in (q, esc, off))
    assert sub == O.SUB[t]
    wq, we, wo = O.unpack_i8(t, b, n)
    assert np.array_equal(q, wq)
    assert np.array_equal(esc.view(np.uint32), we.view(np.uint32))
    assert np.array_equal(off.view(np.uint32), wo.view(np.uint32))
    # value = escala * q + desplazamiento reproduces descuantizar exactly
    rec = np.repeat(esc, sub) * q.astype(np.float32) + np.repeat(off, sub)
    assert np.array_equal(rec, O.dequantize(t, b, n))


@pytest.mark.parametrize("t", (O.F32, O.F16))
@pytest.mark.parametrize("m", (1, 5, 9))
def test_matmul_auto_unquantized(ops, dev, t, m):  # src/ops.rs:1064-1071 -> 87-156
    n, k = 300, 2048
    rng = np.random.default_rng(m + t)
    w32 = rng.normal(0, 0.05, (n, k)).astype(np.float32)
    wb = w32 if t == O.F32 else w32.astype(np.float16)
    lhs = rng.normal(0, 1, (m, k)).astype(np.float32)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    ops.matmul_auto((m, k, n), T(lhs, dev), T(wb.view(np.uint8).reshape(-1), dev), t, dst)
    want = lhs.astype(np.float64) @ wb.astype(np.float64).T
    got = dst.cpu().numpy().astype(np.float64)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) <= 1e-5
    # and one row of a batch equals the row alone (src/ops.rs:1364-1393)
    one = torch.empty(n, dtype=torch.float32, device=dev)
    ops.matmul_auto((1, k, n), T(lhs[-1], dev), T(wb.view(np.uint8).reshape(-1), dev), t, one)
    assert torch.equal(one, dst[-1])
