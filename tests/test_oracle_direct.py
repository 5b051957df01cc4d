"""The oracle's buffer path (ops::matmul_i8_directo, src/ops.rs:310-414) for
Q8_0 and Q5_0, the formats of models whose width is not a multiple of 256
(src/gguf.rs:80-82): the reference's own Q8_0 tests (src/ops.rs:1331-1426,
1614-1670) and closed forms."""
import numpy as np
import pytest

from oracle import oracle as O


def q8_identity(n, k):  # src/ops.rs:1336-1351
    b = np.zeros((n, k // 32, 34), np.uint8)
    b[:, :, 0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)  # d = 1
    for r in range(min(n, k)):
        b[r, r // 32, 2 + r % 32] = 1
    return b.reshape(n, -1)


def q5_0_rows(rows, width, seed):
    """Q5_0 rows with any quants and a power-of-two scale per block."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (rows * width // 32, 22), dtype=np.uint8)
    d = rng.choice([0x2000, 0x2400, 0x2800, 0x1C00], rows * width // 32).astype(np.uint16)
    b[:, 0], b[:, 1] = d & 0xFF, d >> 8
    return b.reshape(rows, -1)


def q8_0_rows(rows, width, seed):
    x = np.random.default_rng(seed).normal(0, 0.02, rows * width).astype(np.float32)
    return O.quantize_blocks(O.Q8_0, x).reshape(rows, -1)


def test_identity_gives_the_quantized_input():
    """d = 1, a one on the diagonal: each output is one product, xe * xq,
    of the row's quantized input (src/ops.rs:1353-1361 with the i8 path)."""
    m, k, n = 3, 64, 64
    lhs = (np.arange(m * k, dtype=np.float32) * np.float32(0.25) - np.float32(4.0)).reshape(m, k)
    y = O.matmul_direct(O.Q8_0, lhs, q8_identity(n, k), n)
    for f in range(m):
        xq, xe, _ = O.quantize_act(lhs[f], 32)
        want = (xe[np.arange(k) // 32] * xq.astype(np.float32)).astype(np.float32)
        assert np.array_equal(y[f], want)
        assert np.abs(y[f] - lhs[f]).max() <= 0.51 * xe.max()


def test_one_row_and_many_rows_agree():  # src/ops.rs:1363-1393
    k, n = 64, 96
    w = q8_identity(n, k).reshape(-1).copy()
    idx = np.arange(w.size)
    sel = idx % 34 >= 2
    w[sel] = ((idx[sel] * 31) % 177).astype(np.uint8)
    w = w.reshape(n, -1)
    rows = np.stack([np.sin((np.arange(k) + f) * np.float32(0.13)).astype(np.float32)
                     for f in range(4)])
    batch = O.matmul_direct(O.Q8_0, rows, w, n)
    for f in range(4):
        assert np.array_equal(batch[f], O.matmul_direct(O.Q8_0, rows[f], w, n)[0])


def test_integer_and_f32_paths_agree_within_2pc_of_the_range():  # src/ops.rs:1395-1426
    m, k, n = 3, 128, 64
    w = q8_identity(n, k).reshape(-1).copy()
    idx = np.arange(w.size)
    sel = idx % 34 >= 2
    w[sel] = ((idx[sel] * 29) % 200).astype(np.uint8)
    w = w.reshape(n, -1)
    lhs = np.sin(np.arange(m * k, dtype=np.float32) * np.float32(0.07)).reshape(m, k)
    wf = O.dequantize(O.Q8_0, w, n * k).reshape(n, k).astype(np.float64)
    exact = lhs.astype(np.float64) @ wf.T
    got = O.matmul_direct(O.Q8_0, lhs, w, n)
    assert np.abs(got - exact).max() < 0.02 * (exact.max() - exact.min())


@pytest.mark.parametrize("t,k", [(O.Q8_0, 896), (O.Q5_0, 896), (O.Q8_0, 160), (O.Q5_0, 2048)])
def test_rows_are_the_blockwise_closed_form(t, k):
    """Each row is sum over blocks of (d_b * xe_b) * E_b with E_b the exact
    integer dot of the block's quants (dequantized value / d, the weights'
    own dequantizer) and the quantized input, added in block order."""
    n = 24
    w = q8_0_rows(n, k, 3) if t == O.Q8_0 else q5_0_rows(n, k, 3)
    x = np.random.default_rng(9).normal(0, 1, k).astype(np.float32)
    xq, xe, _ = O.quantize_act(x, 32)
    y = O.matmul_direct(t, x, w, n)[0]
    deq = O.dequantize(t, w, n * k).reshape(n, k)
    bpb = 34 if t == O.Q8_0 else 22
    for r in range(n):
        blocks = w[r].reshape(-1, bpb)
        d = blocks[:, :2].copy().view(np.float16).astype(np.float32).ravel()
        q = np.round(deq[r].reshape(-1, 32) / np.where(d == 0, 1, d)[:, None]).astype(np.int64)
        lo, hi = (-128, 127) if t == O.Q8_0 else (-16, 15)
        assert q.min() >= lo and q.max() <= hi
        e = (q * xq.reshape(-1, 32).astype(np.int64)).sum(1)
        acc = np.float32(0)
        for b in range(k // 32):
            acc = np.float32(acc + np.float32(np.float32(d[b] * xe[b]) * np.float32(e[b])))
        assert acc == y[r], (r, acc, y[r])


def test_q5_0_high_bits_sit_where_the_dequantizer_puts_them():
    """A block whose quants differ only in qh: the unpacked i8 values and the
    dequantized floats must agree value for value (q * d)."""
    b = np.zeros(22, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    qh = 0x8001_0003
    b[2:6] = np.frombuffer(np.uint32(qh).tobytes(), np.uint8)
    b[6:22] = np.arange(16, dtype=np.uint8) * 0x11
    q, e, o = O.unpack_i8(O.Q5_0, b, 32)
    y = O.dequantize(O.Q5_0, b, 32)
    assert e[0] == 1.0 and o[0] == 0.0
    assert np.array_equal(q.astype(np.float32), y)
    want = [(j % 16) + 16 * ((qh >> j) & 1) - 16 for j in range(32)]
    assert q.tolist() == want


def test_multi_with_buffer_formats_is_bit_identical_to_separate_calls():  # src/ops.rs:1614-1670
    k = 512
    w8 = q8_identity(5, k).reshape(-1).copy()
    idx = np.arange(w8.size)
    sel = idx % 34 >= 2
    w8[sel] = (((idx[sel] * 29) % 253) - 126).astype(np.int8).view(np.uint8)
    mats = [(O.daiss_matrix(1, "q", 70, k, 0.02, O.Q3_K), O.Q3_K, 70),
            (O.daiss_matrix(1, "k", 33, k, 0.02, O.Q4_K), O.Q4_K, 33),
            (w8.reshape(5, -1), O.Q8_0, 5),
            (q5_0_rows(40, k, 4), O.Q5_0, 40)]
    x = np.cos(np.arange(k, dtype=np.float32) * np.float32(0.021)).astype(np.float32)
    outs = O.matmul_multi_1row(x, mats, threads=4)
    for (w, t, n), o in zip(mats, outs):
        one = O.matmul_fused(t, x, w, n)[0] if t in (O.Q3_K, O.Q4_K) else O.matmul_direct(t, x, w, n)[0]
        assert np.array_equal(o, one), t


def test_shape_errors():  # src/ops.rs:1692-1697
    w = q8_identity(32, 64)
    with pytest.raises(ValueError):
        O.matmul_direct(O.Q8_0, np.zeros(63, np.float32), w, 32)
    with pytest.raises(ValueError):
        O.matmul_direct(O.F32, np.zeros(64, np.float32), w, 32)
