"""Writes tests/golden/kquant_rows.npz: row-kernel golden vectors.

Inputs are made here (seeded daiss rows quantized by the oracle, the
reference's closed-form byte pattern (i*131+17)%251 of
src/kernels/mod.rs:815-817, and extreme activations at +-127); the expected
outputs come from the REFERENCE's OWN compiled native x86 kernels
(oracle/_ref/libcxref.so, built by `make -C oracle ref` from
/root/reference/kernels): cosxamix_q2k_{c,asm}, cosxamix_q3k_{c,completo},
cosxamix_q4k_completo, cosxamix_q5k_{c,asm}.

Run in the dev container (it needs /root/reference):
    python tests/golden/make_golden.py
The .npz is data (inputs and f32 outputs); it carries no reference source.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kquant_rows.npz")


# where each format keeps its f16 d (and dmin) inside a block
F16_AT = {O.Q2_K: (80, 82), O.Q3_K: (108,), O.Q4_K: (0, 2), O.Q5_K: (0, 2)}


def pattern_rows(t: int, rows: int, k: int) -> np.ndarray:
    """(i*131+17)%251 bytes with finite f16 scales patched in (0x2C00, 0x2400),
    as the reference's own tests do (src/ops.rs:1630-1642): the raw pattern
    can hit f16 exponent 31 (inf/NaN)."""
    rb, bpb = O.row_bytes(t, k), O.BYTES_PER_BLOCK[t]
    i = np.arange(rows * rb, dtype=np.int64)
    w = ((i * 131 + 17) % 251).astype(np.uint8).reshape(rows, rb)
    for b in range(k // 256):
        for off, h in zip(F16_AT[t], (0x2C00, 0x2400)):
            w[:, b * bpb + off] = h & 0xFF
            w[:, b * bpb + off + 1] = h >> 8
    return w


def main():
    r = O.load_ref()
    if r is None:
        raise SystemExit("oracle/_ref/libcxref.so is not built: run `make -C oracle ref`")
    kernels = O.ref_kernels(r)
    data = {}
    for t in (O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K):
        for k in (2048, 11008):
            sub = O.SUB[t]
            name = f"{O.NAMES[t]}_{k}"
            w = np.concatenate([
                O.daiss_matrix(7, f"golden.{name}", 4, k, 0.02, t),
                pattern_rows(t, 2, k),
            ])
            x = O.daiss_row(11, f"golden.x.{k}", 0, 1.0, k)
            acts = {"normal": O.quantize_act(x, sub)}
            # extremes at the edge of the contract (-128 never appears)
            xq = np.where(np.arange(k) % 3 == 0, 127, -127).astype(np.int8)
            xe = np.full(k // sub, 1.0 / 127.0, np.float32)
            xs = xq.reshape(-1, sub).astype(np.int32).sum(1).astype(np.float32)
            acts["extreme"] = (xq, xe, xs)
            data[f"{name}_w"] = w
            for an, (xq, xe, xs) in acts.items():
                data[f"{name}_{an}_xq"] = xq
                data[f"{name}_{an}_xe"] = xe
                data[f"{name}_{an}_xs"] = xs
                for kn, fn in kernels[t]:
                    ys = np.array([fn(O._p(np.ascontiguousarray(row), O._u8p), O._p(xq, O._i8p),
                                      O._p(xe, O._f32p), O._p(xs, O._f32p), k // 256)
                                   for row in w], dtype=np.float32)
                    data[f"{name}_{an}_ref_{kn}"] = ys
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT}: {os.path.getsize(OUT)} bytes, {len(data)} arrays")


if __name__ == "__main__":
    main()
