"""The kernel contract (level 1 of the boundary) on host arrays.

Mirrors ``kernels::dot_q{2,3,4,5,6}k_i8`` (src/kernels/mod.rs:347-493,
src/kernels/q2k.rs:262-292): one row of super-blocks against an i8
activation with one f32 scale and one f32 sum per sub-block. Preconditions
are checked like the reference's ``assert!``s (here: ``ValueError``).
"""
from __future__ import annotations

import math

import numpy as np

from . import _lib as L

_lib = L.load()
_SUB = {L.Q2_K: 16, L.Q3_K: 16, L.Q4_K: 32, L.Q5_K: 32, L.Q6_K: 16}
_BPB = {L.Q2_K: 84, L.Q3_K: 110, L.Q4_K: 144, L.Q5_K: 176, L.Q6_K: 210}
_FN = {L.Q2_K: "cx_dot_q2k_i8", L.Q3_K: "cx_dot_q3k_i8", L.Q4_K: "cx_dot_q4k_i8",
       L.Q5_K: "cx_dot_q5k_i8", L.Q6_K: "cx_dot_q6k_i8"}


def dot_qk_i8(tipo: int, bloques: np.ndarray, xq: np.ndarray, xe: np.ndarray,
              xs: np.ndarray) -> float:
    bloques = np.ascontiguousarray(bloques, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    xe = np.ascontiguousarray(xe, dtype=np.float32)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    if xq.size % 256:
        raise ValueError("la fila tiene que ser multiplo de 256")
    if xe.size != xq.size // _SUB[tipo]:
        raise ValueError("faltan escalas")
    if xs.size != xe.size:
        raise ValueError("faltan sumas")
    if bloques.size < xq.size // 256 * _BPB[tipo]:
        raise ValueError("faltan bytes de pesos")
    y = getattr(_lib, _FN[tipo])(bloques.ctypes.data_as(L._u8p), xq.ctypes.data_as(L._i8p),
                                 xe.ctypes.data_as(L._f32p), xs.ctypes.data_as(L._f32p),
                                 xq.size // 256)
    if math.isnan(y) and L.last_error():
        raise L.CxError(L.last_error())
    return y


def dot_q2k_i8(b, xq, xe, xs):
    return dot_qk_i8(L.Q2_K, b, xq, xe, xs)


def dot_q3k_i8(b, xq, xe, xs):
    return dot_qk_i8(L.Q3_K, b, xq, xe, xs)


def dot_q4k_i8(b, xq, xe, xs):
    return dot_qk_i8(L.Q4_K, b, xq, xe, xs)


def dot_q5k_i8(b, xq, xe, xs):
    return dot_qk_i8(L.Q5_K, b, xq, xe, xs)


def dot_q6k_i8(b, xq, xe, xs):
    return dot_qk_i8(L.Q6_K, b, xq, xe, xs)
