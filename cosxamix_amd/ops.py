"""Operators of the decode path on the GPU — the host-side mirror of the
reference's ``ops`` / ``kernels`` / ``sampler`` API (src/ops.rs,
src/kernels/mod.rs, src/sampler.rs), called through the C ABI.

Tensors are torch tensors on a ROCm device (torch is the device-memory and
stream plumbing); every call is enqueued on the current torch stream.
Shape errors raise ``ValueError`` where the reference returns ``Err``.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib as L
from ._lib import Q2_K, Q3_K, Q4_K, Q5_K, Q6_K  # noqa: F401

_lib = L.load()

BYTES_PER_BLOCK = {L.F32: 4, L.F16: 2, L.Q5_0: 22, L.Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144,
                   Q5_K: 176, Q6_K: 210}
VALUES_PER_BLOCK = {L.F32: 1, L.F16: 1, L.Q5_0: 32, L.Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256,
                    Q5_K: 256, Q6_K: 256}


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: torch.Tensor):
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return C.c_void_p(t.data_ptr())


def _call(fn, *args, what=""):
    rc = fn(*args)
    if rc != 0:
        msg = L.last_error()
        raise ValueError(f"{what}: {msg}") if rc == -1 else L.CxError(f"{what}: {msg}")


def sub_block(tipo: int):
    """quant::sub_bloque (src/quant.rs:213-219); None for types without one."""
    s = _lib.cx_sub_block(tipo)
    return s or None


def row_bytes(tipo: int, k: int) -> int:
    return k // VALUES_PER_BLOCK[tipo] * BYTES_PER_BLOCK[tipo]


def cuantizar_i8_en(x: torch.Tensor, bloque: int):
    """ops::cuantizar_i8_en + the per-sub-block sums (src/ops.rs:178-198,
    472-483). x: f32 [rows, k] or [k]. Returns (xq i8, xe f32, xs f32)."""
    rows, k = (1, x.numel()) if x.dim() == 1 else tuple(x.shape)
    xq = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    ns = k // bloque
    shape = (ns,) if x.dim() == 1 else (rows, ns)
    xe = torch.empty(shape, dtype=torch.float32, device=x.device)
    xs = torch.empty(shape, dtype=torch.float32, device=x.device)
    _call(_lib.cx_quantize_act, _ptr(x), rows, k, bloque, _ptr(xq), _ptr(xe), _ptr(xs), _stream(),
          what="cuantizar_i8_en")
    return xq, xe, xs


def gemv(tipo: int, pesos: torch.Tensor, n: int, k: int, xq, xe, xs) -> torch.Tensor:
    """y[r] = fused dot of row r (the per-row kernel of matmul_i8_fusionado)."""
    y = torch.empty(n, dtype=torch.float32, device=pesos.device)
    _call(_lib.cx_gemv, tipo, _ptr(pesos), n, k, _ptr(xq), _ptr(xe), _ptr(xs), _ptr(y), _stream(),
          what="gemv")
    return y


def gemv_subsums(tipo: int, pesos: torch.Tensor, n: int, k: int, xq, xe, xs) -> torch.Tensor:
    """Integer per-sub-block sums formed by the GEMV kernel's lanes."""
    out = torch.empty((n, k // sub_block(tipo)), dtype=torch.int32, device=pesos.device)
    _call(_lib.cx_gemv_subsums, tipo, _ptr(pesos), n, k, _ptr(xq), _ptr(xe), _ptr(xs), _ptr(out),
          _stream(), what="gemv_subsums")
    return out


def cuantizar_bloques(tipo: int, x: torch.Tensor) -> torch.Tensor:
    """quant::cuantizar_bloques for Q2_K..Q5_K (src/quant.rs:744-805) on the GPU."""
    out = torch.empty(row_bytes(tipo, x.numel()), dtype=torch.uint8, device=x.device)
    _call(_lib.cx_quantize_blocks, tipo, _ptr(x), x.numel(), _ptr(out), _stream(),
          what="cuantizar_bloques")
    return out


def descuantizar(tipo: int, bloques: torch.Tensor, n: int) -> torch.Tensor:
    """quant::descuantizar (src/quant.rs:124-162): n values of GGUF bytes to f32."""
    vpb = VALUES_PER_BLOCK.get(tipo)
    if vpb is None:
        raise ValueError(f"tipo {tipo}: sin descuantizador")
    if n % vpb:
        raise ValueError(f"pedí {n} valores y el bloque es de {vpb}")
    if bloques.numel() < row_bytes(tipo, n):
        raise ValueError("faltan bytes")
    y = torch.empty(n, dtype=torch.float32, device=bloques.device)
    _call(_lib.cx_dequantize, tipo, _ptr(bloques), n, _ptr(y), _stream(), what="descuantizar")
    return y


def descuantizar_filas(tipo: int, datos: torch.Tensor, ancho: int, filas) -> torch.Tensor:
    """quant::descuantizar_filas (src/quant.rs:172-205): the rows `filas` of a
    row-major matrix of `ancho` values per row, as f32 [len(filas), ancho]."""
    total = datos.numel() // row_bytes(tipo, ancho)
    ids = (C.c_size_t * len(filas))(*[int(f) for f in filas])
    y = torch.empty((len(filas), ancho), dtype=torch.float32, device=datos.device)
    _call(_lib.cx_dequantize_rows, tipo, _ptr(datos), ancho, total, ids, len(filas), _ptr(y),
          _stream(), what="descuantizar_filas")
    return y


def desempaquetar_i8(tipo: int, bloques: torch.Tensor, n: int):
    """quant::desempaquetar_i8 (src/quant.rs:238-468): (q i8[n], escalas,
    desplazamientos f32[n/sub], sub) with value = escala*q + desplazamiento."""
    sub = sub_block(tipo)
    if sub is None:
        raise ValueError(f"tipo {tipo}: sin desempaquetado directo a i8")
    q = torch.empty(n, dtype=torch.int8, device=bloques.device)
    esc = torch.empty(n // sub, dtype=torch.float32, device=bloques.device)
    off = torch.empty(n // sub, dtype=torch.float32, device=bloques.device)
    out = C.c_int(0)
    _call(_lib.cx_unpack_i8, tipo, _ptr(bloques), n, _ptr(q), _ptr(esc), _ptr(off), C.byref(out),
          _stream(), what="desempaquetar_i8")
    return q, esc, off, out.value


def matmul_auto(mkn, lhs: torch.Tensor, pesos: torch.Tensor, tipo: int, dst: torch.Tensor) -> None:
    """ops::matmul_auto (src/ops.rs:1056-1093): dst[m,n] = lhs[m,k] . W[n,k]^T."""
    m, k, n = mkn
    if lhs.numel() != m * k:
        raise ValueError(f"lhs mide {lhs.numel()} y deberia medir {m}*{k}")
    if dst.numel() != m * n:
        raise ValueError(f"dst mide {dst.numel()} y deberia medir {m}*{n}")
    if pesos.numel() < n * row_bytes(tipo, k):
        raise ValueError("faltan bytes de pesos")
    _call(_lib.cx_matmul_auto, m, k, n, _ptr(lhs), _ptr(pesos), tipo, _ptr(dst), _stream(),
          what="matmul_auto")


def matmul_varias_una_fila(x: torch.Tensor, pesos, destinos) -> None:
    """ops::matmul_varias_una_fila (src/ops.rs:895-1009): destinos[i] = x . W_i^T.
    pesos: list of (bytes tensor, type)."""
    if len(pesos) != len(destinos):
        raise ValueError("hace falta un destino por matriz")
    k = x.numel()
    cnt = len(pesos)
    for (w, t), d in zip(pesos, destinos):
        if w.numel() < d.numel() * row_bytes(t, k):
            raise ValueError("faltan bytes de pesos")
    ws = (C.c_void_p * cnt)(*[w.data_ptr() for w, _ in pesos])
    ts = (C.c_int * cnt)(*[t for _, t in pesos])
    ns = (C.c_size_t * cnt)(*[d.numel() for d in destinos])
    ds = (C.c_void_p * cnt)(*[d.data_ptr() for d in destinos])
    _call(_lib.cx_matmul_multi_1row, _ptr(x), k, cnt, ws, ts, ns, ds, _stream(),
          what="matmul_varias_una_fila")


def rmsnorm(salida: torch.Tensor, entrada: torch.Tensor, peso: torch.Tensor, eps: float) -> None:
    """kernels::rmsnorm (src/kernels/mod.rs:511-536), row by row."""
    n = peso.numel()
    if entrada.numel() % n or salida.numel() != entrada.numel():
        raise ValueError("rmsnorm: salida y entrada miden distinto")
    _call(_lib.cx_rmsnorm, _ptr(salida), _ptr(entrada), _ptr(peso), entrada.numel() // n, n, eps,
          _stream(), what="rmsnorm")


def silu(salida: torch.Tensor, entrada: torch.Tensor) -> None:
    """kernels::silu (src/kernels/mod.rs:495-509)."""
    if salida.numel() != entrada.numel():
        raise ValueError("silu: salida y entrada miden distinto")
    _call(_lib.cx_silu, _ptr(salida), _ptr(entrada), entrada.numel(), _stream(), what="silu")


def frecuencias_rope(dim_cabeza: int, base: float, contexto: int):
    """ops::frecuencias_rope (src/ops.rs:1108-1129), computed on the host."""
    half = dim_cabeza // 2
    c = np.zeros(contexto * half, np.float32)
    s = np.zeros_like(c)
    _call(_lib.cx_rope_tables, dim_cabeza, base, contexto, c.ctypes.data_as(L._f32p),
          s.ctypes.data_as(L._f32p), what="frecuencias_rope")
    return c, s


def rope(x: torch.Tensor, forma, cos: torch.Tensor, sin: torch.Tensor, posicion: int) -> None:
    """ops::rope (src/ops.rs:1150-1193), in place. forma = (tokens, cabezas, dim_cabeza)."""
    tokens, cabezas, dim_cabeza = forma
    if x.numel() != tokens * cabezas * dim_cabeza:
        raise ValueError("rope: x no cuadra con la forma")
    ctx = cos.numel() // (dim_cabeza // 2)
    _call(_lib.cx_rope, _ptr(x), tokens, cabezas, dim_cabeza, _ptr(cos), _ptr(sin), ctx, posicion,
          _stream(), what="rope")


def softmax(x: torch.Tensor, ancho: int) -> None:
    """ops::softmax (src/ops.rs:1206-1230), in place by rows of `ancho`."""
    _call(_lib.cx_softmax, _ptr(x), x.numel(), ancho, _stream(), what="softmax")


def atencion(q, k, v, forma, salida) -> None:
    """ops::atencion (src/ops.rs:1258-1325). forma = (tokens, total, cabezas,
    cabezas_kv, dim_cabeza)."""
    tokens, total, cabezas, cabezas_kv, dim_cabeza = forma
    _call(_lib.cx_attention, _ptr(q), _ptr(k), _ptr(v), tokens, total, cabezas, cabezas_kv,
          dim_cabeza, _ptr(salida), _stream(), what="atencion")


def atencion_decode(q, k, v, forma, salida, modo: int = 0) -> None:
    """ops::atencion at tokens = 1 with the model's decode kernels.
    forma = (total, cabezas, cabezas_kv, dim_cabeza); modo 0 auto, 1 order-
    exact, 2 split-K."""
    total, cabezas, cabezas_kv, dim_cabeza = forma
    _call(_lib.cx_attention_decode, _ptr(q), _ptr(k), _ptr(v), total, cabezas, cabezas_kv,
          dim_cabeza, modo, _ptr(salida), _stream(), what="atencion_decode")


def argmax(v: torch.Tensor) -> int:
    """sampler::argmax (src/sampler.rs:129-137)."""
    out = torch.empty(1, dtype=torch.int32, device=v.device)
    _call(_lib.cx_argmax, _ptr(v), v.numel(), _ptr(out), _stream(), what="argmax")
    return int(out.item())
