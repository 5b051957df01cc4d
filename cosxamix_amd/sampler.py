"""``sampler::Muestreador`` (src/sampler.rs:27-152) over the C ABI: the
temperature / top-p sampler running on the GPU (cx_sample). The generator is
the reference's ``Azar`` (xorshift64*, src/daiss.rs:317-337), kept on the
host between calls exactly as the reference's struct keeps it."""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib as L
from .ops import _call, _ptr, _stream, argmax  # noqa: F401

_lib = L.load()


def semilla_azar(s: int) -> int:
    """Azar::con_semilla (src/daiss.rs:322-328): zero is xorshift's fixed point."""
    return s if s else 0x9E3779B97F4A7C15


class Muestreador:
    """Chooses tokens with temperature and top-p (src/sampler.rs:27-47)."""

    def __init__(self, semilla: int, temperatura: float, top_p: float):
        self.estado = semilla_azar(semilla & (2**64 - 1))
        self.temperatura = float(temperatura)
        self.top_p = float(top_p)
        self.semilla = semilla

    @classmethod
    def voraz(cls) -> "Muestreador":
        """Muestreador::voraz (src/sampler.rs:49-51): always the argmax."""
        return cls(0, 0.0, 1.0)

    def avanzar(self, n: int) -> None:
        """n draws of Azar::siguiente (src/daiss.rs:330-337) whose values
        are not needed."""
        M = 2**64 - 1
        x = self.estado
        for _ in range(n):
            x ^= x >> 12
            x ^= (x << 25) & M
            x ^= x >> 27
        self.estado = x

    def elegir(self, logits: torch.Tensor) -> int:
        """Muestreador::elegir (src/sampler.rs:61-125) on device logits."""
        st = C.c_uint64(self.estado)
        out = C.c_uint32()
        _call(_lib.cx_sample, _ptr(logits) if logits.numel() else None, logits.numel(),
              self.temperatura, self.top_p, C.byref(st), C.byref(out), _stream(), what="elegir")
        self.estado = st.value
        return out.value
