"""GGUF files — the host-side mirror of the reference's ``gguf`` module
(src/gguf.rs:119-436: ``Gguf::abrir``, ``meta_entero``, ``meta_decimal``,
``tensor``, ``datos_de``), through the library's C ABI (no device work).
Errors raise ``ValueError`` where the reference returns ``Err``."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib as L

_lib = L.load()


# TipoGgml block geometry (src/gguf.rs:83-111): type -> (values, bytes)
GEOMETRIA = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
             8: (32, 34), 9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144),
             13: (256, 176), 14: (256, 210), 15: (256, 292)}


@dataclass
class InfoTensor:
    """InfoTensor (src/gguf.rs:172-194): dims as stored in the file
    (fastest-varying first), offset from the start of the data section."""
    nombre: str
    dims: list
    tipo: int
    offset: int

    def elementos(self) -> int:
        n = 1
        for d in self.dims:
            n *= int(d)
        return n

    def bytes(self) -> int:
        vpb, bpb = GEOMETRIA[self.tipo]
        return self.elementos() // vpb * bpb


class Gguf:
    def __init__(self, handle):
        self._h = handle
        v, nt, nm, ds, al = (C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_uint64(), C.c_uint64())
        L.check(_lib.cx_gguf_header(self._h, C.byref(v), C.byref(nt), C.byref(nm), C.byref(ds),
                                    C.byref(al)), "gguf")
        self.version = v.value
        self.inicio_datos = ds.value
        self.alineacion = al.value
        self.n_metadatos = nm.value
        self.tensores = []
        for i in range(nt.value):
            t = L.CxGgufTensor()
            L.check(_lib.cx_gguf_tensor_info(self._h, i, C.byref(t)), "gguf")
            self.tensores.append(InfoTensor(t.name.decode(), [int(d) for d in t.dims[:t.n_dims]],
                                            t.type, int(t.offset)))

    @classmethod
    def abrir(cls, ruta) -> "Gguf":
        """Gguf::abrir (src/gguf.rs:274-342): header, metadata and tensor
        table; the weights are not read."""
        h = C.c_void_p()
        if _lib.cx_gguf_open(str(ruta).encode(), C.byref(h)) != 0:
            raise ValueError(L.last_error())
        return cls(h)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.cx_gguf_free(h)
            except Exception:
                pass
            self._h = None

    def meta_entero(self, clave: str):
        v = C.c_uint64()
        return v.value if _lib.cx_gguf_meta_int(self._h, clave.encode(), C.byref(v)) == 0 else None

    def meta_decimal(self, clave: str):
        v = C.c_double()
        return v.value if _lib.cx_gguf_meta_float(self._h, clave.encode(), C.byref(v)) == 0 else None

    def meta_texto(self, clave: str, indice: int = -1):
        """Valor::texto of a string, or of element `indice` of a list."""
        n = C.c_size_t()
        if _lib.cx_gguf_meta_str(self._h, clave.encode(), indice, None, 0, C.byref(n)) != 0:
            return None
        buf = C.create_string_buffer(n.value + 1)
        L.check(_lib.cx_gguf_meta_str(self._h, clave.encode(), indice, buf, n.value + 1, None),
                "gguf")
        return buf.raw[:n.value].decode()

    def meta_tipo(self, clave: str):
        """(GGUF value type, element count) of a key, or None."""
        t, n = C.c_uint32(), C.c_uint64()
        if _lib.cx_gguf_meta_type(self._h, clave.encode(), C.byref(t), C.byref(n)) != 0:
            return None
        return t.value, n.value

    def tensor(self, nombre: str):
        """Gguf::tensor (src/gguf.rs:344-346)."""
        i = _lib.cx_gguf_find(self._h, nombre.encode())
        return None if i < 0 else self.tensores[i]

    def datos_de(self, info: InfoTensor) -> np.ndarray:
        """The tensor's bytes (Gguf::datos_de / Pesos::de, src/gguf.rs:357-436):
        an error, not a read, when it reaches past the end of the file."""
        n = info.bytes()
        if n >= 1 << 63 or info.offset >= 1 << 64:
            raise ValueError(f"{info.nombre}: the size overflows")
        raw = L.CxGgufTensor()
        raw.name = info.nombre.encode()[:127]
        raw.type = info.tipo
        raw.n_dims = len(info.dims)
        for d in range(4):
            raw.dims[d] = int(info.dims[d]) if d < len(info.dims) else 1
        raw.offset = int(info.offset)
        raw.elements = info.elementos() & ((1 << 64) - 1)
        raw.bytes = n
        # the range is checked before any allocation of the tensor's size
        if _lib.cx_gguf_tensor_read(self._h, C.byref(raw), None, 0) != 0:
            msg = L.last_error()
            if "needs" not in msg:
                raise ValueError(msg)
        out = np.empty(max(n, 1), dtype=np.uint8)
        if _lib.cx_gguf_tensor_read(self._h, C.byref(raw), out.ctypes.data_as(C.c_void_p),
                                    out.size) != 0:
            raise ValueError(L.last_error())
        return out[:n]
