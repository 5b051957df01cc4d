"""The model level of the boundary: ``forward::{Config, Cache, Modelo}``
(src/forward.rs:36-137, 375-559) over the C ABI.

A ``Modelo`` owns its weights in HBM; a ``Cache`` owns the f32 KV cache and
the captured decode step. ``forward`` appends tokens and returns the logits
of the last one; ``generar`` is the greedy token loop of Modelo::generar.
"""
from __future__ import annotations

import ctypes as C
import weakref
from dataclasses import dataclass

import numpy as np

from . import _lib as L

_lib = L.load()


@dataclass(frozen=True)
class Config:
    """forward::Config (src/forward.rs:36-55) plus the daiss family shapes
    (src/daiss.rs:77-139)."""
    capas: int
    dim: int
    cabezas: int
    cabezas_kv: int
    ffn: int
    vocab: int
    contexto: int
    eps: float = 1e-6
    rope: float = 1_000_000.0

    def dim_cabeza(self) -> int:
        return self.dim // self.cabezas

    def dim_kv(self) -> int:
        return self.cabezas_kv * self.dim_cabeza()

    def c(self) -> L.CxConfig:
        return L.CxConfig(self.capas, self.dim, self.cabezas, self.cabezas_kv, self.ffn, self.vocab,
                          self.contexto, self.eps, self.rope)


# daiss-0.5b (src/daiss.rs:91-102): dim 896 is 3.5 blocks of 256, so its
# matrices are Q8_0 (the reference's writer) or Q5_0 (real Qwen2.5-0.5B GGUFs)
DAISS_0_5B = Config(24, 896, 14, 2, 4864, 151936, 32768, 1e-6, 1_000_000.0)
# daiss-3b (src/daiss.rs:103-114) = the Qwen2.5-3B shape of the benchmark
DAISS_3B = Config(36, 2048, 16, 2, 11008, 151936, 32768, 1e-6, 1_000_000.0)
# Llama-3-8B shape written as a qwen2-architecture model (zero biases)
LLAMA3_8B = Config(32, 4096, 32, 8, 14336, 128256, 8448 + 256, 1e-5, 500_000.0)


def bytes_de_cache_por_token(cfg: Config) -> int:
    """forward::bytes_de_cache_por_token (src/forward.rs:563-565)."""
    return 2 * cfg.capas * cfg.dim_kv() * 4


class Modelo:
    """A Qwen2 model resident in HBM: daiss-style seeded weights made on the
    GPU (the constructor), or a GGUF file (``Modelo.abrir``)."""

    def __init__(self, cfg: Config, tipo=L.Q4_K, semilla: int = 42, tipo_down=None,
                 tipo_salida=None):
        self.cfg = cfg
        h = C.c_void_p()
        L.check(_lib.cx_model_create_daiss(C.byref(cfg.c()), tipo, tipo_down or tipo,
                                           tipo_salida or tipo, semilla, C.byref(h)),
                "Modelo")
        self._h = h
        self._caches = weakref.WeakSet()

    @classmethod
    def abrir(cls, ruta) -> "Modelo":
        """Modelo::abrir (src/forward.rs:187-266): a GGUF file into HBM."""
        h = C.c_void_p()
        if _lib.cx_model_open(str(ruta).encode(), C.byref(h)) != 0:
            raise ValueError(L.last_error())
        m = cls.__new__(cls)
        m._h = h
        m._caches = weakref.WeakSet()
        c = L.CxConfig()
        L.check(_lib.cx_model_config(h, C.byref(c)), "Modelo")
        m.cfg = Config(c.layers, c.dim, c.heads, c.kv_heads, c.ffn, c.vocab, c.ctx, c.eps,
                       c.rope_base)
        return m

    def guardar(self, ruta) -> None:
        """The model as a GGUF file (the daiss writer's metadata, src/daiss.rs:422-468)."""
        L.check(_lib.cx_model_save_gguf(self._h, str(ruta).encode()), "guardar")

    def close(self):
        """Frees the model and, first, every cache still open on it."""
        for c in list(getattr(self, "_caches", ())):
            c.close()
        if getattr(self, "_h", None) and _lib is not None:
            _lib.cx_model_free(self._h)
        self._h = None

    def __del__(self):
        self.close()

    def bytes_por_token(self) -> int:
        """Weight bytes streamed per decode token (matrices + one embedding row)."""
        return int(_lib.cx_model_weight_bytes(self._h))

    def tensores(self):
        """[(name, type, (width, rows), bytes)] in GGUF declaration order."""
        out = []
        for i in range(_lib.cx_model_tensor_count(self._h)):
            name = C.create_string_buffer(128)
            t = C.c_int()
            dims = (C.c_uint64 * 2)()
            nb = C.c_size_t()
            L.check(_lib.cx_model_tensor_info(self._h, i, name, 128, C.byref(t), dims, C.byref(nb)),
                    "tensor_info")
            out.append((name.value.decode(), t.value, (dims[0], dims[1]), nb.value))
        return out

    def tensor(self, idx: int) -> np.ndarray:
        name, t, dims, nb = self.tensores()[idx]
        buf = np.empty(nb, dtype=np.uint8)
        L.check(_lib.cx_model_tensor_copy(self._h, idx, buf.ctypes.data_as(C.c_void_p), nb),
                "tensor_copy")
        if t == L.F32:
            return buf.view(np.float32)
        return buf.reshape(dims[1], -1)

    def tensor_ptr(self, idx: int) -> int:
        """Device address of tensor `idx` (a view owned by the model)."""
        p = _lib.cx_model_tensor_data(self._h, idx)
        if not p:
            raise L.CxError(L.last_error())
        return p

    def nueva_cache(self, capacidad: int) -> "Cache":
        return Cache(self, capacidad)

    def forward(self, tokens, cache: "Cache", logits: bool = True):
        """Modelo::forward: logits (f32[vocab]) of the last token, and its argmax."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        lg = np.empty(self.cfg.vocab, np.float32) if logits else None
        am = C.c_uint32()
        L.check(_lib.cx_forward(self._h, cache._h, t.ctypes.data_as(L._u32p), t.size,
                                lg.ctypes.data_as(L._f32p) if logits else None, C.byref(am)),
                "forward")
        return lg, am.value

    def generar(self, prompt, max_nuevos: int, cache: "Cache", fin: int | None = None,
                tiempos: bool = False, muestreador=None, al_token=None, fines=None):
        """Modelo::generar (src/forward.rs:533-559): greedy, or with a
        ``sampler.Muestreador`` (its seed, temperature and top_p; the draws
        happen on the GPU). Returns the tokens, and if `tiempos` the decode
        time in ms of each step that forwarded a returned token (one per
        token the cache grew by). ``al_token(t) -> bool`` is called with each token
        as it is pushed (False stops at once, src/forward.rs:549-551);
        ``fines`` is a list of stop tokens (MotorPropio stops at the end
        token and the chat's end of turn, src/engine_own.rs:259-261)."""
        if al_token is not None or fines is not None:
            if tiempos:
                raise ValueError("generar: tiempos with al_token/fines is not supported")
            return self._generar_stream(prompt, max_nuevos, cache,
                                        ([] if fin is None else [fin]) + list(fines or []),
                                        muestreador, al_token)
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(max_nuevos, 1), np.uint32)
        n = C.c_size_t()
        ms = np.zeros(max(max_nuevos, 1), np.float32) if tiempos else None
        eos = 0xFFFFFFFF if fin is None else fin
        inicio = cache.largo()
        if muestreador is None:
            rc = _lib.cx_generate(self._h, cache._h, p.ctypes.data_as(L._u32p), p.size,
                                  max_nuevos, eos, out.ctypes.data_as(L._u32p), C.byref(n),
                                  ms.ctypes.data_as(L._f32p) if tiempos else None)
        else:
            # the sampler's generator as it stands; afterwards it is advanced
            # by the draws the reference makes: one per token, one more for
            # the end token, none past the context
            rc = _lib.cx_generate_sampled(self._h, cache._h, p.ctypes.data_as(L._u32p), p.size,
                                          max_nuevos, eos, muestreador.estado,
                                          muestreador.temperatura, muestreador.top_p,
                                          out.ctypes.data_as(L._u32p), C.byref(n),
                                          ms.ctypes.data_as(L._f32p) if tiempos else None)
            if rc == 0 and muestreador.temperatura > 0.0:
                pasos = min(p.size + max_nuevos, self.cfg.contexto - inicio)
                hechos = min(max_nuevos, pasos - p.size + 1)
                muestreador.avanzar(n.value + (1 if n.value < hechos else 0))
            elif rc == L.CX_ENOMEM and muestreador.temperatura > 0.0:
                muestreador.avanzar(n.value)  # one draw per token made
        toks = out[: n.value].copy()
        if tiempos:
            # the steps that forwarded a returned token: the cache's growth
            ms = ms[: max(0, min(cache.largo() - inicio - p.size, n.value))].copy()
        _check_generation(rc, toks, ms)
        return (toks, ms) if tiempos else toks

    def _generar_stream(self, prompt, max_nuevos, cache, fines, muestreador, al_token):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(max_nuevos, 1), np.uint32)
        stops = np.ascontiguousarray(fines, dtype=np.uint32)
        n = C.c_size_t()
        estado = {"error": None, "parado": False}

        def cb(t, _user):
            try:
                sigue = bool(al_token(int(t)))
            except BaseException as e:  # stops generation; raised once the call returns
                estado["error"] = e
                sigue = False
            estado["parado"] = not sigue
            return 1 if sigue else 0

        fn = L.TOKEN_FN(cb) if al_token is not None else L.TOKEN_FN()
        seed, temp, top_p = ((muestreador.estado, muestreador.temperatura, muestreador.top_p)
                             if muestreador is not None else (0, 0.0, 1.0))
        inicio = cache.largo()
        rc = _lib.cx_generate_stream(self._h, cache._h, p.ctypes.data_as(L._u32p), p.size,
                                     max_nuevos, stops.ctypes.data_as(L._u32p), stops.size,
                                     seed, temp, top_p, fn, None, out.ctypes.data_as(L._u32p),
                                     C.byref(n))
        if estado["error"] is not None:
            raise estado["error"]
        _check_generation(rc, out[: n.value].copy())
        if muestreador is not None and temp > 0.0:
            # one draw per pushed token, and one more for a stop token: the
            # loop stopped short of max_nuevos and of the context, not by al_token
            hechos = min(max_nuevos, self.cfg.contexto - inicio - p.size + 1)
            fin = n.value < hechos and not estado["parado"]
            muestreador.avanzar(n.value + (1 if fin else 0))
        return out[: n.value].copy()


def _check_generation(rc, tokens, tiempos=None):
    """Raises for a failed generation; when the cache filled first
    (CX_ENOMEM) the error carries the tokens made until then."""
    if rc == L.CX_ENOMEM:
        raise L.CacheLlena(f"generar: {L.last_error()} (status {rc})", tokens, tiempos)
    L.check(rc, "generar")


class Cache:
    """forward::Cache (src/forward.rs:62-137) with room for `capacidad` tokens."""

    def __init__(self, modelo: Modelo, capacidad: int):
        self.modelo = modelo
        h = C.c_void_p()
        L.check(_lib.cx_cache_new(modelo._h, capacidad, C.byref(h)), "Cache")
        self._h = h
        modelo._caches.add(self)

    def largo(self) -> int:
        return int(_lib.cx_cache_len(self._h))

    def bytes(self) -> int:
        """Cache::bytes (src/forward.rs:130-136): K and V bytes held."""
        return int(_lib.cx_cache_bytes(self._h))

    def prefijo(self, n: int, capacidad: int = 0) -> "Cache":
        """Cache::prefijo (src/forward.rs:117-128): a new cache holding a copy
        of the first min(n, largo) tokens (room for `capacidad`, 0 = this
        cache's)."""
        h = C.c_void_p()
        L.check(_lib.cx_cache_prefix(self._h, n, capacidad, C.byref(h)), "prefijo")
        c = Cache.__new__(Cache)
        c.modelo = self.modelo
        c._h = h
        self.modelo._caches.add(c)
        return c

    def truncar(self, n: int) -> None:
        L.check(_lib.cx_cache_truncate(self._h, n), "truncar")

    def limpiar(self) -> None:
        _lib.cx_cache_clear(self._h)

    def close(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.cx_cache_free(self._h)
        self._h = None

    def __del__(self):
        self.close()
