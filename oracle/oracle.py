"""ctypes view of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this module. It loads ``oracle/liboracle.so`` (the C
restatement of the reference's scalar arithmetic, see ``cx_oracle.h``) and,
when present, ``oracle/_ref/libcxref.so`` (the reference's own native x86
kernels compiled from ``/root/reference/kernels`` by ``oracle/Makefile``).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# CX_ORACLE_LIB names another build of cx_oracle.c (tests/test_oracle_mutants.py
# loads deliberately broken copies through it to show the pinning tests fail)
LIB_PATH = os.environ.get("CX_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libcxref.so")

F32, F16, Q5_0, Q8_0 = 0, 1, 6, 8
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 10, 11, 12, 13, 14
BYTES_PER_BLOCK = {F32: 4, F16: 2, Q5_0: 22, Q8_0: 34, Q2_K: 84, Q3_K: 110,
                   Q4_K: 144, Q5_K: 176, Q6_K: 210}
VALUES_PER_BLOCK = {F32: 1, F16: 1, Q5_0: 32, Q8_0: 32, Q2_K: 256, Q3_K: 256,
                    Q4_K: 256, Q5_K: 256, Q6_K: 256}
SUB = {Q8_0: 32, Q5_0: 32, Q4_K: 32, Q5_K: 32, Q2_K: 16, Q3_K: 16, Q6_K: 16}
NAMES = {Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}

_u8p = C.POINTER(C.c_uint8)
_i8p = C.POINTER(C.c_int8)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_u32p = C.POINTER(C.c_uint32)
ROW_KERNEL = C.CFUNCTYPE(C.c_float, _u8p, _i8p, _f32p, _f32p, C.c_size_t)


def row_bytes(t: int, k: int) -> int:
    return k // VALUES_PER_BLOCK[t] * BYTES_PER_BLOCK[t]


def _p(a: np.ndarray, typ):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data_as(typ)


class OrcConfig(C.Structure):
    _fields_ = [("layers", C.c_size_t), ("dim", C.c_size_t), ("heads", C.c_size_t),
                ("kv_heads", C.c_size_t), ("ffn", C.c_size_t), ("vocab", C.c_size_t),
                ("ctx", C.c_size_t), ("eps", C.c_float), ("rope_base", C.c_float)]


class OrcLayer(C.Structure):
    _fields_ = [(n, _f32p) for n in ("attn_norm", "q_bias", "k_bias", "v_bias", "ffn_norm")] + \
               [(n, _u8p) for n in ("q", "k", "v", "o", "gate", "up", "down")] + \
               [(n, C.c_int) for n in ("t_q", "t_k", "t_v", "t_o", "t_gate", "t_up", "t_down")]


class OrcModel(C.Structure):
    _fields_ = [("cfg", OrcConfig), ("embd", _f32p), ("out_norm", _f32p), ("out", _u8p),
                ("t_out", C.c_int), ("layers", C.POINTER(OrcLayer)), ("cos_t", _f32p),
                ("sin_t", _f32p), ("kern_override", C.c_void_p), ("threads", C.c_int),
                ("attn_chunk", C.c_int)]


class OrcCache(C.Structure):
    _fields_ = [("len", C.c_size_t), ("cap", C.c_size_t),
                ("k", C.POINTER(_f32p)), ("v", C.POINTER(_f32p))]


def _load():
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"oracle library missing: build it with `make -C {HERE}`")
    lib = C.CDLL(LIB_PATH)
    sig = {
        "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
        "orc_dequantize": (C.c_int, [C.c_int, _u8p, _f32p, C.c_size_t]),
        "orc_unpack_i8": (C.c_int, [C.c_int, _u8p, C.c_size_t, _i8p, _f32p, _f32p]),
        "orc_quantize_blocks": (C.c_long, [C.c_int, _f32p, C.c_size_t, _u8p]),
        "orc_kquant_search": (C.c_int, [C.c_int, _f32p, _f32p, _f32p, _i32p]),
        "orc_seed_of": (C.c_uint64, [C.c_uint64, C.c_char_p, C.c_uint64]),
        "orc_daiss_row": (None, [C.c_uint64, C.c_char_p, C.c_uint64, C.c_float, _f32p, C.c_size_t]),
        "orc_daiss_matrix": (C.c_int, [C.c_uint64, C.c_char_p, C.c_size_t, C.c_size_t, C.c_float,
                                       C.c_int, _u8p, C.c_int]),
        "orc_quantize_act": (None, [_f32p, C.c_size_t, C.c_int, _i8p, _f32p, _f32p]),
        "orc_subsums": (C.c_int, [C.c_int, _u8p, _i8p, C.c_size_t, _i32p]),
        "orc_dot_f32": (C.c_float, [_f32p, _f32p, C.c_size_t]),
        "orc_rmsnorm": (None, [_f32p, _f32p, _f32p, C.c_size_t, C.c_float]),
        "orc_silu": (None, [_f32p, _f32p, C.c_size_t]),
        "orc_argmax": (C.c_uint32, [_f32p, C.c_size_t]),
        "orc_rope_tables": (None, [C.c_size_t, C.c_float, C.c_size_t, _f32p, _f32p]),
        "orc_rope": (C.c_int, [_f32p, C.c_size_t, C.c_size_t, C.c_size_t, _f32p, _f32p,
                               C.c_size_t, C.c_size_t]),
        "orc_softmax": (C.c_int, [_f32p, C.c_size_t, C.c_size_t]),
        "orc_attention": (C.c_int, [_f32p, _f32p, _f32p] + [C.c_size_t] * 5 + [_f32p]),
        "orc_matmul_fused": (C.c_int, [C.c_size_t] * 3 + [_f32p, _u8p, C.c_int, _f32p,
                                                          C.c_void_p, C.c_int, C.c_int]),
        "orc_matmul_direct": (C.c_int, [C.c_size_t] * 3 + [_f32p, _u8p, C.c_int, _f32p, C.c_int]),
        "orc_dot_i8_scaled": (C.c_float, [_i8p, _i8p, _f32p, _f32p, C.c_size_t, C.c_int]),
        "orc_matmul_multi_1row": (C.c_int, [_f32p, C.c_size_t, C.c_size_t, C.POINTER(_u8p),
                                            C.POINTER(C.c_int), C.POINTER(C.c_size_t),
                                            C.POINTER(_f32p), C.c_int]),
        "orc_model_init": (C.c_int, [C.POINTER(OrcModel), C.POINTER(OrcConfig), _f32p, _f32p,
                                     _u8p, C.c_int, C.POINTER(OrcLayer), C.c_int]),
        "orc_model_release": (None, [C.POINTER(OrcModel)]),
        "orc_cache_init": (C.c_int, [C.POINTER(OrcCache), C.POINTER(OrcConfig), C.c_size_t]),
        "orc_cache_release": (None, [C.POINTER(OrcCache), C.POINTER(OrcConfig)]),
        "orc_forward": (C.c_int, [C.POINTER(OrcModel), _u32p, C.c_size_t, C.POINTER(OrcCache),
                                  _f32p]),
        "orc_generate": (C.c_int, [C.POINTER(OrcModel), _u32p, C.c_size_t, C.c_size_t,
                                   C.POINTER(OrcCache), _u32p, C.POINTER(C.c_size_t)]),
        "orc_sampler_init": (None, [C.c_void_p, C.c_uint64, C.c_float, C.c_float]),
        "orc_sample": (C.c_uint32, [C.c_void_p, _f32p, C.c_size_t]),
        "orc_generate_sampled": (C.c_int, [C.POINTER(OrcModel), _u32p, C.c_size_t, C.c_size_t,
                                           C.c_void_p, C.c_uint32, C.POINTER(OrcCache), _u32p,
                                           C.POINTER(C.c_size_t)]),
        "orc_last_error": (C.c_char_p, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    for t in (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K):
        fn = getattr(lib, f"orc_dot_{NAMES[t][:2].lower()}k")
        fn.restype, fn.argtypes = C.c_float, [_u8p, _i8p, _f32p, _f32p, C.c_size_t]
    return lib


lib = _load()


def err() -> str:
    return lib.orc_last_error().decode()


# ------------------------------------------------------------------ formats
def f16_to_f32(h: int) -> float:
    return lib.orc_f16_to_f32(h)


def f32_to_f16(x: float) -> int:
    return lib.orc_f32_to_f16(x)


def quantize_blocks(t: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(row_bytes(t, x.size), dtype=np.uint8)
    n = lib.orc_quantize_blocks(t, _p(x, _f32p), x.size, _p(out, _u8p))
    if n < 0:
        raise ValueError(err())
    return out


def kquant_search(t: int, x: np.ndarray):
    """The per-sub-block search of one 256-value block as the quantizer runs
    it: (scales, -mins, codes[256]) before the scales and mins are
    themselves quantized (src/quant_kquants.rs:29-157, 236-257, 301-313)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    assert x.size == 256
    sc, mn = np.zeros(16, np.float32), np.zeros(16, np.float32)
    codes = np.zeros(256, np.int32)
    n = lib.orc_kquant_search(t, _p(x, _f32p), _p(sc, _f32p), _p(mn, _f32p), _p(codes, _i32p))
    if n < 0:
        raise ValueError(err())
    return sc[:n], mn[:n], codes


def dequantize(t: int, b: np.ndarray, n: int) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint8)
    y = np.zeros(n, dtype=np.float32)
    if lib.orc_dequantize(t, _p(b, _u8p), _p(y, _f32p), n):
        raise ValueError(err())
    return y


def unpack_i8(t: int, b: np.ndarray, n: int):
    b = np.ascontiguousarray(b, dtype=np.uint8)
    q = np.zeros(n, dtype=np.int8)
    ns = n // SUB[t]
    e = np.zeros(ns, dtype=np.float32)
    o = np.zeros(ns, dtype=np.float32)
    if lib.orc_unpack_i8(t, _p(b, _u8p), n, _p(q, _i8p), _p(e, _f32p), _p(o, _f32p)) < 0:
        raise ValueError(err())
    return q, e, o


def seed_of(model: int, name: str, row: int) -> int:
    return lib.orc_seed_of(model, name.encode(), row)


def daiss_row(seed: int, name: str, row: int, sigma: float, width: int) -> np.ndarray:
    out = np.zeros(width, dtype=np.float32)
    lib.orc_daiss_row(seed, name.encode(), row, sigma, _p(out, _f32p), width)
    return out


def daiss_matrix(seed: int, name: str, rows: int, width: int, sigma: float, t: int) -> np.ndarray:
    """`rows` rows of `width` N(0, sigma) values from per-row seeds, quantized
    to type `t` row by row (src/daiss.rs:539-571)."""
    out = np.zeros((rows, row_bytes(t, width)), dtype=np.uint8)
    if lib.orc_daiss_matrix(seed, name.encode(), rows, width, sigma, t, _p(out, _u8p),
                            os.cpu_count() or 1):
        raise ValueError(err())
    return out


def quantize_act(x: np.ndarray, sub: int):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    k = x.size
    ns = (k + sub - 1) // sub
    q = np.zeros(k, dtype=np.int8)
    e = np.zeros(ns, dtype=np.float32)
    s = np.zeros(ns, dtype=np.float32)
    lib.orc_quantize_act(_p(x, _f32p), k, sub, _p(q, _i8p), _p(e, _f32p), _p(s, _f32p))
    return q, e, s


def dot_row(t: int, blocks: np.ndarray, xq, xe, xs) -> float:
    fn = getattr(lib, f"orc_dot_{NAMES[t][:2].lower()}k")
    return fn(_p(np.ascontiguousarray(blocks, np.uint8), _u8p), _p(xq, _i8p), _p(xe, _f32p),
              _p(xs, _f32p), xq.size // 256)


def subsums(t: int, blocks: np.ndarray, xq: np.ndarray) -> np.ndarray:
    nb = xq.size // 256
    out = np.zeros(nb * (256 // SUB[t]), dtype=np.int32)
    if lib.orc_subsums(t, _p(np.ascontiguousarray(blocks, np.uint8), _u8p), _p(xq, _i8p), nb,
                       _p(out, _i32p)):
        raise ValueError(err())
    return out


def matmul_fused(t: int, lhs: np.ndarray, w: np.ndarray, n: int, threads: int = 1,
                 kernel=None, prefetch: int = 2) -> np.ndarray:
    """dst[m, n] = lhs[m, k] . W^T with the fused per-row path (ops.rs:435-522).
    `kernel` is a ctypes ROW_KERNEL (e.g. a reference _ref kernel) or None for
    the scalar restatement."""
    lhs = np.ascontiguousarray(lhs, dtype=np.float32)
    m, k = lhs.shape if lhs.ndim == 2 else (1, lhs.size)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    dst = np.zeros((m, n), dtype=np.float32)
    kp = C.cast(kernel, C.c_void_p) if kernel is not None else None
    if lib.orc_matmul_fused(m, k, n, _p(lhs, _f32p), _p(w, _u8p), t, _p(dst, _f32p), kp,
                            threads, prefetch):
        raise ValueError(err())
    return dst


def matmul_direct(t: int, lhs: np.ndarray, w: np.ndarray, n: int, threads: int = 1) -> np.ndarray:
    """dst[m, n] = lhs[m, k] . W^T by the buffer path (ops::matmul_i8_directo,
    src/ops.rs:310-414): Q8_0, Q5_0 and the k-quants."""
    lhs = np.ascontiguousarray(lhs, dtype=np.float32)
    m, k = lhs.shape if lhs.ndim == 2 else (1, lhs.size)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    dst = np.zeros((m, n), dtype=np.float32)
    if lib.orc_matmul_direct(m, k, n, _p(lhs, _f32p), _p(w, _u8p), t, _p(dst, _f32p), threads):
        raise ValueError(err())
    return dst


def matmul_multi_1row(x: np.ndarray, mats, threads: int = 1):
    """mats: list of (bytes ndarray, type, n). Returns list of outputs."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    cnt = len(mats)
    outs = [np.zeros(n, dtype=np.float32) for (_, _, n) in mats]
    ws = (_u8p * cnt)(*[_p(np.ascontiguousarray(w, np.uint8), _u8p) for (w, _, _) in mats])
    ts = (C.c_int * cnt)(*[t for (_, t, _) in mats])
    ns = (C.c_size_t * cnt)(*[n for (_, _, n) in mats])
    ds = (_f32p * cnt)(*[_p(o, _f32p) for o in outs])
    if lib.orc_matmul_multi_1row(_p(x, _f32p), x.size, cnt, ws, ts, ns, ds, threads):
        raise ValueError(err())
    return outs


# ------------------------------------------------------------ per-token ops
def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    lib.orc_rmsnorm(_p(out, _f32p), _p(x, _f32p), _p(w, _f32p), x.size, eps)
    return out


def silu(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    lib.orc_silu(_p(out, _f32p), _p(x, _f32p), x.size)
    return out


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(lib.orc_argmax(_p(v, _f32p), v.size))


def rope_tables(head_dim: int, base: float, ctx: int):
    c = np.zeros(ctx * (head_dim // 2), np.float32)
    s = np.zeros_like(c)
    lib.orc_rope_tables(head_dim, base, ctx, _p(c, _f32p), _p(s, _f32p))
    return c, s


def rope(x: np.ndarray, tokens: int, heads: int, head_dim: int, cos_t, sin_t, pos: int):
    x = np.array(x, dtype=np.float32, copy=True)
    ctx = cos_t.size // (head_dim // 2)
    if lib.orc_rope(_p(x, _f32p), tokens, heads, head_dim, _p(cos_t, _f32p), _p(sin_t, _f32p),
                    ctx, pos):
        raise ValueError(err())
    return x


def softmax(x: np.ndarray, width: int) -> np.ndarray:
    x = np.array(x, dtype=np.float32, copy=True)
    if lib.orc_softmax(_p(x, _f32p), x.size, width):
        raise ValueError(err())
    return x


def attention(q, k, v, tokens, total, heads, kv_heads, head_dim) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    out = np.zeros(tokens * heads * head_dim, np.float32)
    if lib.orc_attention(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), tokens, total, heads,
                         kv_heads, head_dim, _p(out, _f32p)):
        raise ValueError(err())
    return out


# --------------------------------------------------------------- the model
class Model:
    """A Qwen2 model held in host memory for the oracle forward
    (src/forward.rs:375-505). `tensors` maps GGUF-style names to numpy arrays
    (F32 vectors/embedding as float32, quantized matrices as uint8 rows) and
    `types` maps names to GGML type ids."""

    def __init__(self, cfg: dict, tensors: dict, types: dict, threads: int = 8, ref_q4k=None):
        self._keep = []
        c = OrcConfig(cfg["layers"], cfg["dim"], cfg["heads"], cfg["kv_heads"], cfg["ffn"],
                      cfg["vocab"], cfg["ctx"], cfg["eps"], cfg["rope_base"])
        self.cfg = cfg
        self.c_cfg = c
        arr = (OrcLayer * cfg["layers"])()

        def fp(name):
            a = np.ascontiguousarray(tensors[name], np.float32)
            self._keep.append(a)
            return _p(a, _f32p)

        def bp(name):
            a = tensors[name]
            # F32/F16 matrices travel as their bytes (ops::matmul's path)
            a = (np.ascontiguousarray(a).view(np.uint8) if a.dtype in (np.float32, np.float16)
                 else np.ascontiguousarray(a, np.uint8))
            self._keep.append(a)
            return _p(a, _u8p)

        for i in range(cfg["layers"]):
            p = f"blk.{i}."
            L = arr[i]
            L.attn_norm, L.ffn_norm = fp(p + "attn_norm.weight"), fp(p + "ffn_norm.weight")
            L.q_bias, L.k_bias, L.v_bias = (fp(p + "attn_q.bias"), fp(p + "attn_k.bias"),
                                            fp(p + "attn_v.bias"))
            for fld, nm in (("q", "attn_q"), ("k", "attn_k"), ("v", "attn_v"), ("o", "attn_output"),
                            ("gate", "ffn_gate"), ("up", "ffn_up"), ("down", "ffn_down")):
                setattr(L, fld, bp(p + nm + ".weight"))
                setattr(L, "t_" + fld, types[p + nm + ".weight"])
        self.layers = arr
        self.m = OrcModel()
        if lib.orc_model_init(C.byref(self.m), C.byref(c), fp("token_embd.weight"),
                              fp("output_norm.weight"), bp("output.weight"),
                              types["output.weight"], arr, threads):
            raise RuntimeError(err())
        if ref_q4k is not None:
            self.m.kern_override = C.cast(ref_q4k, C.c_void_p)

    def __del__(self):
        try:
            lib.orc_model_release(C.byref(self.m))
        except Exception:
            pass

    def set_q4k_kernel(self, ref_q4k=None):
        """The Q4_K row kernel of later forwards: a reference _ref kernel, or
        None for the oracle's own (scalar order)."""
        self.m.kern_override = C.cast(ref_q4k, C.c_void_p) if ref_q4k is not None else None

    def set_threads(self, n: int):
        self.m.threads = max(1, int(n))

    def set_attention_chunk(self, n: int):
        """0: the reference's attention order; n > 0: a test hook, the
        softmax and P.V sums split over chunks of n positions (the order of
        a split-K kernel, orc_attention_split)."""
        self.m.attn_chunk = max(0, int(n))

    def new_cache(self, cap: int) -> "Cache":
        return Cache(self, cap)

    def forward(self, toks, cache: "Cache") -> np.ndarray:
        t = np.ascontiguousarray(toks, np.uint32)
        lg = np.zeros(self.cfg["vocab"], np.float32)
        if lib.orc_forward(C.byref(self.m), _p(t, _u32p), t.size, C.byref(cache.c), _p(lg, _f32p)):
            raise RuntimeError(err())
        return lg

    def generate(self, prompt, max_new: int, cache: "Cache"):
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(max_new, np.uint32)
        n = C.c_size_t(0)
        if lib.orc_generate(C.byref(self.m), _p(p, _u32p), p.size, max_new, C.byref(cache.c),
                            _p(out, _u32p), C.byref(n)):
            raise RuntimeError(err())
        return out[: n.value]


class Cache:
    def __init__(self, model: Model, cap: int):
        self.model = model
        self.c = OrcCache()
        if lib.orc_cache_init(C.byref(self.c), C.byref(model.c_cfg), cap):
            raise MemoryError("oracle cache")

    @property
    def len(self) -> int:
        return self.c.len

    def __del__(self):
        try:
            lib.orc_cache_release(C.byref(self.c), C.byref(self.model.c_cfg))
        except Exception:
            pass


# ------------------------------------------- the reference's own kernels
def load_ref():
    """The reference's compiled native kernels (oracle/_ref), or None when
    they were not built (the GPU box has no /root/reference; build() builds
    them here and the .so travels with the tree)."""
    if not os.path.exists(REF_PATH):
        return None
    r = C.CDLL(REF_PATH)
    for name in ("cosxamix_q2k_c", "cosxamix_q2k_asm", "cosxamix_q3k_c", "cosxamix_q3k_completo",
                 "cosxamix_q5k_c", "cosxamix_q5k_asm", "cxref_q4k_row"):
        fn = getattr(r, name)
        fn.restype, fn.argtypes = C.c_float, [_u8p, _i8p, _f32p, _f32p, C.c_size_t]
    return r


def ref_kernels(r):
    """type -> list of (name, ctypes function) of the reference's native row
    kernels available for that type."""
    return {
        Q2_K: [("cosxamix_q2k_c", r.cosxamix_q2k_c), ("cosxamix_q2k_asm", r.cosxamix_q2k_asm)],
        Q3_K: [("cosxamix_q3k_c", r.cosxamix_q3k_c),
               ("cosxamix_q3k_completo", r.cosxamix_q3k_completo)],
        Q4_K: [("cosxamix_q4k_completo", r.cxref_q4k_row)],
        Q5_K: [("cosxamix_q5k_c", r.cosxamix_q5k_c), ("cosxamix_q5k_asm", r.cosxamix_q5k_asm)],
    }


def ref_row_kernel(r, t: int):
    """A ctypes ROW_KERNEL pointer for the fastest reference kernel of `t`."""
    name = {Q2_K: "cosxamix_q2k_asm", Q3_K: "cosxamix_q3k_completo", Q4_K: "cxref_q4k_row",
            Q5_K: "cosxamix_q5k_asm"}[t]
    return C.cast(getattr(r, name), ROW_KERNEL)


class OrcSampler(C.Structure):
    _fields_ = [("azar", C.c_uint64), ("temp", C.c_float), ("top_p", C.c_float)]


class Sampler:
    """sampler::Muestreador (src/sampler.rs:27-152), restated in C."""

    def __init__(self, seed: int, temp: float, top_p: float):
        self.s = OrcSampler()
        lib.orc_sampler_init(C.byref(self.s), seed & (2**64 - 1), temp, top_p)

    @property
    def state(self) -> int:
        return self.s.azar

    def choose(self, logits) -> int:
        x = np.ascontiguousarray(logits, np.float32)
        return int(lib.orc_sample(C.byref(self.s), _p(x, _f32p), x.size))


def generate_sampled(model: "Model", prompt, max_new: int, sampler: Sampler, cache: "Cache",
                     eos: int = 0xFFFFFFFF):
    p = np.ascontiguousarray(prompt, np.uint32)
    out = np.zeros(max(max_new, 1), np.uint32)
    n = C.c_size_t(0)
    if lib.orc_generate_sampled(C.byref(model.m), _p(p, _u32p), p.size, max_new,
                                C.byref(sampler.s), eos, C.byref(cache.c), _p(out, _u32p),
                                C.byref(n)):
        raise RuntimeError(err())
    return out[: n.value]
