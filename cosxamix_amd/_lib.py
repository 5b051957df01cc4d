"""ctypes binding of libcosxamix_hip.so (the C ABI in include/cosxamix_hip.h).

The library is built in-tree by ``cosxamix_amd/build.py`` (or
``__graft_entry__.build()``). There is no fallback: if the library is missing
or cannot be loaded, importing the package's compute modules raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libcosxamix_hip.so")

# GGML type ids (src/gguf.rs:39-54)
F32, F16, Q5_0, Q8_0 = 0, 1, 6, 8
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 10, 11, 12, 13, 14
TYPE_NAMES = {F32: "F32", F16: "F16", Q5_0: "Q5_0", Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K",
              Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}

_u8p = C.POINTER(C.c_uint8)
_i8p = C.POINTER(C.c_int8)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_u32p = C.POINTER(C.c_uint32)
_vp = C.c_void_p
_sz = C.c_size_t


class CxConfig(C.Structure):
    """forward::Config (src/forward.rs:36-55)."""
    _fields_ = [("layers", C.c_uint32), ("dim", C.c_uint32), ("heads", C.c_uint32),
                ("kv_heads", C.c_uint32), ("ffn", C.c_uint32), ("vocab", C.c_uint32),
                ("ctx", C.c_uint32), ("eps", C.c_float), ("rope_base", C.c_float)]


class CxGgufTensor(C.Structure):
    """InfoTensor (src/gguf.rs:172-194) as cx_gguf_tensor."""
    _fields_ = [("name", C.c_char * 128), ("type", C.c_int), ("n_dims", C.c_uint32),
                ("dims", C.c_uint64 * 4), ("offset", C.c_uint64), ("elements", C.c_uint64),
                ("bytes", C.c_uint64)]


# cx_token_fn: int (*)(uint32_t token, void *user)
TOKEN_FN = C.CFUNCTYPE(C.c_int, C.c_uint32, C.c_void_p)

# name -> (restype, argtypes); every symbol include/cosxamix_hip.h declares
SIGNATURES = {
    "cx_last_error": (C.c_char_p, []),
    "cx_init": (C.c_int, [C.c_int]),
    "cx_row_bytes": (_sz, [C.c_int, _sz]),
    "cx_sub_block": (C.c_int, [C.c_int]),
    "cx_dot_q2k_i8": (C.c_float, [_u8p, _i8p, _f32p, _f32p, _sz]),
    "cx_dot_q3k_i8": (C.c_float, [_u8p, _i8p, _f32p, _f32p, _sz]),
    "cx_dot_q4k_i8": (C.c_float, [_u8p, _i8p, _f32p, _f32p, _sz]),
    "cx_dot_q5k_i8": (C.c_float, [_u8p, _i8p, _f32p, _f32p, _sz]),
    "cx_dot_q6k_i8": (C.c_float, [_u8p, _i8p, _f32p, _f32p, _sz]),
    "cx_quantize_act": (C.c_int, [_vp, _sz, _sz, C.c_int, _vp, _vp, _vp, _vp]),
    "cx_gemv": (C.c_int, [C.c_int, _vp, _sz, _sz, _vp, _vp, _vp, _vp, _vp]),
    "cx_gemv_subsums": (C.c_int, [C.c_int, _vp, _sz, _sz, _vp, _vp, _vp, _vp, _vp]),
    "cx_quantize_blocks": (C.c_int, [C.c_int, _vp, _sz, _vp, _vp]),
    "cx_dequantize": (C.c_int, [C.c_int, _vp, _sz, _vp, _vp]),
    "cx_dequantize_rows": (C.c_int, [C.c_int, _vp, _sz, _sz, C.POINTER(_sz), _sz, _vp, _vp]),
    "cx_unpack_i8": (C.c_int, [C.c_int, _vp, _sz, _vp, _vp, _vp, C.POINTER(C.c_int), _vp]),
    "cx_matmul_auto": (C.c_int, [_sz, _sz, _sz, _vp, _vp, C.c_int, _vp, _vp]),
    "cx_matmul_auto_noalloc": (C.c_int, [_sz, _sz, _sz, _vp, _vp, C.c_int, _vp, _vp]),
    "cx_matmul_multi_1row": (C.c_int, [_vp, _sz, _sz, C.POINTER(_vp), C.POINTER(C.c_int),
                                       C.POINTER(_sz), C.POINTER(_vp), _vp]),
    "cx_rmsnorm": (C.c_int, [_vp, _vp, _vp, _sz, _sz, C.c_float, _vp]),
    "cx_silu": (C.c_int, [_vp, _vp, _sz, _vp]),
    "cx_rope_tables": (C.c_int, [_sz, C.c_float, _sz, _f32p, _f32p]),
    "cx_rope": (C.c_int, [_vp, _sz, _sz, _sz, _vp, _vp, _sz, _sz, _vp]),
    "cx_softmax": (C.c_int, [_vp, _sz, _sz, _vp]),
    "cx_attention": (C.c_int, [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp]),
    "cx_attention_decode": (C.c_int, [_vp, _vp, _vp, _sz, _sz, _sz, _sz, C.c_int, _vp, _vp]),
    "cx_argmax": (C.c_int, [_vp, _sz, _vp, _vp]),
    "cx_stream_read": (C.c_int, [_vp, _sz, _vp, _vp]),
    "cx_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(_vp)]),
    "cx_gguf_free": (None, [_vp]),
    "cx_gguf_header": (C.c_int, [_vp, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
                                 C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                 C.POINTER(C.c_uint64)]),
    "cx_gguf_meta_int": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_uint64)]),
    "cx_gguf_meta_float": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_double)]),
    "cx_gguf_meta_str": (C.c_int, [_vp, C.c_char_p, C.c_long, C.c_char_p, _sz, C.POINTER(_sz)]),
    "cx_gguf_meta_type": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_uint32),
                                    C.POINTER(C.c_uint64)]),
    "cx_gguf_find": (C.c_int, [_vp, C.c_char_p]),
    "cx_gguf_tensor_info": (C.c_int, [_vp, C.c_int, C.POINTER(CxGgufTensor)]),
    "cx_gguf_tensor_read": (C.c_int, [_vp, C.POINTER(CxGgufTensor), _vp, _sz]),
    "cx_model_create_daiss": (C.c_int, [C.POINTER(CxConfig), C.c_int, C.c_int, C.c_int,
                                        C.c_uint64, C.POINTER(_vp)]),
    "cx_model_open": (C.c_int, [C.c_char_p, C.POINTER(_vp)]),
    "cx_model_save_gguf": (C.c_int, [_vp, C.c_char_p]),
    "cx_model_free": (None, [_vp]),
    "cx_model_config": (C.c_int, [_vp, C.POINTER(CxConfig)]),
    "cx_model_tensor_count": (C.c_int, [_vp]),
    "cx_model_tensor_info": (C.c_int, [_vp, C.c_int, C.c_char_p, _sz, C.POINTER(C.c_int),
                                       C.POINTER(C.c_uint64), C.POINTER(_sz)]),
    "cx_model_tensor_copy": (C.c_int, [_vp, C.c_int, _vp, _sz]),
    "cx_model_tensor_data": (_vp, [_vp, C.c_int]),
    "cx_model_weight_bytes": (_sz, [_vp]),
    "cx_cache_new": (C.c_int, [_vp, _sz, C.POINTER(_vp)]),
    "cx_cache_len": (_sz, [_vp]),
    "cx_cache_truncate": (C.c_int, [_vp, _sz]),
    "cx_cache_clear": (None, [_vp]),
    "cx_cache_free": (None, [_vp]),
    "cx_cache_bytes": (_sz, [_vp]),
    "cx_cache_prefix": (C.c_int, [_vp, _sz, _sz, C.POINTER(_vp)]),
    "cx_forward": (C.c_int, [_vp, _vp, _u32p, _sz, _f32p, _u32p]),
    "cx_generate": (C.c_int, [_vp, _vp, _u32p, _sz, _sz, C.c_uint32, _u32p, C.POINTER(_sz),
                              _f32p]),
    "cx_generate_sampled": (C.c_int, [_vp, _vp, _u32p, _sz, _sz, C.c_uint32, C.c_uint64, C.c_float,
                                      C.c_float, _u32p, C.POINTER(_sz), _f32p]),
    "cx_generate_stream": (C.c_int, [_vp, _vp, _u32p, _sz, _sz, _u32p, _sz, C.c_uint64, C.c_float,
                                     C.c_float, TOKEN_FN, _vp, _u32p, C.POINTER(_sz)]),
    "cx_sample": (C.c_int, [_vp, _sz, C.c_float, C.c_float, C.POINTER(C.c_uint64),
                            C.POINTER(C.c_uint32), _vp]),
}


CX_OK, CX_EINVAL, CX_EHIP, CX_ENOMEM, CX_ENOTSUP = 0, -1, -2, -3, -4


class CxError(RuntimeError):
    pass


class CacheLlena(CxError):
    """Generation stopped because the cache was full before it ended
    (CX_ENOMEM). ``tokens`` holds the tokens made until then, as the C ABI
    returns them in out/n_out, and ``tiempos`` their step times when they
    were asked for."""

    def __init__(self, msg, tokens, tiempos=None):
        super().__init__(msg)
        self.tokens = tokens
        self.tiempos = tiempos


_lib = None


def load():
    """Loads the library once; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python cosxamix_amd/build.py` "
                          "or __graft_entry__.build(); there is no CPU fallback")
    # One process can hold only one ROCm runtime instance. PyTorch's wheel
    # bundles its own libamdhip64 (SONAME libamdhip64.so.7, the same as
    # /opt/rocm's); loading torch first makes this library bind to that copy,
    # so torch tensors, streams and graphs share the runtime with our kernels.
    # Loaded the other way round, torch would bring a second copy that can no
    # longer acquire the GPU.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    _lib = lib
    return lib


def last_error() -> str:
    return load().cx_last_error().decode(errors="replace")


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        raise CxError(f"{what}: {last_error()} (status {rc})")
