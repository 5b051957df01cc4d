"""cosxamix_amd — the batch-1 decode token loop of Brashkie/Cosxamix on
MI355X (gfx950): k-quant GEMV, per-token ops and the greedy loop as
hand-written HIP kernels behind a C ABI (include/cosxamix_hip.h).

Submodules:
  _lib     ctypes binding of libcosxamix_hip.so (no fallback when missing)
  kernels  level 1: the row-kernel contract on host arrays
  ops      level 2: operators on device tensors
  forward  level 3: Config / Modelo / Cache
  build    the hipcc recipe
"""
from ._lib import (F32, F16, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q5_0, Q8_0, LIB_PATH,  # noqa: F401
                   TYPE_NAMES)

__all__ = ["F32", "F16", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q5_0", "Q8_0", "LIB_PATH"]
