// cx_internal.h — launch-level interfaces shared between translation units.
#pragma once

#include "cx_common.h"

// One matrix of a (possibly multi-matrix) GEMV launch. All segments of one
// launch share the activation, the row width k and the weight type.
struct cx_seg {
  const uint8_t* w;     // rows x row_bytes, GGUF raw
  float* y;             // rows
  const float* bias;    // rows or nullptr (Qwen2 q/k/v bias, src/forward.rs:360-366)
  uint32_t rows;
};

// Where the GEMV's activation comes from. Every workgroup builds the same
// i8 activation (xq, xe, xs) in LDS from it, with the same arithmetic as
// cx_quantize_act, so the result is bit-identical across workgroups.
enum cx_act_src {
  CX_ACT_QUANTIZED = 0,  // xq/xe/xs given in device memory
  CX_ACT_NORM = 1,       // rmsnorm(x, w, eps) then quantize   (kernels/mod.rs:511 + ops.rs:178)
  CX_ACT_PLAIN = 2,      // quantize x                           (ops.rs:178)
  CX_ACT_SWIGLU = 3,     // quantize silu(x) * x2               (forward.rs:483-487)
};

struct cx_act {
  int src;
  const int8_t* xq;
  const float* xe;
  const float* xs;
  const float* x;
  const float* x2;
  const float* norm_w;
  float eps;
};

enum cx_epi { CX_EPI_STORE = 0, CX_EPI_ACCUM = 1 };

// GEMV over `nseg` segments: seg[i].y[r] (=|+=) row r of seg[i].w . act.
int cx_launch_gemv(int type, const cx_seg* segs, int nseg, uint32_t k,
                   const cx_act& act, int epi, int32_t* dbg, hipStream_t s);

// Activation quantization for `rows` rows (bit-exact, ops.rs:178-198).
int cx_launch_quantize(const float* x, size_t rows, size_t k, int sub,
                       int8_t* xq, float* xe, float* xs, hipStream_t s);
int cx_launch_rmsnorm(float* out, const float* in, const float* w,
                      size_t rows, size_t n, float eps, hipStream_t s);
