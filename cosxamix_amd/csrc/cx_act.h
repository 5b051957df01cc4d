// cx_act.h — device arithmetic for the activation side of the GEMV.
//
// cx_quant_lane() is ops::cuantizar_i8_en (src/ops.rs:178-198) plus the
// per-sub-block integer sum (src/ops.rs:472-483), with one value per lane and
// one sub-block per group of SUB consecutive lanes:
//   amax = max|x| (f32::max ignores NaN -> fmaxf)
//   xe   = amax / 127        (IEEE division, correctly rounded)
//   inv  = 127 / amax        (0 when amax == 0)
//   xq   = round(x * inv) as i32 as i8   (half away from zero; saturating)
//   xs   = sum of xq, as f32 (exact)
// The maximum and the integer sum do not depend on the order in which they
// are formed, so the lane-parallel form is bit-identical to the reference's
// sequential loop. Nothing here may be contracted into an FMA; the whole
// library is built with -ffp-contract=off.
#pragma once

#include "cx_common.h"

// Each lane holds 8 consecutive values v[0..8) at position i (i % 8 == 0);
// the SUB/8 lanes of one sub-block are consecutive lanes of one quad and
// must call this together. cx_quant8_vals gives the lane's 8 quantized bytes
// (lo, hi) and the sub-block's xe (d) and integer sum (s); cx_quant8 writes
// the 8 bytes of xq and, from the sub-block's first lane, its xe and xs.
template <int SUB>
__device__ inline void cx_quant8_vals(const float (&v)[8], uint32_t& lo, uint32_t& hi, float& d,
                                      int32_t& s) {
  static_assert(SUB == 16 || SUB == 32, "sub-blocks of 16 or 32");
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[j]));
  amax = fmaxf(amax, cx_xor1f(amax));
  if (SUB == 32) amax = fmaxf(amax, cx_xor2f(amax));
  float inv = 0.0f;
  d = 0.0f;
  if (amax > 0.0f) {
    d = amax / 127.0f;
    inv = 127.0f / amax;
  }
  s = 0;
  lo = 0;
  hi = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int8_t q = cx_rust_i8(roundf(v[j] * inv));
    s += q;
    if (j < 4)
      lo |= (uint32_t)(uint8_t)q << (8 * j);
    else
      hi |= (uint32_t)(uint8_t)q << (8 * (j - 4));
  }
  s += cx_xor1(s);
  if (SUB == 32) s += cx_xor2(s);
}

template <int SUB>
__device__ inline void cx_quant8(const float (&v)[8], size_t i, int8_t* xq, float* xe,
                                 float* xs) {
  uint32_t lo, hi;
  float d;
  int32_t s;
  cx_quant8_vals<SUB>(v, lo, hi, d, s);
  *reinterpret_cast<uint2*>(xq + i) = make_uint2(lo, hi);
  if ((i & (SUB - 1)) == 0) {
    xe[i / SUB] = d;
    xs[i / SUB] = (float)s;
  }
}

__device__ inline void cx_load8(const float* p, float (&v)[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

#include "cx_expf.h"

// kernels::silu (src/kernels/scalar.rs:63-67) with the reference's exp
// (glibc expf, reproduced bit for bit by cx_expf): SiLU feeds an i8
// quantization whose rounding a one-ulp difference can flip.
__device__ inline float cx_silu1(float x) { return x / (1.0f + cx_expf(-x)); }

// silu(gate) * up (src/forward.rs:483-487)
__device__ inline float cx_swiglu(float g, float u) {
  float a = cx_silu1(g);
  return a * u;
}

// f64 sum of squares of x[0..n) over a 256-thread workgroup, then the rmsnorm
// factor 1 / sqrt(sum / n + eps) in f64 (src/kernels/scalar.rs:46-47).
// `red` is 4 doubles of shared memory. Deterministic: fixed tree. Every
// square is exact in f64, so the tree differs from the sequential sum only
// in f64 roundings (relative 1e-16), far below the f32 result's ulp.
__device__ inline double cx_rms_scale(const float* x, uint32_t n, float eps,
                                      double* red) {
  const int tid = threadIdx.x;
  double s = 0.0;
  for (uint32_t i = 4 * tid; i < n; i += 4 * 256) {
    float4 f = *reinterpret_cast<const float4*>(x + i);
    s += (double)f.x * (double)f.x;
    s += (double)f.y * (double)f.y;
    s += (double)f.z * (double)f.z;
    s += (double)f.w * (double)f.w;
  }
  s = cx_wave_sum_d(s);
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  double tot = ((red[0] + red[1]) + red[2]) + red[3];
  __syncthreads();
  return 1.0 / sqrt(tot / (double)n + (double)eps);
}
