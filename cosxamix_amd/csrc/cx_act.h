// cx_act.h — device arithmetic for the activation side of the GEMV.
//
// quant_sub() is ops::cuantizar_i8_en for one sub-block (src/ops.rs:178-198)
// plus its integer sum (src/ops.rs:472-483):
//   amax = max|x| (f32::max ignores NaN -> fmaxf)
//   xe   = amax / 127        (IEEE division, correctly rounded)
//   inv  = 127 / amax        (0 when amax == 0)
//   xq   = round(x * inv) as i32 as i8   (half away from zero; saturating)
//   xs   = sum of xq, as f32 (exact)
// Nothing here may be contracted into an FMA; the whole library is built
// with -ffp-contract=off.
#pragma once

#include "cx_common.h"

template <int SUB>
__device__ inline void cx_quant_sub(const float (&v)[SUB], int8_t* q, float* xe,
                                    float* xs) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < SUB; i++) amax = fmaxf(amax, fabsf(v[i]));
  float d = 0.0f, inv = 0.0f;
  if (amax > 0.0f) {
    d = amax / 127.0f;
    inv = 127.0f / amax;
  }
  int32_t s = 0;
  uint32_t packed[SUB / 4];
#pragma unroll
  for (int i = 0; i < SUB / 4; i++) packed[i] = 0;
#pragma unroll
  for (int i = 0; i < SUB; i++) {
    int8_t qi = cx_rust_i8(roundf(v[i] * inv));
    s += qi;
    packed[i / 4] |= (uint32_t)(uint8_t)qi << (8 * (i % 4));
  }
#pragma unroll
  for (int i = 0; i < SUB / 4; i++) reinterpret_cast<uint32_t*>(q)[i] = packed[i];
  *xe = d;
  *xs = (float)s;
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

// Builds the i8 activation of one row of k values in (shared or global)
// memory: xq[k], xe[k/SUB], xs[k/SUB]. One thread per sub-block, strided over
// the workgroup. For CX_ACT_NORM `scale` is the f64 rmsnorm factor.
template <int SUB>
__device__ inline void cx_build_act_rows(int src, const float* x, const float* x2,
                                         const float* nw, double scale, uint32_t k,
                                         int8_t* xq, float* xe, float* xs,
                                         int tid, int nthreads) {
  const uint32_t nsub = k / SUB;
  for (uint32_t sb = tid; sb < nsub; sb += nthreads) {
    float v[SUB];
    const float4* px = reinterpret_cast<const float4*>(x + (size_t)sb * SUB);
#pragma unroll
    for (int i = 0; i < SUB / 4; i++) {
      float4 f = px[i];
      v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
    }
    if (src == 1) {  // rmsnorm: (x as f64 * scale) as f32 * w   (scalar.rs:50-52)
      const float4* pw = reinterpret_cast<const float4*>(nw + (size_t)sb * SUB);
#pragma unroll
      for (int i = 0; i < SUB / 4; i++) {
        float4 w = pw[i];
        v[4 * i] = (float)((double)v[4 * i] * scale) * w.x;
        v[4 * i + 1] = (float)((double)v[4 * i + 1] * scale) * w.y;
        v[4 * i + 2] = (float)((double)v[4 * i + 2] * scale) * w.z;
        v[4 * i + 3] = (float)((double)v[4 * i + 3] * scale) * w.w;
      }
    } else if (src == 3) {
      const float4* pu = reinterpret_cast<const float4*>(x2 + (size_t)sb * SUB);
#pragma unroll
      for (int i = 0; i < SUB / 4; i++) {
        float4 u = pu[i];
        v[4 * i] = cx_swiglu(v[4 * i], u.x);
        v[4 * i + 1] = cx_swiglu(v[4 * i + 1], u.y);
        v[4 * i + 2] = cx_swiglu(v[4 * i + 2], u.z);
        v[4 * i + 3] = cx_swiglu(v[4 * i + 3], u.w);
      }
    }
    cx_quant_sub<SUB>(v, xq + (size_t)sb * SUB, xe + sb, xs + sb);
  }
}

// f64 sum of squares of x[0..n) over a 256-thread workgroup, then the rmsnorm
// factor 1 / sqrt(sum / n + eps) in f64 (src/kernels/scalar.rs:46-47).
// `red` is 4 doubles of shared memory. Deterministic: fixed tree.
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
