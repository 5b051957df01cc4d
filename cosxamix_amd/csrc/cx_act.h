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

// ------------------------------------------------ rmsnorm's exact scale
// The reference sums the squares in f64 in order from 0 and takes
// scale = 1 / sqrt(sum / n + eps) (src/kernels/scalar.rs:47-48); a
// workgroup sums them as a tree. Every square t_i = x_i^2 is exact in f64,
// so each sum differs from the exact S only by its own roundings (u = 2^-53):
//   in order:  |S_seq - S| <= u * (S_1 + ... + S_{n-1}) <= u * W,
//              W = sum_i t_i * (n - i)   (S_k the partial sums);
//   a tree:    |S_tree - S| <= D * u * S  (D its depth).
// The scales of the two sums then differ by at most half their relative
// difference plus the roundings of the f64 operations on each side, which
// moves v = x * scale by a bounded number of its ulps (cx_rms_reach). Where
// no value's f32 rounding can change within that (cx_rms_risk), the tree's
// scale gives the reference's outputs bit for bit;
// otherwise the workgroup sums the squares again in order (cx_rms_seq_sum).
// About one random vector in 300 takes the second sum at n = 2048, one in
// 80 at n = 4096.
// A lane's share of the tree: its sum of squares s, and w >= the share of
// W of its values, from whole groups: a group of G consecutive values from
// index i0 adds its f64 sum times (n - i0) (>= t_i * (n - i) for each of
// its values), kept in f32 (the bound carries the margin).
struct cx_rms_part {
  double s = 0.0;
  float w = 0.0f;
  template <int G>
  __device__ void add(const float* a, uint32_t i0, uint32_t n) {
    double g = 0.0;
#pragma unroll
    for (int e = 0; e < G; e++) g += (double)a[e] * (double)a[e];
    s += g;
    w = fmaf((float)g, (float)(n - i0), w);
  }
};
__device__ inline cx_rms_part cx_wave_sum_rms(cx_rms_part p) {
  p.s = cx_wave_sum_d(p.s);
  float w = p.w;  // only a bound: any order
  w += __uint_as_float(cx_dpp<CX_DPP_XOR1>(__float_as_uint(w)));
  w += __uint_as_float(cx_dpp<CX_DPP_XOR2>(__float_as_uint(w)));
  w += __uint_as_float(cx_dpp<CX_DPP_HALF_MIRROR>(__float_as_uint(w)));
  w += __uint_as_float(cx_dpp<CX_DPP_MIRROR>(__float_as_uint(w)));
  w += __shfl_xor(w, 16, CX_WAVE);
  w += __shfl_xor(w, 32, CX_WAVE);
  p.w = w;
  return p;
}
__device__ inline double cx_rms_factor(double sum, uint32_t n, float eps) {
  return 1.0 / sqrt(sum / (double)n + (double)eps);
}
// The reach of the check: how far (in f64 ulps of v = x * scale) v may
// move between the tree's sum `tot` (of depth at most `depth`, with W's
// bound w) and the sum in order. A relative bound e moves v by at most
// e * |v| < e * 2^53 ulps, and e * 2^53 = 0.51 (W / tot + depth) + 16 plus
// the f32 roundings of w / tot (an approximate reciprocal, within 1 ulp),
// covered by 0.52 and 20. 0 when the two
// cannot differ (all zeros) or cannot matter (inf, NaN); outside
// [1e-30, 1e30] W / tot takes its largest value, n.
__device__ inline uint32_t cx_rms_reach(double tot, float w, uint32_t n, uint32_t depth) {
  if (!(tot > 0.0) || !(tot < INFINITY)) return 0u;
  float q = (float)n;
  if (tot > 1e-30 && tot < 1e30) q = fminf(w * __builtin_amdgcn_rcpf((float)tot), q);
  return (uint32_t)(0.52f * (q + (float)depth)) + 20u;
}
// Whether (float)(a * scale) may round differently when v = a * scale moves
// by up to `reach` ulps, over all of a thread's values: for v in f32's
// normal range its f32 rounding drops the low 29 of its 52 mantissa bits
// and turns at 2^28 (the midpoint), so v is at risk when those bits are
// within reach of 2^28; below 2^-126 (f32's subnormals round at a fixed
// quantum) every nonzero v counts as at risk. The distances are kept as
// running minima (three vector operations a test) and compared once.
struct cx_rms_risk {
  uint32_t mid = 0xFFFFFFFFu;  // min over values of 8 * (low 29 bits) - c, wrapping
  uint32_t low = 0xFFFFFFFFu;  // min over values of (|v|'s high word) - 1
  // c = 2^31 - 8 * reach: a value's 8 * (low bits) - c is at most 16 * reach
  // exactly when its low bits are within reach of 2^28
  __device__ void add(float a, double scale, uint32_t c) {
    const uint64_t b = (uint64_t)__double_as_longlong((double)a * scale);
    mid = min(mid, ((uint32_t)b << 3) - c);
    low = min(low, ((uint32_t)(b >> 32) & 0x7FFFFFFFu) - 1u);  // zeros wrap past the test
  }
  __device__ bool unsure(uint32_t reach) const {
    return mid <= 16u * reach || low < (897u << 20) - 1u;  // 0 < |v| < 2^-126
  }
};
__device__ inline uint32_t cx_rms_c(uint32_t reach) { return 0x80000000u - 8u * reach; }
// The f64 sum of squares of x[0..n) in order from 0, by one wave: lane l
// loads x[64q + l] (coalesced) and writes its square to a 64-double LDS
// buffer, then lane 0 adds the chunk's 64 squares to the running sum in
// order, two per 16-byte LDS read (one dependent f64 add an element; reading
// the squares across lanes with readlane took ~41 clocks an element). Lanes
// past n write +0.0, which leaves a sum of squares as it is. Every lane ends
// with the sum. x may be in global memory or in LDS. The LDS writes and lane
// 0's reads are one wave's, so LDS performs them in issue order.
__device__ inline double cx_rms_seq_sum(const float* x, uint32_t n) {
  __shared__ __align__(16) double sq[2][64];
  const uint32_t lane = threadIdx.x & 63;
  double s = 0.0;
  float nxt = lane < n ? x[lane] : 0.0f;
  uint32_t b = 0;
  for (uint32_t q = 0; q < n; q += 64, b ^= 1) {
    sq[b][lane] = (double)nxt * (double)nxt;
    // the next chunk's load under this chunk's adds
    nxt = q + 64 + lane < n ? x[q + 64 + lane] : 0.0f;
    if (lane == 0) {
      const double2* p = reinterpret_cast<const double2*>(sq[b]);
#pragma unroll
      for (int j = 0; j < 32; j++) {
        const double2 v = p[j];
        s += v.x;
        s += v.y;
      }
    }
  }
  return __shfl(s, 0, 64);
}

// The rmsnorm factor of x[0..n) (n % 4 == 0, x 16-byte aligned) over a
// 256-thread workgroup, bit for bit the reference's: the tree (4 values a
// lane, wave sums, ((w0 + w1) + w2) + w3), the check above, and the sum in
// order when the check asks for it. `red` is 9 doubles and `flag` an int of
// shared memory; every thread of the workgroup calls it.
__device__ inline double cx_rms_scale(const float* x, uint32_t n, float eps, double* red,
                                      int* flag) {
  const int tid = threadIdx.x;
  cx_rms_part p;
  for (uint32_t i = 4 * tid; i < n; i += 4 * 256) {
    const float4 f = *reinterpret_cast<const float4*>(x + i);
    const float a[4] = {f.x, f.y, f.z, f.w};
    p.add<4>(a, i, n);
  }
  p = cx_wave_sum_rms(p);
  if ((tid & 63) == 0) {
    red[tid >> 6] = p.s;
    red[4 + (tid >> 6)] = (double)p.w;
  }
  if (tid == 0) *flag = 0;
  __syncthreads();
  const double tot = ((red[0] + red[1]) + red[2]) + red[3];
  const float w = (float)(((red[4] + red[5]) + red[6]) + red[7]);
  double scale = cx_rms_factor(tot, n, eps);
  const uint32_t reach = cx_rms_reach(tot, w, n, (n + 1023) / 1024 * 4 + 16);
  cx_rms_risk risk;
  const uint32_t c = cx_rms_c(reach);
  for (uint32_t i = 4 * tid; i < n; i += 4 * 256) {
    const float4 f = *reinterpret_cast<const float4*>(x + i);
    risk.add(f.x, scale, c);
    risk.add(f.y, scale, c);
    risk.add(f.z, scale, c);
    risk.add(f.w, scale, c);
  }
  if (reach && risk.unsure(reach)) *flag = 1;
  __syncthreads();
  if (*flag) {  // the same for every thread
    if (tid < 64) {
      const double seq = cx_rms_seq_sum(x, n);
      if (tid == 0) red[8] = seq;
    }
    __syncthreads();
    scale = cx_rms_factor(red[8], n, eps);
  }
  __syncthreads();  // red and flag are free again
  return scale;
}
