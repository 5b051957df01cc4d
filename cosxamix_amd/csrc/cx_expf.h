// cx_expf.h — e^x bit-identical to glibc's expf (x86-64, FMA build).
//
// The reference computes SiLU and softmax with Rust's f32::exp, which is the
// C library's expf: on Linux, glibc's implementation of the published
// "optimized-routines" method: x*N/ln2 = k + r (N = 32), 2^(k/N) from a
// 32-entry table of 2^(i/N), 2^(r/N) by a cubic, all in double, one rounding
// to float at the end. On FMA hardware glibc's build fuses the range
// reduction and the polynomial steps; the fused form below reproduces it for
// every float input (checked exhaustively on the host against libm's expf).
// Usable from host and device code.
#pragma once

#include <math.h>
#include <stdint.h>
#include <string.h>

#ifndef CX_HD
#if defined(__HIPCC__)
#define CX_HD __host__ __device__
#else
#define CX_HD
#endif
#endif

// 2^(i/32) as doubles, minus (i << 47) so that adding k << 47 yields 2^(k/32)
#define CX_EXP2_TAB                                                            \
  {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,        \
   0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,        \
   0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,        \
   0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,        \
   0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,        \
   0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,        \
   0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,        \
   0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,        \
   0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,        \
   0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,        \
   0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

// `tab` holds CX_EXP2_TAB (a device kernel may keep a copy in LDS, so that
// exp issues no global loads)
CX_HD static inline float cx_expf_tab(float x, const uint64_t* tab) {
  uint32_t ux;
  memcpy(&ux, &x, 4);
  const uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= 0x42b) {                   // |x| >= 88 or NaN
    if (ux == 0xff800000u) return 0.0f;    // -inf
    if (abstop >= 0x7f8) return x + x;     // inf or NaN
    if (x > 0x1.62e42ep6f) return INFINITY;  // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;     // underflow
  }
  const double N = 32.0;
  const double inv_ln2_n = 0x1.71547652b82fep+0 * N, shift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / N / N / N, c1 = 0x1.ebfce50fac4f3p-3 / N / N,
               c2 = 0x1.62e42ff0c52d6p-1 / N;
  const double xd = (double)x;
  double kd = fma(inv_ln2_n, xd, shift);
  uint64_t ki;
  memcpy(&ki, &kd, 8);
  kd -= shift;
  const double r = fma(inv_ln2_n, xd, -kd);
  uint64_t t = tab[ki % 32];
  t += ki << (52 - 5);
  double s;
  memcpy(&s, &t, 8);
  const double z = fma(c0, r, c1);
  const double r2 = r * r;
  double y = fma(c2, r, 1.0);
  y = fma(z, r2, y);
  y = y * s;
  return (float)y;
}

CX_HD static inline float cx_expf(float x) {
  const uint64_t t[32] = CX_EXP2_TAB;
  return cx_expf_tab(x, t);
}
