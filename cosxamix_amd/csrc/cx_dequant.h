// cx_dequant.h — one lane's 8 consecutive values of a GGUF block, as
// quant::descuantizar (src/quant.rs:124-162, formats 501-679) and
// quant::desempaquetar_i8 (src/quant.rs:238-468) form them, with the same f32
// expressions and rounding (no FMA contraction: the library is built with
// -ffp-contract=off).
//
// `b` points at the block (global or LDS), `pos` is the first of the 8
// values inside the block (a multiple of 8; blocks hold 256 values for the
// k-quants, 32 for Q8_0/Q5_0, 1 for F32/F16 — those take `b` at the value).
#pragma once

#include "cx_common.h"

namespace cxq {

__device__ inline float f16_at(const uint8_t* p) { return cx_h2f((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

// quant::escala_y_minimo (src/quant.rs:108-117): 6-bit scale and min of
// sub-block j from the 12 bytes at q
__device__ inline void scale_min_k4(int j, const uint8_t* q, uint32_t& sc, uint32_t& mn) {
  if (j < 4) {
    sc = q[j] & 63;
    mn = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

// quant::escalas_q3k (src/quant.rs:87-106): the signed 6-bit scale of
// sub-block `is` (before the -32) from the 12 bytes at b + 96
__device__ inline int q3k_scale(const uint8_t* b, int is) {
  auto rd = [&](int o) {
    return (uint32_t)b[o] | ((uint32_t)b[o + 1] << 8) | ((uint32_t)b[o + 2] << 16) |
           ((uint32_t)b[o + 3] << 24);
  };
  const uint32_t m1 = 0x03030303u, m2 = 0x0F0F0F0Fu;
  const uint32_t a0 = rd(96), a1 = rd(100), tmp = rd(104);
  uint32_t aux;
  switch (is / 4) {
    case 0: aux = (a0 & m2) | ((tmp & m1) << 4); break;
    case 1: aux = (a1 & m2) | (((tmp >> 2) & m1) << 4); break;
    case 2: aux = ((a0 >> 4) & m2) | (((tmp >> 4) & m1) << 4); break;
    default: aux = ((a1 >> 4) & m2) | (((tmp >> 6) & m1) << 4); break;
  }
  return (int)(int8_t)(uint8_t)(aux >> (8 * (is % 4)));
}

// descuantizar: 8 f32 values
template <int T> __device__ void dequant8(const uint8_t* b, uint32_t pos, float (&y)[8]);

template <> __device__ inline void dequant8<CX_F32>(const uint8_t* b, uint32_t, float (&y)[8]) {
  const float* f = reinterpret_cast<const float*>(b);
#pragma unroll
  for (int i = 0; i < 8; i++) y[i] = f[i];
}
template <> __device__ inline void dequant8<CX_F16>(const uint8_t* b, uint32_t, float (&y)[8]) {
#pragma unroll
  for (int i = 0; i < 8; i++) y[i] = f16_at(b + 2 * i);
}
template <> __device__ inline void dequant8<CX_Q8_0>(const uint8_t* b, uint32_t pos, float (&y)[8]) {
  const float d = f16_at(b);
#pragma unroll
  for (int i = 0; i < 8; i++) y[i] = (float)(int8_t)b[2 + pos + i] * d;
}
template <> __device__ inline void dequant8<CX_Q5_0>(const uint8_t* b, uint32_t pos, float (&y)[8]) {
  const float d = f16_at(b);
  const uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) |
                      ((uint32_t)b[5] << 24);
  const uint8_t* qs = b + 6;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    int q;
    if (pos < 16) {
      const uint32_t j = pos + i;
      q = (int)((qs[j] & 0x0F) | (((qh >> j) << 4) & 0x10)) - 16;
    } else {
      const uint32_t j = pos - 16 + i;
      q = (int)((qs[j] >> 4) | ((qh >> (j + 12)) & 0x10)) - 16;
    }
    y[i] = (float)q * d;
  }
}
template <> __device__ inline void dequant8<CX_Q2_K>(const uint8_t* b, uint32_t pos, float (&y)[8]) {
  const uint32_t half = pos / 128, r = pos % 128 / 32, l0 = pos % 32, is = half * 8 + r * 2 + l0 / 16;
  const float d = f16_at(b + 80), mn = f16_at(b + 82);
  const uint8_t sc = b[is];
  const float dl = d * (float)(sc & 0xF), ml = mn * (float)(sc >> 4);
  const uint8_t* qs = b + 16 + half * 32 + l0;
#pragma unroll
  for (int i = 0; i < 8; i++) y[i] = dl * (float)((qs[i] >> (2 * r)) & 3) - ml;
}
template <> __device__ inline void dequant8<CX_Q3_K>(const uint8_t* b, uint32_t pos, float (&y)[8]) {
  const uint32_t half = pos / 128, r = pos % 128 / 32, l0 = pos % 32, is = half * 8 + r * 2 + l0 / 16;
  const float dall = f16_at(b + 108);
  const float dl = dall * ((float)q3k_scale(b, is) - 32.0f);
  const uint32_t m = 1u << (half * 4 + r);
  const uint8_t* qs = b + 32 + half * 32;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t idx = l0 + i;
    const int hi = (b[idx] & m) == 0 ? 4 : 0;
    y[i] = dl * (float)((int)((qs[idx] >> (2 * r)) & 3) - hi);
  }
}
template <> __device__ inline void dequant8<CX_Q4_K>(const uint8_t* b, uint32_t pos, float (&y)[8]) {
  const uint32_t pair = pos / 64, hi = pos % 64 / 32, l0 = pos % 32;
  const float d = f16_at(b), mn = f16_at(b + 2);
  uint32_t sc, m;
  scale_min_k4((int)(2 * pair + hi), b + 4, sc, m);
  const float d1 = d * (float)sc, m1 = mn * (float)m;
  const uint8_t* q = b + 16 + pair * 32 + l0;
#pragma unroll
  for (int i = 0; i < 8; i++) y[i] = d1 * (float)(hi ? (q[i] >> 4) : (q[i] & 0xF)) - m1;
}
template <> __device__ inline void dequant8<CX_Q5_K>(const uint8_t* b, uint32_t pos, float (&y)[8]) {
  const uint32_t pair = pos / 64, hi = pos % 64 / 32, l0 = pos % 32;
  const float d = f16_at(b), mn = f16_at(b + 2);
  uint32_t sc, m;
  scale_min_k4((int)(2 * pair + hi), b + 4, sc, m);
  const float d1 = d * (float)sc, m1 = mn * (float)m;
  const uint8_t u = (uint8_t)(1u << (2 * pair + hi));
  const uint8_t *qh = b + 16 + l0, *q = b + 48 + pair * 32 + l0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float ex = (qh[i] & u) ? 16.0f : 0.0f;
    y[i] = d1 * ((float)(hi ? (q[i] >> 4) : (q[i] & 0xF)) + ex) - m1;
  }
}
// the 6-bit quant (0..63) of Q6_K at `pos` of half `half`, quarter `qt`
__device__ inline int q6k_quant(const uint8_t* b, uint32_t half, uint32_t qt, uint32_t l) {
  const uint8_t *ql = b + 64 * half, *qh = b + 128 + 32 * half;
  switch (qt) {
    case 0: return (ql[l] & 0xF) | ((qh[l] & 3) << 4);
    case 1: return (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4);
    case 2: return (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
    default: return (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4);
  }
}
template <> __device__ inline void dequant8<CX_Q6_K>(const uint8_t* b, uint32_t pos, float (&y)[8]) {
  const uint32_t half = pos / 128, qt = pos % 128 / 32, l0 = pos % 32;
  const float d = f16_at(b + 208);
  const float sc = (float)(int8_t)b[192 + 8 * half + l0 / 16 + 2 * qt];
#pragma unroll
  for (int i = 0; i < 8; i++)
    y[i] = d * sc * (float)(int8_t)(q6k_quant(b, half, qt, l0 + i) - 32);
}

// desempaquetar_i8: 8 i8 values and, for the lane holding the start of a
// sub-block, its scale and offset (value = scale * q + offset)
template <int T> __device__ void unpack8(const uint8_t* b, uint32_t pos, int8_t (&q)[8],
                                         float& esc, float& off);

template <> __device__ inline void unpack8<CX_Q8_0>(const uint8_t* b, uint32_t pos, int8_t (&q)[8],
                                                    float& esc, float& off) {
#pragma unroll
  for (int i = 0; i < 8; i++) q[i] = (int8_t)b[2 + pos + i];
  esc = f16_at(b);
  off = 0.0f;
}
template <> __device__ inline void unpack8<CX_Q5_0>(const uint8_t* b, uint32_t pos, int8_t (&q)[8],
                                                    float& esc, float& off) {
  const uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) |
                      ((uint32_t)b[5] << 24);
  const uint8_t* qs = b + 6;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    if (pos < 16) {
      const uint32_t j = pos + i;
      q[i] = (int8_t)((int)((qs[j] & 0x0F) | (((qh >> j) << 4) & 0x10)) - 16);
    } else {
      const uint32_t j = pos - 16 + i;
      q[i] = (int8_t)((int)((qs[j] >> 4) | ((qh >> (j + 12)) & 0x10)) - 16);
    }
  }
  esc = f16_at(b);
  off = 0.0f;
}
template <> __device__ inline void unpack8<CX_Q2_K>(const uint8_t* b, uint32_t pos, int8_t (&q)[8],
                                                    float& esc, float& off) {
  const uint32_t half = pos / 128, r = pos % 128 / 32, l0 = pos % 32, is = half * 8 + r * 2 + l0 / 16;
  const float d = f16_at(b + 80), mn = f16_at(b + 82);
  const uint8_t sc = b[is];
  esc = d * (float)(sc & 0xF);
  off = -(mn * (float)(sc >> 4));
  const uint8_t* qs = b + 16 + half * 32 + l0;
#pragma unroll
  for (int i = 0; i < 8; i++) q[i] = (int8_t)((qs[i] >> (2 * r)) & 3);
}
template <> __device__ inline void unpack8<CX_Q3_K>(const uint8_t* b, uint32_t pos, int8_t (&q)[8],
                                                    float& esc, float& off) {
  const uint32_t half = pos / 128, r = pos % 128 / 32, l0 = pos % 32, is = half * 8 + r * 2 + l0 / 16;
  esc = f16_at(b + 108) * ((float)q3k_scale(b, is) - 32.0f);
  off = 0.0f;
  const uint32_t m = 1u << (half * 4 + r);
  const uint8_t* qs = b + 32 + half * 32;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t idx = l0 + i;
    q[i] = (int8_t)((int)((qs[idx] >> (2 * r)) & 3) - ((b[idx] & m) == 0 ? 4 : 0));
  }
}
template <> __device__ inline void unpack8<CX_Q4_K>(const uint8_t* b, uint32_t pos, int8_t (&q)[8],
                                                    float& esc, float& off) {
  const uint32_t pair = pos / 64, hi = pos % 64 / 32, l0 = pos % 32;
  uint32_t sc, m;
  scale_min_k4((int)(2 * pair + hi), b + 4, sc, m);
  esc = f16_at(b) * (float)sc;
  off = -(f16_at(b + 2) * (float)m);
  const uint8_t* qs = b + 16 + pair * 32 + l0;
#pragma unroll
  for (int i = 0; i < 8; i++) q[i] = (int8_t)(hi ? (qs[i] >> 4) : (qs[i] & 0xF));
}
template <> __device__ inline void unpack8<CX_Q5_K>(const uint8_t* b, uint32_t pos, int8_t (&q)[8],
                                                    float& esc, float& off) {
  const uint32_t pair = pos / 64, hi = pos % 64 / 32, l0 = pos % 32;
  uint32_t sc, m;
  scale_min_k4((int)(2 * pair + hi), b + 4, sc, m);
  esc = f16_at(b) * (float)sc;
  off = -(f16_at(b + 2) * (float)m);
  const uint8_t u = (uint8_t)(1u << (2 * pair + hi));
  const uint8_t *qh = b + 16 + l0, *qs = b + 48 + pair * 32 + l0;
#pragma unroll
  for (int i = 0; i < 8; i++)
    q[i] = (int8_t)((hi ? (qs[i] >> 4) : (qs[i] & 0xF)) + ((qh[i] & u) ? 16 : 0));
}
template <> __device__ inline void unpack8<CX_Q6_K>(const uint8_t* b, uint32_t pos, int8_t (&q)[8],
                                                    float& esc, float& off) {
  const uint32_t half = pos / 128, qt = pos % 128 / 32, l0 = pos % 32;
  esc = f16_at(b + 208) * (float)(int8_t)b[192 + 8 * half + l0 / 16 + 2 * qt];
  off = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) q[i] = (int8_t)(q6k_quant(b, half, qt, l0 + i) - 32);
}

}  // namespace cxq
