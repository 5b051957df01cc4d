/*
 * cx_oracle.c — CPU oracle (TEST INFRASTRUCTURE ONLY; see cx_oracle.h).
 *
 * A plain-C restatement of the reference's scalar arithmetic. Built with
 * -O2 -ffp-contract=off and no fast-math so every f32 operation rounds where
 * the Rust source rounds (Rust never contracts a*b+c into an FMA).
 *
 * Rust semantics reproduced explicitly:
 *   f32::round        -> roundf (half away from zero)
 *   `as i32` on f32   -> saturating, NaN -> 0        (sat_i32)
 *   `as i8`  on i32   -> keep the low 8 bits         ((int8_t)(uint8_t))
 *   f32::max / ::min  -> fmaxf / fminf (a NaN operand is ignored)
 *   iterator .sum()   -> sequential left fold
 */
#include "cx_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_err[256];
static void set_err(const char *m) { snprintf(g_err, sizeof g_err, "%s", m); }
const char *orc_last_error(void) { return g_err; }

static int32_t sat_i32(float f) {
  if (isnan(f)) return 0;
  if (f >= 2147483648.0f) return INT32_MAX;
  if (f <= -2147483648.0f) return INT32_MIN;
  return (int32_t)f;
}
/* quant_kquants.rs:22-24 */
static int32_t entero(float x) { return sat_i32(roundf(x)); }
static int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}
static uint32_t rd_u32(const uint8_t *b) {
  return (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 |
         (uint32_t)b[3] << 24;
}
static float rd_f16(const uint8_t *b) {
  return orc_f16_to_f32((uint16_t)(b[0] | b[1] << 8));
}

/* ---------------------------------------------------------------- types */
size_t orc_values_per_block(int t) {
  switch (t) {
  case ORC_F32: case ORC_F16: return 1;
  case ORC_Q5_0: case ORC_Q8_0: return 32;
  case ORC_Q2_K: case ORC_Q3_K: case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K:
    return 256;
  default: return 0;
  }
}
size_t orc_bytes_per_block(int t) {
  switch (t) {
  case ORC_F32: return 4;
  case ORC_F16: return 2;
  case ORC_Q5_0: return 22;
  case ORC_Q8_0: return 34;
  case ORC_Q2_K: return 84;
  case ORC_Q3_K: return 110;
  case ORC_Q4_K: return 144;
  case ORC_Q5_K: return 176;
  case ORC_Q6_K: return 210;
  default: return 0;
  }
}
int orc_sub_block(int t) {
  switch (t) {
  case ORC_Q8_0: case ORC_Q5_0: case ORC_Q4_K: case ORC_Q5_K: return 32;
  case ORC_Q2_K: case ORC_Q3_K: case ORC_Q6_K: return 16;
  default: return 0;
  }
}

/* ----------------------------------------------------------- f16 <-> f32 */
/* src/quant.rs:38-60 */
float orc_f16_to_f32(uint16_t bits) {
  uint32_t sign = (uint32_t)(bits >> 15) << 31;
  uint32_t e = (bits >> 10) & 0x1F, man = bits & 0x3FF, out;
  if (e == 0 && man == 0) {
    out = sign;
  } else if (e == 0) {
    int32_t ee = 1;
    uint32_t m = man;
    while (!(m & 0x400)) { m <<= 1; ee -= 1; }
    m &= 0x3FF;
    out = sign | ((uint32_t)(ee - 15 + 127) << 23) | (m << 13);
  } else if (e == 0x1F) {
    out = sign | 0x7F800000u | (man << 13);
  } else {
    out = sign | ((e + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}

/* src/quant.rs:691-731 — round to nearest even, subnormals, saturate to inf */
uint16_t orc_f32_to_f16(float x) {
  uint32_t bits;
  memcpy(&bits, &x, 4);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
  uint32_t mag = bits & 0x7FFFFFFF;
  if (mag >= 0x7F800000u) {
    int nanm = (mag & 0x007FFFFF) != 0;
    return sign | 0x7C00 | (nanm ? 0x0200 : 0);
  }
  int32_t exp = (int32_t)(mag >> 23) - 127;
  if (exp > 15) return sign | 0x7C00;
  if (exp < -14) {
    uint32_t sh = (uint32_t)(-14 - exp);
    if (sh > 24) return sign;
    /* For sh in 19..24 (|x| in [2^-38, 2^-32)) these u32 shifts reach 32..37
     * bits. A Rust release build wraps the shift amount (mod 32), so the
     * reference returns a wrapped value there; the `& 31` states that
     * behaviour instead of relying on C's undefined one. */
    uint32_t man = (mag & 0x007FFFFF) | 0x00800000;
    uint32_t val = man >> ((sh + 13) & 31);
    uint32_t rest = man & ((1u << ((sh + 13) & 31)) - 1);
    uint32_t half = 1u << ((sh + 12) & 31);
    uint32_t up = (rest > half || (rest == half && (val & 1))) ? 1 : 0;
    return sign | (uint16_t)(val + up);
  }
  uint32_t man = mag & 0x007FFFFF;
  uint32_t val = ((uint32_t)(exp + 15) << 10) | (man >> 13);
  uint32_t rest = man & 0x1FFF;
  uint32_t up = (rest > 0x1000 || (rest == 0x1000 && (val & 1))) ? 1 : 0;
  return sign | (uint16_t)(val + up);
}

/* --------------------------------------------------------- scale unpack */
/* src/quant.rs:108-117 */
void orc_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn) {
  if (j < 4) {
    *sc = q[j] & 63;
    *mn = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
    *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* src/quant.rs:87-106 */
void orc_scales_q3k(const uint8_t *b, int8_t out[16]) {
  const uint32_t m1 = 0x03030303u, m2 = 0x0F0F0F0Fu;
  uint32_t aux[4];
  aux[0] = rd_u32(b + 96);
  aux[1] = rd_u32(b + 100);
  aux[2] = rd_u32(b + 104);
  uint32_t tmp = aux[2];
  aux[2] = ((aux[0] >> 4) & m2) | (((tmp >> 4) & m1) << 4);
  aux[3] = ((aux[1] >> 4) & m2) | (((tmp >> 6) & m1) << 4);
  aux[0] = (aux[0] & m2) | ((tmp & m1) << 4);
  aux[1] = (aux[1] & m2) | (((tmp >> 2) & m1) << 4);
  for (int j = 0; j < 16; j++)
    out[j] = (int8_t)(uint8_t)(aux[j / 4] >> (8 * (j % 4)));
}

/* ----------------------------------------------------------- dequantize */
/* src/quant.rs:124-162 dispatch; formats at 501-679 */
int orc_dequantize(int type, const uint8_t *b, float *y, size_t n) {
  size_t vpb = orc_values_per_block(type);
  if (!vpb || n % vpb) { set_err("dequantize: bad type or length"); return -1; }
  size_t nb = n / vpb;
  switch (type) {
  case ORC_F32:
    memcpy(y, b, n * 4);
    break;
  case ORC_F16:
    for (size_t i = 0; i < n; i++) y[i] = rd_f16(b + 2 * i);
    break;
  case ORC_Q8_0: /* quant.rs:501-509 region (q8_0) */
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 34;
      float d = rd_f16(o);
      for (int j = 0; j < 32; j++) y[i * 32 + j] = (float)(int8_t)o[2 + j] * d;
    }
    break;
  case ORC_Q5_0: /* q5_0 */
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 22;
      float d = rd_f16(o);
      uint32_t qh = rd_u32(o + 2);
      const uint8_t *qs = o + 6;
      for (int j = 0; j < 16; j++) {
        uint8_t h0 = (uint8_t)(((qh >> j) << 4) & 0x10);
        uint8_t h1 = (uint8_t)((qh >> (j + 12)) & 0x10);
        y[i * 32 + j] = (float)(((qs[j] & 0x0F) | h0) - 16) * d;
        y[i * 32 + 16 + j] = (float)(((qs[j] >> 4) | h1) - 16) * d;
      }
    }
    break;
  case ORC_Q2_K: /* quant.rs:501-533 */
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 84, *esc = o, *qs0 = o + 16;
      float d = rd_f16(o + 80), mn = rd_f16(o + 82);
      size_t is = 0, k = i * 256;
      for (int half = 0; half < 2; half++) {
        const uint8_t *qs = qs0 + half * 32;
        int sh = 0;
        for (int r = 0; r < 4; r++) {
          for (int tr = 0; tr < 2; tr++) {
            uint8_t sc = esc[is++];
            float dl = d * (float)(sc & 0xF), ml = mn * (float)(sc >> 4);
            for (int l = 0; l < 16; l++)
              y[k + tr * 16 + l] = dl * (float)((qs[tr * 16 + l] >> sh) & 3) - ml;
          }
          k += 32;
          sh += 2;
        }
      }
    }
    break;
  case ORC_Q3_K: /* quant.rs:535-580 */
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 110, *hm = o, *qs0 = o + 32;
      float dall = rd_f16(o + 108);
      int8_t esc[16];
      orc_scales_q3k(o, esc);
      uint8_t m = 1;
      size_t is = 0, k = i * 256;
      for (int half = 0; half < 2; half++) {
        const uint8_t *qs = qs0 + half * 32;
        int sh = 0;
        for (int r = 0; r < 4; r++) {
          for (int tr = 0; tr < 2; tr++) {
            float dl = dall * ((float)esc[is] - 32.0f);
            is++;
            for (int l = 0; l < 16; l++) {
              int idx = tr * 16 + l;
              int8_t hi = (hm[idx] & m) == 0 ? 4 : 0;
              y[k + idx] = dl * (float)((int8_t)((qs[idx] >> sh) & 3) - hi);
            }
          }
          k += 32;
          sh += 2;
          m <<= 1;
        }
      }
    }
    break;
  case ORC_Q4_K: /* quant.rs:582-609 */
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 144, *esc = o + 4, *qs = o + 16;
      float d = rd_f16(o), mn = rd_f16(o + 2);
      size_t k = i * 256;
      for (int j = 0, is = 0; j < 256; j += 64, is += 2) {
        const uint8_t *q = qs + j / 2;
        uint8_t sc, m;
        orc_scale_min_k4(is, esc, &sc, &m);
        float d1 = d * (float)sc, m1 = mn * (float)m;
        orc_scale_min_k4(is + 1, esc, &sc, &m);
        float d2 = d * (float)sc, m2 = mn * (float)m;
        for (int l = 0; l < 32; l++) y[k + l] = d1 * (float)(q[l] & 0xF) - m1;
        for (int l = 0; l < 32; l++) y[k + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
        k += 64;
      }
    }
    break;
  case ORC_Q5_K: /* quant.rs:611-645 */
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 176, *esc = o + 4, *qh = o + 16, *ql = o + 48;
      float d = rd_f16(o), mn = rd_f16(o + 2);
      uint8_t u1 = 1, u2 = 2;
      size_t k = i * 256;
      for (int j = 0, is = 0; j < 256; j += 64, is += 2) {
        const uint8_t *q = ql + j / 2;
        uint8_t sc, m;
        orc_scale_min_k4(is, esc, &sc, &m);
        float d1 = d * (float)sc, m1 = mn * (float)m;
        orc_scale_min_k4(is + 1, esc, &sc, &m);
        float d2 = d * (float)sc, m2 = mn * (float)m;
        for (int l = 0; l < 32; l++) {
          float ex = (qh[l] & u1) ? 16.0f : 0.0f;
          y[k + l] = d1 * ((float)(q[l] & 0xF) + ex) - m1;
        }
        for (int l = 0; l < 32; l++) {
          float ex = (qh[l] & u2) ? 16.0f : 0.0f;
          y[k + 32 + l] = d2 * ((float)(q[l] >> 4) + ex) - m2;
        }
        k += 64;
        u1 <<= 2;
        u2 <<= 2;
      }
    }
    break;
  case ORC_Q6_K: /* quant.rs:647-679 */
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 210;
      float d = rd_f16(o + 208);
      for (int half = 0; half < 2; half++) {
        size_t base = i * 256 + half * 128;
        const uint8_t *ql = o + 64 * half, *qh = o + 128 + 32 * half;
        const uint8_t *sc = o + 192 + 8 * half;
        for (int l = 0; l < 32; l++) {
          int is = l / 16;
          int8_t q1 = (int8_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
          int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
          int8_t q3 = (int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
          int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
          y[base + l] = d * (float)(int8_t)sc[is] * (float)q1;
          y[base + 32 + l] = d * (float)(int8_t)sc[is + 2] * (float)q2;
          y[base + 64 + l] = d * (float)(int8_t)sc[is + 4] * (float)q3;
          y[base + 96 + l] = d * (float)(int8_t)sc[is + 6] * (float)q4;
        }
      }
    }
    break;
  default:
    set_err("dequantize: type not implemented");
    return -1;
  }
  return 0;
}

/* --------------------------------------------------------------- unpack */
/* src/quant.rs:238-468 */
int orc_unpack_i8(int type, const uint8_t *b, size_t n, int8_t *q,
                  float *esc, float *off) {
  size_t vpb = orc_values_per_block(type);
  int sub = orc_sub_block(type);
  if (!vpb || !sub || n % vpb) { set_err("unpack: bad type/len"); return -1; }
  size_t nb = n / vpb, nsub = n / (size_t)sub;
  for (size_t i = 0; i < nsub; i++) off[i] = 0.0f;
  switch (type) {
  case ORC_Q8_0:
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 34;
      esc[i] = rd_f16(o);
      for (int j = 0; j < 32; j++) q[i * 32 + j] = (int8_t)o[2 + j];
    }
    break;
  case ORC_Q4_K:
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 144, *e = o + 4, *qs = o + 16;
      float d = rd_f16(o), mn = rd_f16(o + 2);
      for (int p = 0; p < 4; p++) {
        uint8_t sc, m, sc2, m2;
        orc_scale_min_k4(p * 2, e, &sc, &m);
        orc_scale_min_k4(p * 2 + 1, e, &sc2, &m2);
        size_t s0 = i * 8 + p * 2;
        esc[s0] = d * (float)sc;
        off[s0] = -(mn * (float)m);
        esc[s0 + 1] = d * (float)sc2;
        off[s0 + 1] = -(mn * (float)m2);
        size_t from = i * 256 + p * 64;
        for (int l = 0; l < 32; l++) {
          q[from + l] = (int8_t)(qs[p * 32 + l] & 0xF);
          q[from + 32 + l] = (int8_t)(qs[p * 32 + l] >> 4);
        }
      }
    }
    break;
  case ORC_Q5_0:
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 22;
      esc[i] = rd_f16(o);
      uint32_t qh = rd_u32(o + 2);
      const uint8_t *qs = o + 6;
      for (int j = 0; j < 16; j++) {
        uint8_t h0 = (uint8_t)(((qh >> j) << 4) & 0x10);
        uint8_t h1 = (uint8_t)((qh >> (j + 12)) & 0x10);
        q[i * 32 + j] = (int8_t)((qs[j] & 0x0F) | h0) - 16;
        q[i * 32 + 16 + j] = (int8_t)((qs[j] >> 4) | h1) - 16;
      }
    }
    break;
  case ORC_Q5_K:
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 176, *e = o + 4, *qh = o + 16, *ql = o + 48;
      float d = rd_f16(o), mn = rd_f16(o + 2);
      uint8_t u1 = 1, u2 = 2;
      size_t k = i * 256;
      for (int j = 0, is = 0; j < 256; j += 64, is += 2) {
        const uint8_t *qv = ql + j / 2;
        uint8_t sc, m;
        orc_scale_min_k4(is, e, &sc, &m);
        esc[i * 8 + is] = d * (float)sc;
        off[i * 8 + is] = -(mn * (float)m);
        orc_scale_min_k4(is + 1, e, &sc, &m);
        esc[i * 8 + is + 1] = d * (float)sc;
        off[i * 8 + is + 1] = -(mn * (float)m);
        for (int l = 0; l < 32; l++)
          q[k + l] = (int8_t)((qv[l] & 0xF) + ((qh[l] & u1) ? 16 : 0));
        for (int l = 0; l < 32; l++)
          q[k + 32 + l] = (int8_t)((qv[l] >> 4) + ((qh[l] & u2) ? 16 : 0));
        k += 64;
        u1 <<= 2;
        u2 <<= 2;
      }
    }
    break;
  case ORC_Q2_K:
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 84, *e = o, *qs0 = o + 16;
      float d = rd_f16(o + 80), mn = rd_f16(o + 82);
      size_t is = 0, k = i * 256;
      for (int half = 0; half < 2; half++) {
        const uint8_t *qs = qs0 + half * 32;
        int sh = 0;
        for (int r = 0; r < 4; r++) {
          for (int t = 0; t < 2; t++) {
            uint8_t sc = e[is + t];
            esc[i * 16 + is + t] = d * (float)(sc & 0xF);
            off[i * 16 + is + t] = -(mn * (float)(sc >> 4));
          }
          is += 2;
          for (int l = 0; l < 32; l++) q[k + l] = (int8_t)((qs[l] >> sh) & 3);
          k += 32;
          sh += 2;
        }
      }
    }
    break;
  case ORC_Q3_K:
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 110, *hm = o, *qs0 = o + 32;
      float dall = rd_f16(o + 108);
      int8_t e[16];
      orc_scales_q3k(o, e);
      uint8_t m = 1;
      size_t is = 0, k = i * 256;
      for (int half = 0; half < 2; half++) {
        const uint8_t *qs = qs0 + half * 32;
        int sh = 0;
        for (int r = 0; r < 4; r++) {
          for (int t = 0; t < 2; t++)
            esc[i * 16 + is + t] = dall * ((float)e[is + t] - 32.0f);
          is += 2;
          for (int l = 0; l < 32; l++) {
            int8_t hi = (hm[l] & m) == 0 ? 4 : 0;
            q[k + l] = (int8_t)((qs[l] >> sh) & 3) - hi;
          }
          k += 32;
          sh += 2;
          m <<= 1;
        }
      }
    }
    break;
  case ORC_Q6_K:
    for (size_t i = 0; i < nb; i++) {
      const uint8_t *o = b + i * 210;
      float d = rd_f16(o + 208);
      for (int half = 0; half < 2; half++) {
        size_t base = i * 256 + half * 128;
        const uint8_t *ql = o + 64 * half, *qh = o + 128 + 32 * half;
        const uint8_t *sc = o + 192 + 8 * half;
        for (int p = 0; p < 8; p++)
          esc[i * 16 + half * 8 + p] = d * (float)(int8_t)sc[p];
        for (int l = 0; l < 32; l++) {
          uint8_t h = qh[l];
          q[base + l] = (int8_t)((ql[l] & 0xF) | ((h & 3) << 4)) - 32;
          q[base + 32 + l] = (int8_t)((ql[l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32;
          q[base + 64 + l] = (int8_t)((ql[l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
          q[base + 96 + l] = (int8_t)((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
        }
      }
    }
    break;
  default:
    set_err("unpack: type not implemented");
    return -1;
  }
  return sub;
}

/* ----------------------------------------------------------- quantizers */
#define EPSILON_Q 1e-15f /* quant_kquants.rs:19 */

/* quant_kquants.rs:29-84 (cuantos_q3) */
static float quants_q3(const float *x, int nmax, int32_t *l) {
  float big = 0.0f, amax = 0.0f;
  for (int i = 0; i < 16; i++)
    if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); big = x[i]; }
  if (amax < EPSILON_Q) {
    for (int i = 0; i < 16; i++) l[i] = 0;
    return 0.0f;
  }
  float iscale = -(float)nmax / big;
  float sumlx = 0.0f, suml2 = 0.0f;
  for (int i = 0; i < 16; i++) {
    l[i] = clampi(entero(iscale * x[i]), -nmax, nmax - 1);
    float w = x[i] * x[i];
    sumlx += w * x[i] * (float)l[i];
    suml2 += w * (float)(l[i] * l[i]);
  }
  for (int it = 0; it < 5; it++) {
    int changes = 0;
    for (int i = 0; i < 16; i++) {
      float w = x[i] * x[i];
      float cur = (float)l[i];
      float slx = sumlx - w * x[i] * cur;
      if (slx > 0.0f) {
        float sl2 = suml2 - w * cur * cur;
        int32_t nw = clampi(entero(x[i] * sl2 / slx), -nmax, nmax - 1);
        if (nw != l[i]) {
          slx += w * x[i] * (float)nw;
          sl2 += w * (float)(nw * nw);
          if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
            l[i] = nw;
            sumlx = slx;
            suml2 = sl2;
            changes++;
          }
        }
      }
    }
    if (!changes) break;
  }
  for (int i = 0; i < 16; i++) l[i] += nmax;
  return suml2 > 0.0f ? sumlx / suml2 : 0.0f;
}

typedef struct { int nmax; float from, step; int steps; int absolute; } search_t;

static float err_of(float d, int absolute) { return absolute ? fabsf(d) : d * d; }

/* quant_kquants.rs:99-157 (cuantos_qkx); returns scale, *neg_min = -min */
static float quants_qkx(const float *x, const float *w, int n, int32_t *l,
                        int32_t *aux, const search_t *b, float *neg_min) {
  float mn = x[0], mx = x[0], sum_w = w[0], sum_x = w[0] * x[0];
  for (int i = 1; i < n; i++) {
    mn = fminf(mn, x[i]);
    mx = fmaxf(mx, x[i]);
    sum_w += w[i];
    sum_x += w[i] * x[i];
  }
  if (mn > 0.0f) mn = 0.0f;
  if (mn == mx) {
    for (int i = 0; i < n; i++) l[i] = 0;
    *neg_min = -mn;
    return 0.0f;
  }
  float iscale = (float)b->nmax / (mx - mn);
  float scale = 1.0f / iscale;
  float best = 0.0f;
  for (int i = 0; i < n; i++) {
    l[i] = clampi(entero(iscale * (x[i] - mn)), 0, b->nmax);
    best += w[i] * err_of(scale * (float)l[i] + mn - x[i], b->absolute);
  }
  for (int k = 0; k <= b->steps; k++) {
    iscale = (b->from + b->step * (float)k + (float)b->nmax) / (mx - mn);
    float sl = 0.0f, sl2 = 0.0f, sxl = 0.0f;
    for (int i = 0; i < n; i++) {
      aux[i] = clampi(entero(iscale * (x[i] - mn)), 0, b->nmax);
      float lf = (float)aux[i];
      float wl = w[i] * lf;
      sl += wl;
      sl2 += wl * lf;
      sxl += wl * x[i];
    }
    float D = sum_w * sl2 - sl * sl;
    if (D > 0.0f) {
      float this_scale = (sum_w * sxl - sum_x * sl) / D;
      float this_min = (sl2 * sum_x - sl * sxl) / D;
      if (this_min > 0.0f) {
        this_min = 0.0f;
        this_scale = sxl / sl2;
      }
      float e = 0.0f;
      for (int i = 0; i < n; i++)
        e += w[i] * err_of(this_scale * (float)aux[i] + this_min - x[i], b->absolute);
      if (e < best) {
        for (int i = 0; i < n; i++) l[i] = aux[i];
        best = e;
        scale = this_scale;
        mn = this_min;
      }
    }
  }
  *neg_min = -mn;
  return scale;
}

static void put_f16(uint8_t *o, uint16_t h) { o[0] = (uint8_t)h; o[1] = (uint8_t)(h >> 8); }

/* quant_kquants.rs:160-228 (bloque_q3k) -> 110 bytes */
static void block_q3k(const float *x, uint8_t *out) {
  int32_t l[16][16];
  float scales[16], big = 0.0f, amax = 0.0f;
  for (int j = 0; j < 16; j++) {
    scales[j] = quants_q3(x + j * 16, 4, l[j]);
    if (fabsf(scales[j]) > amax) { amax = fabsf(scales[j]); big = scales[j]; }
  }
  uint8_t hmask[32] = {0}, qs[64] = {0}, packed[12] = {0};
  uint16_t dstore;
  if (amax < EPSILON_Q) {
    dstore = 0;
    for (int j = 0; j < 16; j++)
      for (int i = 0; i < 16; i++) l[j][i] = 4;
  } else {
    float iscale = -32.0f / big;
    dstore = orc_f32_to_f16(1.0f / iscale);
    float d = orc_f16_to_f32(dstore);
    for (int j = 0; j < 16; j++) {
      int32_t e = clampi(entero(iscale * scales[j]), -32, 31);
      float sc = d * (float)e;
      if (sc != 0.0f) {
        float inv = 1.0f / sc;
        for (int i = 0; i < 16; i++)
          l[j][i] = clampi(entero(x[j * 16 + i] * inv), -4, 3) + 4;
      } else {
        for (int i = 0; i < 16; i++) l[j][i] = 4;
      }
      uint8_t u = (uint8_t)(e + 32);
      if (j < 8) packed[j] |= u & 0xF;
      else packed[j - 8] |= (uint8_t)((u & 0xF) << 4);
      packed[8 + j % 4] |= (uint8_t)((u >> 4) << (2 * (j / 4)));
    }
  }
  for (int idx = 0; idx < 256; idx++) {
    uint8_t val = (uint8_t)l[idx / 16][idx % 16];
    int half = idx / 128, round = (idx % 128) / 32, place = idx % 32;
    qs[half * 32 + place] |= (uint8_t)((val & 3) << (round * 2));
    if (val & 4) hmask[place] |= (uint8_t)(1 << (half * 4 + round));
  }
  memcpy(out, hmask, 32);
  memcpy(out + 32, qs, 64);
  memcpy(out + 96, packed, 12);
  put_f16(out + 108, dstore);
}

/* quant_kquants.rs:236-257: the search of each 16-value sub-block of a
 * Q2_K block, weights |v|, absolute error */
static void search_q2k(const float *x, float scales[16], float mins[16], int32_t l[16][16]) {
  int32_t aux[16];
  float w[16];
  const search_t s = {3, -0.5f, 0.1f, 15, 1};
  for (int j = 0; j < 16; j++) {
    const float *sub = x + j * 16;
    for (int i = 0; i < 16; i++) w[i] = fabsf(sub[i]);
    scales[j] = quants_qkx(sub, w, 16, l[j], aux, &s, &mins[j]);
  }
}

/* quant_kquants.rs:231-291 (bloque_q2k) -> 84 bytes */
static void block_q2k(const float *x, uint8_t *out) {
  int32_t l[16][16];
  float scales[16], mins[16], max_sc = 0.0f, max_mn = 0.0f;
  search_q2k(x, scales, mins, l);
  for (int j = 0; j < 16; j++) {
    max_sc = fmaxf(max_sc, scales[j]);
    max_mn = fmaxf(max_mn, mins[j]);
  }
  float inv_sc = max_sc > 0.0f ? 15.0f / max_sc : 0.0f;
  float inv_mn = max_mn > 0.0f ? 15.0f / max_mn : 0.0f;
  uint16_t dstore = orc_f32_to_f16(max_sc > 0.0f ? 1.0f / inv_sc : 0.0f);
  uint16_t mstore = orc_f32_to_f16(max_mn > 0.0f ? 1.0f / inv_mn : 0.0f);
  float d = orc_f16_to_f32(dstore), dm = orc_f16_to_f32(mstore);
  uint8_t pack[16], qs[64] = {0};
  for (int j = 0; j < 16; j++) {
    int32_t le = clampi(entero(inv_sc * scales[j]), 0, 15);
    int32_t lm = clampi(entero(inv_mn * mins[j]), 0, 15);
    pack[j] = (uint8_t)(le | (lm << 4));
    float dl = d * (float)le, ml = dm * (float)lm;
    for (int i = 0; i < 16; i++)
      l[j][i] = dl > 0.0f ? clampi(entero((x[j * 16 + i] + ml) / dl), 0, 3) : 0;
  }
  for (int idx = 0; idx < 256; idx++) {
    int half = idx / 128, round = (idx % 128) / 32;
    uint8_t val = (uint8_t)l[idx / 16][idx % 16];
    qs[half * 32 + idx % 32] |= (uint8_t)(val << (round * 2));
  }
  memcpy(out, pack, 16);
  memcpy(out + 16, qs, 64);
  put_f16(out + 80, dstore);
  put_f16(out + 82, mstore);
}

/* quant_kquants.rs:301-313: the search of each 32-value sub-block of a
 * Q4_K/Q5_K block, weights media + |v| (media: the block's RMS) */
static void search_32(const float *x, const search_t *b, float scales[8], float mins[8],
                      int32_t l[8][32]) {
  int32_t aux[32];
  float w[32];
  float ss = 0.0f;
  for (int i = 0; i < 256; i++) ss += x[i] * x[i];
  float mean = sqrtf(ss / 256.0f);
  for (int j = 0; j < 8; j++) {
    const float *sub = x + j * 32;
    for (int i = 0; i < 32; i++) w[i] = mean + fabsf(sub[i]);
    scales[j] = quants_qkx(sub, w, 32, l[j], aux, b, &mins[j]);
  }
}

/* quant_kquants.rs:295-348 (sub_bloques_de_32) */
static void subblocks_32(const float *x, const search_t *b, uint16_t *dstore,
                         uint16_t *mstore, uint8_t packed[12],
                         int32_t l[8][32]) {
  float scales[8], mins[8], max_sc = 0.0f, max_mn = 0.0f;
  search_32(x, b, scales, mins, l);
  for (int j = 0; j < 8; j++) {
    max_sc = fmaxf(max_sc, scales[j]);
    max_mn = fmaxf(max_mn, mins[j]);
  }
  float inv_sc = max_sc > 0.0f ? 63.0f / max_sc : 0.0f;
  float inv_mn = max_mn > 0.0f ? 63.0f / max_mn : 0.0f;
  *dstore = orc_f32_to_f16(max_sc > 0.0f ? 1.0f / inv_sc : 0.0f);
  *mstore = orc_f32_to_f16(max_mn > 0.0f ? 1.0f / inv_mn : 0.0f);
  float d = orc_f16_to_f32(*dstore), dm = orc_f16_to_f32(*mstore);
  memset(packed, 0, 12);
  for (int j = 0; j < 8; j++) {
    uint8_t le = (uint8_t)clampi(entero(inv_sc * scales[j]), 0, 63);
    uint8_t lm = (uint8_t)clampi(entero(inv_mn * mins[j]), 0, 63);
    if (j < 4) {
      packed[j] |= le;
      packed[j + 4] |= lm;
    } else {
      packed[j + 4] = (uint8_t)((le & 0xF) | ((lm & 0xF) << 4));
      packed[j - 4] |= (uint8_t)((le >> 4) << 6);
      packed[j] |= (uint8_t)((lm >> 4) << 6);
    }
    float dl = d * (float)le, ml = dm * (float)lm;
    for (int i = 0; i < 32; i++)
      l[j][i] = dl > 0.0f ? clampi(entero((x[j * 32 + i] + ml) / dl), 0, b->nmax) : 0;
  }
}

/* quant_kquants.rs:353-359, 375-381: the searches of Q4_K and Q5_K */
static const search_t SEARCH_Q4K = {15, -1.0f, 0.1f, 20, 0};
static const search_t SEARCH_Q5K = {31, -0.5f, 0.1f, 15, 0};

/* quant_kquants.rs:351-369 (bloque_q4k) -> 144 bytes */
static void block_q4k(const float *x, uint8_t *out) {
  const search_t s = SEARCH_Q4K;
  uint16_t d, m;
  uint8_t packed[12];
  int32_t l[8][32];
  subblocks_32(x, &s, &d, &m, packed, l);
  put_f16(out, d);
  put_f16(out + 2, m);
  memcpy(out + 4, packed, 12);
  for (int p = 0; p < 4; p++)
    for (int i = 0; i < 32; i++)
      out[16 + p * 32 + i] = (uint8_t)(l[2 * p][i] | (l[2 * p + 1][i] << 4));
}

/* quant_kquants.rs:373-399 (bloque_q5k) -> 176 bytes */
static void block_q5k(const float *x, uint8_t *out) {
  const search_t s = SEARCH_Q5K;
  uint16_t d, m;
  uint8_t packed[12], qh[32] = {0};
  int32_t l[8][32];
  subblocks_32(x, &s, &d, &m, packed, l);
  for (int p = 0; p < 4; p++)
    for (int i = 0; i < 32; i++) {
      qh[i] |= (uint8_t)((l[2 * p][i] >> 4) << (2 * p));
      qh[i] |= (uint8_t)((l[2 * p + 1][i] >> 4) << (2 * p + 1));
    }
  put_f16(out, d);
  put_f16(out + 2, m);
  memcpy(out + 4, packed, 12);
  memcpy(out + 16, qh, 32);
  for (int p = 0; p < 4; p++)
    for (int i = 0; i < 32; i++)
      out[48 + p * 32 + i] =
          (uint8_t)((l[2 * p][i] & 0xF) | ((l[2 * p + 1][i] & 0xF) << 4));
}

/* The per-sub-block search of one 256-value block, as the block quantizers
 * above run it, before the scales and mins are themselves quantized:
 * Q2_K 16 sub-blocks (scale, -min, codes 0..3), Q4_K/Q5_K 8 sub-blocks
 * (codes 0..15 / 0..31), Q3_K 16 sub-blocks (cuantos_q3's scale, codes
 * 0..7, mins 0). l holds 256 codes. A test hook of the oracle. */
int orc_kquant_search(int type, const float *x, float *scales, float *neg_mins, int32_t *l) {
  switch (type) {
    case ORC_Q2_K:
      search_q2k(x, scales, neg_mins, (int32_t(*)[16])l);
      return 16;
    case ORC_Q3_K:
      for (int j = 0; j < 16; j++) {
        scales[j] = quants_q3(x + j * 16, 4, l + j * 16);
        neg_mins[j] = 0.0f;
      }
      return 16;
    case ORC_Q4_K:
      search_32(x, &SEARCH_Q4K, scales, neg_mins, (int32_t(*)[32])l);
      return 8;
    case ORC_Q5_K:
      search_32(x, &SEARCH_Q5K, scales, neg_mins, (int32_t(*)[32])l);
      return 8;
    default:
      set_err("kquant_search: not a k-quant with a quantizer");
      return -1;
  }
}

/* src/quant.rs:744-805 (cuantizar_bloques) */
long orc_quantize_blocks(int type, const float *x, size_t n, uint8_t *out) {
  size_t vpb = orc_values_per_block(type), bpb = orc_bytes_per_block(type);
  if (!vpb || n % vpb) { set_err("quantize_blocks: bad type/len"); return -1; }
  size_t nb = n / vpb;
  switch (type) {
  case ORC_F32:
    memcpy(out, x, n * 4);
    break;
  case ORC_F16:
    for (size_t i = 0; i < n; i++) put_f16(out + 2 * i, orc_f32_to_f16(x[i]));
    break;
  case ORC_Q8_0:
    for (size_t i = 0; i < nb; i++) {
      const float *c = x + 32 * i;
      uint8_t *o = out + 34 * i;
      float amax = 0.0f;
      for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(c[j]));
      float d = amax / 127.0f;
      put_f16(o, orc_f32_to_f16(d));
      float read = orc_f16_to_f32(orc_f32_to_f16(d));
      float inv = read > 0.0f ? 1.0f / read : 0.0f;
      for (int j = 0; j < 32; j++)
        o[2 + j] = (uint8_t)(int8_t)clampi(sat_i32(roundf(c[j] * inv)), -127, 127);
    }
    break;
  case ORC_Q2_K: for (size_t i = 0; i < nb; i++) block_q2k(x + 256 * i, out + bpb * i); break;
  case ORC_Q3_K: for (size_t i = 0; i < nb; i++) block_q3k(x + 256 * i, out + bpb * i); break;
  case ORC_Q4_K: for (size_t i = 0; i < nb; i++) block_q4k(x + 256 * i, out + bpb * i); break;
  case ORC_Q5_K: for (size_t i = 0; i < nb; i++) block_q5k(x + 256 * i, out + bpb * i); break;
  default:
    set_err("quantize_blocks: no quantizer for this type");
    return -1;
  }
  return (long)(nb * bpb);
}

/* ------------------------------------------------------------ Azar RNG */
/* src/daiss.rs:317-357 */
void orc_azar_seed(orc_azar *a, uint64_t s) {
  a->state = s == 0 ? 0x9E3779B97F4A7C15ull : s;
}
uint64_t orc_azar_next(orc_azar *a) {
  uint64_t x = a->state;
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  a->state = x;
  return x * 0x2545F4914F6CDD1Dull;
}
static float azar_uniform(orc_azar *a) {
  uint64_t bits = orc_azar_next(a) >> 40;
  return ((float)bits + 1.0f) / 16777216.0f;
}
void orc_azar_normals(orc_azar *a, float sigma, float *z0, float *z1) {
  float u1 = azar_uniform(a), u2 = azar_uniform(a);
  float r = sigma * sqrtf(-2.0f * logf(u1));
  float ang = 6.28318530717958647692f * u2; /* std::f32::consts::TAU */
  *z0 = r * cosf(ang);
  *z1 = r * sinf(ang);
}
/* src/daiss.rs:364-379 (FNV-1a 64 of the name, then the row, then the seed) */
uint64_t orc_seed_of(uint64_t model, const char *name, uint64_t row) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (const unsigned char *p = (const unsigned char *)name; *p; p++) {
    h ^= *p;
    h *= 0x00000100000001B3ull;
  }
  h ^= row;
  h *= 0x00000100000001B3ull;
  return h ^ ((model << 17) | (model >> 47));
}
/* src/daiss.rs:552-564 */
void orc_daiss_row(uint64_t seed, const char *name, uint64_t row, float sigma,
                   float *out, size_t width) {
  orc_azar a;
  orc_azar_seed(&a, orc_seed_of(seed, name, row));
  size_t i = 0;
  for (; i + 1 < width; i += 2) orc_azar_normals(&a, sigma, &out[i], &out[i + 1]);
  if (i < width) {
    float z1;
    orc_azar_normals(&a, sigma, &out[i], &z1);
  }
}

int orc_daiss_matrix(uint64_t seed, const char *name, size_t rows, size_t width,
                     float sigma, int type, uint8_t *out, int threads) {
  size_t vpb = orc_values_per_block(type);
  if (!vpb || width % vpb) { set_err("daiss_matrix: width/type"); return -1; }
  size_t rb = width / vpb * orc_bytes_per_block(type);
  int err = 0;
  if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
  {
    float *row = (float *)malloc(width * sizeof(float));
    if (!row) {
#pragma omp atomic write
      err = 1;
    }
#pragma omp for schedule(static)
    for (size_t r = 0; r < rows; r++) {
      if (!row) continue;
      orc_daiss_row(seed, name, r, sigma, row, width);
      if (orc_quantize_blocks(type, row, width, out + r * rb) < 0) {
#pragma omp atomic write
        err = 1;
      }
    }
    free(row);
  }
  if (err) { set_err("daiss_matrix failed"); return -1; }
  return 0;
}

/* ------------------------------------------------- activation quantizer */
/* src/ops.rs:178-198 and the per-sub-block sums of ops.rs:472-483 */
void orc_quantize_act(const float *x, size_t k, int sub, int8_t *xq, float *xe,
                      float *xs) {
  size_t nsub = (k + (size_t)sub - 1) / (size_t)sub;
  for (size_t b = 0; b < nsub; b++) {
    size_t from = b * (size_t)sub, to = from + (size_t)sub;
    if (to > k) to = k;
    float amax = 0.0f;
    for (size_t i = from; i < to; i++) amax = fmaxf(amax, fabsf(x[i]));
    float d = 0.0f, inv = 0.0f;
    if (amax > 0.0f) {
      d = amax / 127.0f;
      inv = 127.0f / amax;
    }
    xe[b] = d;
    int32_t s = 0;
    for (size_t i = from; i < to; i++) {
      int8_t q = (int8_t)(uint8_t)sat_i32(roundf(x[i] * inv));
      xq[i] = q;
      s += q;
    }
    if (xs) xs[b] = (float)s;
  }
}

/* ------------------------------------------------------------- row dots */
/* src/kernels/scalar.rs:132-170 */
float orc_dot_q4k(const uint8_t *B, const int8_t *xq, const float *xe,
                  const float *xs, size_t nb) {
  float total = 0.0f;
  for (size_t bl = 0; bl < nb; bl++) {
    const uint8_t *o = B + bl * 144, *esc = o + 4, *qs = o + 16;
    float d = rd_f16(o), dmin = rd_f16(o + 2);
    for (int p = 0; p < 4; p++)
      for (int h = 0; h < 2; h++) {
        int j = p * 2 + h;
        uint8_t sc, mn;
        orc_scale_min_k4(j, esc, &sc, &mn);
        size_t sub = bl * 8 + (size_t)j;
        const int8_t *x = xq + bl * 256 + p * 64 + h * 32;
        int32_t e = 0;
        for (int i = 0; i < 32; i++) {
          int q = h == 0 ? (qs[p * 32 + i] & 0x0F) : (qs[p * 32 + i] >> 4);
          e += (int32_t)x[i] * q;
        }
        total += xe[sub] * (d * (float)sc * (float)e - dmin * (float)mn * xs[sub]);
      }
  }
  return total;
}

/* src/kernels/scalar.rs:179-217 */
float orc_dot_q5k(const uint8_t *B, const int8_t *xq, const float *xe,
                  const float *xs, size_t nb) {
  float total = 0.0f;
  for (size_t bl = 0; bl < nb; bl++) {
    const uint8_t *o = B + bl * 176, *esc = o + 4, *qh = o + 16, *qs = o + 48;
    float d = rd_f16(o), dmin = rd_f16(o + 2);
    for (int p = 0; p < 4; p++)
      for (int h = 0; h < 2; h++) {
        int j = p * 2 + h;
        uint8_t sc, mn;
        orc_scale_min_k4(j, esc, &sc, &mn);
        size_t sub = bl * 8 + (size_t)j;
        const int8_t *x = xq + bl * 256 + p * 64 + h * 32;
        int32_t e = 0;
        for (int i = 0; i < 32; i++) {
          int nib = h == 0 ? (qs[p * 32 + i] & 0x0F) : (qs[p * 32 + i] >> 4);
          int hi = (qh[i] & (1 << j)) ? 16 : 0;
          e += (int32_t)x[i] * (nib + hi);
        }
        total += xe[sub] * (d * (float)sc * (float)e - dmin * (float)mn * xs[sub]);
      }
  }
  return total;
}

/* src/kernels/scalar.rs:236-275 */
float orc_dot_q3k(const uint8_t *B, const int8_t *xq, const float *xe,
                  const float *xs, size_t nb) {
  float total = 0.0f;
  for (size_t bl = 0; bl < nb; bl++) {
    const uint8_t *o = B + bl * 110, *hm = o, *qs = o + 32;
    float d = rd_f16(o + 108);
    int8_t esc[16];
    orc_scales_q3k(o, esc);
    for (int g = 0; g < 8; g++) {
      const uint8_t *qsg = qs + (g / 4) * 32;
      int sh = 2 * (g % 4);
      uint8_t m = (uint8_t)(1u << g);
      const int8_t *x = xq + bl * 256 + g * 32;
      for (int half = 0; half < 2; half++) {
        size_t sub = bl * 16 + (size_t)(g * 2 + half);
        float scale = d * ((float)esc[g * 2 + half] - 32.0f);
        int32_t e = 0;
        for (int l = 0; l < 16; l++) {
          int idx = half * 16 + l;
          int extra = (hm[idx] & m) ? 4 : 0;
          int q = ((qsg[idx] >> sh) & 3) + extra;
          e += (int32_t)x[idx] * q;
        }
        total += xe[sub] * scale * ((float)e - 4.0f * xs[sub]);
      }
    }
  }
  return total;
}

/* src/kernels/q2k.rs:41-69 */
float orc_dot_q2k(const uint8_t *B, const int8_t *xq, const float *xe,
                  const float *xs, size_t nb) {
  float total = 0.0f;
  for (size_t bl = 0; bl < nb; bl++) {
    const uint8_t *o = B + bl * 84, *esc = o, *qs = o + 16;
    float d = rd_f16(o + 80), dm = rd_f16(o + 82);
    for (int g = 0; g < 8; g++) {
      const uint8_t *qsg = qs + (g / 4) * 32;
      int sh = 2 * (g % 4);
      const int8_t *x = xq + bl * 256 + g * 32;
      for (int half = 0; half < 2; half++) {
        int s = g * 2 + half;
        size_t sub = bl * 16 + (size_t)s;
        int32_t e = 0;
        for (int l = 0; l < 16; l++) {
          int idx = half * 16 + l;
          e += (int32_t)x[idx] * ((qsg[idx] >> sh) & 3);
        }
        float es = d * (float)(esc[s] & 0xF);
        float ms = dm * (float)(esc[s] >> 4);
        total += xe[sub] * (es * (float)e - ms * xs[sub]);
      }
    }
  }
  return total;
}

/* src/kernels/scalar.rs:294-324 */
float orc_dot_q6k(const uint8_t *B, const int8_t *xq, const float *xe,
                  const float *xs, size_t nb) {
  float total = 0.0f;
  for (size_t bl = 0; bl < nb; bl++) {
    const uint8_t *o = B + bl * 210, *esc = o + 192;
    float d = rd_f16(o + 208);
    for (int g = 0; g < 8; g++) {
      int half = g / 4, gi = g % 4;
      const uint8_t *ql = o + 64 * half + 32 * (gi % 2);
      const uint8_t *qh = o + 128 + 32 * half;
      const int8_t *x = xq + bl * 256 + g * 32;
      for (int md = 0; md < 2; md++) {
        size_t sub = bl * 16 + (size_t)(g * 2 + md);
        float scale = d * (float)(int8_t)esc[g * 2 + md];
        int32_t e = 0;
        for (int l = 0; l < 16; l++) {
          int i = md * 16 + l;
          int nib = gi < 2 ? (ql[i] & 0x0F) : (ql[i] >> 4);
          int q = nib | (((qh[i] >> (2 * gi)) & 3) << 4);
          e += (int32_t)x[i] * q;
        }
        total += xe[sub] * scale * ((float)e - 32.0f * xs[sub]);
      }
    }
  }
  return total;
}

orc_row_kernel orc_row_kernel_for(int t) {
  switch (t) {
  case ORC_Q2_K: return orc_dot_q2k;
  case ORC_Q3_K: return orc_dot_q3k;
  case ORC_Q4_K: return orc_dot_q4k;
  case ORC_Q5_K: return orc_dot_q5k;
  case ORC_Q6_K: return orc_dot_q6k;
  default: return NULL;
  }
}

/* The integer sums each scalar kernel above forms before its f32 scaling;
 * out has nb*8 (Q4_K/Q5_K) or nb*16 (Q2_K/Q3_K/Q6_K) entries. */
int orc_subsums(int t, const uint8_t *B, const int8_t *xq, size_t nb, int32_t *out) {
  for (size_t bl = 0; bl < nb; bl++) {
    const int8_t *x = xq + bl * 256;
    if (t == ORC_Q4_K || t == ORC_Q5_K) {
      const uint8_t *o = B + bl * (t == ORC_Q4_K ? 144 : 176);
      const uint8_t *qs = o + (t == ORC_Q4_K ? 16 : 48), *qh = o + 16;
      for (int j = 0; j < 8; j++) {
        int p = j / 2, h = j % 2;
        int32_t e = 0;
        for (int i = 0; i < 32; i++) {
          int q = h == 0 ? (qs[p * 32 + i] & 0xF) : (qs[p * 32 + i] >> 4);
          if (t == ORC_Q5_K && (qh[i] & (1 << j))) q += 16;
          e += (int32_t)x[p * 64 + h * 32 + i] * q;
        }
        out[bl * 8 + (size_t)j] = e;
      }
    } else if (t == ORC_Q2_K || t == ORC_Q3_K) {
      const uint8_t *o = B + bl * (t == ORC_Q2_K ? 84 : 110);
      const uint8_t *qs = o + (t == ORC_Q2_K ? 16 : 32), *hm = o;
      for (int s = 0; s < 16; s++) {
        int g = s / 2, half = s % 2, sh = 2 * (g % 4);
        const uint8_t *qsg = qs + (g / 4) * 32;
        int32_t e = 0;
        for (int l = 0; l < 16; l++) {
          int idx = half * 16 + l;
          int q = (qsg[idx] >> sh) & 3;
          if (t == ORC_Q3_K && (hm[idx] & (1 << g))) q += 4;
          e += (int32_t)x[g * 32 + idx] * q;
        }
        out[bl * 16 + (size_t)s] = e;
      }
    } else if (t == ORC_Q6_K) {
      const uint8_t *o = B + bl * 210;
      for (int s = 0; s < 16; s++) {
        int g = s / 2, md = s % 2, half = g / 4, gi = g % 4;
        const uint8_t *ql = o + 64 * half + 32 * (gi % 2), *qh = o + 128 + 32 * half;
        int32_t e = 0;
        for (int l = 0; l < 16; l++) {
          int i = md * 16 + l;
          int nib = gi < 2 ? (ql[i] & 0xF) : (ql[i] >> 4);
          e += (int32_t)x[g * 32 + i] * (nib | (((qh[i] >> (2 * gi)) & 3) << 4));
        }
        out[bl * 16 + (size_t)s] = e;
      }
    } else {
      set_err("subsums: type");
      return -1;
    }
  }
  return 0;
}

/* ------------------------------------------------------- per-token ops */
/* src/kernels/scalar.rs:16-23 */
float orc_dot_f32(const float *a, const float *b, size_t n) {
  float s = 0.0f;
  for (size_t i = 0; i < n; i++) s += a[i] * b[i];
  return s;
}
/* src/kernels/scalar.rs:36-54 (f64 accumulation) */
void orc_rmsnorm(float *out, const float *in, const float *w, size_t n, float eps) {
  if (!n) return;
  double s = 0.0;
  for (size_t i = 0; i < n; i++) s += (double)in[i] * (double)in[i];
  double scale = 1.0 / sqrt(s / (double)n + (double)eps);
  for (size_t i = 0; i < n; i++) out[i] = (float)((double)in[i] * scale) * w[i];
}
/* src/kernels/scalar.rs:63-67 */
void orc_silu(float *out, const float *in, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = in[i] / (1.0f + expf(-in[i]));
}
/* src/sampler.rs:129-137 — strict '>', ties keep the first index */
uint32_t orc_argmax(const float *v, size_t n) {
  size_t best = 0;
  for (size_t i = 0; i < n; i++)
    if (v[i] > v[best]) best = i;
  return (uint32_t)best;
}

/* src/ops.rs:1108-1129 — f32 powf frequency, f64 angle, f64 cos/sin */
void orc_rope_tables(size_t hd, float base, size_t ctx, float *c, float *s) {
  size_t half = hd / 2;
  for (size_t j = 0; j < half; j++) {
    float freq = 1.0f / powf(base, 2.0f * (float)j / (float)hd);
    for (size_t p = 0; p < ctx; p++) {
      double ang = (double)p * (double)freq;
      c[p * half + j] = (float)cos(ang);
      s[p * half + j] = (float)sin(ang);
    }
  }
}
/* src/ops.rs:1150-1193 — split-half rotation */
int orc_rope(float *x, size_t tokens, size_t heads, size_t hd, const float *c,
             const float *s, size_t ctx, size_t pos) {
  if (hd % 2) { set_err("rope: odd head_dim"); return -1; }
  if (pos + tokens > ctx) { set_err("rope: position past table"); return -1; }
  size_t half = hd / 2, width = heads * hd;
  for (size_t t = 0; t < tokens; t++) {
    const float *ct = c + (pos + t) * half, *st = s + (pos + t) * half;
    for (size_t h = 0; h < heads; h++) {
      float *lo = x + t * width + h * hd, *hi = lo + half;
      for (size_t i = 0; i < half; i++) {
        float x0 = lo[i], x1 = hi[i];
        lo[i] = x0 * ct[i] - x1 * st[i];
        hi[i] = x0 * st[i] + x1 * ct[i];
      }
    }
  }
  return 0;
}
/* src/ops.rs:1206-1230 */
int orc_softmax(float *x, size_t len, size_t width) {
  if (!width || len % width) { set_err("softmax: width"); return -1; }
  for (size_t r = 0; r < len / width; r++) {
    float *row = x + r * width;
    float mx = -INFINITY;
    for (size_t i = 0; i < width; i++) mx = fmaxf(mx, row[i]);
    if (!isfinite(mx)) {
      float p = 1.0f / (float)width;
      for (size_t i = 0; i < width; i++) row[i] = p;
      continue;
    }
    float tot = 0.0f;
    for (size_t i = 0; i < width; i++) {
      row[i] = expf(row[i] - mx);
      tot += row[i];
    }
    float inv = 1.0f / tot;
    for (size_t i = 0; i < width; i++) row[i] *= inv;
  }
  return 0;
}
/* src/ops.rs:1258-1325 — causal GQA; head h reads kv group h/(H/Hkv).
 * Each score is kernels::dot's sequential sum from 0 times the scale, and
 * each output value the sum of prob*v in position order from 0. For many
 * query rows the keys are first copied to a [group dim][position] layout so
 * that sixteen positions' sums advance together in AVX lanes, each lane in
 * its own order; the output's dims advance together the same way. */
static void scores16(const float *qh, const float *kg, size_t total, size_t hd, size_t p,
                     float scale, float *pts) {
  __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
  for (size_t d = 0; d < hd; d++) {
    const __m256 qd = _mm256_set1_ps(qh[d]);
    const float *kd = kg + d * total + p;
    s0 = _mm256_add_ps(s0, _mm256_mul_ps(qd, _mm256_loadu_ps(kd)));
    s1 = _mm256_add_ps(s1, _mm256_mul_ps(qd, _mm256_loadu_ps(kd + 8)));
  }
  const __m256 sc = _mm256_set1_ps(scale);
  _mm256_storeu_ps(pts + p, _mm256_mul_ps(s0, sc));
  _mm256_storeu_ps(pts + p + 8, _mm256_mul_ps(s1, sc));
}

/* out[d] = sum_p prob[p] * v[p][d] in position order, 64 dims at a time */
static void weighted_sum(const float *pts, const float *v, size_t wkv, size_t vis, size_t hd,
                         float *dst) {
  size_t d0 = 0;
  for (; d0 + 64 <= hd; d0 += 64) {
    __m256 a[8];
    for (int i = 0; i < 8; i++) a[i] = _mm256_setzero_ps();
    for (size_t p = 0; p < vis; p++) {
      const __m256 w = _mm256_set1_ps(pts[p]);
      const float *vp = v + p * wkv + d0;
      for (int i = 0; i < 8; i++) a[i] = _mm256_add_ps(a[i], _mm256_mul_ps(w, _mm256_loadu_ps(vp + 8 * i)));
    }
    for (int i = 0; i < 8; i++) _mm256_storeu_ps(dst + d0 + 8 * i, a[i]);
  }
  for (; d0 < hd; d0++) {
    float acc = 0.0f;
    for (size_t p = 0; p < vis; p++) acc += pts[p] * v[p * wkv + d0];
    dst[d0] = acc;
  }
}

int orc_attention(const float *q, const float *k, const float *v, size_t tokens,
                  size_t total, size_t heads, size_t kvh, size_t hd, float *out) {
  if (!kvh || heads % kvh) { set_err("attention: groups"); return -1; }
  if (tokens > total) { set_err("attention: tokens > total"); return -1; }
  size_t wq = heads * hd, wkv = kvh * hd, per = heads / kvh, off = total - tokens;
  float scale = 1.0f / sqrtf((float)hd);
  /* the transposed keys pay off when many query rows read them */
  float *kt = tokens * per >= 32 ? (float *)malloc(total * wkv * sizeof(float)) : NULL;
  if (kt) {
#pragma omp parallel for schedule(static)
    for (size_t c0 = 0; c0 < wkv; c0 += 64)
      for (size_t p0 = 0; p0 < total; p0 += 64)
        for (size_t p = p0; p < p0 + 64 && p < total; p++)
          for (size_t c = c0; c < c0 + 64 && c < wkv; c++) kt[c * total + p] = k[p * wkv + c];
  }
  int err = 0;
#pragma omp parallel for schedule(dynamic)
  for (size_t th = 0; th < tokens * heads; th++) {
    const size_t t = th / heads, h = th % heads;
    size_t vis = off + t + 1;
    float *pts = (float *)malloc((vis + 16) * sizeof(float));
    if (!pts) { err = 1; continue; }
    {
      const float *qh = q + t * wq + h * hd;
      size_t base = (h / per) * hd;
      size_t p = 0;
      if (kt) {
        const float *kg = kt + base * total;
        for (; p + 16 <= vis; p += 16) scores16(qh, kg, total, hd, p, scale, pts);
        for (; p < vis; p++) {
          float s = 0.0f;
          for (size_t d = 0; d < hd; d++) s += qh[d] * kg[d * total + p];
          pts[p] = s * scale;
        }
      } else {
        for (; p + 8 <= vis; p += 8) {
          float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
          const float *kp = k + p * wkv + base;
          for (size_t d = 0; d < hd; d++)
            for (int j = 0; j < 8; j++) s[j] += qh[d] * kp[(size_t)j * wkv + d];
          for (int j = 0; j < 8; j++) pts[p + (size_t)j] = s[j] * scale;
        }
        for (; p < vis; p++) pts[p] = orc_dot_f32(qh, k + p * wkv + base, hd) * scale;
      }
      orc_softmax(pts, vis, vis);
      weighted_sum(pts, v + base, wkv, vis, hd, out + t * wq + h * hd);
    }
    free(pts);
  }
  free(kt);
  if (err) { set_err("attention: alloc"); return -1; }
  return 0;
}

/* A test hook (not the reference's order): the attention of orc_attention
 * with its sums split over chunks of positions, combined as a split-K kernel
 * combines them; the scores are the same sequential dots. */
int orc_attention_split(const float *q, const float *k, const float *v, size_t tokens,
                        size_t total, size_t heads, size_t kvh, size_t hd, size_t chunk,
                        float *out) {
  if (!kvh || heads % kvh || !chunk) { set_err("attention_split: groups or chunk"); return -1; }
  if (tokens > total) { set_err("attention_split: tokens > total"); return -1; }
  const size_t wq = heads * hd, wkv = kvh * hd, per = heads / kvh, off = total - tokens;
  const float scale = 1.0f / sqrtf((float)hd);
  const size_t nch = (total + chunk - 1) / chunk;
  int err = 0;
#pragma omp parallel for schedule(dynamic)
  for (size_t th = 0; th < tokens * heads; th++) {
    const size_t t = th / heads, h = th % heads, vis = off + t + 1, base = (h / per) * hd;
    float *sc = (float *)malloc(vis * 4), *m = (float *)malloc(nch * 4), *l = (float *)malloc(nch * 4);
    float *o = (float *)calloc(nch * hd, 4);
    if (!sc || !m || !l || !o) { err = 1; free(sc); free(m); free(l); free(o); continue; }
    const float *qh = q + t * wq + h * hd;
    for (size_t p = 0; p < vis; p++) sc[p] = orc_dot_f32(qh, k + p * wkv + base, hd) * scale;
    size_t used = 0;
    for (size_t c0 = 0; c0 < vis; c0 += chunk, used++) {
      const size_t c1 = c0 + chunk < vis ? c0 + chunk : vis;
      float mx = -INFINITY, sum = 0.0f;
      for (size_t p = c0; p < c1; p++) mx = fmaxf(mx, sc[p]);
      for (size_t p = c0; p < c1; p++) {
        const float e = expf(sc[p] - mx);
        sum += e;
        for (size_t d = 0; d < hd; d++) o[used * hd + d] += e * v[p * wkv + base + d];
      }
      m[used] = mx;
      l[used] = sum;
    }
    float M = -INFINITY, L = 0.0f;
    for (size_t i = 0; i < used; i++) M = fmaxf(M, m[i]);
    for (size_t i = 0; i < used; i++) L += l[i] * expf(m[i] - M);
    const float inv = 1.0f / L;
    for (size_t d = 0; d < hd; d++) {
      float acc = 0.0f;
      for (size_t i = 0; i < used; i++) acc += o[i * hd + d] * expf(m[i] - M);
      out[t * wq + h * hd + d] = acc * inv;
    }
    free(sc); free(m); free(l); free(o);
  }
  if (err) { set_err("attention_split: alloc"); return -1; }
  return 0;
}

/* ------------------------------------------------------------ matmuls */
#define ROWS_PER_TASK 32 /* ops.rs:43 COLUMNAS_MINIMAS */

typedef struct { int8_t *q; float *e, *s; } act_buf;

static int act_alloc(act_buf *a, size_t m, size_t k, int sub) {
  a->q = (int8_t *)malloc(m * k);
  a->e = (float *)malloc(m * (k / (size_t)sub) * 4);
  a->s = (float *)malloc(m * (k / (size_t)sub) * 4);
  return a->q && a->e && a->s ? 0 : -1;
}
static void act_free(act_buf *a) { free(a->q); free(a->e); free(a->s); }

/* The scalar row kernels above (src/kernels/scalar.rs:132-324,
 * src/kernels/q2k.rs:41-69) restructured for speed, bit for bit:
 * a weight row is unpacked once into its levels (the integers each kernel
 * multiplies the activation by) and two f32 coefficients per sub-block (the
 * same products the kernel forms: d*sc and dmin*mn, or d*scale); then its
 * dots with four activation rows run as four independent chains, each
 * adding its sub-block terms in the kernel's order from 0. The integer
 * sub-block sums are exact in any order. tests/test_oracle_ops.py checks
 * this against the per-row kernels for every type. */
enum { TERM_MIN, TERM_OFF4, TERM_OFF32 };

static int prep_row(int type, const uint8_t *row, size_t nb, uint8_t *q, float *A, float *B) {
  for (size_t bl = 0; bl < nb; bl++) {
    uint8_t *qb = q + bl * 256;
    switch (type) {
    case ORC_Q4_K: case ORC_Q5_K: {
      const size_t bpb = type == ORC_Q4_K ? 144 : 176;
      const uint8_t *o = row + bl * bpb, *esc = o + 4, *qh = o + 16;
      const uint8_t *qs = o + (type == ORC_Q4_K ? 16 : 48);
      const float d = rd_f16(o), dmin = rd_f16(o + 2);
      for (int j = 0; j < 8; j++) {
        uint8_t sc, mn;
        orc_scale_min_k4(j, esc, &sc, &mn);
        A[bl * 8 + j] = d * (float)sc;
        B[bl * 8 + j] = dmin * (float)mn;
        const int pr = j / 2, h = j % 2;
        for (int i = 0; i < 32; i++) {
          int v = h == 0 ? (qs[pr * 32 + i] & 0x0F) : (qs[pr * 32 + i] >> 4);
          if (type == ORC_Q5_K && (qh[i] & (1 << j))) v += 16;
          qb[j * 32 + i] = (uint8_t)v;
        }
      }
      break;
    }
    case ORC_Q3_K: {
      const uint8_t *o = row + bl * 110, *hm = o, *qs = o + 32;
      const float d = rd_f16(o + 108);
      int8_t esc[16];
      orc_scales_q3k(o, esc);
      for (int g = 0; g < 8; g++) {
        const uint8_t *qsg = qs + (g / 4) * 32;
        const int sh = 2 * (g % 4);
        const uint8_t m = (uint8_t)(1u << g);
        for (int half = 0; half < 2; half++) A[bl * 16 + g * 2 + half] = d * ((float)esc[g * 2 + half] - 32.0f);
        for (int idx = 0; idx < 32; idx++)
          qb[g * 32 + idx] = (uint8_t)(((qsg[idx] >> sh) & 3) + ((hm[idx] & m) ? 4 : 0));
      }
      break;
    }
    case ORC_Q2_K: {
      const uint8_t *o = row + bl * 84, *esc = o, *qs = o + 16;
      const float d = rd_f16(o + 80), dm = rd_f16(o + 82);
      for (int s = 0; s < 16; s++) {
        A[bl * 16 + s] = d * (float)(esc[s] & 0xF);
        B[bl * 16 + s] = dm * (float)(esc[s] >> 4);
      }
      for (int g = 0; g < 8; g++)
        for (int idx = 0; idx < 32; idx++)
          qb[g * 32 + idx] = (uint8_t)((qs[(g / 4) * 32 + idx] >> (2 * (g % 4))) & 3);
      break;
    }
    case ORC_Q6_K: {
      const uint8_t *o = row + bl * 210, *esc = o + 192;
      const float d = rd_f16(o + 208);
      for (int s = 0; s < 16; s++) A[bl * 16 + s] = d * (float)(int8_t)esc[s];
      for (int g = 0; g < 8; g++) {
        const int half = g / 4, gi = g % 4;
        const uint8_t *ql = o + 64 * half + 32 * (gi % 2), *qh = o + 128 + 32 * half;
        for (int i = 0; i < 32; i++) {
          const int nib = gi < 2 ? (ql[i] & 0x0F) : (ql[i] >> 4);
          qb[g * 32 + i] = (uint8_t)(nib | (((qh[i] >> (2 * gi)) & 3) << 4));
        }
      }
      break;
    }
    default:
      return -1;
    }
  }
  return 0;
}

/* Up to four activation rows against one prepared weight row: SUB values
 * per sub-block, TERM the kernel's term:
 *   TERM_MIN   xe * (A*E - B*xs)     (Q4_K, Q5_K, Q2_K)
 *   TERM_OFF4  (xe*A) * (E - 4*xs)   (Q3_K)
 *   TERM_OFF32 (xe*A) * (E - 32*xs)  (Q6_K) */
/* the exact integer sum of one sub-block: levels (0..63) times i8 values,
 * pairwise in 16 bits (at most 2 * 63 * 128, no saturation), then 32 bits */
static inline int32_t isum32(const uint8_t *q, const int8_t *x) {
  const __m256i p = _mm256_maddubs_epi16(_mm256_loadu_si256((const __m256i *)q),
                                         _mm256_loadu_si256((const __m256i *)x));
  const __m256i w = _mm256_madd_epi16(p, _mm256_set1_epi16(1));
  __m128i v = _mm_add_epi32(_mm256_castsi256_si128(w), _mm256_extracti128_si256(w, 1));
  v = _mm_add_epi32(v, _mm_shuffle_epi32(v, 0x4E));
  v = _mm_add_epi32(v, _mm_shuffle_epi32(v, 0xB1));
  return _mm_cvtsi128_si32(v);
}
static inline int32_t isum16(const uint8_t *q, const int8_t *x) {
  const __m128i p = _mm_maddubs_epi16(_mm_loadu_si128((const __m128i *)q),
                                      _mm_loadu_si128((const __m128i *)x));
  __m128i v = _mm_madd_epi16(p, _mm_set1_epi16(1));
  v = _mm_add_epi32(v, _mm_shuffle_epi32(v, 0x4E));
  v = _mm_add_epi32(v, _mm_shuffle_epi32(v, 0xB1));
  return _mm_cvtsi128_si32(v);
}

#define DOT_ROWS(NAME, SUB, TERM)                                                              \
  static void NAME(size_t ns, const uint8_t *q, const float *A, const float *B,              \
                   const int8_t *const *x, const float *const *xe, const float *const *xs,   \
                   int nr, float *out) {                                                      \
    float t0 = 0.0f, t1 = 0.0f, t2 = 0.0f, t3 = 0.0f;                                         \
    for (size_t s = 0; s < ns; s++) {                                                         \
      const uint8_t *qs = q + s * SUB;                                                        \
      float tm[4];                                                                            \
      for (int r = 0; r < 4; r++) {                                                           \
        const int8_t *xr = x[r < nr ? r : 0] + s * SUB;                                       \
        const int32_t e = SUB == 32 ? isum32(qs, xr) : isum16(qs, xr);                        \
        const float E = (float)e, ve = xe[r < nr ? r : 0][s], vs = xs[r < nr ? r : 0][s];     \
        if (TERM == TERM_MIN) tm[r] = ve * (A[s] * E - B[s] * vs);                            \
        else if (TERM == TERM_OFF4) tm[r] = ve * A[s] * (E - 4.0f * vs);                      \
        else tm[r] = ve * A[s] * (E - 32.0f * vs);                                            \
      }                                                                                       \
      t0 += tm[0];                                                                            \
      t1 += tm[1];                                                                            \
      t2 += tm[2];                                                                            \
      t3 += tm[3];                                                                            \
    }                                                                                         \
    const float t[4] = {t0, t1, t2, t3};                                                      \
    for (int r = 0; r < nr; r++) out[r] = t[r];                                               \
  }
DOT_ROWS(dot_rows_min32, 32, TERM_MIN)
DOT_ROWS(dot_rows_min16, 16, TERM_MIN)
DOT_ROWS(dot_rows_off4, 16, TERM_OFF4)
DOT_ROWS(dot_rows_off32, 16, TERM_OFF32)

/* one activation row (decode): a single chain */
#define DOT_ROW(NAME, SUB, TERM)                                                               \
  static float NAME(size_t ns, const uint8_t *q, const float *A, const float *B,             \
                    const int8_t *x, const float *xe, const float *xs) {                      \
    float t = 0.0f;                                                                           \
    for (size_t s = 0; s < ns; s++) {                                                         \
      const int32_t e = SUB == 32 ? isum32(q + s * SUB, x + s * SUB)                          \
                                  : isum16(q + s * SUB, x + s * SUB);                         \
      const float E = (float)e;                                                               \
      if (TERM == TERM_MIN) t += xe[s] * (A[s] * E - B[s] * xs[s]);                           \
      else if (TERM == TERM_OFF4) t += xe[s] * A[s] * (E - 4.0f * xs[s]);                     \
      else t += xe[s] * A[s] * (E - 32.0f * xs[s]);                                           \
    }                                                                                         \
    return t;                                                                                 \
  }
DOT_ROW(dot_row_min32, 32, TERM_MIN)
DOT_ROW(dot_row_min16, 16, TERM_MIN)
DOT_ROW(dot_row_off4, 16, TERM_OFF4)
DOT_ROW(dot_row_off32, 16, TERM_OFF32)

typedef void (*dot_rows_fn)(size_t, const uint8_t *, const float *, const float *,
                            const int8_t *const *, const float *const *, const float *const *,
                            int, float *);
typedef float (*dot_row_fn)(size_t, const uint8_t *, const float *, const float *,
                            const int8_t *, const float *, const float *);
static dot_rows_fn dot_rows_for(int type, dot_row_fn *one) {
  switch (type) {
  case ORC_Q4_K: case ORC_Q5_K: *one = dot_row_min32; return dot_rows_min32;
  case ORC_Q2_K: *one = dot_row_min16; return dot_rows_min16;
  case ORC_Q3_K: *one = dot_row_off4; return dot_rows_off4;
  case ORC_Q6_K: *one = dot_row_off32; return dot_rows_off32;
  default: return NULL;
  }
}

/* src/ops.rs:435-522 (matmul_i8_fusionado) */
int orc_matmul_fused(size_t m, size_t k, size_t n, const float *lhs,
                     const uint8_t *w, int type, float *dst, orc_row_kernel kern,
                     int threads, int prefetch) {
  int sub = orc_sub_block(type);
  size_t bpb = orc_bytes_per_block(type);
  if (!kern) kern = orc_row_kernel_for(type);
  if (!kern || !sub || k % 256) { set_err("matmul_fused: type/k"); return -1; }
  size_t nsub = k / (size_t)sub, rowb = k / 256 * bpb, nb = k / 256;
  act_buf a;
  if (act_alloc(&a, m, k, sub)) { act_free(&a); set_err("alloc"); return -1; }
  for (size_t f = 0; f < m; f++)
    orc_quantize_act(lhs + f * k, k, sub, a.q + f * k, a.e + f * nsub, a.s + f * nsub);
  size_t tasks = (n + ROWS_PER_TASK - 1) / ROWS_PER_TASK;
  if (threads < 1) threads = 1;
  /* the oracle's own kernel: the restructured form (same bits) */
  dot_row_fn row1 = NULL;
  dot_rows_fn rows4 = kern == orc_row_kernel_for(type) ? dot_rows_for(type, &row1) : NULL;
  int err = 0;
#pragma omp parallel for schedule(dynamic) num_threads(threads)
  for (size_t t = 0; t < tasks; t++) {
    size_t r0 = t * ROWS_PER_TASK, r1 = r0 + ROWS_PER_TASK;
    if (r1 > n) r1 = n;
    if (rows4) {
      /* the task's rows prepared once; each group of four activation rows
       * then meets all of them while it sits in cache */
      const size_t nr_w = r1 - r0;
      uint8_t *q = (uint8_t *)malloc(nr_w * k);
      float *A = (float *)malloc(nr_w * nsub * 4), *B = (float *)malloc(nr_w * nsub * 4);
      if (!q || !A || !B) {
        err = 1;
      } else {
        for (size_t r = 0; r < nr_w && !err; r++)
          if (prep_row(type, w + (r0 + r) * rowb, nb, q + r * k, A + r * nsub, B + r * nsub)) err = 1;
        for (size_t f = 0; f < m && !err; f += 4) {
          const int nr = m - f < 4 ? (int)(m - f) : 4;
          const int8_t *xr[4];
          const float *er[4], *sr[4];
          for (int i = 0; i < 4; i++) {
            const size_t g = f + (size_t)(i < nr ? i : 0);
            xr[i] = a.q + g * k;
            er[i] = a.e + g * nsub;
            sr[i] = a.s + g * nsub;
          }
          for (size_t r = 0; r < nr_w; r++) {
            if (nr == 1) {
              dst[f * n + r0 + r] = row1(nsub, q + r * k, A + r * nsub, B + r * nsub, xr[0], er[0], sr[0]);
              continue;
            }
            float out[4];
            rows4(nsub, q + r * k, A + r * nsub, B + r * nsub, xr, er, sr, nr, out);
            for (int i = 0; i < nr; i++) dst[(f + (size_t)i) * n + r0 + r] = out[i];
          }
        }
      }
      free(q); free(A); free(B);
      continue;
    }
    for (size_t r = r0; r < r1; r++) {
      const uint8_t *row = w + r * rowb;
      if (prefetch > 0 && r + (size_t)prefetch < r1) {
        const uint8_t *nx = row + (size_t)prefetch * rowb;
        for (size_t o = 0; o < rowb; o += 64) __builtin_prefetch(nx + o, 0, 3);
      }
      for (size_t f = 0; f < m; f++)
        dst[f * n + r] = kern(row, a.q + f * k, a.e + f * nsub, a.s + f * nsub, nb);
    }
  }
  act_free(&a);
  if (err) { set_err("matmul_fused: alloc"); return -1; }
  return 0;
}

/* src/kernels/scalar.rs:95-109 (dot_i8_escalado): per block of `block`
 * values the exact i32 dot, then total += (esc_a * esc_b) * (f32)dot, in
 * block order from 0 */
float orc_dot_i8_scaled(const int8_t *a, const int8_t *b, const float *esc_a,
                        const float *esc_b, size_t n, int block) {
  float total = 0.0f;
  for (size_t i = 0, r = 0; r < n; i++, r += (size_t)block) {
    size_t to = r + (size_t)block < n ? r + (size_t)block : n;
    int32_t part = 0;
    for (size_t j = r; j < to; j++) part += (int32_t)a[j] * (int32_t)b[j];
    total += esc_a[i] * esc_b[i] * (float)part;
  }
  return total;
}

/* One weight row of the buffer path (src/ops.rs:377-407, 968-993): unpack
 * the row to (q, scale, offset) per sub-block, the scaled dot, then the
 * offset term when the format has one. A row that does not unpack is left
 * at 0. */
static float direct_row(int type, const uint8_t *row, size_t k, int sub, const int8_t *xq,
                        const float *xe, const float *xs, int8_t *cq, float *ce, float *cd) {
  if (orc_unpack_i8(type, row, k, cq, ce, cd) < 0) return 0.0f;
  size_t nsub = k / (size_t)sub;
  float total = orc_dot_i8_scaled(cq, xq, ce, xe, k, sub);
  int has_off = 0;
  for (size_t b = 0; b < nsub; b++) has_off |= cd[b] != 0.0f;
  if (has_off)
    for (size_t b = 0; b < nsub; b++) total += cd[b] * xe[b] * xs[b];
  return total;
}

/* src/ops.rs:310-414 (matmul_i8_directo): every format with an i8 unpack
 * (Q8_0, Q5_0 and the k-quants); the path matmul_auto takes for Q8_0/Q5_0
 * below its blocked threshold (src/ops.rs:1072-1092) */
int orc_matmul_direct(size_t m, size_t k, size_t n, const float *lhs, const uint8_t *w,
                      int type, float *dst, int threads) {
  int sub = orc_sub_block(type);
  size_t vpb = orc_values_per_block(type), bpb = orc_bytes_per_block(type);
  if (!sub || !vpb) { set_err("matmul_direct: type has no i8 unpack"); return -1; }
  if (k % vpb || k % (size_t)sub) { set_err("matmul_direct: a row is not whole blocks"); return -1; }
  size_t nsub = k / (size_t)sub, rowb = k / vpb * bpb;
  act_buf a;
  if (act_alloc(&a, m, k, sub)) { act_free(&a); set_err("alloc"); return -1; }
  for (size_t f = 0; f < m; f++)
    orc_quantize_act(lhs + f * k, k, sub, a.q + f * k, a.e + f * nsub, a.s + f * nsub);
  size_t tasks = (n + ROWS_PER_TASK - 1) / ROWS_PER_TASK;
  int err = 0;
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(dynamic) num_threads(threads)
  for (size_t t = 0; t < tasks; t++) {
    int8_t *cq = (int8_t *)malloc(k);
    float *ce = (float *)malloc(nsub * 4), *cd = (float *)malloc(nsub * 4);
    if (!cq || !ce || !cd) {
      err = 1;
    } else {
      size_t r0 = t * ROWS_PER_TASK, r1 = r0 + ROWS_PER_TASK;
      if (r1 > n) r1 = n;
      for (size_t r = r0; r < r1; r++)
        for (size_t f = 0; f < m; f++)
          dst[f * n + r] = direct_row(type, w + r * rowb, k, sub, a.q + f * k, a.e + f * nsub,
                                      a.s + f * nsub, cq, ce, cd);
    }
    free(cq); free(ce); free(cd);
  }
  act_free(&a);
  if (err) { set_err("matmul_direct: alloc"); return -1; }
  return 0;
}

/* src/ops.rs:895-1009 (matmul_varias_una_fila) — one activation quantization
 * per sub size, then every 32-row task of every matrix in one region: the
 * fused row kernel where the format has one (src/ops.rs:950-966), the
 * buffer path otherwise (968-993). */
int orc_matmul_multi_1row(const float *x, size_t k, size_t count,
                          const uint8_t *const *ws, const int *types,
                          const size_t *ns, float *const *dsts, int threads) {
  act_buf a16 = {0}, a32 = {0};
  int need16 = 0, need32 = 0;
  for (size_t i = 0; i < count; i++) {
    int s = orc_sub_block(types[i]);
    size_t vpb = orc_values_per_block(types[i]);
    if (!s || !vpb) { set_err("multi: type"); return -1; }
    if (k % vpb || k % (size_t)s) { set_err("multi: a row is not whole blocks"); return -1; }
    if (s == 16) need16 = 1; else need32 = 1;
  }
  if (need16) { act_alloc(&a16, 1, k, 16); orc_quantize_act(x, k, 16, a16.q, a16.e, a16.s); }
  if (need32) { act_alloc(&a32, 1, k, 32); orc_quantize_act(x, k, 32, a32.q, a32.e, a32.s); }
  size_t total_tasks = 0;
  for (size_t i = 0; i < count; i++) total_tasks += (ns[i] + ROWS_PER_TASK - 1) / ROWS_PER_TASK;
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(dynamic) num_threads(threads)
  for (size_t t = 0; t < total_tasks; t++) {
    size_t i = 0, tt = t;
    while (tt >= (ns[i] + ROWS_PER_TASK - 1) / ROWS_PER_TASK) {
      tt -= (ns[i] + ROWS_PER_TASK - 1) / ROWS_PER_TASK;
      i++;
    }
    const int sub = orc_sub_block(types[i]);
    const act_buf *a = sub == 16 ? &a16 : &a32;
    orc_row_kernel kern = k % 256 == 0 ? orc_row_kernel_for(types[i]) : NULL;
    size_t rowb = k / orc_values_per_block(types[i]) * orc_bytes_per_block(types[i]);
    size_t r0 = tt * ROWS_PER_TASK, r1 = r0 + ROWS_PER_TASK;
    if (r1 > ns[i]) r1 = ns[i];
    if (kern) {
      for (size_t r = r0; r < r1; r++) dsts[i][r] = kern(ws[i] + r * rowb, a->q, a->e, a->s, k / 256);
      continue;
    }
    size_t nsub = k / (size_t)sub;
    int8_t *cq = (int8_t *)malloc(k);
    float *ce = (float *)malloc(nsub * 4), *cd = (float *)malloc(nsub * 4);
    if (cq && ce && cd)
      for (size_t r = r0; r < r1; r++)
        dsts[i][r] = direct_row(types[i], ws[i] + r * rowb, k, sub, a->q, a->e, a->s, cq, ce, cd);
    free(cq); free(ce); free(cd);
  }
  if (need16) act_free(&a16);
  if (need32) act_free(&a32);
  return 0;
}

/* ------------------------------------------------------------- forward */
int orc_model_init(orc_model *m, const orc_config *cfg, const float *embd,
                   const float *out_norm, const uint8_t *out, int t_out,
                   const orc_layer *layers, int threads) {
  memset(m, 0, sizeof *m);
  m->cfg = *cfg;
  m->embd = embd;
  m->out_norm = out_norm;
  m->out = out;
  m->t_out = t_out;
  m->layers = layers;
  m->threads = threads < 1 ? 1 : threads;
  size_t hd = cfg->dim / cfg->heads;
  m->cos_t = (float *)malloc(cfg->ctx * (hd / 2) * 4);
  m->sin_t = (float *)malloc(cfg->ctx * (hd / 2) * 4);
  if (!m->cos_t || !m->sin_t) { set_err("alloc"); return -1; }
  orc_rope_tables(hd, cfg->rope_base, cfg->ctx, m->cos_t, m->sin_t);
  return 0;
}
void orc_model_release(orc_model *m) { free(m->cos_t); free(m->sin_t); }

int orc_cache_init(orc_cache *c, const orc_config *cfg, size_t cap) {
  size_t kvd = cfg->kv_heads * (cfg->dim / cfg->heads);
  c->len = 0;
  c->cap = cap;
  c->k = (float **)calloc(cfg->layers, sizeof(float *));
  c->v = (float **)calloc(cfg->layers, sizeof(float *));
  if (!c->k || !c->v) return -1;
  for (size_t i = 0; i < cfg->layers; i++) {
    c->k[i] = (float *)malloc(cap * kvd * 4);
    c->v[i] = (float *)malloc(cap * kvd * 4);
    if (!c->k[i] || !c->v[i]) return -1;
  }
  return 0;
}
void orc_cache_release(orc_cache *c, const orc_config *cfg) {
  for (size_t i = 0; i < cfg->layers; i++) { free(c->k[i]); free(c->v[i]); }
  free(c->k);
  free(c->v);
}
/* src/forward.rs:98-110 */
void orc_cache_truncate(orc_cache *c, size_t n) { if (n < c->len) c->len = n; }

/* src/ops.rs:87-156 (ops::matmul), the path matmul_auto takes for F32 and
 * F16 weights (src/ops.rs:1064-1071): each weight row widened to f32
 * (descuantizar), then kernels::dot with every lhs row (spec
 * src/kernels/scalar.rs:16-23, the sum in order from 0) */
static int matmul_widened(size_t m, size_t k, size_t n, const float *lhs, const uint8_t *w,
                          int type, float *dst, int threads) {
  const size_t rowb = k * orc_bytes_per_block(type);
  int err = 0;
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(dynamic) num_threads(threads)
  for (size_t r = 0; r < n; r++) {
    float *col = (float *)malloc(k * 4);
    if (!col || orc_dequantize(type, w + r * rowb, col, k) < 0) {
      err = 1;
    } else {
      for (size_t f = 0; f < m; f++) dst[f * n + r] = orc_dot_f32(lhs + f * k, col, k);
    }
    free(col);
  }
  if (err) { set_err("matmul_widened: alloc or dequantize"); return -1; }
  return 0;
}

static int proj(const orc_model *M, const float *x, size_t t, size_t k, size_t n,
                const uint8_t *w, int type, const float *bias, float *dst) {
  orc_row_kernel kern = M->kern_override && type == ORC_Q4_K ? M->kern_override : NULL;
  /* matmul_auto (src/ops.rs:1056-1093): the f32 path for F32/F16 weights,
   * the fused row kernel for the k-quants, the buffer path for Q8_0/Q5_0 */
  if (type == ORC_F32 || type == ORC_F16) {
    if (matmul_widened(t, k, n, x, w, type, dst, M->threads)) return -1;
  } else if (orc_row_kernel_for(type) && k % 256 == 0) {
    if (orc_matmul_fused(t, k, n, x, w, type, dst, kern, M->threads, 2)) return -1;
  } else if (orc_matmul_direct(t, k, n, x, w, type, dst, M->threads)) {
    return -1;
  }
  if (bias)
    for (size_t r = 0; r < t; r++)
      for (size_t i = 0; i < n; i++) dst[r * n + i] += bias[i];
  return 0;
}

/* src/forward.rs:375-505. Projections use the fused per-row arithmetic for
 * every token count (the reference's blocked prefill path is the same sum in
 * another order, tolerance 1e-4 of the max by ops.rs:1518-1561). */
int orc_forward(const orc_model *M, const uint32_t *toks, size_t t, orc_cache *c,
                float *logits) {
  const orc_config *g = &M->cfg;
  if (!t) { set_err("forward: no tokens"); return -1; }
  size_t total = c->len + t;
  if (total > g->ctx || total > c->cap) { set_err("forward: context"); return -1; }
  size_t D = g->dim, hd = D / g->heads, kvd = g->kv_heads * hd, I = g->ffn;
  float *x = (float *)malloc(t * D * 4), *xn = (float *)malloc(t * D * 4);
  float *q = (float *)malloc(t * D * 4), *kk = (float *)malloc(t * kvd * 4);
  float *vv = (float *)malloc(t * kvd * 4), *att = (float *)malloc(t * D * 4);
  float *pr = (float *)malloc(t * D * 4), *ga = (float *)malloc(t * I * 4);
  float *up = (float *)malloc(t * I * 4);
  int rc = -1;
  if (!x || !xn || !q || !kk || !vv || !att || !pr || !ga || !up) { set_err("alloc"); goto done; }
  for (size_t i = 0; i < t; i++) {
    if (toks[i] >= g->vocab) { set_err("forward: token out of vocab"); goto done; }
    memcpy(x + i * D, M->embd + (size_t)toks[i] * D, D * 4);
  }
  for (size_t li = 0; li < g->layers; li++) {
    const orc_layer *L = &M->layers[li];
    /* Past the last layer's K and V only the last token's row reaches the
     * logits (and every step is a function of its own row), so that layer
     * computes the rest for the last token alone: the same values the
     * reference computes for it. */
    const size_t r0 = li + 1 == g->layers ? t - 1 : 0, tr = t - r0;
    float *xr = x + r0 * D, *xnr = xn + r0 * D, *qr = q + r0 * D;
    for (size_t r = 0; r < t; r++) orc_rmsnorm(xn + r * D, x + r * D, L->attn_norm, D, g->eps);
    if (proj(M, xnr, tr, D, D, L->q, L->t_q, L->q_bias, qr)) goto done;
    if (proj(M, xn, t, D, kvd, L->k, L->t_k, L->k_bias, kk)) goto done;
    if (proj(M, xn, t, D, kvd, L->v, L->t_v, L->v_bias, vv)) goto done;
    if (orc_rope(qr, tr, g->heads, hd, M->cos_t, M->sin_t, g->ctx, c->len + r0)) goto done;
    if (orc_rope(kk, t, g->kv_heads, hd, M->cos_t, M->sin_t, g->ctx, c->len)) goto done;
    memcpy(c->k[li] + c->len * kvd, kk, t * kvd * 4);
    memcpy(c->v[li] + c->len * kvd, vv, t * kvd * 4);
    if (M->attn_chunk
            ? orc_attention_split(qr, c->k[li], c->v[li], tr, total, g->heads, g->kv_heads, hd,
                                  (size_t)M->attn_chunk, att)
            : orc_attention(qr, c->k[li], c->v[li], tr, total, g->heads, g->kv_heads, hd, att))
      goto done;
    if (proj(M, att, tr, D, D, L->o, L->t_o, NULL, pr)) goto done;
    for (size_t i = 0; i < tr * D; i++) xr[i] += pr[i];
    for (size_t r = 0; r < tr; r++) orc_rmsnorm(xnr + r * D, xr + r * D, L->ffn_norm, D, g->eps);
    if (proj(M, xnr, tr, D, I, L->gate, L->t_gate, NULL, ga)) goto done;
    if (proj(M, xnr, tr, D, I, L->up, L->t_up, NULL, up)) goto done;
    orc_silu(ga, ga, tr * I);
    for (size_t i = 0; i < tr * I; i++) ga[i] *= up[i];
    if (proj(M, ga, tr, I, D, L->down, L->t_down, NULL, pr)) goto done;
    for (size_t i = 0; i < tr * D; i++) xr[i] += pr[i];
  }
  orc_rmsnorm(xn, x + (t - 1) * D, M->out_norm, D, g->eps);
  if (proj(M, xn, 1, D, g->vocab, M->out, M->t_out, NULL, logits)) goto done;
  c->len = total;
  rc = 0;
done:
  free(x); free(xn); free(q); free(kk); free(vv); free(att); free(pr); free(ga); free(up);
  return rc;
}

/* src/forward.rs:533-559 with greedy choice (sampler.rs:65-66) and no EOS */
int orc_generate(const orc_model *M, const uint32_t *prompt, size_t n,
                 size_t max_new, orc_cache *c, uint32_t *out, size_t *n_out) {
  float *lg = (float *)malloc(M->cfg.vocab * 4);
  if (!lg) return -1;
  *n_out = 0;
  int rc = orc_forward(M, prompt, n, c, lg);
  for (size_t i = 0; rc == 0 && i < max_new; i++) {
    uint32_t t = orc_argmax(lg, M->cfg.vocab);
    out[(*n_out)++] = t;
    if (c->len >= M->cfg.ctx) break;
    rc = orc_forward(M, &t, 1, c, lg);
  }
  free(lg);
  return rc;
}

/* ------------------------------------------------------------- sampler */
/* src/sampler.rs:38-47 */
void orc_sampler_init(orc_sampler *s, uint64_t seed, float temp, float top_p) {
  orc_azar_seed(&s->azar, seed);
  s->temp = temp;
  /* f32::clamp(0, 1): a NaN passes through */
  s->top_p = top_p < 0.0f ? 0.0f : (top_p > 1.0f ? 1.0f : top_p);
}

/* f32::total_cmp as an unsigned key: larger key, larger value */
static uint32_t total_key(float p) {
  uint32_t b;
  memcpy(&b, &p, 4);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
static const float *g_sort_p; /* qsort has no context argument */
/* descending probability (total_cmp), then ascending index */
static int by_prob_desc(const void *a, const void *b) {
  const uint32_t i = *(const uint32_t *)a, j = *(const uint32_t *)b;
  const uint32_t ki = total_key(g_sort_p[i]), kj = total_key(g_sort_p[j]);
  if (ki != kj) return ki > kj ? -1 : 1;
  return i < j ? -1 : (i > j);
}

/* src/sampler.rs:139-152 */
static uint32_t sample_running(const float *probs, const uint32_t *idx, size_t len,
                               float u) {
  float acc = 0.0f;
  uint32_t last = 0;
  for (size_t k = 0; k < len; k++) {
    const uint32_t t = idx ? idx[k] : (uint32_t)k;
    acc += probs[t];
    last = t;
    if (acc > u) return t;
  }
  return last;
}

/* src/sampler.rs:61-125 */
uint32_t orc_sample(orc_sampler *s, const float *logits, size_t n) {
  if (n == 0) return 0;
  if (s->temp <= 0.0f) return orc_argmax(logits, n);
  const float u = (float)(orc_azar_next(&s->azar) >> 40) / 16777216.0f;
  float *probs = (float *)malloc(n * 4);
  uint32_t *ord = (uint32_t *)malloc(n * 4);
  if (!probs || !ord) {
    free(probs);
    free(ord);
    return 0;
  }
  const float inv = 1.0f / s->temp;
  for (size_t i = 0; i < n; i++) probs[i] = logits[i] * inv;
  orc_softmax(probs, n, n);
  uint32_t tok;
  if (s->top_p >= 1.0f) {
    tok = sample_running(probs, NULL, n, u);
  } else {
    /* the CANDIDATOS = 1024 most probable, sorted (the top k of a total
     * order are the first k of the full sort), their mass, and the full
     * order when they fall short */
    for (size_t i = 0; i < n; i++) ord[i] = (uint32_t)i;
    g_sort_p = probs;
    qsort(ord, n, 4, by_prob_desc);
    const size_t k = n < 1024 ? n : 1024;
    float masa = 0.0f;
    for (size_t i = 0; i < k; i++) masa += probs[ord[i]];
    size_t len = k;
    if (masa < s->top_p && k < n) len = n;
    float acc = 0.0f;
    size_t corte = len;
    for (size_t i = 0; i < len; i++) {
      acc += probs[ord[i]];
      if (acc >= s->top_p) {
        corte = i + 1;
        break;
      }
    }
    float total = 0.0f;
    for (size_t i = 0; i < corte; i++) total += probs[ord[i]];
    tok = sample_running(probs, ord, corte, u * total);
  }
  free(probs);
  free(ord);
  return tok;
}

/* src/forward.rs:533-559 */
int orc_generate_sampled(const orc_model *M, const uint32_t *prompt, size_t n,
                         size_t max_new, orc_sampler *s, uint32_t eos,
                         orc_cache *c, uint32_t *out, size_t *n_out) {
  float *lg = (float *)malloc(M->cfg.vocab * 4);
  if (!lg) return -1;
  *n_out = 0;
  int rc = orc_forward(M, prompt, n, c, lg);
  for (size_t i = 0; rc == 0 && i < max_new; i++) {
    uint32_t t = orc_sample(s, lg, M->cfg.vocab);
    if (t == eos) break;
    out[(*n_out)++] = t;
    if (c->len >= M->cfg.ctx) break;
    rc = orc_forward(M, &t, 1, c, lg);
  }
  free(lg);
  return rc;
}
