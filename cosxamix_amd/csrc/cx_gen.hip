// cx_gen.hip — daiss-style random models made directly in HBM.
//
// Rows: `Azar` xorshift64* seeded per row with semilla_de (src/daiss.rs:317-379),
// Box-Muller pairs (daiss.rs:343-350), one thread per row. The integer stream
// is exact; logf/cosf/sinf are the device library's, so the normals can
// differ from a host run by an ulp (the reference pins them statistically).
//
// Blocks: the reference's k-quant quantizers (src/quant_kquants.rs:22-399)
// with one thread per 256-value block. Given the same f32 input these produce
// the same bytes as the host restatement: every operation is the same IEEE
// f32 operation in the same order (no contraction, correctly rounded
// division and sqrt, round-half-away).
#include "cx_ops.h"

namespace {

__device__ inline int32_t sat_i32(float f) {
  if (f != f) return 0;
  if (f >= 2147483648.0f) return 2147483647;
  if (f <= -2147483648.0f) return (int32_t)0x80000000u;
  return (int32_t)f;
}
__device__ inline int32_t entero(float x) { return sat_i32(roundf(x)); }
__device__ inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// src/quant.rs:38-60
__device__ inline float f16_to_f32(uint16_t bits) {
  uint32_t sign = (uint32_t)(bits >> 15) << 31, e = (bits >> 10) & 0x1F, man = bits & 0x3FF, out;
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
  return __uint_as_float(out);
}
// src/quant.rs:691-731
__device__ inline uint16_t f32_to_f16(float x) {
  const uint32_t bits = __float_as_uint(x);
  const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
  const uint32_t mag = bits & 0x7FFFFFFF;
  if (mag >= 0x7F800000u) return sign | 0x7C00 | ((mag & 0x007FFFFF) ? 0x0200 : 0);
  const int32_t exp = (int32_t)(mag >> 23) - 127;
  if (exp > 15) return sign | 0x7C00;
  if (exp < -14) {
    const uint32_t sh = (uint32_t)(-14 - exp);
    if (sh > 24) return sign;
    // shift amounts wrap mod 32 like a Rust release build (|x| in [2^-38, 2^-32))
    const uint32_t man = (mag & 0x007FFFFF) | 0x00800000;
    const uint32_t val = man >> ((sh + 13) & 31), rest = man & ((1u << ((sh + 13) & 31)) - 1);
    const uint32_t half = 1u << ((sh + 12) & 31);
    return sign | (uint16_t)(val + ((rest > half || (rest == half && (val & 1))) ? 1 : 0));
  }
  const uint32_t man = mag & 0x007FFFFF;
  const uint32_t val = ((uint32_t)(exp + 15) << 10) | (man >> 13), rest = man & 0x1FFF;
  return sign | (uint16_t)(val + ((rest > 0x1000 || (rest == 0x1000 && (val & 1))) ? 1 : 0));
}
__device__ inline void put16(uint8_t* o, uint16_t h) {
  o[0] = (uint8_t)h;
  o[1] = (uint8_t)(h >> 8);
}

// --------------------------------------------------------------- rows
__global__ void k_gen_rows(float* out, uint64_t name_hash, uint64_t seed, uint32_t rows,
                           uint32_t width, float sigma) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  // semilla_de: FNV-1a of the name (host), then the row, then the model seed
  uint64_t h = name_hash ^ (uint64_t)r;
  h *= 0x00000100000001B3ull;
  uint64_t st = h ^ ((seed << 17) | (seed >> 47));
  if (st == 0) st = 0x9E3779B97F4A7C15ull;
  float* row = out + (size_t)r * width;
  auto uni = [&]() {
    uint64_t x = st;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    st = x;
    const uint64_t bits = (x * 0x2545F4914F6CDD1Dull) >> 40;
    return ((float)bits + 1.0f) / 16777216.0f;
  };
  for (uint32_t i = 0; i < width; i += 2) {
    const float u1 = uni(), u2 = uni();
    const float rr = sigma * sqrtf(-2.0f * logf(u1));
    const float a = 6.28318530717958647692f * u2;
    row[i] = rr * cosf(a);
    if (i + 1 < width) row[i + 1] = rr * sinf(a);
  }
}

__global__ void k_fill(float* out, size_t n, float v) {
  for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) out[i] = v;
}

// --------------------------------------------------------- quantizers
// quant_kquants.rs:29-84
__device__ float quants_q3(const float* x, int nmax, int8_t* l) {
  float big = 0.0f, amax = 0.0f;
  for (int i = 0; i < 16; i++)
    if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); big = x[i]; }
  if (amax < 1e-15f) {
    for (int i = 0; i < 16; i++) l[i] = 0;
    return 0.0f;
  }
  const float iscale = -(float)nmax / big;
  float sumlx = 0.0f, suml2 = 0.0f;
  for (int i = 0; i < 16; i++) {
    l[i] = (int8_t)clampi(entero(iscale * x[i]), -nmax, nmax - 1);
    const float w = x[i] * x[i];
    sumlx += w * x[i] * (float)l[i];
    suml2 += w * (float)(l[i] * l[i]);
  }
  for (int it = 0; it < 5; it++) {
    int changes = 0;
    for (int i = 0; i < 16; i++) {
      const float w = x[i] * x[i], cur = (float)l[i];
      float slx = sumlx - w * x[i] * cur;
      if (slx > 0.0f) {
        float sl2 = suml2 - w * cur * cur;
        const int32_t nw = clampi(entero(x[i] * sl2 / slx), -nmax, nmax - 1);
        if (nw != l[i]) {
          slx += w * x[i] * (float)nw;
          sl2 += w * (float)(nw * nw);
          if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
            l[i] = (int8_t)nw;
            sumlx = slx;
            suml2 = sl2;
            changes++;
          }
        }
      }
    }
    if (!changes) break;
  }
  for (int i = 0; i < 16; i++) l[i] = (int8_t)(l[i] + nmax);
  return suml2 > 0.0f ? sumlx / suml2 : 0.0f;
}

struct Search { int nmax; float from, step; int steps; bool absolute; };
__device__ inline float err_of(float d, bool a) { return a ? fabsf(d) : d * d; }

// quant_kquants.rs:99-157; returns the scale, *neg_min = -min
__device__ float quants_qkx(const float* x, const float* w, int n, int8_t* l, int8_t* aux,
                            const Search& b, float* neg_min) {
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
  float iscale = (float)b.nmax / (mx - mn);
  float scale = 1.0f / iscale;
  float best = 0.0f;
  for (int i = 0; i < n; i++) {
    l[i] = (int8_t)clampi(entero(iscale * (x[i] - mn)), 0, b.nmax);
    best += w[i] * err_of(scale * (float)l[i] + mn - x[i], b.absolute);
  }
  for (int k = 0; k <= b.steps; k++) {
    iscale = (b.from + b.step * (float)k + (float)b.nmax) / (mx - mn);
    float sl = 0.0f, sl2 = 0.0f, sxl = 0.0f;
    for (int i = 0; i < n; i++) {
      aux[i] = (int8_t)clampi(entero(iscale * (x[i] - mn)), 0, b.nmax);
      const float lf = (float)aux[i], wl = w[i] * lf;
      sl += wl;
      sl2 += wl * lf;
      sxl += wl * x[i];
    }
    const float D = sum_w * sl2 - sl * sl;
    if (D > 0.0f) {
      float ts = (sum_w * sxl - sum_x * sl) / D;
      float tm = (sl2 * sum_x - sl * sxl) / D;
      if (tm > 0.0f) {
        tm = 0.0f;
        ts = sxl / sl2;
      }
      float e = 0.0f;
      for (int i = 0; i < n; i++) e += w[i] * err_of(ts * (float)aux[i] + tm - x[i], b.absolute);
      if (e < best) {
        for (int i = 0; i < n; i++) l[i] = aux[i];
        best = e;
        scale = ts;
        mn = tm;
      }
    }
  }
  *neg_min = -mn;
  return scale;
}

// quant_kquants.rs:160-228
__device__ void block_q3k(const float* x, uint8_t* out) {
  int8_t l[256];
  float scales[16], big = 0.0f, amax = 0.0f;
  for (int j = 0; j < 16; j++) {
    scales[j] = quants_q3(x + j * 16, 4, l + j * 16);
    if (fabsf(scales[j]) > amax) { amax = fabsf(scales[j]); big = scales[j]; }
  }
  uint8_t hmask[32], qs[64], packed[12];
  for (int i = 0; i < 32; i++) hmask[i] = 0;
  for (int i = 0; i < 64; i++) qs[i] = 0;
  for (int i = 0; i < 12; i++) packed[i] = 0;
  uint16_t dstore;
  if (amax < 1e-15f) {
    dstore = 0;
    for (int i = 0; i < 256; i++) l[i] = 4;
  } else {
    const float iscale = -32.0f / big;
    dstore = f32_to_f16(1.0f / iscale);
    const float d = f16_to_f32(dstore);
    for (int j = 0; j < 16; j++) {
      const int32_t e = clampi(entero(iscale * scales[j]), -32, 31);
      const float sc = d * (float)e;
      if (sc != 0.0f) {
        const float inv = 1.0f / sc;
        for (int i = 0; i < 16; i++) l[j * 16 + i] = (int8_t)(clampi(entero(x[j * 16 + i] * inv), -4, 3) + 4);
      } else {
        for (int i = 0; i < 16; i++) l[j * 16 + i] = 4;
      }
      const uint8_t u = (uint8_t)(e + 32);
      if (j < 8) packed[j] |= u & 0xF;
      else packed[j - 8] |= (uint8_t)((u & 0xF) << 4);
      packed[8 + j % 4] |= (uint8_t)((u >> 4) << (2 * (j / 4)));
    }
  }
  for (int idx = 0; idx < 256; idx++) {
    const uint8_t val = (uint8_t)l[idx];
    const int half = idx / 128, round = (idx % 128) / 32, place = idx % 32;
    qs[half * 32 + place] |= (uint8_t)((val & 3) << (round * 2));
    if (val & 4) hmask[place] |= (uint8_t)(1 << (half * 4 + round));
  }
  for (int i = 0; i < 32; i++) out[i] = hmask[i];
  for (int i = 0; i < 64; i++) out[32 + i] = qs[i];
  for (int i = 0; i < 12; i++) out[96 + i] = packed[i];
  put16(out + 108, dstore);
}

// quant_kquants.rs:231-291
__device__ void block_q2k(const float* x, uint8_t* out) {
  int8_t l[256], aux[16];
  float w[16], scales[16], mins[16], max_sc = 0.0f, max_mn = 0.0f;
  const Search s{3, -0.5f, 0.1f, 15, true};
  for (int j = 0; j < 16; j++) {
    const float* sub = x + j * 16;
    for (int i = 0; i < 16; i++) w[i] = fabsf(sub[i]);
    float m;
    scales[j] = quants_qkx(sub, w, 16, l + j * 16, aux, s, &m);
    mins[j] = m;
    max_sc = fmaxf(max_sc, scales[j]);
    max_mn = fmaxf(max_mn, mins[j]);
  }
  const float inv_sc = max_sc > 0.0f ? 15.0f / max_sc : 0.0f;
  const float inv_mn = max_mn > 0.0f ? 15.0f / max_mn : 0.0f;
  const uint16_t dstore = f32_to_f16(max_sc > 0.0f ? 1.0f / inv_sc : 0.0f);
  const uint16_t mstore = f32_to_f16(max_mn > 0.0f ? 1.0f / inv_mn : 0.0f);
  const float d = f16_to_f32(dstore), dm = f16_to_f32(mstore);
  uint8_t qs[64];
  for (int i = 0; i < 64; i++) qs[i] = 0;
  for (int j = 0; j < 16; j++) {
    const int32_t le = clampi(entero(inv_sc * scales[j]), 0, 15);
    const int32_t lm = clampi(entero(inv_mn * mins[j]), 0, 15);
    out[j] = (uint8_t)(le | (lm << 4));
    const float dl = d * (float)le, ml = dm * (float)lm;
    for (int i = 0; i < 16; i++)
      l[j * 16 + i] = (int8_t)(dl > 0.0f ? clampi(entero((x[j * 16 + i] + ml) / dl), 0, 3) : 0);
  }
  for (int idx = 0; idx < 256; idx++) {
    const int half = idx / 128, round = (idx % 128) / 32;
    qs[half * 32 + idx % 32] |= (uint8_t)((uint8_t)l[idx] << (round * 2));
  }
  for (int i = 0; i < 64; i++) out[16 + i] = qs[i];
  put16(out + 80, dstore);
  put16(out + 82, mstore);
}

// quant_kquants.rs:295-348; l[8*32]
__device__ void subblocks_32(const float* x, const Search& b, uint16_t* dstore, uint16_t* mstore,
                             uint8_t* packed, int8_t* l) {
  int8_t aux[32];
  float w[32], scales[8], mins[8], max_sc = 0.0f, max_mn = 0.0f, ss = 0.0f;
  for (int i = 0; i < 256; i++) ss += x[i] * x[i];
  const float mean = sqrtf(ss / 256.0f);
  for (int j = 0; j < 8; j++) {
    const float* sub = x + j * 32;
    for (int i = 0; i < 32; i++) w[i] = mean + fabsf(sub[i]);
    float m;
    scales[j] = quants_qkx(sub, w, 32, l + j * 32, aux, b, &m);
    mins[j] = m;
    max_sc = fmaxf(max_sc, scales[j]);
    max_mn = fmaxf(max_mn, mins[j]);
  }
  const float inv_sc = max_sc > 0.0f ? 63.0f / max_sc : 0.0f;
  const float inv_mn = max_mn > 0.0f ? 63.0f / max_mn : 0.0f;
  *dstore = f32_to_f16(max_sc > 0.0f ? 1.0f / inv_sc : 0.0f);
  *mstore = f32_to_f16(max_mn > 0.0f ? 1.0f / inv_mn : 0.0f);
  const float d = f16_to_f32(*dstore), dm = f16_to_f32(*mstore);
  for (int i = 0; i < 12; i++) packed[i] = 0;
  for (int j = 0; j < 8; j++) {
    const uint8_t le = (uint8_t)clampi(entero(inv_sc * scales[j]), 0, 63);
    const uint8_t lm = (uint8_t)clampi(entero(inv_mn * mins[j]), 0, 63);
    if (j < 4) {
      packed[j] |= le;
      packed[j + 4] |= lm;
    } else {
      packed[j + 4] = (uint8_t)((le & 0xF) | ((lm & 0xF) << 4));
      packed[j - 4] |= (uint8_t)((le >> 4) << 6);
      packed[j] |= (uint8_t)((lm >> 4) << 6);
    }
    const float dl = d * (float)le, ml = dm * (float)lm;
    for (int i = 0; i < 32; i++)
      l[j * 32 + i] = (int8_t)(dl > 0.0f ? clampi(entero((x[j * 32 + i] + ml) / dl), 0, b.nmax) : 0);
  }
}

// quant_kquants.rs:351-369
__device__ void block_q4k(const float* x, uint8_t* out) {
  const Search s{15, -1.0f, 0.1f, 20, false};
  uint16_t d, m;
  uint8_t packed[12];
  int8_t l[256];
  subblocks_32(x, s, &d, &m, packed, l);
  put16(out, d);
  put16(out + 2, m);
  for (int i = 0; i < 12; i++) out[4 + i] = packed[i];
  for (int p = 0; p < 4; p++)
    for (int i = 0; i < 32; i++)
      out[16 + p * 32 + i] = (uint8_t)(l[64 * p + i] | (l[64 * p + 32 + i] << 4));
}

// quant_kquants.rs:373-399
__device__ void block_q5k(const float* x, uint8_t* out) {
  const Search s{31, -0.5f, 0.1f, 15, false};
  uint16_t d, m;
  uint8_t packed[12], qh[32];
  int8_t l[256];
  subblocks_32(x, s, &d, &m, packed, l);
  for (int i = 0; i < 32; i++) qh[i] = 0;
  for (int p = 0; p < 4; p++)
    for (int i = 0; i < 32; i++) {
      qh[i] |= (uint8_t)((l[64 * p + i] >> 4) << (2 * p));
      qh[i] |= (uint8_t)((l[64 * p + 32 + i] >> 4) << (2 * p + 1));
    }
  put16(out, d);
  put16(out + 2, m);
  for (int i = 0; i < 12; i++) out[4 + i] = packed[i];
  for (int i = 0; i < 32; i++) out[16 + i] = qh[i];
  for (int p = 0; p < 4; p++)
    for (int i = 0; i < 32; i++)
      out[48 + p * 32 + i] = (uint8_t)((l[64 * p + i] & 0xF) | ((l[64 * p + 32 + i] & 0xF) << 4));
}

template <int T>
__global__ __launch_bounds__(64) void k_quant_blocks(const float* x, size_t nblocks, uint8_t* out) {
  const size_t b = blockIdx.x * 64ull + threadIdx.x;
  if (b >= nblocks) return;
  const float* xb = x + b * 256;
  if (T == CX_Q2_K) block_q2k(xb, out + b * 84);
  if (T == CX_Q3_K) block_q3k(xb, out + b * 110);
  if (T == CX_Q4_K) block_q4k(xb, out + b * 144);
  if (T == CX_Q5_K) block_q5k(xb, out + b * 176);
}

// quant::cuantizar_bloques for Q8_0 (src/quant.rs:765-780), one 32-value
// block a lane: d = max|x| / 127 stored as f16, the quants made with the
// scale as it will be read back, round half away, clamped to [-127, 127]
__global__ __launch_bounds__(64) void k_quant_q8_0(const float* x, size_t nblocks, uint8_t* out) {
  const size_t b = blockIdx.x * 64ull + threadIdx.x;
  if (b >= nblocks) return;
  const float* c = x + b * 32;
  uint8_t* o = out + b * 34;
  float amax = 0.0f;
  for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(c[j]));
  const uint16_t h = f32_to_f16(amax / 127.0f);
  put16(o, h);
  const float read = f16_to_f32(h);
  const float inv = read > 0.0f ? 1.0f / read : 0.0f;
  for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t)(int8_t)clampi(entero(c[j] * inv), -127, 127);
}

}  // namespace

uint64_t cx_fnv_name(const char* name) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (const unsigned char* p = (const unsigned char*)name; *p; p++) {
    h ^= *p;
    h *= 0x00000100000001B3ull;
  }
  return h;
}

int cx_gen_rows_f32(float* out, uint64_t name_hash, uint64_t seed, uint32_t rows, uint32_t width,
                    float sigma, hipStream_t s) {
  if (!rows) return CX_OK;
  hipLaunchKernelGGL(k_gen_rows, dim3((rows + 63) / 64), dim3(64), 0, s, out, name_hash, seed, rows,
                     width, sigma);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_gen_fill(float* out, size_t n, float v, hipStream_t s) {
  if (!n) return CX_OK;
  const unsigned grid = (unsigned)((n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192);
  hipLaunchKernelGGL(k_fill, dim3(grid), dim3(256), 0, s, out, n, v);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_quantize_blocks_dev(int type, const float* x, size_t n, uint8_t* out, hipStream_t s) {
  if (type == CX_Q8_0) {
    CX_REQUIRE(n % 32 == 0, "quantize_blocks: %zu values are not whole blocks of 32", n);
    const size_t nb = n / 32;
    if (!nb) return CX_OK;
    hipLaunchKernelGGL(k_quant_q8_0, dim3((unsigned)((nb + 63) / 64)), dim3(64), 0, s, x, nb, out);
    CX_HIP(hipGetLastError());
    return CX_OK;
  }
  CX_REQUIRE(n % 256 == 0, "quantize_blocks: %zu values are not whole blocks", n);
  const size_t nb = n / 256;
  if (!nb) return CX_OK;
  const dim3 g((unsigned)((nb + 63) / 64));
  switch (type) {
    case CX_Q2_K: hipLaunchKernelGGL(k_quant_blocks<CX_Q2_K>, g, dim3(64), 0, s, x, nb, out); break;
    case CX_Q3_K: hipLaunchKernelGGL(k_quant_blocks<CX_Q3_K>, g, dim3(64), 0, s, x, nb, out); break;
    case CX_Q4_K: hipLaunchKernelGGL(k_quant_blocks<CX_Q4_K>, g, dim3(64), 0, s, x, nb, out); break;
    case CX_Q5_K: hipLaunchKernelGGL(k_quant_blocks<CX_Q5_K>, g, dim3(64), 0, s, x, nb, out); break;
    default: CX_REQUIRE(false, "quantize_blocks: no quantizer for type %d", type);
  }
  CX_HIP(hipGetLastError());
  return CX_OK;
}
