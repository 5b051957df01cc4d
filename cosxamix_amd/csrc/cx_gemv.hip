// cx_gemv.hip — batch-1 k-quant GEMV for gfx950 (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K).
//
// y[r] = sum over super-blocks of row r of the reference's fused dot
// (src/kernels/scalar.rs:132-324, src/kernels/q2k.rs:41-69).
//
// Work split. A super-block (256 values) is handled by 8 consecutive lanes,
// one "slot" each; a wave covers 8 super-blocks per step. A lane loads its
// slice of the block straight from HBM into registers (16-byte loads for
// Q4_K/Q5_K, whose 144/176-byte blocks keep rows 16-byte aligned; dword
// loads for Q2_K; 2-byte-aligned dword loads for Q3_K/Q6_K), unpacks the
// quants and the 6-bit scales in registers, and forms integer partial sums
// with v_dot4c_i32_i8 against the i8 activation held in LDS. The two lanes
// that share a sub-block swap partial sums with one DPP move, so every
// sub-block integer sum E_j is formed exactly. The lane that owns sub-block j
// then computes the reference's f32 term with the reference's rounding:
//   Q4_K/Q5_K/Q2_K : xe[j] * ((d*sc_j)*E_j - (dmin*mn_j)*xs[j])
//   Q3_K           : (xe[j] * (d*(esc_j-32))) * (E'_j - 4*xs[j])
//   Q6_K           : (xe[j] * (d*esc_j)) * (E'_j - 32*xs[j])
// Only the order in which the per-sub-block terms are summed differs from
// the scalar loop (per lane, then a fixed butterfly, then a fixed cross-wave
// order), so results are deterministic run to run.
//
// Rows: one row is handled by 1, 2 or 4 waves of a 256-thread workgroup
// (more waves per row for long rows, so that every wave issues all of its
// loads up front). All loads of a wave are issued before the activation is
// built in LDS, so weight traffic overlaps the prologue.

#include "cx_internal.h"
#include "cx_act.h"

namespace {

constexpr uint32_t M4 = 0x0F0F0F0Fu;

__device__ inline uint32_t ld32u(const uint8_t* p) {
  uint32_t v;
  __builtin_memcpy(&v, p, 4);
  return v;
}
__device__ inline int dot4(uint32_t a, int b, int c) {
  return __builtin_amdgcn_sdot4((int)a, b, c, false);
}

template <int T> struct KQ;

// ------------------------------------------------------------------ Q4_K
// 144 B: d(2) dmin(2) scales(12) qs(128). Slot l: pair p = l/2, half h = l%2,
// qs bytes [16+32p+16h, +16): low nibbles -> sub-block 2p positions
// 16h..16h+15, high nibbles -> sub-block 2p+1 same positions.
template <> struct KQ<CX_Q4_K> {
  static constexpr int BPB = 144, SUB = 32, NW = 8;
  __device__ static void load(const uint8_t* b, int l, uint32_t (&r)[NW]) {
    uint4 h = *reinterpret_cast<const uint4*>(b);
    uint4 q = *reinterpret_cast<const uint4*>(b + 16 + 16 * l);
    r[0] = h.x; r[1] = h.y; r[2] = h.z; r[3] = h.w;
    r[4] = q.x; r[5] = q.y; r[6] = q.z; r[7] = q.w;
  }
  __device__ static void term(const uint32_t (&r)[NW], int l, const int8_t* xb,
                               const float* xe, const float* xs, int32_t* dbg, float* to) {
    const int p = l >> 1, h = l & 1;
    const int4 xa = *reinterpret_cast<const int4*>(xb + 64 * p + 16 * h);
    const int4 xc = *reinterpret_cast<const int4*>(xb + 64 * p + 32 + 16 * h);
    int e0 = dot4(r[4] & M4, xa.x, 0);
    e0 = dot4(r[5] & M4, xa.y, e0);
    e0 = dot4(r[6] & M4, xa.z, e0);
    e0 = dot4(r[7] & M4, xa.w, e0);
    int e1 = dot4((r[4] >> 4) & M4, xc.x, 0);
    e1 = dot4((r[5] >> 4) & M4, xc.y, e1);
    e1 = dot4((r[6] >> 4) & M4, xc.z, e1);
    e1 = dot4((r[7] >> 4) & M4, xc.w, e1);
    finish(r, h ? e0 : e1, h ? e1 : e0, 2 * p + h, xe, xs, dbg, to);
  }
  // shared with Q5_K: exchange, 6-bit scale unpack, the f32 term
  template <int N>
  __device__ static void finish(const uint32_t (&r)[N], int send, int mine, int j,
                                 const float* xe, const float* xs, int32_t* dbg, float* to) {
    const int e = mine + cx_xor1(send);
    // branch-free 6-bit unpack, the word form of src/kernels/x86.rs:437-447;
    // equal to quant::escala_y_minimo (src/quant.rs:108-117)
    const uint32_t a = r[1], b = r[2], c = r[3];
    const int sh = 8 * (j & 3);
    uint32_t sc, mn;
    if (j < 4) {
      sc = (a >> sh) & 63;
      mn = (b >> sh) & 63;
    } else {
      sc = ((c >> sh) & 0xF) | (((a >> sh) >> 6 & 3) << 4);
      mn = ((c >> sh) >> 4 & 0xF) | (((b >> sh) >> 6 & 3) << 4);
    }
    const float d = cx_h2f(r[0] & 0xFFFF), dm = cx_h2f(r[0] >> 16);
    if (dbg) dbg[j] = e;
    if (to) to[j] = xe[j] * (d * (float)sc * (float)e - dm * (float)mn * xs[j]);
  }
};

// ------------------------------------------------------------------ Q5_K
// 176 B: d dmin scales(12) qh(32) qs(128). As Q4_K plus the fifth bit of
// position i of sub-block j = bit j of qh[i] (src/kernels/scalar.rs:205-210).
template <> struct KQ<CX_Q5_K> {
  static constexpr int BPB = 176, SUB = 32, NW = 12;
  __device__ static void load(const uint8_t* b, int l, uint32_t (&r)[NW]) {
    const int p = l >> 1, h = l & 1;
    uint4 hd = *reinterpret_cast<const uint4*>(b);
    uint4 qh = *reinterpret_cast<const uint4*>(b + 16 + 16 * h);
    uint4 q = *reinterpret_cast<const uint4*>(b + 48 + 32 * p + 16 * h);
    r[0] = hd.x; r[1] = hd.y; r[2] = hd.z; r[3] = hd.w;
    r[4] = q.x; r[5] = q.y; r[6] = q.z; r[7] = q.w;
    r[8] = qh.x; r[9] = qh.y; r[10] = qh.z; r[11] = qh.w;
  }
  __device__ static void term(const uint32_t (&r)[NW], int l, const int8_t* xb,
                               const float* xe, const float* xs, int32_t* dbg, float* to) {
    const int p = l >> 1, h = l & 1;
    const int4 xa = *reinterpret_cast<const int4*>(xb + 64 * p + 16 * h);
    const int4 xc = *reinterpret_cast<const int4*>(xb + 64 * p + 32 + 16 * h);
    const int s0 = 2 * p, s1 = 2 * p + 1;
    int e0 = 0, e1 = 0;
    const int xav[4] = {xa.x, xa.y, xa.z, xa.w};
    const int xcv[4] = {xc.x, xc.y, xc.z, xc.w};
#pragma unroll
    for (int w = 0; w < 4; w++) {
      uint32_t qs = r[4 + w], qh = r[8 + w];
      uint32_t lo = (qs & M4) | (((qh >> s0) & 0x01010101u) << 4);
      uint32_t hi = ((qs >> 4) & M4) | (((qh >> s1) & 0x01010101u) << 4);
      e0 = dot4(lo, xav[w], e0);
      e1 = dot4(hi, xcv[w], e1);
    }
    KQ<CX_Q4_K>::finish(r, h ? e0 : e1, h ? e1 : e0, 2 * p + h, xe, xs, dbg, to);
  }
};

// Shared shape of Q2_K / Q3_K / Q6_K: 16-value sub-blocks, 8 groups of 32.
// Slot l: half = l/4, c = l%4 -> positions 8c..8c+7 of each of the four
// groups g = 4*half + r (r = 0..3); sub-block of (g, c) = 2g + c/2. Lanes c
// and c^1 hold the two halves of the same 16-value sub-blocks; after the
// swap the even lane owns r = 0,1 and the odd lane r = 2,3.
struct Swap16 {
  int own0, own1, s0, s1;
  __device__ Swap16(const int (&E)[4], int l) {
    const int half = l >> 2, c = l & 3, odd = c & 1;
    const int r0 = 2 * odd;
    own0 = (odd ? E[2] : E[0]) + cx_xor1(odd ? E[0] : E[2]);
    own1 = (odd ? E[3] : E[1]) + cx_xor1(odd ? E[1] : E[3]);
    s0 = 2 * (4 * half + r0) + (c >> 1);
    s1 = s0 + 2;
  }
};
// The scale bytes of the two owned sub-blocks live in one 32-bit word,
// index 2*half+odd, at byte m and 2+m (m = c/2).
__device__ inline uint32_t sel4(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                int i) {
  return i == 0 ? w0 : (i == 1 ? w1 : (i == 2 ? w2 : w3));
}

// ------------------------------------------------------------------ Q2_K
// 84 B: scales(16) qs(64) d dmin. value = (qs >> 2(g%4)) & 3.
template <> struct KQ<CX_Q2_K> {
  static constexpr int BPB = 84, SUB = 16, NW = 7;
  __device__ static void load(const uint8_t* b, int l, uint32_t (&r)[NW]) {
    const int half = l >> 2, c = l & 3;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(b + 16 + 32 * half + 8 * c);
    const uint32_t* s = reinterpret_cast<const uint32_t*>(b);
    r[0] = q[0]; r[1] = q[1];
    r[2] = s[0]; r[3] = s[1]; r[4] = s[2]; r[5] = s[3];
    r[6] = *reinterpret_cast<const uint32_t*>(b + 80);
  }
  __device__ static void term(const uint32_t (&r)[NW], int l, const int8_t* xb,
                               const float* xe, const float* xs, int32_t* dbg, float* to) {
    const int half = l >> 2, c = l & 3;
    int E[4];
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
      const int2 x = *reinterpret_cast<const int2*>(xb + 32 * (4 * half + rr) + 8 * c);
      E[rr] = dot4((r[1] >> (2 * rr)) & 0x03030303u, x.y,
                   dot4((r[0] >> (2 * rr)) & 0x03030303u, x.x, 0));
    }
    Swap16 sw(E, l);
    const uint32_t word = sel4(r[2], r[3], r[4], r[5], 2 * half + (c & 1));
    const int m = c >> 1;
    const uint32_t sc0 = (word >> (8 * m)) & 0xFF, sc1 = (word >> (8 * (m + 2))) & 0xFF;
    const float d = cx_h2f(r[6] & 0xFFFF), dm = cx_h2f(r[6] >> 16);
    if (dbg) { dbg[sw.s0] = sw.own0; dbg[sw.s1] = sw.own1; }
    float t0 = xe[sw.s0] * (d * (float)(sc0 & 0xF) * (float)sw.own0 -
                            dm * (float)(sc0 >> 4) * xs[sw.s0]);
    float t1 = xe[sw.s1] * (d * (float)(sc1 & 0xF) * (float)sw.own1 -
                            dm * (float)(sc1 >> 4) * xs[sw.s1]);
    if (to) {
      to[sw.s0] = t0;
      to[sw.s1] = t1;
    }
  }
};

// ------------------------------------------------------------------ Q3_K
// 110 B: hmask(32) qs(64) scales(12) d. Biased value (q+4) in 0..7 =
// ((qs >> 2(g%4)) & 3) | ((hmask >> g) & 1) << 2   (src/kernels/scalar.rs:262-268)
template <> struct KQ<CX_Q3_K> {
  static constexpr int BPB = 110, SUB = 16, NW = 8;
  __device__ static void load(const uint8_t* b, int l, uint32_t (&r)[NW]) {
    const int half = l >> 2, c = l & 3;
    r[0] = ld32u(b + 8 * c);
    r[1] = ld32u(b + 8 * c + 4);
    r[2] = ld32u(b + 32 + 32 * half + 8 * c);
    r[3] = ld32u(b + 32 + 32 * half + 8 * c + 4);
    r[4] = ld32u(b + 96);
    r[5] = ld32u(b + 100);
    r[6] = ld32u(b + 104);
    r[7] = (uint32_t)b[108] | ((uint32_t)b[109] << 8);
  }
  __device__ static void term(const uint32_t (&r)[NW], int l, const int8_t* xb,
                               const float* xe, const float* xs, int32_t* dbg, float* to) {
    const int half = l >> 2, c = l & 3;
    int E[4];
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
      const int g = 4 * half + rr;
      const int2 x = *reinterpret_cast<const int2*>(xb + 32 * g + 8 * c);
      uint32_t v0 = ((r[2] >> (2 * rr)) & 0x03030303u) | (((r[0] >> g) & 0x01010101u) << 2);
      uint32_t v1 = ((r[3] >> (2 * rr)) & 0x03030303u) | (((r[1] >> g) & 0x01010101u) << 2);
      E[rr] = dot4(v1, x.y, dot4(v0, x.x, 0));
    }
    Swap16 sw(E, l);
    // escalas_q3k (src/quant.rs:87-106): scale j = low nibble of byte j%4 of
    // (A or B by (j/4)&1) shifted 4*(j/8), plus 2 bits of T at 8*(j%4)+2*(j/4)
    const uint32_t A = r[4], B = r[5], T = r[6];
    const int w = 2 * half + (c & 1), m = c >> 1;
    const uint32_t src = (w & 1) ? B : A;
    const int lsh = 4 * (w >> 1);
    const uint32_t esc0 = ((src >> (8 * m + lsh)) & 0xF) | (((T >> (8 * m + 2 * w)) & 3) << 4);
    const uint32_t esc1 =
        ((src >> (8 * (m + 2) + lsh)) & 0xF) | (((T >> (8 * (m + 2) + 2 * w)) & 3) << 4);
    const float d = cx_h2f(r[7]);
    if (dbg) { dbg[sw.s0] = sw.own0; dbg[sw.s1] = sw.own1; }
    const float sc0 = d * ((float)esc0 - 32.0f), sc1 = d * ((float)esc1 - 32.0f);
    float t0 = xe[sw.s0] * sc0 * ((float)sw.own0 - 4.0f * xs[sw.s0]);
    float t1 = xe[sw.s1] * sc1 * ((float)sw.own1 - 4.0f * xs[sw.s1]);
    if (to) {
      to[sw.s0] = t0;
      to[sw.s1] = t1;
    }
  }
};

// ------------------------------------------------------------------ Q6_K
// 210 B: ql(128) qh(64) scales(16, i8) d. Unsigned value 0..63 =
// nib | ((qh >> 2gi) & 3) << 4   (src/kernels/scalar.rs:305-320)
template <> struct KQ<CX_Q6_K> {
  static constexpr int BPB = 210, SUB = 16, NW = 11;
  __device__ static void load(const uint8_t* b, int l, uint32_t (&r)[NW]) {
    const int half = l >> 2, c = l & 3;
    const uint8_t* qa = b + 64 * half + 8 * c;
    r[0] = ld32u(qa); r[1] = ld32u(qa + 4);
    r[2] = ld32u(qa + 32); r[3] = ld32u(qa + 36);
    r[4] = ld32u(b + 128 + 32 * half + 8 * c);
    r[5] = ld32u(b + 128 + 32 * half + 8 * c + 4);
    r[6] = ld32u(b + 192); r[7] = ld32u(b + 196); r[8] = ld32u(b + 200); r[9] = ld32u(b + 204);
    r[10] = (uint32_t)b[208] | ((uint32_t)b[209] << 8);
  }
  __device__ static void term(const uint32_t (&r)[NW], int l, const int8_t* xb,
                               const float* xe, const float* xs, int32_t* dbg, float* to) {
    const int half = l >> 2, c = l & 3;
    int E[4];
#pragma unroll
    for (int gi = 0; gi < 4; gi++) {
      const int g = 4 * half + gi;
      const int2 x = *reinterpret_cast<const int2*>(xb + 32 * g + 8 * c);
      const uint32_t s0 = (gi & 1) ? r[2] : r[0], s1 = (gi & 1) ? r[3] : r[1];
      uint32_t n0 = gi < 2 ? (s0 & M4) : ((s0 >> 4) & M4);
      uint32_t n1 = gi < 2 ? (s1 & M4) : ((s1 >> 4) & M4);
      uint32_t v0 = n0 | (((r[4] >> (2 * gi)) & 0x03030303u) << 4);
      uint32_t v1 = n1 | (((r[5] >> (2 * gi)) & 0x03030303u) << 4);
      E[gi] = dot4(v1, x.y, dot4(v0, x.x, 0));
    }
    Swap16 sw(E, l);
    const uint32_t word = sel4(r[6], r[7], r[8], r[9], 2 * half + (c & 1));
    const int m = c >> 1;
    const int8_t e0 = (int8_t)((word >> (8 * m)) & 0xFF);
    const int8_t e1 = (int8_t)((word >> (8 * (m + 2))) & 0xFF);
    const float d = cx_h2f(r[10]);
    if (dbg) { dbg[sw.s0] = sw.own0; dbg[sw.s1] = sw.own1; }
    const float sc0 = d * (float)e0, sc1 = d * (float)e1;
    float t0 = xe[sw.s0] * sc0 * ((float)sw.own0 - 32.0f * xs[sw.s0]);
    float t1 = xe[sw.s1] * sc1 * ((float)sw.own1 - 32.0f * xs[sw.s1]);
    if (to) {
      to[sw.s0] = t0;
      to[sw.s1] = t1;
    }
  }
};

// -------------------------------------------------------------- kernel
struct GemvParams {
  cx_seg seg[4];
  uint32_t seg_end[4];  // cumulative rows
  int nseg;
  uint32_t k, nb, nsub;
  uint32_t waves_per_row, rows_per_wg, slots_per_wave;
  int src;
  const int8_t* xq;
  const float* xe;
  const float* xs;
  const float* x;
  const float* x2;
  const float* nw;
  float eps;
  int epi;
  int32_t* dbg;
};

template <int T, int MAXIT>
__global__ __launch_bounds__(256) void k_gemv(GemvParams P) {
  using Q = KQ<T>;
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ double red[4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t row_in_wg = wave / P.waves_per_row, part = wave % P.waves_per_row;
  const uint32_t grow = blockIdx.x * P.rows_per_wg + row_in_wg;
  const bool row_ok = grow < P.seg_end[P.nseg - 1];
  int sg = 0;
  uint32_t rbase = 0;
  if (row_ok) {
    while (grow >= P.seg_end[sg]) sg++;
    rbase = sg ? P.seg_end[sg - 1] : 0;
  }
  const uint32_t row = grow - rbase;
  const size_t row_bytes = (size_t)P.nb * Q::BPB;
  const uint8_t* wrow = row_ok ? P.seg[sg].w + (size_t)row * row_bytes : nullptr;
  const uint32_t nslots = P.nb * 8, s_begin = part * P.slots_per_wave;

  // 1. every weight load of this wave, issued up front
  uint32_t regs[MAXIT][Q::NW];
  bool valid[MAXIT];
#pragma unroll
  for (int it = 0; it < MAXIT; it++) {
    const uint32_t off = it * 64 + lane, slot = s_begin + off;
    valid[it] = row_ok && off < P.slots_per_wave && slot < nslots;
    if (valid[it]) {
      Q::load(wrow + (size_t)(slot >> 3) * Q::BPB, slot & 7, regs[it]);
    } else {
#pragma unroll
      for (int w = 0; w < Q::NW; w++) regs[it][w] = 0;
    }
  }

  // 2. the i8 activation of this launch, built in LDS by every workgroup
  int8_t* sq = reinterpret_cast<int8_t*>(lds);
  float* se = reinterpret_cast<float*>(lds + P.k);
  float* ss = se + P.nsub;
  if (P.src == CX_ACT_QUANTIZED) {
    const uint4* gq = reinterpret_cast<const uint4*>(P.xq);
    for (uint32_t i = tid; i < P.k / 16; i += 256) reinterpret_cast<uint4*>(sq)[i] = gq[i];
    for (uint32_t i = tid; i < P.nsub; i += 256) {
      se[i] = P.xe[i];
      ss[i] = P.xs[i];
    }
  } else {
    double scale = 1.0;
    if (P.src == CX_ACT_NORM) scale = cx_rms_scale(P.x, P.k, P.eps, red);
    cx_build_act_rows<Q::SUB>(P.src, P.x, P.x2, P.nw, scale, P.k, sq, se, ss, tid, 256);
  }
  __syncthreads();

  // 3. integer dots + the reference's per-sub-block f32 terms, staged in LDS
  //    by sub-block index (every sub-block of the row is owned by one lane)
  float* terms = ss + P.nsub + row_in_wg * P.nsub;
  constexpr int SPB = 256 / Q::SUB;  // sub-blocks per super-block
#pragma unroll
  for (int it = 0; it < MAXIT; it++) {
    const uint32_t slot = s_begin + it * 64 + lane;
    const uint32_t blk = valid[it] ? (slot >> 3) : 0;
    int32_t* dbg = (P.dbg && valid[it]) ? P.dbg + (size_t)grow * P.nsub + blk * SPB : nullptr;
    float* to = valid[it] ? terms + blk * SPB : nullptr;
    Q::term(regs[it], lane & 7, sq + blk * 256, se + blk * SPB, ss + blk * SPB, dbg, to);
  }
  __syncthreads();

  // 4. the row's sum in the scalar spec's order: total = 0; total += term_s
  //    for s = 0, 1, ... (src/kernels/scalar.rs:141-167), so a row's result
  //    is bit-identical to the reference's scalar kernel.
  if (part == 0 && lane == 0 && row_ok) {
    float acc = 0.0f;
    for (uint32_t s = 0; s < P.nsub; s++) acc += terms[s];
    const cx_seg& S = P.seg[sg];
    if (P.epi == CX_EPI_ACCUM) {
      S.y[row] += acc;
    } else {
      S.y[row] = S.bias ? acc + S.bias[row] : acc;
    }
  }
}

template <int T>
int launch_t(GemvParams& P, uint32_t total_rows, hipStream_t s) {
  const uint32_t nslots = P.nb * 8;
  int maxit = 0;
  for (int m : {1, 2, 4, 8}) {
    for (uint32_t S : {1u, 2u, 4u}) {
      uint32_t spw = ((nslots + S - 1) / S + 7) / 8 * 8;
      if (spw <= 64u * m) {
        P.waves_per_row = S;
        P.slots_per_wave = spw;
        maxit = m;
        break;
      }
    }
    if (maxit) break;
  }
  CX_REQUIRE(maxit, "gemv: row of %u values is too long", P.k);
  P.rows_per_wg = 4 / P.waves_per_row;
  const uint32_t grid = (total_rows + P.rows_per_wg - 1) / P.rows_per_wg;
  // activation (k + 8 * nsub) + one row of f32 terms per row of the workgroup
  const size_t lds = P.k + 8 * (size_t)P.nsub + 4 * (size_t)P.nsub * P.rows_per_wg;
  switch (maxit) {
    case 1: hipLaunchKernelGGL((k_gemv<T, 1>), dim3(grid), dim3(256), lds, s, P); break;
    case 2: hipLaunchKernelGGL((k_gemv<T, 2>), dim3(grid), dim3(256), lds, s, P); break;
    case 4: hipLaunchKernelGGL((k_gemv<T, 4>), dim3(grid), dim3(256), lds, s, P); break;
    default: hipLaunchKernelGGL((k_gemv<T, 8>), dim3(grid), dim3(256), lds, s, P); break;
  }
  CX_HIP(hipGetLastError());
  return CX_OK;
}

}  // namespace

int cx_launch_gemv(int type, const cx_seg* segs, int nseg, uint32_t k, const cx_act& act,
                   int epi, int32_t* dbg, hipStream_t s) {
  CX_REQUIRE(nseg >= 1 && nseg <= 4, "gemv: 1..4 matrices per launch");
  CX_REQUIRE(cx_is_kquant(type), "gemv: type %d has no fused GEMV", type);
  CX_REQUIRE(k > 0 && k % 256 == 0, "gemv: k=%u is not a multiple of 256", k);
  GemvParams P{};
  uint32_t total = 0;
  for (int i = 0; i < nseg; i++) {
    CX_REQUIRE(segs[i].w && segs[i].y, "gemv: null matrix or output");
    P.seg[i] = segs[i];
    total += segs[i].rows;
    P.seg_end[i] = total;
  }
  if (total == 0) return CX_OK;
  P.nseg = nseg;
  P.k = k;
  P.nb = k / 256;
  P.nsub = k / cx_sub(type);
  P.src = act.src;
  P.xq = act.xq; P.xe = act.xe; P.xs = act.xs;
  P.x = act.x; P.x2 = act.x2; P.nw = act.norm_w; P.eps = act.eps;
  P.epi = epi;
  P.dbg = dbg;
  if (act.src == CX_ACT_QUANTIZED)
    CX_REQUIRE(act.xq && act.xe && act.xs, "gemv: missing quantized activation");
  else
    CX_REQUIRE(act.x && (act.src != CX_ACT_NORM || act.norm_w) &&
                   (act.src != CX_ACT_SWIGLU || act.x2),
               "gemv: missing activation");
  switch (type) {
    case CX_Q2_K: return launch_t<CX_Q2_K>(P, total, s);
    case CX_Q3_K: return launch_t<CX_Q3_K>(P, total, s);
    case CX_Q4_K: return launch_t<CX_Q4_K>(P, total, s);
    case CX_Q5_K: return launch_t<CX_Q5_K>(P, total, s);
    default: return launch_t<CX_Q6_K>(P, total, s);
  }
}

// ------------------------------------------------- activation kernels
namespace {
template <int SUB>
__global__ __launch_bounds__(256) void k_quantize(const float* x, size_t rows, uint32_t k,
                                                  int8_t* xq, float* xe, float* xs) {
  const uint32_t nsub = k / SUB;
  const size_t total = rows * nsub;
  for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    float v[SUB];
    const float4* px = reinterpret_cast<const float4*>(x + i * SUB);
#pragma unroll
    for (int j = 0; j < SUB / 4; j++) {
      float4 f = px[j];
      v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
    }
    cx_quant_sub<SUB>(v, xq + i * SUB, xe + i, xs + i);
  }
}

__global__ __launch_bounds__(256) void k_rmsnorm(float* out, const float* in, const float* w,
                                                 uint32_t n, float eps) {
  __shared__ double red[4];
  const float* x = in + (size_t)blockIdx.x * n;
  float* y = out + (size_t)blockIdx.x * n;
  const double scale = cx_rms_scale(x, n, eps, red);
  for (uint32_t i = threadIdx.x; i < n; i += 256) y[i] = (float)((double)x[i] * scale) * w[i];
}
}  // namespace

int cx_launch_quantize(const float* x, size_t rows, size_t k, int sub, int8_t* xq, float* xe,
                       float* xs, hipStream_t s) {
  CX_REQUIRE(sub == 16 || sub == 32, "quantize: sub must be 16 or 32, got %d", sub);
  CX_REQUIRE(k % (size_t)sub == 0 && k % 4 == 0, "quantize: k=%zu not a multiple of %d", k, sub);
  CX_REQUIRE(x && xq && xe && xs, "quantize: null pointer");
  const size_t total = rows * (k / sub);
  if (!total) return CX_OK;
  const unsigned grid = (unsigned)((total + 255) / 256 < 65535 ? (total + 255) / 256 : 65535);
  if (sub == 16)
    hipLaunchKernelGGL(k_quantize<16>, dim3(grid), dim3(256), 0, s, x, rows, (uint32_t)k, xq, xe, xs);
  else
    hipLaunchKernelGGL(k_quantize<32>, dim3(grid), dim3(256), 0, s, x, rows, (uint32_t)k, xq, xe, xs);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_rmsnorm(float* out, const float* in, const float* w, size_t rows, size_t n,
                      float eps, hipStream_t s) {
  CX_REQUIRE(out && in && w, "rmsnorm: null pointer");
  CX_REQUIRE(n % 4 == 0, "rmsnorm: n=%zu must be a multiple of 4", n);
  if (!rows || !n) return CX_OK;
  hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)rows), dim3(256), 0, s, out, in, w, (uint32_t)n, eps);
  CX_HIP(hipGetLastError());
  return CX_OK;
}
