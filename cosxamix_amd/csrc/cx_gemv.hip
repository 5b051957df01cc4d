// cx_gemv.hip — batch-1 k-quant GEMV for gfx950 (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K).
//
// y[r] = sum over super-blocks of row r of the reference's fused dot
// (src/kernels/scalar.rs:132-324, src/kernels/q2k.rs:41-69) against an i8
// activation quantized beforehand (xq, xe, xs).
//
// Data movement. A workgroup owns a tile of R consecutive rows, i.e. one
// contiguous byte range of the matrix. Its four waves copy that range into
// LDS with global_load_lds_dwordx4 (gfx950's 16-byte direct-to-LDS load):
// every lane moves 16 consecutive bytes, so a wave reads 1 KiB of contiguous
// HBM per instruction, no VGPRs hold weight data, and the whole tile is in
// flight at once. The activation (k bytes + 2*k/sub floats) follows into LDS
// the same way. R is chosen per launch so that there are >= 2 tiles per CU
// and a tile fits in 64 KiB of LDS; with several workgroups resident per CU
// the whole matrix is in flight within one wave of workgroups.
//
// Arithmetic. A super-block (256 values) is handled by 8 consecutive lanes,
// one "slot" each. A lane reads its slice of the block from LDS, unpacks the
// quants and the 6-bit scales in registers and forms integer partial sums
// with v_dot4c_i32_i8. The two lanes that share a sub-block swap partial
// sums with one DPP move, so every sub-block integer sum E_j is formed
// exactly. The lane that owns sub-block j then computes the reference's f32
// term with the reference's rounding:
//   Q4_K/Q5_K/Q2_K : xe[j] * ((d*sc_j)*E_j - (dmin*mn_j)*xs[j])
//   Q3_K           : (xe[j] * (d*(esc_j-32))) * (E'_j - 4*xs[j])
//   Q6_K           : (xe[j] * (d*esc_j)) * (E'_j - 32*xs[j])
// and stores it in LDS at its sub-block index. Finally one lane per row adds
// the row's terms in sub-block order starting from 0.0, as the scalar kernel
// does, so every row is bit-identical to the reference's scalar dot.

#include "cx_internal.h"
#include "cx_act.h"

namespace {

constexpr uint32_t M4 = 0x0F0F0F0Fu;
constexpr uint32_t TILE_LDS_MAX = 64 * 1024;

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ inline int dot4(uint32_t a, int b, int c) {
  return __builtin_amdgcn_sdot4((int)a, b, c, false);
}
// a dword at any byte offset of LDS: two aligned reads and v_alignbyte_b32.
// May read up to 3 bytes past off+4 (the tile region is padded for it).
__device__ inline uint32_t lds32(const uint8_t* lds, uint32_t off) {
  const uint32_t* q = reinterpret_cast<const uint32_t*>(lds + (off & ~3u));
  return __builtin_amdgcn_alignbyte(q[1], q[0], off & 3u);
}

template <int T> struct KQ;

// ------------------------------------------------------------------ Q4_K
// 144 B: d(2) dmin(2) scales(12) qs(128). Slot l: pair p = l/2, half h = l%2,
// qs bytes [16+32p+16h, +16): low nibbles -> sub-block 2p positions
// 16h..16h+15, high nibbles -> sub-block 2p+1 same positions.
// Blocks are read as 16-byte words: the tile must start 16-byte aligned.
template <> struct KQ<CX_Q4_K> {
  static constexpr int BPB = 144, SUB = 32, NW = 8;
  static constexpr bool ALIGNED = true;
  __device__ static void load(const uint8_t* lds, uint32_t off, int l, uint32_t (&r)[NW]) {
    uint4 h = *reinterpret_cast<const uint4*>(lds + off);
    uint4 q = *reinterpret_cast<const uint4*>(lds + off + 16 + 16 * l);
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
    to[j] = xe[j] * (d * (float)sc * (float)e - dm * (float)mn * xs[j]);
  }
};

// ------------------------------------------------------------------ Q5_K
// 176 B: d dmin scales(12) qh(32) qs(128). As Q4_K plus the fifth bit of
// position i of sub-block j = bit j of qh[i] (src/kernels/scalar.rs:205-210).
template <> struct KQ<CX_Q5_K> {
  static constexpr int BPB = 176, SUB = 32, NW = 12;
  static constexpr bool ALIGNED = true;
  __device__ static void load(const uint8_t* lds, uint32_t off, int l, uint32_t (&r)[NW]) {
    const int p = l >> 1, h = l & 1;
    uint4 hd = *reinterpret_cast<const uint4*>(lds + off);
    uint4 qh = *reinterpret_cast<const uint4*>(lds + off + 16 + 16 * h);
    uint4 q = *reinterpret_cast<const uint4*>(lds + off + 48 + 32 * p + 16 * h);
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
  static constexpr bool ALIGNED = false;
  __device__ static void load(const uint8_t* lds, uint32_t off, int l, uint32_t (&r)[NW]) {
    const int half = l >> 2, c = l & 3;
    const uint32_t q = off + 16 + 32 * half + 8 * c;
    r[0] = lds32(lds, q); r[1] = lds32(lds, q + 4);
    r[2] = lds32(lds, off); r[3] = lds32(lds, off + 4);
    r[4] = lds32(lds, off + 8); r[5] = lds32(lds, off + 12);
    r[6] = lds32(lds, off + 80);
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
    to[sw.s0] = xe[sw.s0] * (d * (float)(sc0 & 0xF) * (float)sw.own0 -
                             dm * (float)(sc0 >> 4) * xs[sw.s0]);
    to[sw.s1] = xe[sw.s1] * (d * (float)(sc1 & 0xF) * (float)sw.own1 -
                             dm * (float)(sc1 >> 4) * xs[sw.s1]);
  }
};

// ------------------------------------------------------------------ Q3_K
// 110 B: hmask(32) qs(64) scales(12) d. Biased value (q+4) in 0..7 =
// ((qs >> 2(g%4)) & 3) | ((hmask >> g) & 1) << 2   (src/kernels/scalar.rs:262-268)
template <> struct KQ<CX_Q3_K> {
  static constexpr int BPB = 110, SUB = 16, NW = 8;
  static constexpr bool ALIGNED = false;
  __device__ static void load(const uint8_t* lds, uint32_t off, int l, uint32_t (&r)[NW]) {
    const int half = l >> 2, c = l & 3;
    r[0] = lds32(lds, off + 8 * c);
    r[1] = lds32(lds, off + 8 * c + 4);
    r[2] = lds32(lds, off + 32 + 32 * half + 8 * c);
    r[3] = lds32(lds, off + 32 + 32 * half + 8 * c + 4);
    r[4] = lds32(lds, off + 96);
    r[5] = lds32(lds, off + 100);
    r[6] = lds32(lds, off + 104);
    r[7] = lds32(lds, off + 108) & 0xFFFFu;
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
    to[sw.s0] = xe[sw.s0] * sc0 * ((float)sw.own0 - 4.0f * xs[sw.s0]);
    to[sw.s1] = xe[sw.s1] * sc1 * ((float)sw.own1 - 4.0f * xs[sw.s1]);
  }
};

// ------------------------------------------------------------------ Q6_K
// 210 B: ql(128) qh(64) scales(16, i8) d. Unsigned value 0..63 =
// nib | ((qh >> 2gi) & 3) << 4   (src/kernels/scalar.rs:305-320)
template <> struct KQ<CX_Q6_K> {
  static constexpr int BPB = 210, SUB = 16, NW = 11;
  static constexpr bool ALIGNED = false;
  __device__ static void load(const uint8_t* lds, uint32_t off, int l, uint32_t (&r)[NW]) {
    const int half = l >> 2, c = l & 3;
    const uint32_t qa = off + 64 * half + 8 * c;
    r[0] = lds32(lds, qa); r[1] = lds32(lds, qa + 4);
    r[2] = lds32(lds, qa + 32); r[3] = lds32(lds, qa + 36);
    r[4] = lds32(lds, off + 128 + 32 * half + 8 * c);
    r[5] = lds32(lds, off + 128 + 32 * half + 8 * c + 4);
    r[6] = lds32(lds, off + 192); r[7] = lds32(lds, off + 196);
    r[8] = lds32(lds, off + 200); r[9] = lds32(lds, off + 204);
    r[10] = lds32(lds, off + 208) & 0xFFFFu;
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
    to[sw.s0] = xe[sw.s0] * sc0 * ((float)sw.own0 - 32.0f * xs[sw.s0]);
    to[sw.s1] = xe[sw.s1] * sc1 * ((float)sw.own1 - 32.0f * xs[sw.s1]);
  }
};

// -------------------------------------------------------------- kernel
struct GemvParams {
  cx_seg seg[4];
  uint32_t tile_end[4];  // cumulative tile counts
  int nseg;
  uint32_t k, nb, nsub;
  uint32_t R;            // rows per tile
  uint32_t row_bytes;
  uint32_t tstride;      // floats between two rows' terms (nsub + 4)
  uint32_t lds_act;      // byte offsets in LDS: activation, xe/xs, terms
  uint32_t lds_scale;
  uint32_t lds_terms;
  cx_qact act;
  int epi;
  int32_t* dbg;
};

// 16-byte chunks [0, n) of `g` into LDS at `l`, 1 KiB per wave instruction.
// global_load_lds writes lane i's 16 bytes at (wave-uniform LDS address) +
// 16*i; lanes past the end are masked off.
__device__ inline void copy_to_lds(const uint8_t* g, uint8_t* l, uint32_t n, int wave, int lane,
                                   int nwaves) {
  for (uint32_t c0 = 64u * wave; c0 < n; c0 += 64u * nwaves) {
    if (c0 + lane < n)
      __builtin_amdgcn_global_load_lds(g + 16 * (size_t)(c0 + lane), (lds_ptr_t)(l + 16 * c0), 16,
                                       0, 0);
  }
}

template <int T>
__global__ __launch_bounds__(256) void k_gemv(GemvParams P) {
  using Q = KQ<T>;
  constexpr int SPB = 256 / Q::SUB;  // sub-blocks per super-block
  extern __shared__ __align__(16) uint8_t lds[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t tile = blockIdx.x;
  int sg = 0;
  while (tile >= P.tile_end[sg]) sg++;
  if (sg) tile -= P.tile_end[sg - 1];
  const cx_seg S = P.seg[sg];
  const uint32_t row0 = tile * P.R;
  const uint32_t rows = min(P.R, S.rows - row0);

  // 1. the tile (rows * row_bytes contiguous bytes) and the activation into
  //    LDS; the tile starts `skew` bytes into LDS when the rows are not
  //    16-byte aligned (Q2_K/Q3_K/Q6_K rows of some widths)
  const uint8_t* src = S.w + (size_t)row0 * P.row_bytes;
  const uint32_t skew = (uint32_t)((uintptr_t)src & 15u);
  copy_to_lds(src - skew, lds, (skew + rows * P.row_bytes + 15) >> 4, wave, lane, 4);
  int8_t* sq = reinterpret_cast<int8_t*>(lds + P.lds_act);
  copy_to_lds(reinterpret_cast<const uint8_t*>(P.act.xq), reinterpret_cast<uint8_t*>(sq),
              P.k >> 4, wave, lane, 4);
  float* se = reinterpret_cast<float*>(lds + P.lds_scale);
  float* ss = se + P.nsub;
  for (uint32_t i = tid; i < P.nsub; i += 256) {
    se[i] = P.act.xe[i];
    ss[i] = P.act.xs[i];
  }
  __builtin_amdgcn_s_waitcnt(0);  // the direct-to-LDS loads have landed
  __syncthreads();

  // 2. integer dots + the reference's per-sub-block f32 terms, staged in LDS
  //    by (row, sub-block); every sub-block of a row is owned by one lane
  float* terms = reinterpret_cast<float*>(lds + P.lds_terms);
  const uint32_t nb8 = P.nb * 8, total = rows * nb8;
  for (uint32_t slot = tid; slot < total; slot += 256) {
    const uint32_t r = slot / nb8, w = slot - r * nb8, blk = w >> 3;
    const int l = (int)(w & 7);
    uint32_t regs[Q::NW];
    Q::load(lds, skew + r * P.row_bytes + blk * Q::BPB, l, regs);
    int32_t* dbg = P.dbg ? P.dbg + (size_t)(row0 + r) * P.nsub + blk * SPB : nullptr;
    Q::term(regs, l, sq + blk * 256, se + blk * SPB, ss + blk * SPB, dbg,
            terms + r * P.tstride + blk * SPB);
  }
  __syncthreads();

  // 3. the row's sum in the scalar spec's order: total = 0; total += term_s
  //    for s = 0, 1, ... (src/kernels/scalar.rs:141-167)
  if ((uint32_t)tid < rows) {
    const float4* t = reinterpret_cast<const float4*>(terms + tid * P.tstride);
    float acc = 0.0f;
    for (uint32_t s = 0; s < P.nsub / 4; s++) {
      const float4 v = t[s];
      acc += v.x;
      acc += v.y;
      acc += v.z;
      acc += v.w;
    }
    const uint32_t row = row0 + tid;
    if (P.epi == CX_EPI_ACCUM)
      S.y[row] += acc;
    else
      S.y[row] = S.bias ? acc + S.bias[row] : acc;
  }
}

struct TilePlan {
  uint32_t R, tiles, lds, lds_act, lds_scale, lds_terms;
};

// LDS layout of a tile of R rows: [16 skew + R*row_bytes + 16 pad] [xq k]
// [xe, xs] [terms R x (nsub+4)]
TilePlan plan_tile(uint32_t R, uint32_t row_bytes, uint32_t k, uint32_t nsub,
                   const uint32_t* rows, int nseg) {
  TilePlan t{};
  t.R = R;
  for (int i = 0; i < nseg; i++) t.tiles += (rows[i] + R - 1) / R;
  t.lds_act = (16 + R * row_bytes + 16 + 15) / 16 * 16;
  t.lds_scale = t.lds_act + k;
  t.lds_terms = t.lds_scale + (8 * nsub + 15) / 16 * 16;
  t.lds = t.lds_terms + 4 * R * (nsub + 4);
  return t;
}

template <int T>
int launch_t(GemvParams& P, const uint32_t* rows, hipStream_t s) {
  using Q = KQ<T>;
  if (Q::ALIGNED) {
    for (int i = 0; i < P.nseg; i++)
      CX_REQUIRE(((uintptr_t)P.seg[i].w & 15u) == 0,
                 "gemv: %s weights must start 16-byte aligned", T == CX_Q4_K ? "Q4_K" : "Q5_K");
  }
  // largest tile (<= 64 rows) that fits the LDS budget and leaves >= 2
  // tiles per CU; small matrices fall back to the smallest tiles
  TilePlan best{};
  for (uint32_t R = 64; R >= 1; R >>= 1) {
    TilePlan t = plan_tile(R, P.row_bytes, P.k, P.nsub, rows, P.nseg);
    if (t.lds > TILE_LDS_MAX) continue;
    best = t;
    if (t.tiles >= 512) break;
  }
  CX_REQUIRE(best.R, "gemv: a row of %u values does not fit in LDS", P.k);
  P.R = best.R;
  P.lds_act = best.lds_act;
  P.lds_scale = best.lds_scale;
  P.lds_terms = best.lds_terms;
  uint32_t acc = 0;
  for (int i = 0; i < P.nseg; i++) {
    acc += (rows[i] + best.R - 1) / best.R;
    P.tile_end[i] = acc;
  }
  hipLaunchKernelGGL((k_gemv<T>), dim3(best.tiles), dim3(256), best.lds, s, P);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

}  // namespace

int cx_launch_gemv(int type, const cx_seg* segs, int nseg, uint32_t k, const cx_qact& act,
                   int epi, int32_t* dbg, hipStream_t s) {
  CX_REQUIRE(nseg >= 1 && nseg <= 4, "gemv: 1..4 matrices per launch");
  CX_REQUIRE(cx_is_kquant(type), "gemv: type %d has no fused GEMV", type);
  CX_REQUIRE(k > 0 && k % 256 == 0, "gemv: k=%u is not a multiple of 256", k);
  CX_REQUIRE(act.xq && act.xe && act.xs, "gemv: missing quantized activation");
  CX_REQUIRE(((uintptr_t)act.xq & 15u) == 0, "gemv: xq must be 16-byte aligned");
  CX_REQUIRE(!dbg || nseg == 1, "gemv: sub-block sums need a single matrix");
  GemvParams P{};
  uint32_t rows[4], total = 0;
  for (int i = 0; i < nseg; i++) {
    CX_REQUIRE(segs[i].w && segs[i].y, "gemv: null matrix or output");
    P.seg[i] = segs[i];
    rows[i] = segs[i].rows;
    total += segs[i].rows;
  }
  if (total == 0) return CX_OK;
  // empty segments would own no tile; keep them out of the tile table
  int n = 0;
  for (int i = 0; i < nseg; i++)
    if (rows[i]) {
      P.seg[n] = segs[i];
      rows[n++] = segs[i].rows;
    }
  P.nseg = n;
  P.k = k;
  P.nb = k / 256;
  P.nsub = k / cx_sub(type);
  P.row_bytes = P.nb * cx_bpb(type);
  P.tstride = P.nsub + 4;
  P.act = act;
  P.epi = epi;
  P.dbg = dbg;
  switch (type) {
    case CX_Q2_K: return launch_t<CX_Q2_K>(P, rows, s);
    case CX_Q3_K: return launch_t<CX_Q3_K>(P, rows, s);
    case CX_Q4_K: return launch_t<CX_Q4_K>(P, rows, s);
    case CX_Q5_K: return launch_t<CX_Q5_K>(P, rows, s);
    default: return launch_t<CX_Q6_K>(P, rows, s);
  }
}

// ------------------------------------------------- activation kernels
namespace {
// 8 values per lane; n % SUB == 0, so a lane group is either wholly inside
// [0, n) or wholly past it. x: rows*k values; a sub-block never straddles
// two rows (k % SUB == 0).
template <int SUB>
__global__ __launch_bounds__(256) void k_quantize(const float* x, size_t n, int8_t* xq,
                                                  float* xe, float* xs) {
  const size_t i = 8 * (blockIdx.x * 256ull + threadIdx.x);
  if (i >= n) return;
  float v[8];
  cx_load8(x + i, v);
  cx_quant8<SUB>(v, i, xq, xe, xs);
}

template <int SUB>
__global__ __launch_bounds__(256) void k_swiglu_quant(const float* g, const float* u, uint32_t n,
                                                      int8_t* xq, float* xe, float* xs) {
  const uint32_t i = 8 * (blockIdx.x * 256u + threadIdx.x);
  if (i >= n) return;
  float v[8], w[8];
  cx_load8(g + i, v);
  cx_load8(u + i, w);
#pragma unroll
  for (int j = 0; j < 8; j++) v[j] = cx_swiglu(v[j], w[j]);
  cx_quant8<SUB>(v, i, xq, xe, xs);
}

// rmsnorm (src/kernels/scalar.rs:40-53) of one row, then its quantization:
// (x as f64 * scale) as f32 * w
template <int SUB>
__global__ __launch_bounds__(256) void k_norm_quant(const float* x, const float* w, uint32_t n,
                                                    float eps, int8_t* xq, float* xe, float* xs) {
  __shared__ double red[4];
  const double scale = cx_rms_scale(x, n, eps, red);
  for (uint32_t i = 8 * threadIdx.x; i < n; i += 8 * 256) {  // n % SUB == 0: whole groups
    float v[8], nw[8];
    cx_load8(x + i, v);
    cx_load8(w + i, nw);
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = (float)((double)v[j] * scale) * nw[j];
    cx_quant8<SUB>(v, i, xq, xe, xs);
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
  CX_REQUIRE(k % (size_t)sub == 0, "quantize: k=%zu not a multiple of %d", k, sub);
  CX_REQUIRE(x && xq && xe && xs, "quantize: null pointer");
  CX_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)xq & 7) == 0,
             "quantize: x must be 16-byte and xq 8-byte aligned");
  const size_t n = rows * k;
  if (!n) return CX_OK;
  const size_t grid = (n / 8 + 255) / 256;
  CX_REQUIRE(grid < (1ull << 31), "quantize: %zu values is too many", n);
  if (sub == 16)
    hipLaunchKernelGGL(k_quantize<16>, dim3((unsigned)grid), dim3(256), 0, s, x, n, xq, xe, xs);
  else
    hipLaunchKernelGGL(k_quantize<32>, dim3((unsigned)grid), dim3(256), 0, s, x, n, xq, xe, xs);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_swiglu_quant(const float* g, const float* u, size_t n, int sub, int8_t* xq,
                           float* xe, float* xs, hipStream_t s) {
  CX_REQUIRE(sub == 16 || sub == 32, "swiglu: sub must be 16 or 32, got %d", sub);
  CX_REQUIRE(n % (size_t)sub == 0 && n < (1u << 31), "swiglu: bad width %zu", n);
  const unsigned grid = (unsigned)((n / 8 + 255) / 256);
  if (sub == 16)
    hipLaunchKernelGGL(k_swiglu_quant<16>, dim3(grid), dim3(256), 0, s, g, u, (uint32_t)n, xq, xe, xs);
  else
    hipLaunchKernelGGL(k_swiglu_quant<32>, dim3(grid), dim3(256), 0, s, g, u, (uint32_t)n, xq, xe, xs);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_norm_quant(const float* x, const float* w, size_t n, float eps, int sub,
                         int8_t* xq, float* xe, float* xs, hipStream_t s) {
  CX_REQUIRE(sub == 16 || sub == 32, "norm: sub must be 16 or 32, got %d", sub);
  CX_REQUIRE(n % 256 == 0 && n < (1u << 31), "norm: width %zu must be a multiple of 256", n);
  if (sub == 16)
    hipLaunchKernelGGL(k_norm_quant<16>, dim3(1), dim3(256), 0, s, x, w, (uint32_t)n, eps, xq, xe, xs);
  else
    hipLaunchKernelGGL(k_norm_quant<32>, dim3(1), dim3(256), 0, s, x, w, (uint32_t)n, eps, xq, xe, xs);
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
