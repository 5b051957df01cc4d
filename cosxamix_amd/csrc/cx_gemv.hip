// cx_gemv.hip — batch-1 GEMV for gfx950: the k-quants (Q2_K, Q3_K, Q4_K,
// Q5_K, Q6_K) and the 32-value block formats (Q8_0, Q5_0).
//
// y[r] = sum over super-blocks of row r of the reference's fused dot
// (src/kernels/scalar.rs:132-324, src/kernels/q2k.rs:41-69) against an i8
// activation quantized beforehand (xq, xe, xs). Q8_0/Q5_0 rows take the
// reference's buffer path instead (k_gemv32 below).
//
// Data movement. A workgroup owns a tile of R consecutive rows, i.e. one
// contiguous byte range of the matrix. Its four waves copy that range into
// LDS with global_load_lds_dwordx4 (gfx950's 16-byte direct-to-LDS load):
// every lane moves 16 consecutive bytes, so a wave reads 1 KiB of contiguous
// HBM per instruction, no VGPRs hold weight data, and the whole tile is in
// flight at once. The activation (k bytes + 2*k/sub floats) follows into LDS
// the same way, or — for the launches that start a layer half — every
// workgroup makes it itself from the f32 residual (rmsnorm + quantization)
// while its weights stream in. R is chosen per launch (see launch_t) so that
// all tiles are resident at once: the whole matrix is in flight within one
// wave of workgroups.
//
// Arithmetic. One lane handles one super-block (256 values) of one row: it
// reads the block from LDS, unpacks the quants and the 6-bit scales in
// registers (the sub-block index is a compile-time constant, so every shift
// is an immediate) and forms each sub-block's integer sum E_j exactly with
// v_dot4c_i32_i8 against the i8 activation in LDS (lanes of different rows
// read the same activation bytes: LDS broadcast). It then computes each
// sub-block's f32 term with the reference's rounding:
//   Q4_K/Q5_K/Q2_K : xe[j] * ((d*sc_j)*E_j - (dmin*mn_j)*xs[j])
//   Q3_K           : (xe[j] * (d*(esc_j-32))) * (E'_j - 4*xs[j])
//   Q6_K           : (xe[j] * (d*esc_j)) * (E'_j - 32*xs[j])
// and stores it in LDS at its sub-block index. Finally one lane per row adds
// the row's terms in sub-block order starting from 0.0, as the scalar kernel
// does, so every row is bit-identical to the reference's scalar dot.

#include "cx_internal.h"
#include "cx_act.h"

namespace {

constexpr uint32_t M4 = 0x0F0F0F0Fu, M2 = 0x03030303u, M1 = 0x01010101u;
constexpr uint32_t TILE_LDS_MAX = 64 * 1024;
constexpr uint32_t TILE_LDS_NORM_MAX = 80 * 1024;  // two workgroups per CU

__device__ inline int dot4(uint32_t a, int b, int c) {
  return __builtin_amdgcn_sdot4((int)a, b, c, false);
}
// N dwords starting at any byte offset of LDS: N+1 aligned reads and
// v_alignbyte_b32. May read up to 7 bytes past off + 4N (the tile region is
// padded for it).
template <int N>
__device__ inline void lds_words(const uint8_t* lds, uint32_t off, uint32_t (&w)[N]) {
  const uint32_t* q = reinterpret_cast<const uint32_t*>(lds + (off & ~3u));
  const uint32_t sh = off & 3u;
  uint32_t a[N + 1];
#pragma unroll
  for (int i = 0; i <= N; i++) a[i] = q[i];
#pragma unroll
  for (int i = 0; i < N; i++) w[i] = __builtin_amdgcn_alignbyte(a[i + 1], a[i], sh);
}
// 8 activation words (32 bytes) of one 32-value group
__device__ inline void act8(const int8_t* x, int (&v)[8]) {
  const int4 a = reinterpret_cast<const int4*>(x)[0], b = reinterpret_cast<const int4*>(x)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Two lanes per super-block: lane half h = 0, 1 computes the terms of
// sub-blocks [SPB/2 h, SPB/2 (h+1)) — the integer sums E_j with
// v_dot4c_i32_i8 (exact), then the reference's f32 term with the reference's
// rounding, written to to[j]; dbg (if set) receives E_j. xb points at the
// block's 256 activation bytes.
template <int T> struct KQ;

// The activation of one half super-block of a 32-value sub-block type
// (Q4_K, Q5_K), in registers: the i8 values of pairs 2h and 2h + 1 (low
// and high sub-block of each) and the four sub-blocks' xe and xs. A lane
// whose items all fall on the same (block, half) reads it once.
struct Pre4 {
  int xa[2][8], xc[2][8];
  float e[4], s[4];
};
__device__ inline void pre4(int h, const int8_t* xb, const float* xe, const float* xs, Pre4& a) {
#pragma unroll
  for (int pp = 0; pp < 2; pp++) {
    act8(xb + 64 * (2 * h + pp), a.xa[pp]);
    act8(xb + 64 * (2 * h + pp) + 32, a.xc[pp]);
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    a.e[j] = xe[4 * h + j];
    a.s[j] = xs[4 * h + j];
  }
}

// ------------------------------------------------------------------ Q4_K
// 144 B: d(2) dmin(2) scales(12) qs(128). Pair p = 0..3: qs bytes
// [32p, 32p+32) hold sub-block 2p (low nibbles) and 2p+1 (high nibbles),
// positions 0..31 (src/kernels/scalar.rs:132-170). Half h owns pairs 2h and
// 2h+1. Blocks are read as 16-byte words: the tile must start 16-byte
// aligned.
template <> struct KQ<CX_Q4_K> {
  static constexpr int BPB = 144, SUB = 32;
  static constexpr bool ALIGNED = true;
  // quant::escala_y_minimo (src/quant.rs:108-117) for sub-blocks 4h..4h+3,
  // four at a time, one per byte: h = 0 takes the low 6 bits of bytes 0..3
  // (a: scales, b: mins); h = 1 the nibbles of c plus the top 2 bits of a/b
  __device__ static void scales_mins(int h, uint32_t a, uint32_t b, uint32_t c, uint32_t& sc,
                                     uint32_t& mn) {
    const uint32_t lo6 = 0x3F3F3F3Fu, top = M2;
    if (h == 0) {
      sc = a & lo6;
      mn = b & lo6;
    } else {
      sc = (c & M4) | (((a >> 6) & top) << 4);
      mn = ((c >> 4) & M4) | (((b >> 6) & top) << 4);
    }
  }
  // The bytes of half h: the 16-byte header and the qs of pairs 2h, 2h+1
  // (64 bytes at 16 + 64h), from LDS or straight from global memory.
  struct Regs {
    uint4 hd, u[4];
  };
  static constexpr int NLOAD = 5;  // 16-byte loads per Regs
  __device__ static void load(const uint8_t* blk, int h, Regs& r) {
    const uint4* bw = reinterpret_cast<const uint4*>(blk);
    r.hd = bw[0];
#pragma unroll
    for (int i = 0; i < 4; i++) r.u[i] = bw[1 + 4 * h + i];
  }
  __device__ static void half(const uint8_t* lds, uint32_t off, int h, const int8_t* xb,
                              const float* xe, const float* xs, int32_t* dbg, float* to) {
    Regs r;
    load(lds + off, h, r);
    half_regs(r, h, xb, xe, xs, dbg, to);
  }
  // sub-block 4h + jj's term in the reference's order:
  // xe * (d * sc * E - dmin * mn * xs)
  __device__ static void term_pre(int jj, int e, float d, float dm, uint32_t sc4, uint32_t mn4,
                                  const Pre4& a, int h, int32_t* dbg, float* to) {
    const uint32_t sc = (sc4 >> (8 * jj)) & 0xFF, mn = (mn4 >> (8 * jj)) & 0xFF;
    if (dbg) dbg[4 * h + jj] = e;
    to[4 * h + jj] = a.e[jj] * (d * (float)sc * (float)e - dm * (float)mn * a.s[jj]);
  }
  __device__ static void half_pre(const Regs& r, int h, const Pre4& a, int32_t* dbg, float* to) {
    const uint4 hd = r.hd;
    const float d = cx_h2f(hd.x & 0xFFFF), dm = cx_h2f(hd.x >> 16);
    uint32_t sc4, mn4;
    scales_mins(h, hd.y, hd.z, hd.w, sc4, mn4);
#pragma unroll
    for (int pp = 0; pp < 2; pp++) {
      const uint4 u0 = r.u[2 * pp], u1 = r.u[2 * pp + 1];
      const uint32_t q[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
      int e0 = 0, e1 = 0;
#pragma unroll
      for (int w = 0; w < 8; w++) {
        e0 = dot4(q[w] & M4, a.xa[pp][w], e0);
        e1 = dot4((q[w] >> 4) & M4, a.xc[pp][w], e1);
      }
      term_pre(2 * pp, e0, d, dm, sc4, mn4, a, h, dbg, to);
      term_pre(2 * pp + 1, e1, d, dm, sc4, mn4, a, h, dbg, to);
    }
  }
  __device__ static void half_regs(const Regs& r, int h, const int8_t* xb, const float* xe,
                                   const float* xs, int32_t* dbg, float* to) {
    Pre4 a;
    pre4(h, xb, xe, xs, a);
    half_pre(r, h, a, dbg, to);
  }
  // half_pre's four terms into registers: t[jj] is sub-block 4h + jj's term;
  // the lane's h selects its scales with selects, not branches
  __device__ static void half_t4(const Regs& r, int h, const Pre4& a, int32_t* dbg,
                                 float (&t)[4]) {
    const uint4 hd = r.hd;
    const float d = cx_h2f(hd.x & 0xFFFF), dm = cx_h2f(hd.x >> 16);
    uint32_t sc0, mn0, sc1, mn1;
    scales_mins(0, hd.y, hd.z, hd.w, sc0, mn0);
    scales_mins(1, hd.y, hd.z, hd.w, sc1, mn1);
    const uint32_t sc4 = h ? sc1 : sc0, mn4 = h ? mn1 : mn0;
#pragma unroll
    for (int pp = 0; pp < 2; pp++) {
      const uint4 u0 = r.u[2 * pp], u1 = r.u[2 * pp + 1];
      const uint32_t q[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
      int e0 = 0, e1 = 0;
#pragma unroll
      for (int w = 0; w < 8; w++) {
        e0 = dot4(q[w] & M4, a.xa[pp][w], e0);
        e1 = dot4((q[w] >> 4) & M4, a.xc[pp][w], e1);
      }
      t[2 * pp] = term_val(2 * pp, e0, d, dm, sc4, mn4, a, h, dbg);
      t[2 * pp + 1] = term_val(2 * pp + 1, e1, d, dm, sc4, mn4, a, h, dbg);
    }
  }
  // term_pre's value, returned
  __device__ static float term_val(int jj, int e, float d, float dm, uint32_t sc4, uint32_t mn4,
                                   const Pre4& a, int h, int32_t* dbg) {
    const uint32_t sc = (sc4 >> (8 * jj)) & 0xFF, mn = (mn4 >> (8 * jj)) & 0xFF;
    if (dbg) dbg[4 * h + jj] = e;
    return a.e[jj] * (d * (float)sc * (float)e - dm * (float)mn * a.s[jj]);
  }
};

// ------------------------------------------------------------------ Q5_K
// 176 B: d dmin scales(12) qh(32) qs(128). As Q4_K plus the fifth bit of
// position i of sub-block j = bit j of qh[i] (src/kernels/scalar.rs:179-217).
template <> struct KQ<CX_Q5_K> {
  static constexpr int BPB = 176, SUB = 32;
  static constexpr bool ALIGNED = true;
  // header, qh (32 bytes) and the qs of pairs 2h, 2h+1 (64 bytes at 48 + 64h)
  struct Regs {
    uint4 hd, h0, h1, u[4];
  };
  static constexpr int NLOAD = 7;
  __device__ static void load(const uint8_t* blk, int h, Regs& r) {
    const uint4* bw = reinterpret_cast<const uint4*>(blk);
    r.hd = bw[0];
    r.h0 = bw[1];
    r.h1 = bw[2];
#pragma unroll
    for (int i = 0; i < 4; i++) r.u[i] = bw[3 + 4 * h + i];
  }
  __device__ static void half(const uint8_t* lds, uint32_t off, int h, const int8_t* xb,
                              const float* xe, const float* xs, int32_t* dbg, float* to) {
    Regs r;
    load(lds + off, h, r);
    half_regs(r, h, xb, xe, xs, dbg, to);
  }
  __device__ static void half_pre(const Regs& r, int h, const Pre4& a, int32_t* dbg, float* to) {
    const uint4 hd = r.hd, h0 = r.h0, h1 = r.h1;
    const uint32_t qh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    const float d = cx_h2f(hd.x & 0xFFFF), dm = cx_h2f(hd.x >> 16);
    uint32_t sc4, mn4;
    KQ<CX_Q4_K>::scales_mins(h, hd.y, hd.z, hd.w, sc4, mn4);
#pragma unroll
    for (int pp = 0; pp < 2; pp++) {
      const int p = 2 * h + pp;
      const uint4 u0 = r.u[2 * pp], u1 = r.u[2 * pp + 1];
      const uint32_t q[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
      int e0 = 0, e1 = 0;
#pragma unroll
      for (int w = 0; w < 8; w++) {
        const uint32_t lo = (q[w] & M4) | (((qh[w] >> (2 * p)) & M1) << 4);
        const uint32_t hi = ((q[w] >> 4) & M4) | (((qh[w] >> (2 * p + 1)) & M1) << 4);
        e0 = dot4(lo, a.xa[pp][w], e0);
        e1 = dot4(hi, a.xc[pp][w], e1);
      }
      KQ<CX_Q4_K>::term_pre(2 * pp, e0, d, dm, sc4, mn4, a, h, dbg, to);
      KQ<CX_Q4_K>::term_pre(2 * pp + 1, e1, d, dm, sc4, mn4, a, h, dbg, to);
    }
  }
  __device__ static void half_regs(const Regs& r, int h, const int8_t* xb, const float* xe,
                                   const float* xs, int32_t* dbg, float* to) {
    Pre4 a;
    pre4(h, xb, xe, xs, a);
    half_pre(r, h, a, dbg, to);
  }
  // half_pre's four terms into registers (as KQ<CX_Q4_K>::half_t4)
  __device__ static void half_t4(const Regs& r, int h, const Pre4& a, int32_t* dbg,
                                 float (&t)[4]) {
    const uint4 hd = r.hd, h0 = r.h0, h1 = r.h1;
    const uint32_t qh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    const float d = cx_h2f(hd.x & 0xFFFF), dm = cx_h2f(hd.x >> 16);
    uint32_t sc0, mn0, sc1, mn1;
    KQ<CX_Q4_K>::scales_mins(0, hd.y, hd.z, hd.w, sc0, mn0);
    KQ<CX_Q4_K>::scales_mins(1, hd.y, hd.z, hd.w, sc1, mn1);
    const uint32_t sc4 = h ? sc1 : sc0, mn4 = h ? mn1 : mn0;
#pragma unroll
    for (int pp = 0; pp < 2; pp++) {
      const uint4 u0 = r.u[2 * pp], u1 = r.u[2 * pp + 1];
      const uint32_t q[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
      const uint32_t p2 = 2 * (2 * (uint32_t)h + pp);  // pair p = 2h + pp: bits 2p, 2p + 1
      int e0 = 0, e1 = 0;
#pragma unroll
      for (int w = 0; w < 8; w++) {
        const uint32_t lo = (q[w] & M4) | (((qh[w] >> p2) & M1) << 4);
        const uint32_t hi = ((q[w] >> 4) & M4) | (((qh[w] >> (p2 + 1)) & M1) << 4);
        e0 = dot4(lo, a.xa[pp][w], e0);
        e1 = dot4(hi, a.xc[pp][w], e1);
      }
      t[2 * pp] = KQ<CX_Q4_K>::term_val(2 * pp, e0, d, dm, sc4, mn4, a, h, dbg);
      t[2 * pp + 1] = KQ<CX_Q4_K>::term_val(2 * pp + 1, e1, d, dm, sc4, mn4, a, h, dbg);
    }
  }
};

// Shared shape of Q2_K / Q3_K / Q6_K: 16-value sub-blocks. Group g = 0..7
// holds 32 values, positions 0..15 in sub-block 2g and 16..31 in 2g+1. Half
// h owns groups 4h..4h+3, whose 2-bit fields (Q2_K, Q3_K) or nibbles (Q6_K)
// live in the h-th half of the quant bytes.

// ------------------------------------------------------------------ Q2_K
// 84 B: scales(16: low nibble scale, high nibble min) qs(64) d dmin.
// value = (qs[32(g/4) + i] >> 2(g%4)) & 3   (src/kernels/q2k.rs:41-69)
template <> struct KQ<CX_Q2_K> {
  static constexpr int BPB = 84, SUB = 16;
  static constexpr bool ALIGNED = false;
  __device__ static void half(const uint8_t* lds, uint32_t off, int h, const int8_t* xb,
                              const float* xe, const float* xs, int32_t* dbg, float* to) {
    uint32_t sw[2], qw[8], dw[1];
    lds_words<2>(lds, off + 8 * h, sw);  // scales of sub-blocks 8h..8h+7
    lds_words<8>(lds, off + 16 + 32 * h, qw);
    lds_words<1>(lds, off + 80, dw);
    const float d = cx_h2f(dw[0] & 0xFFFF), dm = cx_h2f(dw[0] >> 16);
#pragma unroll
    for (int gi = 0; gi < 4; gi++) {
      const int g = 4 * h + gi, sh = 2 * gi;
      int x[8];
      act8(xb + 32 * g, x);
      int e0 = 0, e1 = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        e0 = dot4((qw[i] >> sh) & M2, x[i], e0);
        e1 = dot4((qw[4 + i] >> sh) & M2, x[4 + i], e1);
      }
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
        const int s8 = 2 * gi + hf, sb = 8 * h + s8, e = hf ? e1 : e0;
        const uint32_t sc = (sw[s8 / 4] >> (8 * (s8 % 4))) & 0xFF;
        if (dbg) dbg[sb] = e;
        to[sb] = xe[sb] * (d * (float)(sc & 0xF) * (float)e - dm * (float)(sc >> 4) * xs[sb]);
      }
    }
  }
};

// ------------------------------------------------------------------ Q3_K
// 110 B: hmask(32) qs(64) scales(12) d. Biased value (q+4) in 0..7 =
// ((qs[32(g/4) + i] >> 2(g%4)) & 3) | ((hmask[i] >> g) & 1) << 2
// (src/kernels/scalar.rs:236-275); scales as quant::escalas_q3k
// (src/quant.rs:87-106): aux words 2h, 2h+1 hold sub-blocks 8h..8h+7
template <> struct KQ<CX_Q3_K> {
  static constexpr int BPB = 110, SUB = 16;
  static constexpr bool ALIGNED = false;
  __device__ static void half(const uint8_t* lds, uint32_t off, int h, const int8_t* xb,
                              const float* xe, const float* xs, int32_t* dbg, float* to) {
    uint32_t hm[8], qw[8], tw[4];
    lds_words<8>(lds, off, hm);
    lds_words<8>(lds, off + 32 + 32 * h, qw);
    lds_words<4>(lds, off + 96, tw);  // scales(12) d(2)
    const float d = cx_h2f(tw[3] & 0xFFFF);
    const uint32_t A = tw[0], B = tw[1], T = tw[2];
    // aux[2h] and aux[2h+1] of escalas_q3k
    const uint32_t X = h ? (A >> 4) : A, Y = h ? (B >> 4) : B, Ts = h ? (T >> 4) : T;
    const uint32_t aux[2] = {(X & M4) | ((Ts & M2) << 4), (Y & M4) | (((Ts >> 2) & M2) << 4)};
#pragma unroll
    for (int gi = 0; gi < 4; gi++) {
      const int g = 4 * h + gi, sh = 2 * gi;
      int x[8];
      act8(xb + 32 * g, x);
      int e0 = 0, e1 = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t v0 = ((qw[i] >> sh) & M2) | (((hm[i] >> g) & M1) << 2);
        const uint32_t v1 = ((qw[4 + i] >> sh) & M2) | (((hm[4 + i] >> g) & M1) << 2);
        e0 = dot4(v0, x[i], e0);
        e1 = dot4(v1, x[4 + i], e1);
      }
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
        const int s8 = 2 * gi + hf, sb = 8 * h + s8, e = hf ? e1 : e0;
        const float esc = (float)(int8_t)(uint8_t)(aux[s8 / 4] >> (8 * (s8 % 4)));
        const float scale = d * (esc - 32.0f);
        if (dbg) dbg[sb] = e;
        to[sb] = xe[sb] * scale * ((float)e - 4.0f * xs[sb]);
      }
    }
  }
};

// ------------------------------------------------------------------ Q6_K
// 210 B: ql(128) qh(64) scales(16, i8) d. Group g: half = g/4, gi = g%4;
// value 0..63 = nib | ((qh[32 half + i] >> 2gi) & 3) << 4, nib = low (gi < 2)
// or high nibble of ql[64 half + 32 (gi%2) + i]   (src/kernels/scalar.rs:294-324)
template <> struct KQ<CX_Q6_K> {
  static constexpr int BPB = 210, SUB = 16;
  static constexpr bool ALIGNED = false;
  __device__ static void half(const uint8_t* lds, uint32_t off, int h, const int8_t* xb,
                              const float* xe, const float* xs, int32_t* dbg, float* to) {
    uint32_t ql[16], qh[8], sw[2], dw[1];
    lds_words<16>(lds, off + 64 * h, ql);
    lds_words<8>(lds, off + 128 + 32 * h, qh);
    lds_words<2>(lds, off + 192 + 8 * h, sw);  // scales of sub-blocks 8h..8h+7
    lds_words<1>(lds, off + 208, dw);
    const float d = cx_h2f(dw[0] & 0xFFFF);
#pragma unroll
    for (int gi = 0; gi < 4; gi++) {
      const int g = 4 * h + gi, lw = 8 * (gi % 2);
      int x[8];
      act8(xb + 32 * g, x);
      int e0 = 0, e1 = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t n0 = gi < 2 ? (ql[lw + i] & M4) : ((ql[lw + i] >> 4) & M4);
        const uint32_t n1 = gi < 2 ? (ql[lw + 4 + i] & M4) : ((ql[lw + 4 + i] >> 4) & M4);
        e0 = dot4(n0 | (((qh[i] >> (2 * gi)) & M2) << 4), x[i], e0);
        e1 = dot4(n1 | (((qh[4 + i] >> (2 * gi)) & M2) << 4), x[4 + i], e1);
      }
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
        const int s8 = 2 * gi + hf, sb = 8 * h + s8, e = hf ? e1 : e0;
        const float scale = d * (float)(int8_t)(uint8_t)(sw[s8 / 4] >> (8 * (s8 % 4)));
        if (dbg) dbg[sb] = e;
        to[sb] = xe[sb] * scale * ((float)e - 32.0f * xs[sb]);
      }
    }
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
  uint32_t lds_act;      // byte offsets in LDS: activation, xe/xs, terms, norm input
  uint32_t lds_scale;
  uint32_t lds_terms;
  uint32_t lds_norm;
  cx_qact act;           // the quantized activation, or
  const float* nx;       // the rmsnorm input and weight it is made from here
  const float* nw;
  float eps;
  int epi;
  int32_t* dbg;
  float* apv;     // per tile: the largest output and its index (the argmax's first step)
  uint32_t* api;
};

// 16-byte chunks [0, n) of global `g` into LDS at `l`, 1 KiB per wave load
// (wave w moves chunks 64*(w + 4j) + lane). Returns the loads this wave
// issued; they are untracked by the compiler (see cx_dma16_async).
__device__ inline uint32_t copy_to_lds(const void* g, void* l, uint32_t n, int wave, int lane) {
  uint32_t issued = 0;
  for (uint32_t c0 = 64u * wave; c0 < n; c0 += 256) {
    if (c0 + lane < n)
      cx_dma16_async(static_cast<const uint8_t*>(g) + 16 * (size_t)(c0 + lane),
                     static_cast<uint8_t*>(l) + 16 * c0);
    issued++;
  }
  return issued;
}

// The activation's 256-byte blocks sit ACT_LDS_BLOCK bytes apart in LDS: the
// lanes of one wave read up to 8 different blocks at once, and a 272-byte
// stride puts them on different LDS banks (a 256-byte stride would put all
// eight on the same ones). The direct loads write 16 bytes per lane at
// consecutive LDS addresses, so the 17th chunk of each block loads a dummy.
constexpr uint32_t ACT_LDS_BLOCK = 272;
__device__ inline void copy_act_padded(const int8_t* xq, int8_t* l, uint32_t nb, int wave,
                                       int lane) {
  const uint32_t n = nb * (ACT_LDS_BLOCK / 16);
  for (uint32_t c0 = 64u * wave; c0 < n; c0 += 256) {
    const uint32_t c = c0 + lane, b = c / 17, r = c % 17;
    if (c < n)
      cx_dma16_async(xq + (r < 16 ? 256 * (size_t)b + 16 * r : 0), l + 16 * c0);
  }
}
// cx_quant8 into the padded LDS layout (8 values never straddle a block)
template <int SUB>
__device__ inline void cx_quant8_padded(const float (&v)[8], uint32_t i, int8_t* sq, float* se,
                                        float* ss) {
  int8_t* blk = sq + (i / 256) * ACT_LDS_BLOCK - (i / 256) * 256;
  cx_quant8<SUB>(v, i, blk, se, ss);
}

// Waits until at most n (wave-uniform) of this wave's loads are outstanding,
// or fewer: a smaller count only waits longer.
__device__ inline void wait_all_but(uint32_t n) {
  if (n >= 48) cx_wait_vm<48>();
  else if (n >= 32) cx_wait_vm<32>();
  else if (n >= 16) cx_wait_vm<16>();
  else if (n >= 8) cx_wait_vm<8>();
  else if (n >= 4) cx_wait_vm<4>();
  else if (n >= 2) cx_wait_vm<2>();
  else cx_wait_vm<0>();
}

// Row tid's epilogue operand: y (CX_EPI_ACCUM: y += acc), else the bias
// (y = acc + bias) or 0. f32 addition is commutative, so acc + addend is
// the reference's y + acc and acc + bias bit for bit.
__device__ inline float epi_addend(const GemvParams& P, const cx_seg& S, uint32_t row0,
                                   uint32_t rows, int tid) {
  if ((uint32_t)tid >= rows) return 0.0f;
  if (P.epi == CX_EPI_ACCUM) return S.y[row0 + tid];
  return S.bias ? S.bias[row0 + tid] : 0.0f;
}

// total = 0; total += term_s for s = 0 .. n-1 (n % 4 == 0), in that order.
// The terms are read eight float4s at a time, and the next 32 are read
// while the current 32 are added: the adds are one dependent chain (~9
// clocks each), and the LDS latency is paid once, not once per batch.
__device__ inline void ld8(const float4* t, float4 (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 8; i++) v[i] = t[i];
}
__device__ inline void add8(float& acc, const float4 (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 8; i++) {
    acc += v[i].x;
    acc += v[i].y;
    acc += v[i].z;
    acc += v[i].w;
  }
}
__device__ inline float row_sum(const float* terms, uint32_t n) {
  const float4* t = reinterpret_cast<const float4*>(terms);
  const uint32_t n4 = n / 4;
  float acc = 0.0f;
  uint32_t s = 0;
  float4 a[8], b[8];
  if (s + 8 <= n4) ld8(t + s, a);
  while (s + 8 <= n4) {  // a holds batch s
    const bool more = s + 16 <= n4;
    if (more) ld8(t + s + 8, b);
    add8(acc, a);
    s += 8;
    if (!more) break;  // b holds batch s
    const bool more2 = s + 16 <= n4;
    if (more2) ld8(t + s + 8, a);
    add8(acc, b);
    s += 8;
    if (!more2) break;
  }
  for (; s < n4; s++) {
    const float4 v = t[s];
    acc += v.x;
    acc += v.y;
    acc += v.z;
    acc += v.w;
  }
  return acc;
}

template <int T, bool NORM>
__global__ __launch_bounds__(256) void k_gemv(GemvParams P) {
  using Q = KQ<T>;
  constexpr int SPB = 256 / Q::SUB;  // sub-blocks per super-block
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ double red[9];
  __shared__ int nflag;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t tile = blockIdx.x;
  int sg = 0;
  while (tile >= P.tile_end[sg]) sg++;
  if (sg) tile -= P.tile_end[sg - 1];
  const cx_seg S = P.seg[sg];
  const uint32_t row0 = tile * P.R;
  const uint32_t rows = min(P.R, S.rows - row0);
  // the epilogue's other operand (the residual, or the bias), loaded first:
  // its latency passes under the tile's, not after the row sum
  const float addend = epi_addend(P, S, row0, rows, tid);
  int8_t* sq = reinterpret_cast<int8_t*>(lds + P.lds_act);
  float* se = reinterpret_cast<float*>(lds + P.lds_scale);
  float* ss = se + P.nsub;
  float* sx = reinterpret_cast<float*>(lds + P.lds_norm);

  // 1. every input into LDS with direct loads: the rmsnorm input first (so
  //    the prologue can start before the weights land), then the tile (rows *
  //    row_bytes contiguous bytes, `skew` bytes into LDS when the rows are not
  //    16-byte aligned: Q2_K/Q3_K/Q6_K rows of some widths), then the
  //    quantized activation when it comes ready-made
  if (NORM) {
    copy_to_lds(P.nx, sx, P.k / 4, wave, lane);
    copy_to_lds(P.nw, sx + P.k, P.k / 4, wave, lane);
  }
  const uint8_t* src = S.w + (size_t)row0 * P.row_bytes;
  const uint32_t skew = (uint32_t)((uintptr_t)src & 15u);
  const uint32_t ntile =
      copy_to_lds(src - skew, lds, (skew + rows * P.row_bytes + 15) >> 4, wave, lane);
  if (!NORM) {
    copy_act_padded(P.act.xq, sq, P.nb, wave, lane);
    copy_to_lds(P.act.xe, se, P.nsub / 4, wave, lane);
    copy_to_lds(P.act.xs, ss, P.nsub / 4, wave, lane);
  }
  // rmsnorm (src/kernels/scalar.rs:40-53) and quantization of the
  // activation while the weights stream in: f64 sum of squares (8
  // consecutive values a lane, a tree), scale = 1/sqrt(sum/k + eps),
  // v = (x as f64 * scale) as f32 * w, then ops::cuantizar_i8_en; the
  // reference's factor bit for bit (cx_rms_reach: the sum in order when an
  // output could round apart)
  const float* sw = sx + P.k;
  double scale = 0.0;
  uint32_t reach = 0, c = 0;
  if (NORM) {
    wait_all_but(ntile);
    if (tid == 0) nflag = 0;
    cx_barrier();  // every wave's share of x and w has landed
    cx_rms_part part;
    for (uint32_t i = 8 * tid; i < P.k; i += 2048) {
      float a[8];
      cx_load8(sx + i, a);  // two 16-byte LDS reads
      part.add<8>(a, i, P.k);
    }
    part = cx_wave_sum_rms(part);
    if (lane == 0) {
      red[wave] = part.s;
      red[4 + wave] = (double)part.w;
    }
    cx_wait_lds();
    cx_barrier();
    const double tot = ((red[0] + red[1]) + red[2]) + red[3];
    const float wt = (float)(((red[4] + red[5]) + red[6]) + red[7]);
    scale = cx_rms_factor(tot, P.k, P.eps);
    reach = cx_rms_reach(tot, wt, P.k, P.k / 256 + 16);
    c = cx_rms_c(reach);
  }
  // the activation from the tree's factor; a second pass, when an output
  // could round apart, from the sum in order
#pragma unroll 1
  for (int pass = 0;; pass++) {
    if (NORM) {
      cx_rms_risk risk;
      for (uint32_t i = 8 * tid; i < P.k; i += 2048) {
        float v[8], a[8], b[8];
        cx_load8(sx + i, a);
        cx_load8(sw + i, b);
#pragma unroll
        for (int j = 0; j < 8; j++) {
          risk.add(a[j], scale, c);
          v[j] = (float)((double)a[j] * scale) * b[j];
        }
        cx_quant8_padded<Q::SUB>(v, i, sq, se, ss);
      }
      if (pass == 0 && reach && risk.unsure(reach)) nflag = 1;
    }
    cx_wait_vm<0>();  // every direct load has landed
    cx_wait_lds();
    __syncthreads();
    if (!NORM || pass == 1 || !nflag) break;  // the same for every thread
    if (wave == 0) {
      const double seq = cx_rms_seq_sum(sx, P.k);
      if (lane == 0) red[8] = seq;
    }
    __syncthreads();
    scale = cx_rms_factor(red[8], P.k, P.eps);
  }

  // 2. integer dots + the reference's per-sub-block f32 terms, staged in LDS
  //    by (row, sub-block): two lanes per (row, super-block)
  float* terms = reinterpret_cast<float*>(lds + P.lds_terms);
  const uint32_t items = 2 * rows * P.nb;
  for (uint32_t it = tid; it < items; it += 256) {
    const uint32_t q = it >> 1, r = q / P.nb, blk = q - r * P.nb;
    const int h = (int)(it & 1);
    int32_t* dbg = P.dbg ? P.dbg + (size_t)(row0 + r) * P.nsub + blk * SPB : nullptr;
    Q::half(lds, skew + r * P.row_bytes + blk * Q::BPB, h, sq + blk * ACT_LDS_BLOCK,
            se + blk * SPB, ss + blk * SPB, dbg, terms + r * P.tstride + blk * SPB);
  }
  __syncthreads();

  // 3. the row's sum in the scalar spec's order: total = 0; total += term_s
  //    for s = 0, 1, ... (src/kernels/scalar.rs:141-167)
  if ((uint32_t)tid < rows) {
    const float acc = row_sum(terms + tid * P.tstride, P.nsub);
    const uint32_t row = row0 + tid;
    S.y[row] = (P.epi == CX_EPI_ACCUM || S.bias) ? acc + addend : acc;
  }
}

// The same GEMV for Q4_K/Q5_K (16-byte aligned blocks) with the weights
// loaded straight into VGPRs: each weight byte is used once, so staging it in
// LDS only costs LDS bandwidth (the direct-load write and the read). Each
// lane loads the bytes of its (row, super-block, half) items — the first
// one's loads are in flight from the start, each later one is loaded while
// the previous one is computed — and LDS holds only the shared activation and
// the terms.
template <int T>
__global__ __launch_bounds__(256) void k_gemv_reg(GemvParams P) {
  using Q = KQ<T>;
  constexpr int SPB = 256 / Q::SUB;
  extern __shared__ __align__(16) uint8_t lds[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t tile = blockIdx.x;
  int sg = 0;
  while (tile >= P.tile_end[sg]) sg++;
  if (sg) tile -= P.tile_end[sg - 1];
  const cx_seg S = P.seg[sg];
  const uint32_t row0 = tile * P.R;
  const uint32_t rows = min(P.R, S.rows - row0);
  // the epilogue's other operand (the residual, or the bias), loaded first:
  // its latency passes under the tile's, not after the row sum
  const float addend = epi_addend(P, S, row0, rows, tid);
  int8_t* sq = reinterpret_cast<int8_t*>(lds + P.lds_act);
  float* se = reinterpret_cast<float*>(lds + P.lds_scale);
  float* ss = se + P.nsub;
  float* terms = reinterpret_cast<float*>(lds + P.lds_terms);

  copy_act_padded(P.act.xq, sq, P.nb, wave, lane);
  copy_to_lds(P.act.xe, se, P.nsub / 4, wave, lane);
  copy_to_lds(P.act.xs, ss, P.nsub / 4, wave, lane);
  const uint32_t items = 2 * rows * P.nb;
  auto block_of = [&](uint32_t it) {
    const uint32_t q = it >> 1, r = q / P.nb, blk = q - r * P.nb;
    return S.w + (size_t)(row0 + r) * P.row_bytes + (size_t)blk * Q::BPB;
  };
  // a two-slot ring: the lane's first two items are loaded from the start
  // (a wave's loads complete in order, so waiting for all but its weight
  // loads waits for the activation); item j + 2 is loaded into item j's
  // slot once j is computed
  typename Q::Regs buf[2];
  const uint32_t wave_first = tid & ~63u;  // wave-uniform count of item loads issued
  const uint32_t issued = (wave_first < items) + (wave_first + 256 < items);
  if (tid < items) Q::load(block_of(tid), (int)(tid & 1), buf[0]);
  if (tid + 256 < items) Q::load(block_of(tid + 256), (int)((tid + 256) & 1), buf[1]);
  if (issued == 2) cx_wait_vm<2 * Q::NLOAD>();
  else if (issued == 1) cx_wait_vm<Q::NLOAD>();
  else cx_wait_vm<0>();  // a wave with no items: its activation loads only
  cx_barrier();
  for (uint32_t base = tid; base < items; base += 512) {
#pragma unroll
    for (int d = 0; d < 2; d++) {
      const uint32_t it = base + 256u * d;
      if (it < items) {
        const uint32_t q = it >> 1, r = q / P.nb, blk = q - r * P.nb;
        int32_t* dbg = P.dbg ? P.dbg + (size_t)(row0 + r) * P.nsub + blk * SPB : nullptr;
        Q::half_regs(buf[d], (int)(it & 1), sq + blk * ACT_LDS_BLOCK, se + blk * SPB,
                     ss + blk * SPB, dbg, terms + r * P.tstride + blk * SPB);
        const uint32_t nx = it + 512;
        if (nx < items) Q::load(block_of(nx), (int)(nx & 1), buf[d]);
      }
    }
  }
  __syncthreads();

  // the row's sum in the scalar spec's order (src/kernels/scalar.rs:141-167)
  if ((uint32_t)tid < rows) {
    const float acc = row_sum(terms + tid * P.tstride, P.nsub);
    const uint32_t row = row0 + tid;
    S.y[row] = (P.epi == CX_EPI_ACCUM || S.bias) ? acc + addend : acc;
  }
}

// The plain Q4_K/Q5_K GEMV for rows of NB = 8 or 16 super-blocks (k = 2048
// or 4096), one (row, super-block, half) item a lane: the row's 2*NB lanes
// are consecutive lanes of one wave, lane 2b + h holding half h of
// super-block b, so its four terms are terms 8b + 4h .. 8b + 4h + 3 of the
// row. The scalar spec's sum (total = 0; total += term_s in order,
// src/kernels/scalar.rs:141-167) then runs along the lanes: at step s every
// lane takes its left neighbour's running sum (DPP wave_shr:1, lane 0 reads
// +0.0) and adds its four terms in order, so after 2*NB steps the row's last
// lane holds the row total, rounded add by add as the reference rounds it.
// Every lane starts at +0.0, so the first lane of each row also reads +0.0
// at step 0, and at step s lane 2*NB*r + s reads lane 2*NB*r + s - 1 of the
// same row. No workgroup barrier follows the loads: the activation (k bytes
// + 2k/32 floats) is the only data shared across waves, and it arrives from
// L2 long before the weights, which go straight from HBM into registers, a
// lane's 80 (Q4_K) or 112 (Q5_K) bytes issued at the start.
// Chunk c of the activation of a row-kernel launch, 16 bytes: xq's NB*16
// chunks, then xe's NB*2 and xs's NB*2 (c past the end: the last one). The
// address is picked with masks, not branches: a load behind branches is
// issued late.
template <int NB>
__device__ inline int4 row_act_load(uint64_t xq, uint64_t xe, uint64_t xs, int c) {
  constexpr int NX = NB * 16, NE = NB * 2;
  c = min(c, NX + 2 * NE - 1);
  const uint64_t me = 0 - (uint64_t)(c >= NX), ms = 0 - (uint64_t)(c >= NX + NE);
  uint64_t a = xq + 16 * (uint64_t)c;
  a = (a & ~me) | ((xe + 16 * (uint64_t)(c - NX)) & me);
  a = (a & ~ms) | ((xs + 16 * (uint64_t)(c - NX - NE)) & ms);
  return *(const int4*)reinterpret_cast<const __attribute__((address_space(1))) int4*>(a);
}
// ... and its place in LDS (xq blocks ACT_LDS_BLOCK bytes apart)
template <int NB>
__device__ inline void row_act_store(int8_t* sq, float* se, float* ss, int c, const int4& v) {
  constexpr int NX = NB * 16, NE = NB * 2;
  if (c >= NX + 2 * NE) return;
  int4* p = c < NX ? reinterpret_cast<int4*>(sq + (c >> 4) * ACT_LDS_BLOCK + 16 * (c & 15))
            : c < NX + NE ? reinterpret_cast<int4*>(se) + (c - NX)
                          : reinterpret_cast<int4*>(ss) + (c - NX - NE);
  *p = v;
}
template <int T, int NB, bool MULTI, bool DBG, bool AMAX = false>
__global__ __launch_bounds__(1024) void k_gemv_row(GemvParams P) {
  using Q = KQ<T>;
  constexpr int AP = (NB * 20 + 63) / 64;  // activation chunks a lane of wave 0 loads
  constexpr int LPR = 2 * NB;     // lanes per row
  constexpr int RPW = 64 / LPR;   // rows per wave
  __shared__ __align__(16) int8_t sq[NB * ACT_LDS_BLOCK];
  __shared__ __align__(16) float se[8 * NB], ss[8 * NB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the kernel arguments the loads need, read up front in one batch of
  // scalar loads (the empty asms hold them in SGPRs here; left alone, the
  // compiler reads each one where it is first used, a round trip each)
  uint64_t xq = (uint64_t)P.act.xq, xe = (uint64_t)P.act.xe, xs = (uint64_t)P.act.xs;
  uint32_t tile = blockIdx.x;
  int sg = 0;
  if constexpr (MULTI) {
    while (tile >= P.tile_end[sg]) sg++;
    if (sg) tile -= P.tile_end[sg - 1];
  }
  const cx_seg S = P.seg[sg];
  uint64_t wbase = (uint64_t)S.w;
  uint32_t R = P.R, rb = P.row_bytes, srows = S.rows;
  asm volatile("" : "+s"(xq), "+s"(xe), "+s"(xs), "+s"(wbase), "+s"(R), "+s"(rb), "+s"(srows));
  const uint32_t row0 = tile * R;
  const uint32_t rows = min(R, srows - row0);
  const uint32_t lr = (uint32_t)(wave * RPW + lane / LPR);  // the lane's row in the tile
  const int b = (lane % LPR) >> 1, h = lane & 1;
  const bool owner = lr < rows && lane % LPR == LPR - 1;     // stores the row

  // 1. wave 0 loads the activation's 16-byte chunks into registers (L2
  //    hits; a lane past the last chunk reloads it), every wave its weights.
  //    Named registers, not an array: an array here ends up in memory.
  //    (Activation loads spread over every wave measured 0.3 us slower at
  //    config 1: each wave's weight loads then queue behind its share.)
  int4 av0{}, av1{}, av2{}, av3{}, av4{};
  if (wave == 0) {
    av0 = row_act_load<NB>(xq, xe, xs, lane);
    av1 = row_act_load<NB>(xq, xe, xs, lane + 64);
    av2 = row_act_load<NB>(xq, xe, xs, lane + 128);
    if constexpr (AP > 3) av3 = row_act_load<NB>(xq, xe, xs, lane + 192);
    if constexpr (AP > 4) av4 = row_act_load<NB>(xq, xe, xs, lane + 256);
  }
  __builtin_amdgcn_sched_barrier(0);
  typename Q::Regs r;
  const uint32_t row = row0 + (lr < rows ? lr : rows - 1);
  // (an address formed from an integer is generic; cast through the global
  // address space, the loads are global loads)
  Q::load((const uint8_t*)reinterpret_cast<const __attribute__((address_space(1))) uint8_t*>(wbase) +
              (size_t)row * rb + (size_t)b * Q::BPB, h, r);
  const bool add = P.epi == CX_EPI_ACCUM || S.bias;
  const float* addp = P.epi == CX_EPI_ACCUM ? S.y : S.bias;
  const float addend = add ? addp[row] : 0.0f;
  __builtin_amdgcn_sched_barrier(0);
  if (wave == 0) {
    row_act_store<NB>(sq, se, ss, lane, av0);
    row_act_store<NB>(sq, se, ss, lane + 64, av1);
    row_act_store<NB>(sq, se, ss, lane + 128, av2);
    if constexpr (AP > 3) row_act_store<NB>(sq, se, ss, lane + 192, av3);
    if constexpr (AP > 4) row_act_store<NB>(sq, se, ss, lane + 256, av4);
  }
  // a plain barrier (__syncthreads() would also wait for the weights), and
  // nothing that needs the weights moved above it
  __builtin_amdgcn_sched_barrier(0);
  cx_wait_lds();
  cx_barrier();
  __builtin_amdgcn_sched_barrier(0);

  // 2. the lane's four terms
  Pre4 a;
  pre4(h, sq + b * ACT_LDS_BLOCK, se + 8 * b, ss + 8 * b, a);
  int32_t* dbg = DBG ? P.dbg + (size_t)row * P.nsub + 8 * b : nullptr;
  float t[4];
  Q::half_t4(r, h, a, DBG && lr < rows ? dbg : nullptr, t);

  // 3. the row sums along the lanes
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < LPR; s++) {
    float v = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x138, 0xF, 0xF,
                                                         true));  // wave_shr:1
    v += t[0];
    v += t[1];
    v += t[2];
    v += t[3];
    acc = v;
  }
  const float y = add ? acc + addend : acc;
  if (owner) S.y[row] = y;
  if constexpr (AMAX) {
    // the tile's (largest output, its row) for the argmax, NaN left out:
    // every row slot's last lane, then one wave over the slots (rows past
    // the matrix hold the empty pair)
    static_assert(!MULTI, "one matrix");
    __shared__ VI am[64];
    if (lane % LPR == LPR - 1)
      am[lr] = lr < rows && !(y != y) ? VI{y, row0 + lr} : VI{-INFINITY, 0xFFFFFFFFu};
    __syncthreads();
    if (wave == 0) {
      VI best = (uint32_t)lane < R ? am[lane] : VI{-INFINITY, 0xFFFFFFFFu};
      best = vi_wave(best);
      if (lane == 0) {
        P.apv[tile] = best.v;
        P.api[tile] = best.i;
      }
    }
  }
}

// The row kernel with the rmsnorm prologue (the q/k/v launch): every
// workgroup makes the normalized, quantized activation itself from the f32
// residual x and the norm weight w while its weights are in flight. The
// f64 sum of squares is a tree over 256 virtual lanes, lane v holding
// x[8v + 2048j + e]^2 summed over j, then e, in order; each virtual wave's
// butterfly (cx_wave_sum_d); ((r0 + r1) + r2) + r3. With W < 4 waves a
// thread holds 4/W virtual lanes (virtual wave w + W m), with W > 4 only
// waves 0-3 take part. The factor is the reference's bit for bit
// (cx_rms_reach: the sum in order when an output could round apart). The
// normalization and quantization (src/kernels/scalar.rs:40-53, then
// ops::cuantizar_i8_en) use the same groups of 8 values, into LDS.
template <int T, int NB, int W, bool MULTI>
__global__ __launch_bounds__(64 * W) void k_gemv_row_norm(GemvParams P) {
  using Q = KQ<T>;
  constexpr int LPR = 2 * NB;     // lanes per row
  constexpr int RPW = 64 / LPR;   // rows per wave
  constexpr int NT = 64 * W;
  constexpr int VT = NT >= 256 ? 1 : 256 / NT;  // virtual lanes a thread
  constexpr int GJ = NB / 8;                    // 8-value groups a virtual lane (k / 2048)
  static_assert(W == 1 || W == 2 || W == 4 || W == 8 || W == 16, "power-of-two waves");
  __shared__ __align__(16) int8_t sq[NB * ACT_LDS_BLOCK];
  __shared__ __align__(16) float se[8 * NB], ss[8 * NB];
  __shared__ double red[9];
  __shared__ int nflag;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint64_t xb = (uint64_t)P.nx, wb = (uint64_t)P.nw;
  uint32_t tile = blockIdx.x;
  int sg = 0;
  if constexpr (MULTI) {
    // the tile ends and the count in one batch, then three compares (a
    // search loop waited for one load after another)
    const uint32_t e0 = P.tile_end[0], e1 = P.tile_end[1], e2 = P.tile_end[2];
    const int n = P.nseg;
    sg = (n > 1 && tile >= e0) + (n > 2 && tile >= e1) + (n > 3 && tile >= e2);
    tile -= sg == 0 ? 0u : sg == 1 ? e0 : sg == 2 ? e1 : e2;
  }
  const cx_seg S = P.seg[sg];
  uint64_t wbase = (uint64_t)S.w;
  uint32_t R = P.R, rb = P.row_bytes, srows = S.rows;
  asm volatile("" : "+s"(xb), "+s"(wb), "+s"(wbase), "+s"(R), "+s"(rb), "+s"(srows));
  const uint32_t row0 = tile * R;
  const uint32_t rows = min(R, srows - row0);
  const uint32_t lr = (uint32_t)(wave * RPW + lane / LPR);
  const int b = (lane % LPR) >> 1, h = lane & 1;
  const bool owner = lr < rows && lane % LPR == LPR - 1;

  // 1. x and w of the thread's groups (L2 hits; with more than 256 threads
  //    only the first 256, the tree's, load them: a CU's loads pass its
  //    address unit at a bounded rate, and at k = 4096 the other twelve
  //    waves' copies held back the weights' issue by ~2 us), then the weights
  const float4* const xg = (const float4*)reinterpret_cast<const __attribute__((address_space(1))) float4*>(xb);
  const float4* const wg = (const float4*)reinterpret_cast<const __attribute__((address_space(1))) float4*>(wb);
  float4 xv[VT * GJ * 2], wv[VT * GJ * 2];
  if (NT <= 256 || tid < 256) {  // whole waves
#pragma unroll
    for (int m = 0; m < VT; m++)
#pragma unroll
      for (int j = 0; j < GJ; j++) {
        const uint32_t g = (uint32_t)(tid + NT * m) + 256u * (uint32_t)j;
        xv[2 * (m * GJ + j)] = xg[2 * g];
        xv[2 * (m * GJ + j) + 1] = xg[2 * g + 1];
        wv[2 * (m * GJ + j)] = wg[2 * g];
        wv[2 * (m * GJ + j) + 1] = wg[2 * g + 1];
      }
  } else {
#pragma unroll
    for (int i = 0; i < VT * GJ * 2; i++) xv[i] = wv[i] = float4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  __builtin_amdgcn_sched_barrier(0);
  typename Q::Regs r;
  const uint32_t row = row0 + (lr < rows ? lr : rows - 1);
  Q::load((const uint8_t*)reinterpret_cast<const __attribute__((address_space(1))) uint8_t*>(wbase) +
              (size_t)row * rb + (size_t)b * Q::BPB, h, r);
  const bool add = P.epi == CX_EPI_ACCUM || S.bias;
  const float* addp = P.epi == CX_EPI_ACCUM ? S.y : S.bias;
  const float addend = add ? addp[row] : 0.0f;
  __builtin_amdgcn_sched_barrier(0);

  // 2. the f64 sum of squares over the tree, with the bound's weighted sum
  constexpr uint32_t K = NB * 256;
  const bool in_tree = NT <= 256 || tid < 256;
  if (tid == 0) nflag = 0;
#pragma unroll
  for (int m = 0; m < VT; m++) {
    cx_rms_part part;
#pragma unroll
    for (int j = 0; j < GJ; j++) {
      const float4 a0 = xv[2 * (m * GJ + j)], a1 = xv[2 * (m * GJ + j) + 1];
      const float a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      const uint32_t g = min((uint32_t)(tid + NT * m), 255u) + 256u * (uint32_t)j;
      part.add<8>(a, 8 * g, K);
    }
    part = cx_wave_sum_rms(part);
    if (in_tree && lane == 0) {
      red[wave + W * m] = part.s;
      red[4 + wave + W * m] = (double)part.w;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  cx_wait_lds();
  cx_barrier();
  __builtin_amdgcn_sched_barrier(0);
  const double tot = ((red[0] + red[1]) + red[2]) + red[3];
  const float wt = (float)(((red[4] + red[5]) + red[6]) + red[7]);
  // 3. v = (x as f64 * scale) as f32 * w, quantized into LDS, from the
  //    tree's factor; a second pass, when an output could round apart, from
  //    the sum in order (x from L2). The lane's activation for step 4 is
  //    read with the flag.
  double scale = cx_rms_factor(tot, K, P.eps);
  const uint32_t reach = cx_rms_reach(tot, wt, K, 8 * GJ + 16);
  const uint32_t c = cx_rms_c(reach);
  Pre4 a;
#pragma unroll 1
  for (int pass = 0;; pass++) {
    cx_rms_risk risk;
    if (in_tree) {
#pragma unroll
      for (int m = 0; m < VT; m++)
#pragma unroll
        for (int j = 0; j < GJ; j++) {
          const float4 a0 = xv[2 * (m * GJ + j)], a1 = xv[2 * (m * GJ + j) + 1];
          const float4 b0 = wv[2 * (m * GJ + j)], b1 = wv[2 * (m * GJ + j) + 1];
          const float x8[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
          const float bw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
          float v[8];
#pragma unroll
          for (int q = 0; q < 8; q++) {
            risk.add(x8[q], scale, c);
            v[q] = (float)((double)x8[q] * scale) * bw[q];
          }
          const uint32_t g = (uint32_t)(tid + NT * m) + 256u * (uint32_t)j;
          cx_quant8_padded<Q::SUB>(v, 8 * g, sq, se, ss);
        }
    }
    if (pass == 0 && reach && risk.unsure(reach)) nflag = 1;
    __builtin_amdgcn_sched_barrier(0);
    cx_wait_lds();
    cx_barrier();
    __builtin_amdgcn_sched_barrier(0);
    pre4(h, sq + b * ACT_LDS_BLOCK, se + 8 * b, ss + 8 * b, a);
    if (pass == 1 || !nflag) break;  // the same for every thread
    if (wave == 0) {
      const double seq = cx_rms_seq_sum(P.nx, K);
      if (lane == 0) red[8] = seq;
    }
    cx_wait_lds();
    cx_barrier();
    scale = cx_rms_factor(red[8], K, P.eps);
  }
  // 4. the lane's four terms and the row sums along the lanes (k_gemv_row)
  float t[4];
  Q::half_t4(r, h, a, nullptr, t);
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < LPR; s++) {
    float v = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x138, 0xF, 0xF,
                                                         true));  // wave_shr:1
    v += t[0];
    v += t[1];
    v += t[2];
    v += t[3];
    acc = v;
  }
  if (owner) S.y[row] = add ? acc + addend : acc;
}

// k_gemv_reg with one (row, super-block, half) item a lane: the launch has
// 2 * R * nb lanes rounded up to a wave (at most 1024), and every lane's
// loads are issued at the start. Used where that fits (the 3B down
// projection: 8 rows of 43 super-blocks, 688 items, 11 waves): k_gemv_reg's
// two-slot ring loads a lane's third item only once its first is computed,
// and the launch waits for that round trip (7.68 -> 7.12 us at 2048 x 11008).
template <int T>
__global__ __launch_bounds__(1024) void k_gemv_reg1(GemvParams P) {
  using Q = KQ<T>;
  constexpr int SPB = 256 / Q::SUB;
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t tile = blockIdx.x;
  int sg = 0;
  while (tile >= P.tile_end[sg]) sg++;
  if (sg) tile -= P.tile_end[sg - 1];
  const cx_seg S = P.seg[sg];
  const uint32_t row0 = tile * P.R;
  const uint32_t rows = min(P.R, S.rows - row0);
  const float addend = epi_addend(P, S, row0, rows, tid);
  int8_t* sq = reinterpret_cast<int8_t*>(lds + P.lds_act);
  float* se = reinterpret_cast<float*>(lds + P.lds_scale);
  float* ss = se + P.nsub;
  float* terms = reinterpret_cast<float*>(lds + P.lds_terms);
  // the activation into LDS by waves 0-3 (the copies' wave strides assume
  // four waves), then each lane's item
  if (wave < 4) {
    copy_act_padded(P.act.xq, sq, P.nb, wave, lane);
    copy_to_lds(P.act.xe, se, P.nsub / 4, wave, lane);
    copy_to_lds(P.act.xs, ss, P.nsub / 4, wave, lane);
  }
  const uint32_t items = 2 * rows * P.nb;
  const uint32_t it = (uint32_t)tid;
  const uint32_t q = it >> 1, r = q / P.nb, blk = q - r * P.nb;
  typename Q::Regs buf;
  if (it < items)
    Q::load(S.w + (size_t)(row0 + r) * P.row_bytes + (size_t)blk * Q::BPB, (int)(it & 1), buf);
  // a wave's loads complete in order: waiting for all but its item's loads
  // waits for its activation loads (a wave with no item: all of them)
  if ((uint32_t)(tid & ~63) < items) cx_wait_vm<Q::NLOAD>();
  else cx_wait_vm<0>();
  cx_barrier();
  if (it < items) {
    int32_t* dbg = P.dbg ? P.dbg + (size_t)(row0 + r) * P.nsub + blk * SPB : nullptr;
    Q::half_regs(buf, (int)(it & 1), sq + blk * ACT_LDS_BLOCK, se + blk * SPB, ss + blk * SPB, dbg,
                 terms + r * P.tstride + blk * SPB);
  }
  __syncthreads();

  // the row's sum in the scalar spec's order (src/kernels/scalar.rs:141-167)
  if ((uint32_t)tid < rows) {
    const float acc = row_sum(terms + tid * P.tstride, P.nsub);
    const uint32_t row = row0 + tid;
    S.y[row] = (P.epi == CX_EPI_ACCUM || S.bias) ? acc + addend : acc;
  }
}

// The plain Q4_K/Q5_K GEMV for long rows (the down projections: k = 11008,
// 43 super-blocks, or 14336, 56; any 16 < nb <= 64): one row a wave, lane
// b < nb holding super-block b whole, both halves' eight terms in order. The
// scalar spec's sum (total = 0; total += term_s, src/kernels/scalar.rs:
// 141-167) runs along the row's lanes as in k_gemv_row: nb steps, each
// taking the left neighbour's running sum (wave_shr:1, lane 0 reads +0.0)
// and adding the lane's eight terms, so after step s lane s holds terms
// 0 .. 8s + 7 summed from +0.0 in order, and lane nb - 1 ends with the row
// total. Lanes past nb reload the last block; lanes below them never read
// their sums. No term passes through LDS and no barrier waits for the
// weights: a wave starts its chain once its own row has landed. With nb a
// template argument (NB > 0) the chain is unrolled: a dependent f32 add
// issues every ~4.5 clocks on gfx950, and a loop's branch per step cost as
// much again. The activation (nb*20 chunks of 16 bytes: xq, then xe, then
// xs) is loaded by every thread, ROWL_AP chunks each, and staged in LDS as
// in k_gemv_row.
constexpr uint32_t ROWL_NB_MAX = 64;
template <int W>
struct RowlShape {
  static constexpr uint32_t AP = (ROWL_NB_MAX * 20 + 64 * W - 1) / (64 * W);
};
__device__ inline int4 rowl_act_load(const cx_qact& act, uint32_t nb, uint32_t c) {
  const uint32_t nx = nb * 16, ne = nb * 2;
  const int4* p = c < nx        ? reinterpret_cast<const int4*>(act.xq) + c
                  : c < nx + ne ? reinterpret_cast<const int4*>(act.xe) + (c - nx)
                                : reinterpret_cast<const int4*>(act.xs) + (c - nx - ne);
  return *p;
}
__device__ inline float rowl_step(float acc, const float (&t)[8]) {
  float v = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x138, 0xF, 0xF,
                                                       true));  // wave_shr:1
#pragma unroll
  for (int j = 0; j < 8; j++) v += t[j];
  return v;
}
template <int T, int W, int NB>
__global__ __launch_bounds__(64 * W) void k_gemv_rowl(GemvParams P) {
  using Q = KQ<T>;
  constexpr uint32_t AP = NB ? (NB * 20 + 64 * W - 1) / (64 * W) : RowlShape<W>::AP;
  constexpr uint32_t NBL = NB ? NB : ROWL_NB_MAX;  // LDS blocks
  __shared__ __align__(16) int8_t sq[NBL * ACT_LDS_BLOCK];
  __shared__ __align__(16) float se[8 * NBL], ss[8 * NBL];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t tile = blockIdx.x;
  int sg = 0;
  while (tile >= P.tile_end[sg]) sg++;
  if (sg) tile -= P.tile_end[sg - 1];
  const cx_seg S = P.seg[sg];
  const uint32_t nb = NB ? (uint32_t)NB : P.nb, nch = nb * 20;
  const uint32_t row0 = tile * W;
  const uint32_t rows = min((uint32_t)W, S.rows - row0);
  const uint32_t row = row0 + min((uint32_t)wave, rows - 1);
  const uint32_t b = min((uint32_t)lane, nb - 1);
  // 1. the thread's activation chunks (L2 hits; past the end: the last one),
  //    then the row's weights straight into registers
  int4 av[AP];
  // (a local copy: handed P.act itself, the compiler picked each lane's
  // pointer out of the kernel arguments with a vector load and waited for
  // it before the activation's load, two round trips instead of one)
  const cx_qact act = P.act;
#pragma unroll
  for (uint32_t i = 0; i < AP; i++) av[i] = rowl_act_load(act, nb, min(tid + 64 * W * i, nch - 1));
  __builtin_amdgcn_sched_barrier(0);
  typename Q::Regs r0, r1;
  const uint8_t* blk = S.w + (size_t)row * P.row_bytes + (size_t)b * Q::BPB;
  Q::load(blk, 0, r0);
  Q::load(blk, 1, r1);
  const bool add = P.epi == CX_EPI_ACCUM || S.bias;
  const float* addp = P.epi == CX_EPI_ACCUM ? S.y : S.bias;
  const float addend = add ? addp[row] : 0.0f;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (uint32_t i = 0; i < AP; i++) {
    const uint32_t c = tid + 64 * W * i;
    if (c >= nch) continue;
    const uint32_t nx = nb * 16, ne = nb * 2;
    int4* p = c < nx        ? reinterpret_cast<int4*>(sq + (c >> 4) * ACT_LDS_BLOCK + 16 * (c & 15))
              : c < nx + ne ? reinterpret_cast<int4*>(se) + (c - nx)
                            : reinterpret_cast<int4*>(ss) + (c - nx - ne);
    *p = av[i];
  }
  // a plain barrier (__syncthreads() would also wait for the weights)
  __builtin_amdgcn_sched_barrier(0);
  cx_wait_lds();
  cx_barrier();
  __builtin_amdgcn_sched_barrier(0);
  // 2. the lane's eight terms: half 0's sub-blocks 0-3, then half 1's 4-7
  float t[8];
  {
    Pre4 a;
    float t4[4];
    pre4(0, sq + b * ACT_LDS_BLOCK, se + 8 * b, ss + 8 * b, a);
    Q::half_t4(r0, 0, a, nullptr, t4);
#pragma unroll
    for (int j = 0; j < 4; j++) t[j] = t4[j];
    pre4(1, sq + b * ACT_LDS_BLOCK, se + 8 * b, ss + 8 * b, a);
    Q::half_t4(r1, 1, a, nullptr, t4);
#pragma unroll
    for (int j = 0; j < 4; j++) t[4 + j] = t4[j];
  }
  // 3. the row sum along the lanes
  float acc = 0.0f;
  if constexpr (NB > 0) {
#pragma unroll
    for (int s = 0; s < NB; s++) acc = rowl_step(acc, t);
  } else {
    for (uint32_t s = 0; s < nb; s++) acc = rowl_step(acc, t);
  }
  if ((uint32_t)wave < rows && (uint32_t)lane == nb - 1) S.y[row] = add ? acc + addend : acc;
}

// total = 0; total += term_s for s = 0 .. n-1 (any n), in that order
__device__ inline float row_sum_any(const float* terms, uint32_t n) {
  float acc = row_sum(terms, n & ~3u);
  for (uint32_t s = n & ~3u; s < n; s++) acc += terms[s];
  return acc;
}

// ------------------------------------- gate/up + SwiGLU in one launch
// The MLP's first half of one decode step (src/forward.rs:472-487) for
// gate and up of one type (Q4_K or Q5_K): tile t holds gate rows
// [32t, 32t+32) and the same rows of up. Every workgroup makes the rmsnorm +
// quantization of x itself (the prologue of k_gemv, the same f64 tree) while
// its weights stream straight into registers (as k_gemv_reg), forms the 64
// rows' terms and row sums in the reference's order, then
// act[i] = silu(gate[i]) * up[i] for its 32 values and their i8 quantization
// (sub-blocks of the down projection's size, 16 or 32) — the bytes
// k_gemv_norm + k_swiglu_quant would write, without the launch between them.
struct GluParams {
  const uint8_t* wg;
  const uint8_t* wu;
  const float* nx;
  const float* nw;
  float eps;
  uint32_t k, nb, nsub, row_bytes, tstride;
  uint32_t lds_scale, lds_terms, lds_gu;
  int8_t* xq;  // the down projection's activation
  float* xe;
  float* xs;
};
constexpr uint32_t GLU_ROWS = 32;
// The row-layout gate/up launch's tile (k = 2048): 64 rows of gate and of up
// in 16 waves when the rows divide so (172 tiles at the 3B shape, one a CU),
// else 32 in 8. With 344 tiles of 32 on 256 CUs, 88 CUs ran two and the
// launch ended with them (stamps: the median tile done at 4.4 us, the last
// at 6.8).
// Q4_K only: the Q5_K kernel's registers do not fit 1024 threads (it
// spilled one VGPR to scratch).
inline uint32_t glu_row_tile(int type, uint32_t k, uint32_t I) {
  return type == CX_Q4_K && k == 2048 && I % 64 == 0 ? 64u : GLU_ROWS;
}

// Every thread keeps GLU_DEPTH items' weights in flight: all of them at
// k = 2048 (4 items a thread), a ring refilled one item behind at larger k.
constexpr int GLU_DEPTH = 4;

// HOIST (nb divides 128): item it + 256 d has the (block, half) of item it,
// so a lane reads its activation from LDS once, not once per item.
template <int T, int SUB, bool HOIST>
__global__ __launch_bounds__(256) void k_gemv_glu(GluParams P) {
  using Q = KQ<T>;
  constexpr int SPB = 256 / Q::SUB;
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ double red[9];
  __shared__ int nflag;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t row0 = blockIdx.x * GLU_ROWS;
  int8_t* sq = reinterpret_cast<int8_t*>(lds);
  float* se = reinterpret_cast<float*>(lds + P.lds_scale);
  float* ss = se + P.nsub;
  float* sx = reinterpret_cast<float*>(lds + P.lds_terms);  // the norm input, then the terms
  float* terms = sx;
  float* gu = reinterpret_cast<float*>(lds + P.lds_gu);

  // 1. x and the norm weight by direct loads, then this thread's first
  //    item's weights into registers
  copy_to_lds(P.nx, sx, P.k / 4, wave, lane);
  copy_to_lds(P.nw, sx + P.k, P.k / 4, wave, lane);
  const uint32_t items = 2 * (2 * GLU_ROWS) * P.nb;
  auto block_of = [&](uint32_t it) {
    const uint32_t q = it >> 1, r = q / P.nb, blk = q - r * P.nb;
    const uint8_t* w = r < GLU_ROWS ? P.wg : P.wu;
    return w + (size_t)(row0 + (r & (GLU_ROWS - 1))) * P.row_bytes + (size_t)blk * Q::BPB;
  };
  typename Q::Regs buf[GLU_DEPTH];
  uint32_t issued = 0;  // wave-uniform: items is a multiple of 128
#pragma unroll
  for (int d = 0; d < GLU_DEPTH; d++) {
    const uint32_t it = tid + 256u * d;
    if (it < items) {
      Q::load(block_of(it), (int)(it & 1), buf[d]);
      issued++;
    }
  }
  wait_all_but(issued * Q::NLOAD);  // x and w (issued first) have landed
  if (tid == 0) nflag = 0;
  cx_barrier();
  // 2. rmsnorm + quantization of the activation (k_gemv's prologue, the
  //    reference's factor bit for bit)
  const float* sw = sx + P.k;
  {
    cx_rms_part part;
    for (uint32_t i = 8 * tid; i < P.k; i += 2048) {
      float a[8];
      cx_load8(sx + i, a);  // two 16-byte LDS reads
      part.add<8>(a, i, P.k);
    }
    part = cx_wave_sum_rms(part);
    if (lane == 0) {
      red[wave] = part.s;
      red[4 + wave] = (double)part.w;
    }
    cx_wait_lds();
    cx_barrier();
    const double tot = ((red[0] + red[1]) + red[2]) + red[3];
    const float wt = (float)(((red[4] + red[5]) + red[6]) + red[7]);
    double scale = cx_rms_factor(tot, P.k, P.eps);
    const uint32_t reach = cx_rms_reach(tot, wt, P.k, P.k / 256 + 16);
    const uint32_t c = cx_rms_c(reach);
    // a second pass, when an output could round apart, from the sum in
    // order (x is still in LDS)
#pragma unroll 1
    for (int pass = 0;; pass++) {
      cx_rms_risk risk;
      for (uint32_t i = 8 * tid; i < P.k; i += 2048) {
        float v[8], a[8], b[8];
        cx_load8(sx + i, a);
        cx_load8(sw + i, b);
#pragma unroll
        for (int j = 0; j < 8; j++) {
          risk.add(a[j], scale, c);
          v[j] = (float)((double)a[j] * scale) * b[j];
        }
        cx_quant8_padded<Q::SUB>(v, i, sq, se, ss);
      }
      if (pass == 0 && reach && risk.unsure(reach)) nflag = 1;
      cx_wait_lds();
      cx_barrier();  // the activation is in LDS
      if (pass == 1 || !nflag) break;  // the same for every thread
      if (wave == 0) {
        const double seq = cx_rms_seq_sum(sx, P.k);
        if (lane == 0) red[8] = seq;
      }
      cx_wait_lds();
      cx_barrier();
      scale = cx_rms_factor(red[8], P.k, P.eps);
    }
  }
  // x and w are read: the region becomes the terms
  // 3. the 64 rows' terms; slot d of the ring holds items d, d + DEPTH, ...
  Pre4 pre;
  if (HOIST) {
    const uint32_t blk = (tid >> 1) % P.nb;
    pre4(tid & 1, sq + blk * ACT_LDS_BLOCK, se + blk * SPB, ss + blk * SPB, pre);
  }
  for (uint32_t base = tid; base < items; base += 256u * GLU_DEPTH) {
#pragma unroll
    for (int d = 0; d < GLU_DEPTH; d++) {
      const uint32_t it = base + 256u * d;
      if (it < items) {
        const uint32_t q = it >> 1, r = q / P.nb, blk = q - r * P.nb;
        if (HOIST)
          Q::half_pre(buf[d], (int)(it & 1), pre, nullptr, terms + r * P.tstride + blk * SPB);
        else
          Q::half_regs(buf[d], (int)(it & 1), sq + blk * ACT_LDS_BLOCK, se + blk * SPB,
                       ss + blk * SPB, nullptr, terms + r * P.tstride + blk * SPB);
        const uint32_t nx = it + 256u * GLU_DEPTH;
        if (nx < items) Q::load(block_of(nx), (int)(nx & 1), buf[d]);
      }
    }
  }
  __syncthreads();
  // 4. row sums in the scalar spec's order; SwiGLU one value a lane; then
  //    the quantization, 8 values a lane
  if ((uint32_t)tid < 2 * GLU_ROWS) gu[tid] = row_sum(terms + tid * P.tstride, P.nsub);
  __syncthreads();
  if (tid < (int)GLU_ROWS) gu[tid] = cx_swiglu(gu[tid], gu[GLU_ROWS + tid]);
  __syncthreads();
  if (tid < (int)(GLU_ROWS / 8)) {
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; j++) a[j] = gu[8 * tid + j];
    cx_quant8<SUB>(a, row0 + 8 * tid, P.xq, P.xe, P.xs);
  }
}

// The gate/up/SwiGLU launch on the row kernel's layout (Q4_K or Q5_K; the
// launcher uses it at k = 2048, the template also builds k = 4096): tile t is still gate rows [32t, 32t+32) and the same rows
// of up, but a lane holds one half super-block of a gate row AND the same
// half of the same up row, so its activation registers (pre4) serve both.
// A row's 2·NB lanes sit in one wave (k_gemv_row), the 32 rows fill
// 32·2·NB/64 waves, every weight load is issued at the start, and the
// normalized, quantized activation is made per workgroup from the f64 tree
// of k_gemv_row_norm while the weights are in flight. The gate and up row
// sums run as two interleaved DPP chains along the row's lanes (the
// reference's order, from 0), the row's last lane forms silu(g)·u
// (src/forward.rs:483-487), and four lanes quantize the tile's 32 values
// for the down projection (sub-blocks of SUB) — the bytes k_gemv_glu writes.
template <int T, int NB, int SUB, int ROWS>
__global__ __launch_bounds__(2 * NB * ROWS) void k_gemv_row_glu(GluParams P) {
  using Q = KQ<T>;
  constexpr int LPR = 2 * NB;   // lanes per row
  constexpr int RPW = 64 / LPR; // rows per wave
  constexpr int GJ = NB / 8;    // 8-value groups a virtual lane of the f64 tree
  static_assert(NB == 8 || NB == 16, "k = 2048 or 4096");
  static_assert(ROWS * LPR % 256 == 0 && ROWS * LPR <= 1024, "whole waves, at least the tree's four");
  __shared__ __align__(16) int8_t sq[NB * ACT_LDS_BLOCK];
  __shared__ __align__(16) float se[8 * NB], ss[8 * NB];
  __shared__ double red[9];
  __shared__ int nflag;
  __shared__ __align__(16) float act[ROWS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint64_t xb = (uint64_t)P.nx, wb = (uint64_t)P.nw, gb = (uint64_t)P.wg, ub = (uint64_t)P.wu;
  uint32_t rb = P.row_bytes;
  asm volatile("" : "+s"(xb), "+s"(wb), "+s"(gb), "+s"(ub), "+s"(rb));
  const uint32_t row0 = blockIdx.x * ROWS;
  const uint32_t lr = (uint32_t)(wave * RPW + lane / LPR);  // the lane's row in the tile
  const int b = (lane % LPR) >> 1, h = lane & 1;
  const bool owner = lane % LPR == LPR - 1;

  // 1. waves 0-3 (the tree's 256 virtual lanes) load x and w (L2 hits),
  //    then every lane its gate and up halves
  const float4* const xg = (const float4*)reinterpret_cast<const __attribute__((address_space(1))) float4*>(xb);
  const float4* const wg = (const float4*)reinterpret_cast<const __attribute__((address_space(1))) float4*>(wb);
  float4 xv[GJ * 2], wv[GJ * 2];
  if (wave < 4) {
#pragma unroll
    for (int j = 0; j < GJ; j++) {
      const uint32_t g = (uint32_t)tid + 256u * (uint32_t)j;
      xv[2 * j] = xg[2 * g];
      xv[2 * j + 1] = xg[2 * g + 1];
      wv[2 * j] = wg[2 * g];
      wv[2 * j + 1] = wg[2 * g + 1];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  typename Q::Regs rg, ru;
  const size_t off = (size_t)(row0 + lr) * rb + (size_t)b * Q::BPB;
  Q::load((const uint8_t*)reinterpret_cast<const __attribute__((address_space(1))) uint8_t*>(gb) + off, h, rg);
  Q::load((const uint8_t*)reinterpret_cast<const __attribute__((address_space(1))) uint8_t*>(ub) + off, h, ru);
  __builtin_amdgcn_sched_barrier(0);

  // 2. the f64 sum of squares over the tree (k_gemv_row_norm's), with the
  //    bound's weighted sum
  constexpr uint32_t K = NB * 256;
  if (tid == 0) nflag = 0;
  if (wave < 4) {
    cx_rms_part part;
#pragma unroll
    for (int j = 0; j < GJ; j++) {
      const float4 a0 = xv[2 * j], a1 = xv[2 * j + 1];
      const float a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      const uint32_t g = (uint32_t)tid + 256u * (uint32_t)j;
      part.add<8>(a, 8 * g, K);
    }
    part = cx_wave_sum_rms(part);
    if (lane == 0) {
      red[wave] = part.s;
      red[4 + wave] = (double)part.w;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  cx_wait_lds();
  cx_barrier();
  __builtin_amdgcn_sched_barrier(0);
  const double tot = ((red[0] + red[1]) + red[2]) + red[3];
  const float wt = (float)(((red[4] + red[5]) + red[6]) + red[7]);
  // 3. v = (x as f64 * scale) as f32 * w, quantized into LDS, from the
  //    tree's factor; a second pass, when an output could round apart, from
  //    the sum in order (x from L2). The lane's activation for step 4 is
  //    read with the flag.
  double scale = cx_rms_factor(tot, K, P.eps);
  const uint32_t reach = cx_rms_reach(tot, wt, K, 8 * GJ + 16);
  const uint32_t c = cx_rms_c(reach);
  Pre4 a;
#pragma unroll 1
  for (int pass = 0;; pass++) {
    cx_rms_risk risk;
    if (wave < 4) {
#pragma unroll
      for (int j = 0; j < GJ; j++) {
        const float4 a0 = xv[2 * j], a1 = xv[2 * j + 1];
        const float4 b0 = wv[2 * j], b1 = wv[2 * j + 1];
        const float x8[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const float bw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
        float v[8];
#pragma unroll
        for (int q = 0; q < 8; q++) {
          risk.add(x8[q], scale, c);
          v[q] = (float)((double)x8[q] * scale) * bw[q];
        }
        const uint32_t g = (uint32_t)tid + 256u * (uint32_t)j;
        cx_quant8_padded<Q::SUB>(v, 8 * g, sq, se, ss);
      }
    }
    if (pass == 0 && reach && risk.unsure(reach)) nflag = 1;
    __builtin_amdgcn_sched_barrier(0);
    cx_wait_lds();
    cx_barrier();
    __builtin_amdgcn_sched_barrier(0);
    pre4(h, sq + b * ACT_LDS_BLOCK, se + 8 * b, ss + 8 * b, a);
    if (pass == 1 || !nflag) break;  // the same for every thread
    if (wave == 0) {
      const double seq = cx_rms_seq_sum(P.nx, K);
      if (lane == 0) red[8] = seq;
    }
    cx_wait_lds();
    cx_barrier();
    scale = cx_rms_factor(red[8], K, P.eps);
  }
  // 4. the lane's four gate and four up terms, one activation read for both
  float tg[4], tu[4];
  Q::half_t4(rg, h, a, nullptr, tg);
  Q::half_t4(ru, h, a, nullptr, tu);
  // 5. both row sums along the lanes, then SwiGLU on the row's last lane
  float accg = 0.0f, accu = 0.0f;
#pragma unroll
  for (int s = 0; s < LPR; s++) {
    float vg = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(accg), 0x138, 0xF, 0xF,
                                                          true));  // wave_shr:1
    float vu = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(accu), 0x138, 0xF, 0xF,
                                                          true));
    vg += tg[0];
    vu += tu[0];
    vg += tg[1];
    vu += tu[1];
    vg += tg[2];
    vu += tu[2];
    vg += tg[3];
    vu += tu[3];
    accg = vg;
    accu = vu;
  }
  if (owner) act[lr] = cx_swiglu(accg, accu);
  cx_wait_lds();
  cx_barrier();
  // 6. the down projection's quantization of the tile's 32 values
  if (tid < (int)(ROWS / 8)) {
    const float4 v0 = reinterpret_cast<const float4*>(act)[2 * tid];
    const float4 v1 = reinterpret_cast<const float4*>(act)[2 * tid + 1];
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    cx_quant8<SUB>(v, row0 + 8 * tid, P.xq, P.xe, P.xs);
  }
}

// ------------------------------------------- 32-value blocks (Q8_0, Q5_0)
// The buffer path of the reference for these formats (ops::matmul_i8_directo
// and matmul_varias_una_fila, src/ops.rs:310-414, 968-993): the row unpacked
// to i8 quants and one scale d per 32 values (quant::desempaquetar_i8,
// src/quant.rs:270-330; no offset term), then kernels::dot_i8_escalado
// (src/kernels/scalar.rs:95-109):
//   total = 0; total += (d_b * xe_b) * (f32)E_b   for b = 0, 1, ...
// with E_b the exact i32 dot of the block's quants and the i8 activation.
// One lane per (row, block): it reads the block from LDS at any byte offset,
// forms E_b with v_dot4c_i32_i8 and stores the term; one lane per row adds
// them in block order.
template <int T> struct B32;

// Q8_0, 34 B: d (f16) then 32 signed quants
template <> struct B32<CX_Q8_0> {
  static constexpr int BPB = 34;
  __device__ static float dot(const uint8_t* lds, uint32_t off, const int8_t* xb, int& e) {
    uint32_t dw[1], q[8];
    lds_words<1>(lds, off, dw);
    lds_words<8>(lds, off + 2, q);
    int x[8];
    act8(xb, x);
    e = 0;
#pragma unroll
    for (int w = 0; w < 8; w++) e = dot4(q[w], x[w], e);
    return cx_h2f(dw[0] & 0xFFFF);
  }
};

// Q5_0, 22 B: d (f16), qh (u32: bit i is the fifth bit of value i), qs (16):
// value i < 16 is the low nibble of qs[i], value 16 + i the high one;
// quant = (nibble | fifth bit << 4) - 16
template <> struct B32<CX_Q5_0> {
  static constexpr int BPB = 22;
  __device__ static float dot(const uint8_t* lds, uint32_t off, const int8_t* xb, int& e) {
    uint32_t hw[2], qs[4];
    lds_words<2>(lds, off, hw);
    lds_words<4>(lds, off + 6, qs);
    const uint32_t qh = (hw[0] >> 16) | (hw[1] << 16);
    int x[8];
    act8(xb, x);
    e = 0;
#pragma unroll
    for (int w = 0; w < 8; w++) {
      const uint32_t nib = w < 4 ? (qs[w] & M4) : ((qs[w - 4] >> 4) & M4);
      const uint32_t t = (qh >> (4 * w)) & 0xFu;  // fifth bits of values 4w..4w+3
      const uint32_t hi = ((t & 1u) << 4) | ((t & 2u) << 11) | ((t & 4u) << 18) | ((t & 8u) << 25);
      // (u - 16) in every byte, u in 0..31: bias by 128 so no byte borrows
      const uint32_t v = (((nib | hi) | 0x80808080u) - 0x10101010u) ^ 0x80808080u;
      e = dot4(v, x[w], e);
    }
    return cx_h2f(hw[0] & 0xFFFF);
  }
};

template <int T, bool NORM>
__global__ __launch_bounds__(256) void k_gemv32(GemvParams P) {
  using Q = B32<T>;
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ double red[9];
  __shared__ int nflag;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t tile = blockIdx.x;
  int sg = 0;
  while (tile >= P.tile_end[sg]) sg++;
  if (sg) tile -= P.tile_end[sg - 1];
  const cx_seg S = P.seg[sg];
  const uint32_t row0 = tile * P.R;
  const uint32_t rows = min(P.R, S.rows - row0);
  // the epilogue's other operand (the residual, or the bias), loaded first:
  // its latency passes under the tile's, not after the row sum
  const float addend = epi_addend(P, S, row0, rows, tid);
  int8_t* sq = reinterpret_cast<int8_t*>(lds + P.lds_act);
  float* se = reinterpret_cast<float*>(lds + P.lds_scale);
  float* ss = se + P.nsub;
  float* sx = reinterpret_cast<float*>(lds + P.lds_norm);

  // 1. the rmsnorm input (if any), the tile's rows (`skew` bytes into LDS:
  //    34- and 22-byte blocks leave rows at any even offset) and the
  //    quantized activation, by direct loads; xe by ordinary loads
  if (NORM) {
    copy_to_lds(P.nx, sx, P.k / 4, wave, lane);
    copy_to_lds(P.nw, sx + P.k, P.k / 4, wave, lane);
  }
  const uint8_t* src = S.w + (size_t)row0 * P.row_bytes;
  const uint32_t skew = (uint32_t)((uintptr_t)src & 15u);
  const uint32_t ntile =
      copy_to_lds(src - skew, lds, (skew + rows * P.row_bytes + 15) >> 4, wave, lane);
  if (!NORM) {
    copy_to_lds(P.act.xq, sq, P.k / 16, wave, lane);
    for (uint32_t i = tid; i < P.nsub; i += 256) se[i] = P.act.xe[i];
  }
  // rmsnorm then quantization, as k_gemv's prologue (the reference's factor
  // bit for bit)
  const float* sw = sx + P.k;
  double scale = 0.0;
  uint32_t reach = 0, c = 0;
  if (NORM) {
    wait_all_but(ntile);
    if (tid == 0) nflag = 0;
    cx_barrier();
    cx_rms_part part;
    for (uint32_t i = 8 * tid; i < P.k; i += 2048) {
      float a[8];
      cx_load8(sx + i, a);  // two 16-byte LDS reads
      part.add<8>(a, i, P.k);
    }
    part = cx_wave_sum_rms(part);
    if (lane == 0) {
      red[wave] = part.s;
      red[4 + wave] = (double)part.w;
    }
    cx_wait_lds();
    cx_barrier();
    const double tot = ((red[0] + red[1]) + red[2]) + red[3];
    const float wt = (float)(((red[4] + red[5]) + red[6]) + red[7]);
    scale = cx_rms_factor(tot, P.k, P.eps);
    reach = cx_rms_reach(tot, wt, P.k, (P.k + 2047) / 2048 * 8 + 16);
    c = cx_rms_c(reach);
  }
  // the activation from the tree's factor; a second pass, when an output
  // could round apart, from the sum in order
#pragma unroll 1
  for (int pass = 0;; pass++) {
    if (NORM) {
      cx_rms_risk risk;
      for (uint32_t i = 8 * tid; i < P.k; i += 2048) {
        float v[8], a[8], b[8];
        cx_load8(sx + i, a);
        cx_load8(sw + i, b);
#pragma unroll
        for (int j = 0; j < 8; j++) {
          risk.add(a[j], scale, c);
          v[j] = (float)((double)a[j] * scale) * b[j];
        }
        cx_quant8<32>(v, i, sq, se, ss);
      }
      if (pass == 0 && reach && risk.unsure(reach)) nflag = 1;
    }
    cx_wait_vm<0>();
    cx_wait_lds();
    __syncthreads();
    if (!NORM || pass == 1 || !nflag) break;  // the same for every thread
    if (wave == 0) {
      const double seq = cx_rms_seq_sum(sx, P.k);
      if (lane == 0) red[8] = seq;
    }
    __syncthreads();
    scale = cx_rms_factor(red[8], P.k, P.eps);
  }

  // 2. one (row, block) a lane: E_b exactly, then (d_b * xe_b) * E_b
  float* terms = reinterpret_cast<float*>(lds + P.lds_terms);
  const uint32_t items = rows * P.nsub;
  for (uint32_t it = tid; it < items; it += 256) {
    const uint32_t r = it / P.nsub, b = it - r * P.nsub;
    int e;
    const float d = Q::dot(lds, skew + r * P.row_bytes + b * Q::BPB, sq + 32 * b, e);
    if (P.dbg) P.dbg[(size_t)(row0 + r) * P.nsub + b] = e;
    terms[r * P.tstride + b] = d * se[b] * (float)e;
  }
  __syncthreads();

  // 3. the row's sum in block order from 0 (src/kernels/scalar.rs:97-107)
  if ((uint32_t)tid < rows) {
    const float acc = row_sum_any(terms + tid * P.tstride, P.nsub);
    const uint32_t row = row0 + tid;
    S.y[row] = (P.epi == CX_EPI_ACCUM || S.bias) ? acc + addend : acc;
  }
}

// Gate and up of one 32-value-block type (Q8_0, Q5_0) and SwiGLU in one
// launch, as k_gemv_glu for the k-quants: tile t holds gate rows [32t,
// 32t+32) and the same rows of up, both in LDS (each at its own skew); every
// workgroup makes the rmsnorm + quantization of x (k_gemv32's prologue), forms
// the 64 rows' terms and block-order row sums (k_gemv32's steps 2 and 3),
// then act[i] = silu(gate[i]) * up[i] for its 32 values and their i8
// quantization in sub-blocks of SUB (the down projection's) — the bytes
// k_gemv32<T, true> over gate and up and k_swiglu_quant would write.
struct Glu32Params {
  const uint8_t* wg;
  const uint8_t* wu;
  const float* nx;
  const float* nw;
  float eps;
  uint32_t k, nsub, row_bytes, tstride;
  uint32_t lds_up, lds_act, lds_scale, lds_terms, lds_gu;  // byte offsets
  int8_t* xq;  // the down projection's activation
  float* xe;
  float* xs;
};

template <int T, int SUB>
__global__ __launch_bounds__(256) void k_gemv32_glu(Glu32Params P) {
  using Q = B32<T>;
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ double red[9];
  __shared__ int nflag;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t row0 = blockIdx.x * GLU_ROWS;
  int8_t* sq = reinterpret_cast<int8_t*>(lds + P.lds_act);
  float* se = reinterpret_cast<float*>(lds + P.lds_scale);
  float* ss = se + P.nsub;
  float* sx = reinterpret_cast<float*>(lds + P.lds_terms);  // the norm input, then the terms
  float* terms = sx;
  float* gu = reinterpret_cast<float*>(lds + P.lds_gu);

  // 1. x and the norm weight, then the gate tile and the up tile, by
  //    direct loads
  copy_to_lds(P.nx, sx, P.k / 4, wave, lane);
  copy_to_lds(P.nw, sx + P.k, P.k / 4, wave, lane);
  const uint8_t* src_g = P.wg + (size_t)row0 * P.row_bytes;
  const uint8_t* src_u = P.wu + (size_t)row0 * P.row_bytes;
  const uint32_t skg = (uint32_t)((uintptr_t)src_g & 15u), sku = (uint32_t)((uintptr_t)src_u & 15u);
  uint32_t ntile = copy_to_lds(src_g - skg, lds, (skg + GLU_ROWS * P.row_bytes + 15) >> 4, wave, lane);
  ntile += copy_to_lds(src_u - sku, lds + P.lds_up, (sku + GLU_ROWS * P.row_bytes + 15) >> 4, wave,
                       lane);
  // 2. rmsnorm then quantization, as k_gemv32's prologue (the reference's
  //    factor bit for bit)
  wait_all_but(ntile);
  if (tid == 0) nflag = 0;
  cx_barrier();
  const float* sw = sx + P.k;
  {
    cx_rms_part part;
    for (uint32_t i = 8 * tid; i < P.k; i += 2048) {
      float a[8];
      cx_load8(sx + i, a);
      part.add<8>(a, i, P.k);
    }
    part = cx_wave_sum_rms(part);
    if (lane == 0) {
      red[wave] = part.s;
      red[4 + wave] = (double)part.w;
    }
    cx_wait_lds();
    cx_barrier();
    const double tot = ((red[0] + red[1]) + red[2]) + red[3];
    const float wt = (float)(((red[4] + red[5]) + red[6]) + red[7]);
    double scale = cx_rms_factor(tot, P.k, P.eps);
    const uint32_t reach = cx_rms_reach(tot, wt, P.k, (P.k + 2047) / 2048 * 8 + 16);
    const uint32_t c = cx_rms_c(reach);
    // a second pass, when an output could round apart, from the sum in
    // order (x is still in LDS)
#pragma unroll 1
    for (int pass = 0;; pass++) {
      cx_rms_risk risk;
      for (uint32_t i = 8 * tid; i < P.k; i += 2048) {
        float v[8], a[8], b[8];
        cx_load8(sx + i, a);
        cx_load8(sw + i, b);
#pragma unroll
        for (int j = 0; j < 8; j++) {
          risk.add(a[j], scale, c);
          v[j] = (float)((double)a[j] * scale) * b[j];
        }
        cx_quant8<32>(v, i, sq, se, ss);
      }
      if (pass == 0 && reach && risk.unsure(reach)) nflag = 1;
      cx_wait_vm<0>();
      cx_wait_lds();
      __syncthreads();
      if (pass == 1 || !nflag) break;  // the same for every thread
      if (wave == 0) {
        const double seq = cx_rms_seq_sum(sx, P.k);
        if (lane == 0) red[8] = seq;
      }
      __syncthreads();
      scale = cx_rms_factor(red[8], P.k, P.eps);
    }
  }
  // x and w are read: the region becomes the terms
  // 3. one (row, block) a lane: rows 0-31 are gate's, 32-63 up's
  const uint32_t items = 2 * GLU_ROWS * P.nsub;
  for (uint32_t it = tid; it < items; it += 256) {
    const uint32_t r = it / P.nsub, b = it - r * P.nsub;
    const uint32_t off = r < GLU_ROWS ? skg + r * P.row_bytes + b * Q::BPB
                                      : P.lds_up + sku + (r - GLU_ROWS) * P.row_bytes + b * Q::BPB;
    int e;
    const float d = Q::dot(lds, off, sq + 32 * b, e);
    terms[r * P.tstride + b] = d * se[b] * (float)e;
  }
  __syncthreads();
  // 4. row sums in block order from 0; SwiGLU one value a lane; then the
  //    quantization, 8 values a lane
  if ((uint32_t)tid < 2 * GLU_ROWS) gu[tid] = row_sum_any(terms + tid * P.tstride, P.nsub);
  __syncthreads();
  if (tid < (int)GLU_ROWS) gu[tid] = cx_swiglu(gu[tid], gu[GLU_ROWS + tid]);
  __syncthreads();
  if (tid < (int)(GLU_ROWS / 8)) {
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; j++) a[j] = gu[8 * tid + j];
    cx_quant8<SUB>(a, row0 + 8 * tid, P.xq, P.xe, P.xs);
  }
}

// LDS of the block-32 gate/up launch: [gate tile][up tile] (16 skew + 32
// rows + 16 pad each) [xq, k bytes][xe, xs][norm input (2k floats), then
// the terms (64 x (nsub + 4))][64 row sums]
Glu32Params plan_glu32(int type, uint32_t k, uint32_t* lds) {
  Glu32Params P{};
  P.k = k;
  P.nsub = k / 32;
  P.row_bytes = P.nsub * (uint32_t)cx_bpb(type);
  P.tstride = P.nsub + 4;
  const uint32_t tile = (16 + GLU_ROWS * P.row_bytes + 16 + 15) / 16 * 16;
  P.lds_up = tile;
  P.lds_act = 2 * tile;
  P.lds_scale = P.lds_act + (k + 15) / 16 * 16;
  P.lds_terms = P.lds_scale + (8 * P.nsub + 15) / 16 * 16;
  const uint32_t terms = 4 * 2 * GLU_ROWS * P.tstride, nin = 8 * k;
  P.lds_gu = P.lds_terms + (terms > nin ? terms : nin);
  *lds = P.lds_gu + 4 * 2 * GLU_ROWS;
  return P;
}

struct TilePlan {
  uint32_t R, tiles, lds, lds_act, lds_scale, lds_terms, lds_norm;
};

// LDS layout of a tile of R rows: [16 skew + R*row_bytes + 16 pad]
// [xq, 272 bytes per 256] [xe, xs] then one region used first for the
// rmsnorm input (x, w: 2k floats) and then for the terms (R x (nsub+4))
TilePlan plan_tile(uint32_t R, uint32_t row_bytes, uint32_t k, uint32_t nsub,
                   const uint32_t* rows, int nseg, bool norm, bool reg = false) {
  TilePlan t{};
  t.R = R;
  for (int i = 0; i < nseg; i++) t.tiles += (rows[i] + R - 1) / R;
  t.lds_act = reg ? 0 : (16 + R * row_bytes + 16 + 15) / 16 * 16;
  t.lds_scale = t.lds_act + (k / 256) * ACT_LDS_BLOCK;
  t.lds_terms = t.lds_scale + (8 * nsub + 15) / 16 * 16;
  t.lds_norm = t.lds_terms;
  const uint32_t terms = 4 * R * (nsub + 4), nin = norm ? 8 * k : 0;
  t.lds = t.lds_terms + (terms > nin ? terms : nin);
  return t;
}

// Tiles of a launch without the rmsnorm prologue: about one per CU, the
// largest tile height that leaves at least 7/8 of PLAIN_TILES tiles
// (measured on MI355X: in the 3B decode step 2 tiles per CU took 1.7%
// longer a token and 4 tiles 8% longer; in the daiss-0.5b Q8_0 step 2
// tiles per CU took 1.8% longer, and its 896-row matrices in 224 tiles of
// 4 rows rather than 448 of 2 made the token 0.4% shorter)
constexpr uint32_t PLAIN_TILES = 256;

// The plain (no prologue) launch's tile: the largest R <= 16 that leaves
// 7/8 of PLAIN_TILES tiles
template <int T>
TilePlan plain_plan(uint32_t row_bytes, uint32_t k, uint32_t nsub, const uint32_t* rows, int nseg) {
  constexpr bool REG = T == CX_Q4_K || T == CX_Q5_K;  // weights straight into registers
  TilePlan best{};
  for (uint32_t R = 16; R >= 1; R >>= 1) {
    TilePlan t = plan_tile(R, row_bytes, k, nsub, rows, nseg, false, REG);
    if (t.lds > TILE_LDS_MAX) continue;
    best = t;
    if (t.tiles >= PLAIN_TILES * 7 / 8) break;
  }
  return best;
}

// The row kernel (k_gemv_row) for a plain Q4_K/Q5_K launch of k = 2048 or
// 4096: waves per workgroup W, R = W * 64 / (2k/256) rows a tile. The
// largest W of 16, 12, 8, 4, 2, 1 that leaves at least 7/8 of PLAIN_TILES
// tiles, else W = 1. Measured on MI355X at config 1 (11008 x 2048, 360
// graph-captured launches over 36 matrices): W = 12 (230 tiles of 48 rows)
// 4.45 us, W = 4 (688 of 16) 4.46, W = 11 (251 of 44) 4.51; the
// per-workgroup row-sum kernel (k_gemv_reg) took 5.78.
struct RowPlan {
  uint32_t W, R, tiles;
};
RowPlan row_plan(uint32_t k, const uint32_t* rows, int nseg) {
  RowPlan p{};
  if (k != 2048 && k != 4096) return p;
  const uint32_t rpw = 64 / (2 * (k / 256));
  for (uint32_t W : {16u, 12u, 8u, 4u, 2u, 1u}) {
    uint32_t tiles = 0;
    for (int i = 0; i < nseg; i++) tiles += (rows[i] + rpw * W - 1) / (rpw * W);
    p = RowPlan{W, rpw * W, tiles};
    if (tiles >= PLAIN_TILES * 7 / 8) break;
  }
  return p;
}

template <int T, bool MULTI, bool DBG>
int launch_row_k(GemvParams& P, const RowPlan& rp, hipStream_t s);

template <int T, bool DBG>
int launch_row(GemvParams& P, const uint32_t* rows, const RowPlan& rp, hipStream_t s) {
  P.R = rp.R;
  uint32_t acc = 0;
  for (int i = 0; i < P.nseg; i++) {
    acc += (rows[i] + rp.R - 1) / rp.R;
    P.tile_end[i] = acc;
  }
  if (P.nseg > 1) return launch_row_k<T, true, DBG>(P, rp, s);
  return launch_row_k<T, false, DBG>(P, rp, s);
}

template <int T, bool MULTI, bool DBG>
int launch_row_k(GemvParams& P, const RowPlan& rp, hipStream_t s) {
  const dim3 g(rp.tiles), b(64 * rp.W);
  if (P.k == 2048) hipLaunchKernelGGL((k_gemv_row<T, 8, MULTI, DBG>), g, b, 0, s, P);
  else hipLaunchKernelGGL((k_gemv_row<T, 16, MULTI, DBG>), g, b, 0, s, P);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

// The q/k/v launch's row kernel: W waves a tile (R = W * 64 / (2k/256)
// rows), the largest W of 16, 8, 4, 2, 1 that leaves ROW_NORM_TILES tiles.
// Every workgroup repeats the prologue, so fewer, larger tiles pay:
// measured on MI355X (graph-captured launches over rotating matrices, q/k/v
// shapes of 2048 + 256 + 256 rows at k = 2048 and ~6144 rows at k = 4096):
// 3B 320 tiles of 2 waves 5.10 us, 160 of 4 waves 3.50, 80 of 8 waves 4.49
// (the LDS-tile k_gemv prologue kernel: 5.92); k = 4096 192 tiles of 16
// waves 7.83 us, 384 of 8 waves 7.79 (k_gemv: 13.5). In the config-5 decode
// step (k = 4096), 768 tiles of 4 waves: 298.4 tok/s against 293.5 with 384
// of 8 (whose tree waves, their x loads in a branch, waited for x before
// issuing their weights) and 279.7 with 1536 of 2.
constexpr uint32_t ROW_NORM_TILES = 128;
template <int T, int NB, bool MULTI>
void launch_row_norm_w(uint32_t W, const GemvParams& P, dim3 g, hipStream_t s) {
  switch (W) {
    case 16: hipLaunchKernelGGL((k_gemv_row_norm<T, NB, 16, MULTI>), g, dim3(1024), 0, s, P); break;
    case 8: hipLaunchKernelGGL((k_gemv_row_norm<T, NB, 8, MULTI>), g, dim3(512), 0, s, P); break;
    case 4: hipLaunchKernelGGL((k_gemv_row_norm<T, NB, 4, MULTI>), g, dim3(256), 0, s, P); break;
    case 2: hipLaunchKernelGGL((k_gemv_row_norm<T, NB, 2, MULTI>), g, dim3(128), 0, s, P); break;
    default: hipLaunchKernelGGL((k_gemv_row_norm<T, NB, 1, MULTI>), g, dim3(64), 0, s, P); break;
  }
}
template <int T>
int launch_row_norm(GemvParams& P, const uint32_t* rows, hipStream_t s) {
  const uint32_t rpw = 64 / (2 * (P.k / 256));
  uint32_t W = 1, tiles = 0;
  // at k = 4096 at most 4 waves (with 16, 1024 threads and 128 VGPRs a
  // lane, the prologue's registers spill to scratch; 8 measured slower)
  const uint32_t wmax = P.k == 4096 ? 4u : 16u;
  for (uint32_t w : {16u, 8u, 4u, 2u, 1u}) {
    if (w > wmax) continue;
    tiles = 0;
    for (int i = 0; i < P.nseg; i++) tiles += (rows[i] + rpw * w - 1) / (rpw * w);
    W = w;
    if (tiles >= ROW_NORM_TILES) break;
  }
  P.R = rpw * W;
  uint32_t acc = 0;
  for (int i = 0; i < P.nseg; i++) {
    acc += (rows[i] + P.R - 1) / P.R;
    P.tile_end[i] = acc;
  }
  const dim3 g(acc);
  if (P.k == 2048) {
    if (P.nseg > 1) launch_row_norm_w<T, 8, true>(W, P, g, s);
    else launch_row_norm_w<T, 8, false>(W, P, g, s);
  } else {
    if (P.nseg > 1) launch_row_norm_w<T, 16, true>(W, P, g, s);
    else launch_row_norm_w<T, 16, false>(W, P, g, s);
  }
  CX_HIP(hipGetLastError());
  return CX_OK;
}

// The long-row kernel (k_gemv_rowl) for a plain Q4_K/Q5_K launch of
// 16 < k/256 <= 64 super-blocks: 4 waves (4 rows) a workgroup, the chain
// unrolled at 43 and 56 blocks. Measured on MI355X in the 3B decode step
// (down, 2048 x 11008, 512 tiles): 706 tok/s against 700 with 8 waves, 663
// with 16 and 691 with k_gemv_reg1; at config 5 (4096 x 14336 Q5_K) 8 waves
// 250.0 tok/s against 248.9 with k_gemv_reg1. A two-row ring (wave_ror:1, 32
// lanes a row, one wave a SIMD) took 8.5 us against 7.0: a wave's chain is
// bound by its own dependent adds, so fewer waves only delay the loads.
template <int T>
int launch_rowl(GemvParams& P, const uint32_t* rows, hipStream_t s) {
  constexpr uint32_t W = 4;
  P.R = W;
  uint32_t acc = 0;
  for (int i = 0; i < P.nseg; i++) {
    acc += (rows[i] + W - 1) / W;
    P.tile_end[i] = acc;
  }
  const dim3 g(acc), blk(64 * W);
  if (P.nb == 43) hipLaunchKernelGGL((k_gemv_rowl<T, W, 43>), g, blk, 0, s, P);
  else if (P.nb == 56) hipLaunchKernelGGL((k_gemv_rowl<T, W, 56>), g, blk, 0, s, P);
  else hipLaunchKernelGGL((k_gemv_rowl<T, W, 0>), g, blk, 0, s, P);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

template <int T, bool NORM>
int launch_t(GemvParams& P, const uint32_t* rows, hipStream_t s) {
  using Q = KQ<T>;
  // Q4_K/Q5_K with a ready activation: weights straight into registers
  constexpr bool REG = !NORM && (T == CX_Q4_K || T == CX_Q5_K);
  if (Q::ALIGNED) {
    for (int i = 0; i < P.nseg; i++)
      CX_REQUIRE(((uintptr_t)P.seg[i].w & 15u) == 0,
                 "gemv: %s weights must start 16-byte aligned", T == CX_Q4_K ? "Q4_K" : "Q5_K");
  }
  // Tile rows (measured on MI355X at the 3B projection shapes):
  //  - with the rmsnorm prologue every workgroup repeats the activation
  //    work, so take one tile per CU (R = rows/256) when it fits in LDS, else
  //    two tiles per CU;
  //  - otherwise plain_plan's: the largest R <= 16 that leaves about a
  //    tile per CU (at least 224 tiles).
  if constexpr (REG) {
    const RowPlan rp = row_plan(P.k, rows, P.nseg);
    if (rp.R) return P.dbg ? launch_row<T, true>(P, rows, rp, s) : launch_row<T, false>(P, rows, rp, s);
    if (!P.dbg && P.nb > 16 && P.nb <= ROWL_NB_MAX)
      return launch_rowl<T>(P, rows, s);
  }
  if constexpr (NORM && (T == CX_Q4_K || T == CX_Q5_K)) {
    if (P.k == 2048 || P.k == 4096) return launch_row_norm<T>(P, rows, s);
  }
  uint32_t total_rows = 0;
  for (int i = 0; i < P.nseg; i++) total_rows += rows[i];
  TilePlan best{};
  if (NORM) {
    for (uint32_t per_cu = 1; per_cu <= 8 && !best.R; per_cu *= 2) {
      uint32_t R = (total_rows + 256 * per_cu - 1) / (256 * per_cu);
      R = R < 1 ? 1 : (R > 64 ? 64 : R);
      TilePlan t = plan_tile(R, P.row_bytes, P.k, P.nsub, rows, P.nseg, NORM);
      if (t.lds <= TILE_LDS_NORM_MAX) best = t;
    }
  } else {
    best = plain_plan<T>(P.row_bytes, P.k, P.nsub, rows, P.nseg);
  }
  CX_REQUIRE(best.R, "gemv: a row of %u values does not fit in LDS", P.k);
  P.R = best.R;
  P.lds_act = best.lds_act;
  P.lds_scale = best.lds_scale;
  P.lds_terms = best.lds_terms;
  P.lds_norm = best.lds_norm;
  uint32_t acc = 0;
  for (int i = 0; i < P.nseg; i++) {
    acc += (rows[i] + best.R - 1) / best.R;
    P.tile_end[i] = acc;
  }
  if constexpr (REG) {
    // one item a lane where the tile's items fit 1024 lanes (halving the
    // tile to fit measured slower: config 5's 4096 x 14336 Q5_K down in
    // 512 tiles of 8 rows took 15.1 us against 13.1 in 256 of 16)
    const uint32_t th = (2 * best.R * P.nb + 63) / 64 * 64;
    if (th > 256 && th <= 1024)
      hipLaunchKernelGGL((k_gemv_reg1<T>), dim3(best.tiles), dim3(th), best.lds, s, P);
    else
      hipLaunchKernelGGL((k_gemv_reg<T>), dim3(best.tiles), dim3(256), best.lds, s, P);
  }
  else
    hipLaunchKernelGGL((k_gemv<T, NORM>), dim3(best.tiles), dim3(256), best.lds, s, P);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

// LDS of a 32-value-block tile: [16 skew + R*row_bytes + 16 pad] [xq, k
// bytes] [xe, xs] then the rmsnorm input (2k floats) or the terms
// (R x (nsub+4))
TilePlan plan_tile32(uint32_t R, uint32_t row_bytes, uint32_t k, uint32_t nsub,
                     const uint32_t* rows, int nseg, bool norm) {
  TilePlan t{};
  t.R = R;
  for (int i = 0; i < nseg; i++) t.tiles += (rows[i] + R - 1) / R;
  t.lds_act = (16 + R * row_bytes + 16 + 15) / 16 * 16;
  t.lds_scale = t.lds_act + (k + 15) / 16 * 16;
  t.lds_terms = t.lds_scale + (8 * nsub + 15) / 16 * 16;
  t.lds_norm = t.lds_terms;
  const uint32_t terms = 4 * R * (nsub + 4), nin = norm ? 8 * k : 0;
  t.lds = t.lds_terms + (terms > nin ? terms : nin);
  return t;
}

// The plain block-32 launch's tile: the largest R <= 16 that leaves 7/8 of
// PLAIN_TILES tiles
TilePlan plain_plan32(uint32_t row_bytes, uint32_t k, uint32_t nsub, const uint32_t* rows,
                      int nseg) {
  TilePlan best{};
  for (uint32_t R = 16; R >= 1; R >>= 1) {
    TilePlan t = plan_tile32(R, row_bytes, k, nsub, rows, nseg, false);
    if (t.lds > TILE_LDS_MAX) continue;
    best = t;
    if (t.tiles >= PLAIN_TILES * 7 / 8) break;
  }
  return best;
}

template <int T, bool NORM>
int launch_b32(GemvParams& P, const uint32_t* rows, hipStream_t s) {
  uint32_t total_rows = 0;
  for (int i = 0; i < P.nseg; i++) total_rows += rows[i];
  // the k-quant GEMV's tile choice: with the prologue one or two tiles per
  // CU, otherwise the largest R <= 16 that leaves about a tile per CU
  TilePlan best{};
  if (NORM) {
    for (uint32_t per_cu = 1; per_cu <= 8 && !best.R; per_cu *= 2) {
      uint32_t R = (total_rows + 256 * per_cu - 1) / (256 * per_cu);
      R = R < 1 ? 1 : (R > 64 ? 64 : R);
      TilePlan t = plan_tile32(R, P.row_bytes, P.k, P.nsub, rows, P.nseg, NORM);
      if (t.lds <= TILE_LDS_NORM_MAX) best = t;
    }
  } else {
    best = plain_plan32(P.row_bytes, P.k, P.nsub, rows, P.nseg);
  }
  CX_REQUIRE(best.R, "gemv: a row of %u values does not fit in LDS", P.k);
  P.R = best.R;
  P.lds_act = best.lds_act;
  P.lds_scale = best.lds_scale;
  P.lds_terms = best.lds_terms;
  P.lds_norm = best.lds_norm;
  uint32_t acc = 0;
  for (int i = 0; i < P.nseg; i++) {
    acc += (rows[i] + best.R - 1) / best.R;
    P.tile_end[i] = acc;
  }
  hipLaunchKernelGGL((k_gemv32<T, NORM>), dim3(best.tiles), dim3(256), best.lds, s, P);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

template <bool NORM>
int launch_type(int type, GemvParams& P, const uint32_t* rows, hipStream_t s) {
  switch (type) {
    case CX_Q8_0: return launch_b32<CX_Q8_0, NORM>(P, rows, s);
    case CX_Q5_0: return launch_b32<CX_Q5_0, NORM>(P, rows, s);
    case CX_Q2_K: return launch_t<CX_Q2_K, NORM>(P, rows, s);
    case CX_Q3_K: return launch_t<CX_Q3_K, NORM>(P, rows, s);
    case CX_Q4_K: return launch_t<CX_Q4_K, NORM>(P, rows, s);
    case CX_Q5_K: return launch_t<CX_Q5_K, NORM>(P, rows, s);
    default: return launch_t<CX_Q6_K, NORM>(P, rows, s);
  }
}

// Shared checks and the segment table. Returns CX_OK with *total == 0 when
// there is nothing to do.
int gemv_setup(int type, const cx_seg* segs, int nseg, uint32_t k, int epi, int32_t* dbg,
               GemvParams& P, uint32_t* rows, uint32_t* total) {
  CX_REQUIRE(nseg >= 1 && nseg <= 4, "gemv: 1..4 matrices per launch");
  CX_REQUIRE(cx_has_gemv(type), "gemv: type %d has no GEMV", type);
  const uint32_t vpb = (uint32_t)cx_vpb(type);
  CX_REQUIRE(k > 0 && k % vpb == 0, "gemv: k=%u is not a multiple of %u", k, vpb);
  CX_REQUIRE(!dbg || nseg == 1, "gemv: sub-block sums need a single matrix");
  *total = 0;
  int n = 0;
  for (int i = 0; i < nseg; i++) {
    CX_REQUIRE(segs[i].w && segs[i].y, "gemv: null matrix or output");
    *total += segs[i].rows;
    if (segs[i].rows) {  // empty segments own no tile
      P.seg[n] = segs[i];
      rows[n++] = segs[i].rows;
    }
  }
  P.nseg = n;
  P.k = k;
  P.nb = k / vpb;
  P.nsub = k / cx_sub(type);
  P.row_bytes = P.nb * cx_bpb(type);
  P.tstride = P.nsub + 4;
  P.epi = epi;
  P.dbg = dbg;
  return CX_OK;
}

}  // namespace

int cx_launch_gemv(int type, const cx_seg* segs, int nseg, uint32_t k, const cx_qact& act,
                   int epi, int32_t* dbg, hipStream_t s) {
  CX_REQUIRE(act.xq && act.xe && act.xs, "gemv: missing quantized activation");
  // the 32-value block kernel reads xe with ordinary loads (and no xs)
  const uintptr_t ealign = cx_is_block32(type) ? 3u : 15u;
  CX_REQUIRE(((uintptr_t)act.xq & 15u) == 0 && ((uintptr_t)act.xe & ealign) == 0 &&
                 ((uintptr_t)act.xs & ealign) == 0,
             "gemv: xq must be 16-byte aligned, xe and xs %d-byte", (int)ealign + 1);
  GemvParams P{};
  uint32_t rows[4], total;
  int rc = gemv_setup(type, segs, nseg, k, epi, dbg, P, rows, &total);
  if (rc || !total) return rc;
  P.act = act;
  return launch_type<false>(type, P, rows, s);
}

// The argmax's first step in the GEMV's epilogue (the lm_head): where the
// row kernel takes the matrix (Q4_K/Q5_K, k = 2048 or 4096), the tiles it
// would launch, each writing its (largest output, row) pair; else 0.
uint32_t cx_gemv_argmax_parts(int type, uint32_t n, uint32_t k) {
  if ((type != CX_Q4_K && type != CX_Q5_K) || !n) return 0;
  return row_plan(k, &n, 1).tiles;
}

// y = W·act (CX_EPI_STORE, no bias) and the per-tile argmax pairs in
// apv/api (cx_gemv_argmax_parts(type, n, k) of them); *nparts = 0 and
// nothing launched where the row kernel does not take the matrix.
int cx_launch_gemv_argmax(int type, const cx_seg& seg, uint32_t k, const cx_qact& act, float* apv,
                          uint32_t* api, uint32_t* nparts, hipStream_t s) {
  *nparts = 0;
  const uint32_t parts = cx_gemv_argmax_parts(type, seg.rows, k);
  if (!parts) return CX_OK;
  CX_REQUIRE(apv && api && !seg.bias, "gemv argmax: the pair buffers, no bias");
  CX_REQUIRE(act.xq && act.xe && act.xs && ((uintptr_t)act.xq & 15u) == 0 &&
                 ((uintptr_t)act.xe & 15u) == 0 && ((uintptr_t)act.xs & 15u) == 0,
             "gemv argmax: xq, xe and xs 16-byte aligned");
  CX_REQUIRE(((uintptr_t)seg.w & 15u) == 0, "gemv argmax: weights 16-byte aligned");
  GemvParams P{};
  uint32_t rows[4], total;
  int rc = gemv_setup(type, &seg, 1, k, CX_EPI_STORE, nullptr, P, rows, &total);
  if (rc || !total) return rc;
  P.act = act;
  P.apv = apv;
  P.api = api;
  const RowPlan rp = row_plan(k, rows, 1);
  CX_REQUIRE(rp.R && rp.tiles == parts && rp.R <= 64, "gemv argmax: row plan");
  P.R = rp.R;
  P.tile_end[0] = rp.tiles;
  const dim3 g(rp.tiles), b(64 * rp.W);
#define CX_ROW_AMAX(TT)                                                                   \
  do {                                                                                    \
    if (k == 2048) hipLaunchKernelGGL((k_gemv_row<TT, 8, false, false, true>), g, b, 0, s, P); \
    else hipLaunchKernelGGL((k_gemv_row<TT, 16, false, false, true>), g, b, 0, s, P);          \
  } while (0)
  if (type == CX_Q4_K) CX_ROW_AMAX(CX_Q4_K);
  else CX_ROW_AMAX(CX_Q5_K);
#undef CX_ROW_AMAX
  CX_HIP(hipGetLastError());
  *nparts = parts;
  return CX_OK;
}

int cx_launch_gemv_norm(int type, const cx_seg* segs, int nseg, uint32_t k, const float* x,
                        const float* w, float eps, int epi, hipStream_t s) {
  CX_REQUIRE(x && w, "gemv: missing rmsnorm input");
  CX_REQUIRE(((uintptr_t)x & 15u) == 0 && ((uintptr_t)w & 15u) == 0,
             "gemv: the rmsnorm input and weight must be 16-byte aligned");
  GemvParams P{};
  uint32_t rows[4], total;
  int rc = gemv_setup(type, segs, nseg, k, epi, nullptr, P, rows, &total);
  if (rc || !total) return rc;
  P.nx = x;
  P.nw = w;
  P.eps = eps;
  return launch_type<true>(type, P, rows, s);
}

bool cx_glu_supported(int type) { return type == CX_Q4_K || type == CX_Q5_K; }

bool cx_glu_fits(int type, uint32_t k) {
  if (cx_glu_supported(type)) return k > 0 && k % 256 == 0 && k <= 8192;
  if (type != CX_Q8_0 && type != CX_Q5_0) return false;
  if (!k || k % 32 || k > 8192) return false;
  uint32_t lds = 0;
  (void)plan_glu32(type, k, &lds);
  return lds <= TILE_LDS_NORM_MAX;
}

int cx_launch_gemv_glu(int type, const uint8_t* wg, const uint8_t* wu, uint32_t I, uint32_t k,
                       const float* x, const float* w, float eps, int sub, int8_t* xq, float* xe,
                       float* xs, hipStream_t s) {
  CX_REQUIRE(cx_glu_fits(type, k), "gemv glu: type %d at k=%u (Q4_K or Q5_K with k a multiple "
             "of 256; Q8_0 or Q5_0 whose two tiles fit in LDS)", type, k);
  CX_REQUIRE(sub == 16 || sub == 32, "gemv glu: sub-blocks of 16 or 32, not %d", sub);
  if (type == CX_Q8_0 || type == CX_Q5_0) {
    CX_REQUIRE(I > 0 && I % GLU_ROWS == 0, "gemv glu: %u rows are not tiles of %u", I, GLU_ROWS);
    CX_REQUIRE(wg && wu && x && w && xq && xe && xs, "gemv glu: null pointer");
    CX_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)xq & 7) == 0,
               "gemv glu: x and w 16-byte aligned, xq 8-byte");
    uint32_t lds = 0;
    Glu32Params Q = plan_glu32(type, k, &lds);
    Q.wg = wg;
    Q.wu = wu;
    Q.nx = x;
    Q.nw = w;
    Q.eps = eps;
    Q.xq = xq;
    Q.xe = xe;
    Q.xs = xs;
    const dim3 grid(I / GLU_ROWS);
    if (type == CX_Q8_0) {
      if (sub == 32) hipLaunchKernelGGL((k_gemv32_glu<CX_Q8_0, 32>), grid, dim3(256), lds, s, Q);
      else hipLaunchKernelGGL((k_gemv32_glu<CX_Q8_0, 16>), grid, dim3(256), lds, s, Q);
    } else {
      if (sub == 32) hipLaunchKernelGGL((k_gemv32_glu<CX_Q5_0, 32>), grid, dim3(256), lds, s, Q);
      else hipLaunchKernelGGL((k_gemv32_glu<CX_Q5_0, 16>), grid, dim3(256), lds, s, Q);
    }
    CX_HIP(hipGetLastError());
    return CX_OK;
  }
  CX_REQUIRE(k > 0 && k % 256 == 0 && k <= 8192, "gemv glu: k=%u (a multiple of 256, at most 8192)", k);
  CX_REQUIRE(I > 0 && I % GLU_ROWS == 0, "gemv glu: %u rows are not tiles of %u", I, GLU_ROWS);
  CX_REQUIRE(wg && wu && x && w && xq && xe && xs, "gemv glu: null pointer");
  CX_REQUIRE(((uintptr_t)wg & 15) == 0 && ((uintptr_t)wu & 15) == 0 && ((uintptr_t)x & 15) == 0 &&
                 ((uintptr_t)w & 15) == 0 && ((uintptr_t)xq & 7) == 0,
             "gemv glu: weights, x and w 16-byte aligned, xq 8-byte");
  GluParams P{};
  P.wg = wg;
  P.wu = wu;
  P.nx = x;
  P.nw = w;
  P.eps = eps;
  P.k = k;
  P.nb = k / 256;
  P.nsub = k / cx_sub(type);
  P.row_bytes = P.nb * cx_bpb(type);
  P.tstride = P.nsub + 4;
  P.xq = xq;
  P.xe = xe;
  P.xs = xs;
  if (k == 2048) {
    // the row layout: 32 rows of gate and up in 8 waves (the 3B shape:
    // 8.71 -> 7.75 us a launch, weights in L2). At k = 4096 (16 waves a
    // tile, 448 tiles: config 5's 14336 x 4096, 66 MB past L2) it measured
    // 20.4 us against k_gemv_glu's 16.3, which keeps that shape.
    const uint32_t rows = glu_row_tile(type, k, I);
    const dim3 grid(I / rows), block(2 * (k / 256) * rows);
#define CX_ROW_GLU(TT, NB, R)                                                              \
  do {                                                                                     \
    if (sub == 32) hipLaunchKernelGGL((k_gemv_row_glu<TT, NB, 32, R>), grid, block, 0, s, P); \
    else hipLaunchKernelGGL((k_gemv_row_glu<TT, NB, 16, R>), grid, block, 0, s, P);          \
  } while (0)
    if (rows == 64) {
      CX_ROW_GLU(CX_Q4_K, 8, 64);
    } else {
      if (type == CX_Q4_K) CX_ROW_GLU(CX_Q4_K, 8, 32);
      else CX_ROW_GLU(CX_Q5_K, 8, 32);
    }
#undef CX_ROW_GLU
    CX_HIP(hipGetLastError());
    return CX_OK;
  }
  // LDS: [xq, 272 bytes per 256][xe, xs][norm input (2k floats), then the
  // terms (64 x (nsub + 4))][64 row sums]
  P.lds_scale = P.nb * ACT_LDS_BLOCK;
  P.lds_terms = P.lds_scale + (8 * P.nsub + 15) / 16 * 16;
  const uint32_t terms = 4 * 2 * GLU_ROWS * P.tstride, nin = 8 * k;
  P.lds_gu = P.lds_terms + (terms > nin ? terms : nin);
  const uint32_t lds = P.lds_gu + 4 * 2 * GLU_ROWS;
  const dim3 grid(I / GLU_ROWS);
  const bool hoist = 128 % P.nb == 0;
  if (type == CX_Q4_K) {
    if (sub == 32) {
      if (hoist) hipLaunchKernelGGL((k_gemv_glu<CX_Q4_K, 32, true>), grid, dim3(256), lds, s, P);
      else hipLaunchKernelGGL((k_gemv_glu<CX_Q4_K, 32, false>), grid, dim3(256), lds, s, P);
    } else {
      if (hoist) hipLaunchKernelGGL((k_gemv_glu<CX_Q4_K, 16, true>), grid, dim3(256), lds, s, P);
      else hipLaunchKernelGGL((k_gemv_glu<CX_Q4_K, 16, false>), grid, dim3(256), lds, s, P);
    }
  } else {
    if (sub == 32) {
      if (hoist) hipLaunchKernelGGL((k_gemv_glu<CX_Q5_K, 32, true>), grid, dim3(256), lds, s, P);
      else hipLaunchKernelGGL((k_gemv_glu<CX_Q5_K, 32, false>), grid, dim3(256), lds, s, P);
    } else {
      if (hoist) hipLaunchKernelGGL((k_gemv_glu<CX_Q5_K, 16, true>), grid, dim3(256), lds, s, P);
      else hipLaunchKernelGGL((k_gemv_glu<CX_Q5_K, 16, false>), grid, dim3(256), lds, s, P);
    }
  }
  CX_HIP(hipGetLastError());
  return CX_OK;
}

// ------------------------------------------------------- L2 prefetch
// The bytes workgroup t of a launch reads: tile t of the plain Q4_K/Q5_K
// GEMV (R consecutive rows) or of the gate/up launch (GLU_ROWS rows of each
// matrix). Workgroups go to XCDs by index, round robin, so a prefetch whose
// workgroup t runs on XCD t % 8 leaves the tile in the L2 the GEMV's
// workgroup t reads.
bool cx_gemv_prefetch_plan(int type, const uint8_t* w, uint32_t n, uint32_t k, cx_l2_job* job) {
  if ((type == CX_Q8_0 || type == CX_Q5_0) && k % 32 == 0 && n) {
    const uint32_t rb = k / 32 * (uint32_t)cx_bpb(type), rows[1] = {n};
    const TilePlan t = plain_plan32(rb, k, k / 32, rows, 1);
    if (!t.R) return false;
    *job = cx_l2_job{w, nullptr, (size_t)n * rb, t.R * rb, t.tiles};
    return true;
  }
  if ((type != CX_Q4_K && type != CX_Q5_K) || k % 256 || !n) return false;
  const uint32_t rb = k / 256 * (uint32_t)cx_bpb(type), rows[1] = {n};
  const RowPlan rp = row_plan(k, rows, 1);
  if (rp.R) {
    *job = cx_l2_job{w, nullptr, (size_t)n * rb, rp.R * rb, rp.tiles};
    return true;
  }
  const TilePlan t = type == CX_Q4_K ? plain_plan<CX_Q4_K>(rb, k, k / 32, rows, 1)
                                     : plain_plan<CX_Q5_K>(rb, k, k / 32, rows, 1);
  if (!t.R) return false;
  *job = cx_l2_job{w, nullptr, (size_t)n * rb, t.R * rb, t.tiles};
  return true;
}

bool cx_glu_prefetch_plan(int type, const uint8_t* wg, const uint8_t* wu, uint32_t I, uint32_t k,
                          cx_l2_job* job) {
  if (!cx_glu_fits(type, k) || I % GLU_ROWS) return false;
  const uint32_t rb = (cx_glu_supported(type) ? k / 256 : k / 32) * (uint32_t)cx_bpb(type);
  // the tiles of the launch that reads them (the row kernel's at k = 2048)
  const uint32_t rows = cx_glu_supported(type) ? glu_row_tile(type, k, I) : GLU_ROWS;
  *job = cx_l2_job{wg, wu, (size_t)I * rb, rows * rb, I / rows};
  return true;
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
  __shared__ double red[9];
  __shared__ int flag;
  const double scale = cx_rms_scale(x, n, eps, red, &flag);
  for (uint32_t i = 8 * threadIdx.x; i < n; i += 8 * 256) {  // n % SUB == 0: whole groups
    float v[8], nw[8];
    cx_load8(x + i, v);
    cx_load8(w + i, nw);
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = (float)((double)v[j] * scale) * nw[j];
    cx_quant8<SUB>(v, i, xq, xe, xs);
  }
}

// rmsnorm of row blockIdx.x of x[rows][k]: the reference's factor
// (cx_rms_scale, bit for bit), then v = (x as f64 * scale) as f32 * w, the
// values the decode step's fused GEMV quantizes for the same row, so a
// batched prefill matches token-by-token decoding.
__global__ __launch_bounds__(256) void k_norm_rows(const float* x, const float* w, uint32_t k,
                                                   float eps, float* out) {
  __shared__ double red[9];
  __shared__ int flag;
  const int tid = threadIdx.x;
  const float* xr = x + (size_t)blockIdx.x * k;
  float* yr = out + (size_t)blockIdx.x * k;
  const double scale = cx_rms_scale(xr, k, eps, red, &flag);
  for (uint32_t i = 8 * tid; i < k; i += 2048) {
    float v[8], nw[8];
    cx_load8(xr + i, v);
    cx_load8(w + i, nw);
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = (float)((double)v[j] * scale) * nw[j];
    reinterpret_cast<float4*>(yr + i)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(yr + i)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// silu(g) * u elementwise (src/forward.rs:483-487), 8 values a lane
__global__ __launch_bounds__(256) void k_swiglu_rows(const float* g, const float* u, size_t n,
                                                     float* out) {
  const size_t i = 8 * (blockIdx.x * 256ull + threadIdx.x);
  if (i >= n) return;
  float a[8], b[8];
  cx_load8(g + i, a);
  cx_load8(u + i, b);
#pragma unroll
  for (int j = 0; j < 8; j++) a[j] = cx_swiglu(a[j], b[j]);
  reinterpret_cast<float4*>(out + i)[0] = make_float4(a[0], a[1], a[2], a[3]);
  reinterpret_cast<float4*>(out + i)[1] = make_float4(a[4], a[5], a[6], a[7]);
}

// y[r][i] += a[r % a_rows][i]: the residual add (a_rows = rows) and the bias
// add (a_rows = 1) of src/forward.rs:316-322, 467-469, 489-491, one f32 add
// each, as the GEMV epilogues do
__global__ __launch_bounds__(256) void k_add_rows(float* y, const float* a, uint32_t n,
                                                  uint32_t a_rows, size_t total) {
  const size_t i = blockIdx.x * 256ull + threadIdx.x;
  if (i >= total) return;
  const size_t r = i / n;
  y[i] = y[i] + a[(r % a_rows) * n + i % n];
}

__global__ __launch_bounds__(256) void k_rmsnorm(float* out, const float* in, const float* w,
                                                 uint32_t n, float eps) {
  __shared__ double red[9];
  __shared__ int flag;
  const float* x = in + (size_t)blockIdx.x * n;
  float* y = out + (size_t)blockIdx.x * n;
  const double scale = cx_rms_scale(x, n, eps, red, &flag);
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
  CX_REQUIRE(n % (size_t)sub == 0 && n < (1u << 31), "norm: width %zu must be whole sub-blocks of %d",
             n, sub);
  if (sub == 16)
    hipLaunchKernelGGL(k_norm_quant<16>, dim3(1), dim3(256), 0, s, x, w, (uint32_t)n, eps, xq, xe, xs);
  else
    hipLaunchKernelGGL(k_norm_quant<32>, dim3(1), dim3(256), 0, s, x, w, (uint32_t)n, eps, xq, xe, xs);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_norm_rows(const float* x, const float* w, size_t rows, size_t k, float eps,
                        float* out, hipStream_t s) {
  CX_REQUIRE(x && w && out, "norm rows: null pointer");
  CX_REQUIRE(k % 8 == 0 && rows < (1u << 31), "norm rows: %zu x %zu", rows, k);
  if (!rows || !k) return CX_OK;
  hipLaunchKernelGGL(k_norm_rows, dim3((unsigned)rows), dim3(256), 0, s, x, w, (uint32_t)k, eps,
                     out);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_swiglu_rows(const float* g, const float* u, size_t n, float* out, hipStream_t s) {
  CX_REQUIRE(g && u && out && n % 8 == 0, "swiglu rows: %zu values", n);
  if (!n) return CX_OK;
  const size_t grid = (n / 8 + 255) / 256;
  CX_REQUIRE(grid < (1ull << 31), "swiglu rows: %zu values is too many", n);
  hipLaunchKernelGGL(k_swiglu_rows, dim3((unsigned)grid), dim3(256), 0, s, g, u, n, out);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_add_rows(float* y, const float* a, size_t rows, size_t n, size_t a_rows,
                       hipStream_t s) {
  CX_REQUIRE(y && a && n && a_rows && n < (1u << 31) && a_rows < (1u << 31),
             "add rows: bad arguments");
  const size_t total = rows * n, grid = (total + 255) / 256;
  if (!total) return CX_OK;
  CX_REQUIRE(grid < (1ull << 31), "add rows: %zu values is too many", total);
  hipLaunchKernelGGL(k_add_rows, dim3((unsigned)grid), dim3(256), 0, s, y, a, (uint32_t)n,
                     (uint32_t)a_rows, total);
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
