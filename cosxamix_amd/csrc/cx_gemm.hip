// cx_gemm.hip — multi-row k-quant contraction on int8 MFMA (gfx950):
// dst[a][r] = fused dot of weight row r with activation row a, for m
// activation rows at once (ops::matmul_auto with m > 1, src/ops.rs:1056-1093;
// BASELINE config 4 and prefill-shaped calls).
//
// Q4_K and Q5_K, whose 32-value sub-blocks are exactly the K = 32 of
// v_mfma_i32_16x16x32_i8: one MFMA gives the exact integer sums E_j of one
// sub-block for a 16 (weight rows) x 16 (activation rows) tile. Each lane
// applies the scalar kernel's f32 term to its four results,
//   term_j = xe_j * (d*sc_j * E_j - dmin*mn_j * xs_j),
// and the terms of one output are added sub-block after sub-block from 0
// (src/kernels/scalar.rs:132-217), so every output equals the per-row dot bit
// for bit and a row of a batch equals the row alone (src/ops.rs:1364-1393).
// The reference's own m >= 24 path (src/ops.rs:607-829) adds in another order
// within 1e-4 of the maximum (src/ops.rs:1518-1561); keeping the per-row
// order makes a batched prefill bit-identical to token-by-token.
//
// The per-sub-block f32 term (6 VALU operations per output and sub-block)
// bounds this path, not the MFMA: a 16x16x32 MFMA is followed by 24 VALU
// instructions per lane.
//
// MFMA lane layout (checked on the device): A 16x32 — lane l holds row
// l%16, k = 8(l/16)..+8 as 8 bytes; B 32x16 — lane l holds column l%16,
// same k range; C 16x16 — lane l element i is row 4(l/16)+i, column l%16.
// Activations are the A operand and weights the B operand, so a lane's four
// results share one weight row (l%16): the lane decodes that row's d, dmin
// and 6-bit scales itself, from one 16-byte read of the block header, and
// reads xe, xs of its four activation rows as float4s.
//
// Workgroup: 4 or 8 waves over a TW x MT tile (TW = 16 RW weight rows, MT =
// 16 AW WA activation rows); the waves split rows (RW), activation tiles (AW)
// and, when a tile is too small to give every wave its own rows, the eight
// sub-blocks of each super-block (KS). With KS > 1 the waves write their
// terms to LDS and each thread adds the terms of its outputs in sub-block
// order. The k loop walks super-blocks through an S-stage ring of
// direct-to-LDS loads: a stage is the tile's weight bytes of one super-block,
// the MT activation rows' 256 bytes, and their xe and xs. Every wave issues
// D loads per stage, so the wait for a stage is a fixed vmcnt; loads beyond
// the stage's bytes reload a valid address into the stage's tail.

#include "cx_act.h"
#include "cx_internal.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// The B operand (weights): positions 8g..8g+7 of sub-block j of a block in
// LDS as 8 i8 values. load() reads the raw bytes, operand() unpacks them.
template <int T> struct GQ;
template <> struct GQ<CX_Q4_K> {
  static constexpr int BPB = 144;
  struct Raw {
    uint2 q;  // qs bytes 32(j/2) + 8g .. +8 (low nibbles: even j, high: odd j)
  };
  __device__ static Raw load(const uint8_t* blk, int j, int g) {
    return Raw{*reinterpret_cast<const uint2*>(blk + 16 + 32 * (j >> 1) + 8 * g)};
  }
  __device__ static long operand(const Raw& r, int j) {
    const uint32_t sh = 4 * (j & 1);
    const uint32_t lo = (r.q.x >> sh) & 0x0F0F0F0Fu, hi = (r.q.y >> sh) & 0x0F0F0F0Fu;
    return (long)(((uint64_t)hi << 32) | lo);
  }
};
template <> struct GQ<CX_Q5_K> {
  static constexpr int BPB = 176;
  struct Raw {
    uint2 q;  // qs bytes 32(j/2) + 8g .. +8
    uint2 h;  // qh bytes 8g .. +8: bit j is the fifth bit of sub-block j
  };
  __device__ static Raw load(const uint8_t* blk, int j, int g) {
    return Raw{*reinterpret_cast<const uint2*>(blk + 48 + 32 * (j >> 1) + 8 * g),
               *reinterpret_cast<const uint2*>(blk + 16 + 8 * g)};
  }
  __device__ static long operand(const Raw& r, int j) {
    const uint32_t sh = 4 * (j & 1);
    const uint32_t lo = ((r.q.x >> sh) & 0x0F0F0F0Fu) | (((r.h.x >> j) & 0x01010101u) << 4);
    const uint32_t hi = ((r.q.y >> sh) & 0x0F0F0F0Fu) | (((r.h.y >> j) & 0x01010101u) << 4);
    return (long)(((uint64_t)hi << 32) | lo);
  }
};

// quant::escala_y_minimo (src/quant.rs:108-117) of sub-block j from the 12
// scale bytes q[0..12) held as the words y (q0..q3), z (q4..q7), w (q8..q11)
__device__ inline void scale_min(uint32_t y, uint32_t z, uint32_t w, int j, uint32_t& sc,
                                 uint32_t& mn) {
  if (j < 4) {
    const int s = 8 * j;
    sc = (y >> s) & 63;
    mn = (z >> s) & 63;
  } else {
    const int s = 8 * (j - 4);
    sc = ((w >> s) & 0xF) | (((y >> (s + 6)) & 3) << 4);
    mn = ((w >> (s + 4)) & 0xF) | (((z >> (s + 6)) & 3) << 4);
  }
}

struct GemmParams {
  const uint8_t* w;     // n rows x row_bytes, GGUF raw
  const int8_t* xq;     // m_pad rows x k (rows >= m are zero)
  const float* xexs;    // per sub-block J: xe of the m_pad rows, then their xs
  float* dst;           // m x n
  uint32_t n, k, m, m_pad, nb, row_bytes, row_tiles, act_tiles;
  const float* lhs;     // m x k f32: the quantizer's input (not read by k_gemm)
  uint8_t* scratch;     // where xq and xexs are carved (not read by k_gemm)
  // k_gemm only: with nseg > 1 the n rows are nseg matrices of one type and
  // width, rows [sr[i], sr[i + 1]) matrix i with weights sw[i] and its own
  // output sd[i] (m x (sr[i + 1] - sr[i])); every sr[i] is a multiple of
  // the tile's rows, so a tile lies in one matrix
  uint32_t nseg, sr[CX_GEMM_SEGS + 1];
  const uint8_t* sw[CX_GEMM_SEGS];
  float* sd[CX_GEMM_SEGS];
  // k_gemm only, per matrix (index 0 without segments): a bias added to
  // every output row (dst = acc + bias[r]), and with accum the output added
  // to what dst holds (dst = dst + (acc [+ bias])), f32 adds as written
  const float* sbias[CX_GEMM_SEGS];
  uint32_t accum;
};

template <int T, int RW, int AW, int WA, int KS, int NSB>
struct Shape {
  static constexpr int NW = RW * AW * KS;  // waves
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  static constexpr int BPB = GQ<T>::BPB;
  static constexpr int TW = 16 * RW, MT = 16 * AW * WA;
  static constexpr int NU = 8 * NSB;  // sub-blocks per stage
  static constexpr int NJ = NU / KS;  // sub-blocks per wave per stage
  static_assert(NU % KS == 0 && (NJ >= 8 ? NJ % 8 == 0 : 8 % NJ == 0), "even split");
  static constexpr int NBW = NJ >= 8 ? NJ / 8 : 1;  // blocks a wave touches per stage
  static constexpr int RB = NSB * BPB;              // LDS bytes per weight row
  // LDS bytes per activation row: 68 mod 64 words, so the 8-byte A operand
  // reads of 16 rows x 2 lane groups (one half-wave pass) hit 64 distinct banks
  static constexpr int XS = NSB * 256 + 16;
  static constexpr int WB = TW * RB, XB = MT * XS, EB = NU * MT * 8;
  static constexpr int WCH = WB / 16, XCH = XB / 16, ECH = EB / 16;
  static constexpr int SLOT = NW * 1024;  // bytes of one load of every wave
  static constexpr int STAGE = (WB + XB + EB + SLOT - 1) / SLOT * SLOT;
  static constexpr int D = STAGE / SLOT;  // loads per wave per stage
  static constexpr int TERMS = KS > 1 ? 2 * NU * TW * MT * 4 : 0;
  static constexpr size_t lds(int S) { return (size_t)S * STAGE + TERMS; }
};

// wait until at most `ahead` stages (D loads each) of this wave are in flight
template <int D, int N>
__device__ inline void wait_stages(int ahead) {
  if constexpr (N == 0) {
    cx_wait_vm<0>();
  } else {
    if (ahead >= N)
      cx_wait_vm<N * D>();
    else
      wait_stages<D, N - 1>(ahead);
  }
}

template <int T, int RW, int AW, int WA, int KS, int NSB, int S>
__global__ __launch_bounds__(64 * RW * AW * KS) void k_gemm(GemmParams P) {
  using SH = Shape<T, RW, AW, WA, KS, NSB>;
  constexpr int BPB = SH::BPB, TW = SH::TW, MT = SH::MT, NU = SH::NU, NJ = SH::NJ;
  constexpr int D = SH::D, NW = SH::NW, RB = SH::RB, XS = SH::XS;
  static_assert(S >= 2 && (S - 2) * D <= 63, "stage waits must fit vmcnt");
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int g = lane >> 4, c16 = lane & 15;
  const int ks = wave % KS, aw = (wave / KS) % AW, rw = wave / (KS * AW);

  // blockIdx -> (row tile, activation tile): the activation tiles of one row
  // tile share blockIdx % 8, i.e. one XCD and its L2, which then holds the
  // row tile's weights for all of them
  const uint32_t b = blockIdx.x, A = P.act_tiles;
  const uint32_t rt = b / (8 * A) * 8 + b % 8, at = b / 8 % A;
  if (rt >= P.row_tiles) return;  // whole workgroup, before any load or barrier
  const uint32_t a0 = at * MT;
  // the tile's matrix: its weights W, rows N, output DST; r0 its first row there
  const uint8_t* W = P.w;
  float* DST = P.dst;
  const float* BIAS = P.sbias[0];
  uint32_t N = P.n, r0 = rt * TW;
  if (P.nseg > 1) {
    uint32_t i = 0;
    while (i + 1 < P.nseg && r0 >= P.sr[i + 1]) i++;
    W = P.sw[i];
    DST = P.sd[i];
    BIAS = P.sbias[i];
    N = P.sr[i + 1] - P.sr[i];
    r0 -= P.sr[i];
  }
  auto put = [&](uint32_t a, uint32_t r, float v) {  // output (a, r) of the tile's matrix
    float* d = DST + (size_t)a * N + r;
    if (BIAS) v = v + BIAS[r];
    if (P.accum) v = *d + v;
    *d = v;
  };

  // this lane's load sources: slot s carries chunk NW*64 s + 64 wave + lane
  // of a stage, i.e. LDS bytes [16 c, 16 c + 16) of the stage; the chunk
  // belongs to super-block bis[s] of the stage (a stage past the last
  // super-block loads a valid dummy address instead)
  const uint8_t* src[D];
  uint32_t inc[D];
  uint32_t bis[D];
#pragma unroll
  for (int s = 0; s < D; s++) {
    const uint32_t c = NW * 64 * s + 64 * wave + lane;
    src[s] = W;
    inc[s] = 0;
    bis[s] = 0;
    if (c < (uint32_t)SH::WCH) {
      const uint32_t r = c / (RB / 16), part = c % (RB / 16);
      const uint32_t row = r0 + r < N ? r0 + r : N - 1;  // past the end: a valid row
      src[s] = W + (size_t)row * P.row_bytes + 16 * part;
      inc[s] = RB;
      bis[s] = part / (BPB / 16);
    } else if (c < (uint32_t)(SH::WCH + SH::XCH)) {
      const uint32_t cc = c - SH::WCH, a = cc / (XS / 16);
      uint32_t part = cc % (XS / 16);
      if (part == 16 * NSB) part = 0;  // the row's pad chunk
      src[s] = reinterpret_cast<const uint8_t*>(P.xq) + (size_t)(a0 + a) * P.k + 16 * part;
      inc[s] = 256 * NSB;
      bis[s] = part / 16;
    } else if (c < (uint32_t)(SH::WCH + SH::XCH + SH::ECH)) {
      // sub-block u of the stage: MT xe, then MT xs
      const uint32_t cc = c - SH::WCH - SH::XCH, u = cc / (MT / 2);
      const uint32_t h = cc % (MT / 2) / (MT / 4), part = cc % (MT / 4);
      src[s] = reinterpret_cast<const uint8_t*>(P.xexs + (size_t)(2 * u + h) * P.m_pad + a0) +
               16 * part;
      inc[s] = NU * 2 * P.m_pad * 4;
      bis[s] = u / 8;
    }
  }
  const uint32_t nb = P.nb, nst = (nb + NSB - 1) / NSB;
  auto issue = [&](uint32_t sb) {
    uint8_t* base = lds + (sb % S) * SH::STAGE + 1024 * wave;
#pragma unroll
    for (int s = 0; s < D; s++) {
      const uint8_t* p = sb * NSB + bis[s] < nb ? src[s] + (size_t)sb * inc[s] : W;
      cx_dma16_async(p, base + SH::SLOT * s);
    }
  };

  float* terms = reinterpret_cast<float*>(lds + S * SH::STAGE);  // [2][NU][TW][MT]
  constexpr int NQ = TW * MT;  // outputs of the tile
  constexpr int PP = KS > 1 ? (NQ + 64 * NW - 1) / (64 * NW) : 1;  // outputs chained per thread
  float acc[WA][4];
  float cacc[PP];
#pragma unroll
  for (int t = 0; t < WA; t++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[t][i] = 0.0f;
#pragma unroll
  for (int i = 0; i < PP; i++) cacc[i] = 0.0f;
  // thread `tid` adds, sub-block by sub-block, the terms of outputs
  // q = tid + 64 NW i (weight row q / MT, activation row q % MT) over the
  // first `nu` sub-blocks of a stage
  auto chain = [&](const float* tb, uint32_t nu) {
#pragma unroll
    for (int i = 0; i < PP; i++) {
      const int q = tid + 64 * NW * i;
      if (NQ % (64 * NW) == 0 || q < NQ) {
        float v[NU];  // every load first (all in the buffer), then the adds in order
#pragma unroll
        for (int u = 0; u < NU; u++) v[u] = tb[u * NQ + q];
#pragma unroll
        for (int u = 0; u < NU; u++)
          if ((uint32_t)u < nu) cacc[i] += v[u];
      }
    }
  };
  auto valid_sub = [&](uint32_t sb) { return 8 * (nb - sb * NSB < NSB ? nb - sb * NSB : NSB); };

  for (uint32_t st = 0; st < (uint32_t)(S - 1) && st < nst; st++) issue(st);
  for (uint32_t sb = 0; sb < nst; sb++) {
    const uint32_t last = sb + S - 2 < nst - 1 ? sb + S - 2 : nst - 1;
    wait_stages<D, S - 2>((int)(last - sb));
    cx_wait_lds();  // this wave's reads of the previous stage are done
    cx_barrier();   // stage sb is in LDS for every wave; slot (sb - 1) % S is free
    if (sb + S - 1 < nst) issue(sb + S - 1);
    const uint8_t* cur = lds + (sb % S) * SH::STAGE;
    const uint8_t* X = cur + SH::WB;
    const float* E = reinterpret_cast<const float*>(cur + SH::WB + SH::XB);
    float* tb = terms + (sb & 1) * (NU * NQ);
    const int ub = ks * NJ;  // this wave's first sub-block of the stage
#pragma unroll
    for (int bb = 0; bb < SH::NBW; bb++) {
      const int bi = (ub >> 3) + bb;  // super-block of the stage
      if (sb * NSB + bi >= nb) break;
      // this lane's weight row: d, dmin and the 12 scale bytes in one read
      const uint8_t* wrow = cur + (16 * rw + c16) * RB + bi * BPB;
      const uint4 hd = *reinterpret_cast<const uint4*>(wrow);
      constexpr int NJB = NJ < 8 ? NJ : 8;  // sub-blocks of this block for this wave
      // every operand of the block first when few (one round of LDS latency),
      // else per sub-block
      constexpr bool BATCH = NJB * WA <= 8;
      typename GQ<T>::Raw wr[BATCH ? NJB : 1];
      long axb[BATCH ? NJB : 1][WA];
      float4 xeb[BATCH ? NJB : 1][WA], xsb[BATCH ? NJB : 1][WA];
      auto fetch = [&](int slot, int u, int j) {
        wr[slot] = GQ<T>::load(wrow, j, g);
#pragma unroll
        for (int t = 0; t < WA; t++) {
          const int ab = 16 * (aw * WA + t);  // first activation row of the MFMA tile
          axb[slot][t] = *reinterpret_cast<const long*>(X + (ab + c16) * XS + 32 * u + 8 * g);
          xeb[slot][t] = *reinterpret_cast<const float4*>(E + u * 2 * MT + ab + 4 * g);
          xsb[slot][t] = *reinterpret_cast<const float4*>(E + u * 2 * MT + MT + ab + 4 * g);
        }
      };
      if constexpr (BATCH) {
#pragma unroll
        for (int jj = 0; jj < NJB; jj++) fetch(jj, ub + 8 * bb + jj, (ub + 8 * bb + jj) & 7);
      }
      const float d = cx_h2f(hd.x & 0xFFFFu), dmin = cx_h2f(hd.x >> 16);
#pragma unroll
      for (int jj = 0; jj < NJB; jj++) {
        const int u = ub + 8 * bb + jj, j = u & 7, sl = BATCH ? jj : 0;
        if constexpr (!BATCH) fetch(0, u, j);
        uint32_t sc, mn;
        scale_min(hd.y, hd.z, hd.w, j, sc, mn);
        const float ds = d * (float)sc, dm = dmin * (float)mn;
        const long bw = GQ<T>::operand(wr[sl], j);
#pragma unroll
        for (int t = 0; t < WA; t++) {
          const int ab = 16 * (aw * WA + t);
          v4i e = {0, 0, 0, 0};
          e = __builtin_amdgcn_mfma_i32_16x16x32_i8(axb[sl][t], bw, e, 0, 0, 0);
          const float4 xe = xeb[sl][t], xs = xsb[sl][t];
          const float xev[4] = {xe.x, xe.y, xe.z, xe.w}, xsv[4] = {xs.x, xs.y, xs.z, xs.w};
          float tv[4];
#pragma unroll
          for (int i = 0; i < 4; i++) tv[i] = xev[i] * (ds * (float)e[i] - dm * xsv[i]);
          if constexpr (KS == 1) {
#pragma unroll
            for (int i = 0; i < 4; i++) acc[t][i] += tv[i];
          } else {
            *reinterpret_cast<float4*>(tb + (u * TW + 16 * rw + c16) * MT + ab + 4 * g) =
                make_float4(tv[0], tv[1], tv[2], tv[3]);
          }
        }
      }
    }
    if constexpr (KS > 1) {
      if (sb > 0) chain(terms + ((sb - 1) & 1) * (NU * NQ), valid_sub(sb - 1));
    }
  }

  if constexpr (KS > 1) {
    cx_wait_lds();
    cx_barrier();
    chain(terms + ((nst - 1) & 1) * (NU * NQ), valid_sub(nst - 1));
#pragma unroll
    for (int i = 0; i < PP; i++) {
      const int q = tid + 64 * NW * i;
      const uint32_t a = a0 + q % MT, r = r0 + q / MT;
      if (q < NQ && a < P.m && r < N) put(a, r, cacc[i]);
    }
  } else {
    // lane: weight row r, activation rows 4g .. 4g+3 of each MFMA tile
    const uint32_t r = r0 + 16 * rw + c16;
    if (r < N) {
#pragma unroll
      for (int t = 0; t < WA; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t a = a0 + 16 * (aw * WA + t) + 4 * g + i;
          if (a < P.m) put(a, r, acc[t][i]);
        }
    }
  }
}

// ------------------------------------------- 32-value blocks (Q8_0, Q5_0)
// The reference's buffer path (ops::matmul_i8_directo, src/ops.rs:310-414;
// its m >= 24 blocked path adds in another order, src/ops.rs:726): one
// v_mfma_i32_16x16x32_i8 per block gives a 16 (activation rows) x 16 (weight
// rows) tile of exact block dots E; each lane applies the GEMV's term
// (d * xe) * E to its four outputs and adds them block after block from 0,
// so every output equals k_gemv32's bit for bit. A workgroup of 4 waves
// covers 64 weight rows x 16 activation rows; the operands are read
// straight from global memory (rows of 34- and 22-byte blocks sit at any
// even offset: 16-bit loads), GB32_DEPTH blocks ahead of the MFMA.
template <int T> struct GB;
template <> struct GB<CX_Q8_0> {
  static constexpr int BPB = 34;
  struct Raw {
    uint16_t d, q[4];
  };
  // d and the quants at positions 8g .. 8g+7 of the block
  __device__ static void load(const uint8_t* blk, int g, Raw& r) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
    r.d = h[0];
#pragma unroll
    for (int i = 0; i < 4; i++) r.q[i] = h[1 + 4 * g + i];
  }
  __device__ static long operand(const Raw& r, int) {
    const uint32_t lo = (uint32_t)r.q[0] | ((uint32_t)r.q[1] << 16);
    const uint32_t hi = (uint32_t)r.q[2] | ((uint32_t)r.q[3] << 16);
    return (long)(((uint64_t)hi << 32) | lo);
  }
};
template <> struct GB<CX_Q5_0> {
  static constexpr int BPB = 22;
  struct Raw {
    uint16_t d, qh[2], qs[4];
  };
  // d, the fifth bits and the nibble bytes of positions 8g .. 8g+7: value
  // i < 16 is the low nibble of qs[i], value 16 + i the high one
  __device__ static void load(const uint8_t* blk, int g, Raw& r) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
    r.d = h[0];
    r.qh[0] = h[1];
    r.qh[1] = h[2];
#pragma unroll
    for (int i = 0; i < 4; i++) r.qs[i] = h[3 + 4 * (g & 1) + i];
  }
  __device__ static uint32_t spread4(uint32_t t) {  // bit i -> bit 4 of byte i
    return ((t & 1u) << 4) | ((t & 2u) << 11) | ((t & 4u) << 18) | ((t & 8u) << 25);
  }
  __device__ static long operand(const Raw& r, int g) {
    const uint32_t qh = (uint32_t)r.qh[0] | ((uint32_t)r.qh[1] << 16);
    const uint32_t sh = g < 2 ? 0u : 4u;
    const uint32_t w0 = ((uint32_t)r.qs[0] | ((uint32_t)r.qs[1] << 16)) >> sh;
    const uint32_t w1 = ((uint32_t)r.qs[2] | ((uint32_t)r.qs[3] << 16)) >> sh;
    const uint32_t t = (qh >> (8 * g)) & 0xFFu;
    // (u - 16) in every byte, u in 0..31: biased by 128 so no byte borrows
    const uint32_t lo = (((w0 & 0x0F0F0F0Fu) | spread4(t & 15u)) | 0x80808080u) - 0x10101010u;
    const uint32_t hi = (((w1 & 0x0F0F0F0Fu) | spread4(t >> 4)) | 0x80808080u) - 0x10101010u;
    return (long)(((uint64_t)(hi ^ 0x80808080u) << 32) | (lo ^ 0x80808080u));
  }
};

constexpr int GB32_DEPTH = 4;

template <int T>
__global__ __launch_bounds__(256) void k_gemm32(GemmParams P) {
  using Q = GB<T>;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  // the activation tiles of one row tile share blockIdx % 8 (one XCD's L2)
  const uint32_t b = blockIdx.x, A = P.act_tiles;
  const uint32_t rt = b / (8 * A) * 8 + b % 8, at = b / 8 % A;
  if (rt >= P.row_tiles) return;
  const uint32_t r = rt * 64 + 16 * wave + c16;  // this lane's weight row (B column)
  const uint32_t a0 = at * 16;
  const uint8_t* wrow = P.w + (size_t)min(r, P.n - 1) * P.row_bytes;  // past the end: a valid row
  const int8_t* xrow = P.xq + (size_t)(a0 + c16) * P.k + 8 * g;     // A operand: row a0 + c16
  const float* xe = P.xexs + a0 + 4 * g;  // block J: xe of the tile's rows at J * 2 * m_pad
  const uint32_t nb = P.k / 32;
  typename Q::Raw wr[GB32_DEPTH];
  long ax[GB32_DEPTH];
  float4 xv[GB32_DEPTH];
  auto fetch = [&](uint32_t j, int slot) {
    Q::load(wrow + (size_t)j * Q::BPB, g, wr[slot]);
    ax[slot] = *reinterpret_cast<const long*>(xrow + 32 * j);
    xv[slot] = *reinterpret_cast<const float4*>(xe + (size_t)j * 2 * P.m_pad);
  };
#pragma unroll
  for (int d = 0; d < GB32_DEPTH; d++)
    if ((uint32_t)d < nb) fetch(d, d);
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t j0 = 0; j0 < nb; j0 += GB32_DEPTH) {
#pragma unroll
    for (int d = 0; d < GB32_DEPTH; d++) {
      const uint32_t j = j0 + d;
      if (j < nb) {
        v4i e = {0, 0, 0, 0};
        e = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax[d], Q::operand(wr[d], g), e, 0, 0, 0);
        const float dw = cx_h2f(wr[d].d);
        const float xs4[4] = {xv[d].x, xv[d].y, xv[d].z, xv[d].w};
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] += dw * xs4[i] * (float)e[i];
        if (j + GB32_DEPTH < nb) fetch(j + GB32_DEPTH, d);
      }
    }
  }
  if (r < P.n) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t a = a0 + 4 * g + i;
      if (a < P.m) P.dst[(size_t)a * P.n + r] = acc[i];
    }
  }
}

// ----------------------------- 16-value sub-blocks (Q2_K, Q3_K, Q6_K)
// A 32-value group of a super-block holds two sub-blocks: lanes 16..31 of
// the group's MFMA K range (lane groups g = 0, 1) are sub-block 2G and
// 32..63 (g = 2, 3) sub-block 2G + 1. Two MFMAs per group, each with the
// other sub-block's weight bytes zeroed, give the two exact sums; each lane
// then applies the GEMV's term (k_gemv's KQ<T>) and adds in sub-block order,
// so every output equals the per-row GEMV bit for bit. Operands come
// straight from global memory (16-bit loads: 84-, 110- and 210-byte blocks
// leave rows at any even offset).
template <int T> struct GK;
__device__ inline long pack8(uint32_t lo, uint32_t hi) {
  return (long)(((uint64_t)hi << 32) | lo);
}
__device__ inline uint32_t w16(const uint16_t* h) { return (uint32_t)h[0] | ((uint32_t)h[1] << 16); }

// Q2_K, 84 B: scales(16: low nibble scale, high nibble min) qs(64) d dmin;
// value (qs[32(G/4) + i] >> 2(G%4)) & 3 (src/kernels/q2k.rs:41-69)
template <> struct GK<CX_Q2_K> {
  static constexpr int BPB = 84;
  struct Raw {
    uint16_t q[4], sc, d, dm;
  };
  __device__ static void load(const uint8_t* blk, int G, int g, Raw& r) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
    const int q0 = (16 + 32 * (G / 4) + 8 * g) / 2;
#pragma unroll
    for (int i = 0; i < 4; i++) r.q[i] = h[q0 + i];
    r.sc = h[G];  // the scale bytes of sub-blocks 2G, 2G+1
    r.d = h[40];
    r.dm = h[41];
  }
  __device__ static long operand(const Raw& r, int G, int) {
    const uint32_t sh = 2 * (G % 4);
    return pack8((w16(r.q) >> sh) & 0x03030303u, (w16(r.q + 2) >> sh) & 0x03030303u);
  }
  __device__ static float term(const Raw& r, int G, int hf, int e, float xe, float xs) {
    (void)G;
    const uint32_t sc = hf ? (r.sc >> 8) : (r.sc & 0xFFu);
    const float d = cx_h2f(r.d), dm = cx_h2f(r.dm);
    return xe * (d * (float)(sc & 0xF) * (float)e - dm * (float)(sc >> 4) * xs);
  }
};

// Q3_K, 110 B: hmask(32) qs(64) scales(12) d; value (q + 4) =
// ((qs[32(G/4) + i] >> 2(G%4)) & 3) | ((hmask[i] >> G) & 1) << 2
// (src/kernels/scalar.rs:236-275), scales as quant::escalas_q3k
template <> struct GK<CX_Q3_K> {
  static constexpr int BPB = 110;
  struct Raw {
    uint16_t q[4], hm[4], sw[6], d;
  };
  __device__ static void load(const uint8_t* blk, int G, int g, Raw& r) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
    const int q0 = (32 + 32 * (G / 4) + 8 * g) / 2;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      r.q[i] = h[q0 + i];
      r.hm[i] = h[4 * g + i];
    }
#pragma unroll
    for (int i = 0; i < 6; i++) r.sw[i] = h[48 + i];
    r.d = h[54];
  }
  __device__ static long operand(const Raw& r, int G, int) {
    const uint32_t sh = 2 * (G % 4);
    const uint32_t lo = ((w16(r.q) >> sh) & 0x03030303u) | (((w16(r.hm) >> G) & 0x01010101u) << 2);
    const uint32_t hi =
        ((w16(r.q + 2) >> sh) & 0x03030303u) | (((w16(r.hm + 2) >> G) & 0x01010101u) << 2);
    return pack8(lo, hi);
  }
  // the 6-bit signed scale of sub-block s (src/quant.rs:87-106)
  __device__ static float esc(const Raw& r, int s) {
    const uint32_t m1 = 0x03030303u, m2 = 0x0F0F0F0Fu;
    const uint32_t a0 = w16(r.sw), a1 = w16(r.sw + 2), t = w16(r.sw + 4);
    uint32_t w;
    switch (s / 4) {
      case 0: w = (a0 & m2) | ((t & m1) << 4); break;
      case 1: w = (a1 & m2) | (((t >> 2) & m1) << 4); break;
      case 2: w = ((a0 >> 4) & m2) | (((t >> 4) & m1) << 4); break;
      default: w = ((a1 >> 4) & m2) | (((t >> 6) & m1) << 4); break;
    }
    return (float)(int8_t)(uint8_t)(w >> (8 * (s % 4)));
  }
  __device__ static float term(const Raw& r, int G, int hf, int e, float xe, float xs) {
    const float scale = cx_h2f(r.d) * (esc(r, 2 * G + hf) - 32.0f);
    return xe * scale * ((float)e - 4.0f * xs);
  }
};

// Q6_K, 210 B: ql(128) qh(64) scales(16, i8) d. Group G: half = G/4,
// gi = G%4; value = nibble | ((qh[32 half + i] >> 2gi) & 3) << 4, the nibble
// low (gi < 2) or high of ql[64 half + 32 (gi%2) + i] (src/kernels/scalar.rs:294-324)
template <> struct GK<CX_Q6_K> {
  static constexpr int BPB = 210;
  struct Raw {
    uint16_t ql[4], qh[4], sc, d;
  };
  __device__ static void load(const uint8_t* blk, int G, int g, Raw& r) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
    const int half = G / 4, gi = G % 4;
    const int l0 = (64 * half + 32 * (gi % 2) + 8 * g) / 2, h0 = (128 + 32 * half + 8 * g) / 2;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      r.ql[i] = h[l0 + i];
      r.qh[i] = h[h0 + i];
    }
    r.sc = h[96 + G];
    r.d = h[104];
  }
  __device__ static long operand(const Raw& r, int G, int) {
    const int gi = G % 4;
    const uint32_t ns = gi < 2 ? 0u : 4u, hs = 2 * gi;
    const uint32_t lo = ((w16(r.ql) >> ns) & 0x0F0F0F0Fu) | (((w16(r.qh) >> hs) & 0x03030303u) << 4);
    const uint32_t hi =
        ((w16(r.ql + 2) >> ns) & 0x0F0F0F0Fu) | (((w16(r.qh + 2) >> hs) & 0x03030303u) << 4);
    return pack8(lo, hi);
  }
  __device__ static float term(const Raw& r, int G, int hf, int e, float xe, float xs) {
    (void)G;
    const float scale = cx_h2f(r.d) * (float)(int8_t)(uint8_t)(hf ? (r.sc >> 8) : (r.sc & 0xFFu));
    return xe * scale * ((float)e - 32.0f * xs);
  }
};

constexpr int GK16_DEPTH = 3;

template <int T>
__global__ __launch_bounds__(256) void k_gemm16(GemmParams P) {
  using Q = GK<T>;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const uint32_t b = blockIdx.x, A = P.act_tiles;
  const uint32_t rt = b / (8 * A) * 8 + b % 8, at = b / 8 % A;
  if (rt >= P.row_tiles) return;
  const uint32_t r = rt * 64 + 16 * wave + c16;
  const uint32_t a0 = at * 16;
  const uint8_t* wrow = P.w + (size_t)min(r, P.n - 1) * P.row_bytes;
  const int8_t* xrow = P.xq + (size_t)(a0 + c16) * P.k + 8 * g;
  const float* xe = P.xexs + a0 + 4 * g;  // sub-block J: xe at J * 2 * m_pad, xs m_pad after
  const uint32_t ng = P.k / 32;          // 32-value groups
  typename Q::Raw wr[GK16_DEPTH];
  long ax[GK16_DEPTH];
  float4 xv[GK16_DEPTH][4];  // xe, xs of sub-block 2j, then of 2j + 1
  auto fetch = [&](uint32_t j, int slot) {
    Q::load(wrow + (size_t)(j / 8) * Q::BPB, (int)(j % 8), g, wr[slot]);
    ax[slot] = *reinterpret_cast<const long*>(xrow + 32 * j);
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const float* e = xe + (size_t)(2 * j + h) * 2 * P.m_pad;
      xv[slot][2 * h] = *reinterpret_cast<const float4*>(e);
      xv[slot][2 * h + 1] = *reinterpret_cast<const float4*>(e + P.m_pad);
    }
  };
#pragma unroll
  for (int d = 0; d < GK16_DEPTH; d++)
    if ((uint32_t)d < ng) fetch(d, d);
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t j0 = 0; j0 < ng; j0 += GK16_DEPTH) {
#pragma unroll
    for (int d = 0; d < GK16_DEPTH; d++) {
      const uint32_t j = j0 + d;
      if (j < ng) {
        const int G = (int)(j % 8);
        const long bw = Q::operand(wr[d], G, g);
        v4i e0 = {0, 0, 0, 0}, e1 = {0, 0, 0, 0};
        e0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax[d], g < 2 ? bw : 0l, e0, 0, 0, 0);
        e1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(ax[d], g < 2 ? 0l : bw, e1, 0, 0, 0);
        const float4 xe0 = xv[d][0], xs0 = xv[d][1], xe1 = xv[d][2], xs1 = xv[d][3];
        const float a_e0[4] = {xe0.x, xe0.y, xe0.z, xe0.w}, a_s0[4] = {xs0.x, xs0.y, xs0.z, xs0.w};
        const float a_e1[4] = {xe1.x, xe1.y, xe1.z, xe1.w}, a_s1[4] = {xs1.x, xs1.y, xs1.z, xs1.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          acc[i] += Q::term(wr[d], G, 0, e0[i], a_e0[i], a_s0[i]);
          acc[i] += Q::term(wr[d], G, 1, e1[i], a_e1[i], a_s1[i]);
        }
        if (j + GK16_DEPTH < ng) fetch(j + GK16_DEPTH, d);
      }
    }
  }
  if (r < P.n) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t a = a0 + 4 * g + i;
      if (a < P.m) P.dst[(size_t)a * P.n + r] = acc[i];
    }
  }
}

// ops::cuantizar_i8_en (src/ops.rs:178-198) of m rows into the layout above:
// xq rows [m, m_pad) and their xe, xs are zero
template <int SUB>
__global__ __launch_bounds__(256) void k_quantize_gemm(const float* x, uint32_t m, uint32_t k,
                                                       uint32_t m_pad, int8_t* xq, float* xexs) {
  const size_t i = 8 * (blockIdx.x * 256ull + threadIdx.x);
  if (i >= (size_t)m_pad * k) return;
  const uint32_t a = (uint32_t)(i / k), col = (uint32_t)(i % k);
  float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (a < m) cx_load8(x + i, v);
  uint32_t lo, hi;
  float d;
  int32_t s;
  cx_quant8_vals<SUB>(v, lo, hi, d, s);
  *reinterpret_cast<uint2*>(xq + i) = make_uint2(lo, hi);
  if ((col & (SUB - 1)) == 0) {
    float* e = xexs + (size_t)(col / SUB) * 2 * m_pad + a;
    e[0] = d;
    e[m_pad] = (float)s;
  }
}

// The prefill's row ops straight into that layout, for the contraction that
// reads them: rmsnorm (k_norm_rows' arithmetic: the reference's factor by
// cx_rms_scale, then (float)(x * scale) * w; src/kernels/scalar.rs:36-54),
// one workgroup a row; and silu(g) * u (src/forward.rs:483-487); each
// value is what the row kernel writes, then quantized as k_quantize_gemm
// quantizes it. Rows [m, m_pad) are zero.
template <int SUB>
__global__ __launch_bounds__(256) void k_norm_quant_gemm(const float* x, const float* w,
                                                         uint32_t m, uint32_t k, float eps,
                                                         uint32_t m_pad, int8_t* xq, float* xexs) {
  __shared__ double red[9];
  __shared__ int flag;
  const int tid = threadIdx.x;
  const uint32_t a = blockIdx.x;
  const float* xr = x + (size_t)a * k;
  double scale = 0.0;
  if (a < m) scale = cx_rms_scale(xr, k, eps, red, &flag);  // the same for the whole workgroup
  for (uint32_t i = 8 * tid; i < k; i += 2048) {  // whole quads of lanes (k % 32 == 0)
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (a < m) {
      float nw[8];
      cx_load8(xr + i, v);
      cx_load8(w + i, nw);
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = (float)((double)v[j] * scale) * nw[j];
    }
    uint32_t lo, hi;
    float d;
    int32_t s;
    cx_quant8_vals<SUB>(v, lo, hi, d, s);
    *reinterpret_cast<uint2*>(xq + (size_t)a * k + i) = make_uint2(lo, hi);
    if ((i & (SUB - 1)) == 0) {
      float* e = xexs + (size_t)(i / SUB) * 2 * m_pad + a;
      e[0] = d;
      e[m_pad] = (float)s;
    }
  }
}

template <int SUB>
__global__ __launch_bounds__(256) void k_swiglu_quant_gemm(const float* g, const float* u,
                                                           uint32_t m, uint32_t k, uint32_t m_pad,
                                                           int8_t* xq, float* xexs) {
  const size_t i = 8 * (blockIdx.x * 256ull + threadIdx.x);
  if (i >= (size_t)m_pad * k) return;
  const uint32_t a = (uint32_t)(i / k), col = (uint32_t)(i % k);
  float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (a < m) {
    float b[8];
    cx_load8(g + i, v);
    cx_load8(u + i, b);
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = cx_swiglu(v[j], b[j]);
  }
  uint32_t lo, hi;
  float d;
  int32_t s;
  cx_quant8_vals<SUB>(v, lo, hi, d, s);
  *reinterpret_cast<uint2*>(xq + i) = make_uint2(lo, hi);
  if ((col & (SUB - 1)) == 0) {
    float* e = xexs + (size_t)(col / SUB) * 2 * m_pad + a;
    e[0] = d;
    e[m_pad] = (float)s;
  }
}

struct Config {
  int tw, mt, threads;
  size_t lds;
};

typedef void (*gemm_kernel)(GemmParams);

template <int T, int RW, int AW, int WA, int KS, int NSB, int S>
Config make_config(gemm_kernel* k) {
  using SH = Shape<T, RW, AW, WA, KS, NSB>;
  static_assert(SH::lds(S) <= 160 * 1024, "LDS of one CU");
  *k = k_gemm<T, RW, AW, WA, KS, NSB, S>;
  return Config{SH::TW, SH::MT, 64 * SH::NW, SH::lds(S)};
}

// The tile shapes: weight rows x activation rows, waves, super-blocks per
// stage, ring stages. Each is the fastest of a sweep for some (n, m) of
// BASELINE config 4 (11008 x 2048 and 2048 x 11008, m = 2 .. 512).
template <int T>
Config config(int id, gemm_kernel* k) {
  switch (id) {
    case 0: return make_config<T, 1, 1, 1, 8, 4, 2>(k);  // 16 x 16, 8 waves split k
    case 1: return make_config<T, 1, 1, 1, 8, 2, 3>(k);  // 16 x 16, 8 waves split k
    case 2: return make_config<T, 4, 1, 1, 1, 2, 3>(k);  // 64 x 16
    case 3: return make_config<T, 4, 2, 1, 1, 2, 2>(k);  // 64 x 32, 8 waves
    case 4: return make_config<T, 2, 2, 1, 1, 2, 2>(k);  // 32 x 32
    case 5: return make_config<T, 4, 2, 2, 1, 1, 3>(k);  // 64 x 64, 8 waves
    default: return make_config<T, 8, 1, 4, 1, 1, 2>(k);  // 128 x 64, 8 waves
  }
}

// Few weight rows (n < 4096: 2048 x 11008 and the q/o/k/v shapes) take the
// largest tile (64 x 64, 64 x 32, then 32 x 32) that gives at least 5/8 of
// the CUs a workgroup; below that, 16 x 16 tiles that split k over the
// waves (four super-blocks a stage up to a workgroup per CU, two past it).
// Swept at n = 2048 (k = 2048 and 11008) and n = 256 for m = 64 to 512: the
// rule picks the fastest tile or one within 3% of it; at a prefill
// chunk (m = 256) 2048 x 11008 takes 62 us in 64 x 32 tiles against 88 in
// 64 x 64, 2048 x 2048 16.3 against 20.6, 256 x 2048 9.5 in 16 x 16 against
// 20.8.
int choose(uint32_t n, uint32_t m) {
  if (n >= 4096) return m <= 16 ? 2 : m <= 32 ? 3 : m <= 64 ? 5 : 6;
  auto tiles = [&](uint32_t tw, uint32_t mt) { return (n + tw - 1) / tw * ((m + mt - 1) / mt); };
  constexpr uint32_t ENOUGH = 256 * 5 / 8;  // workgroups, on 256 CUs
  if (tiles(64, 64) >= ENOUGH) return 5;
  if (tiles(64, 32) >= ENOUGH) return 3;
  if (tiles(32, 32) >= ENOUGH) return 4;
  return tiles(16, 16) <= 256 ? 0 : 1;
}

// xq and xexs of m_pad quantized rows in scratch
inline int8_t* scratch_xq(uint8_t* scratch) { return reinterpret_cast<int8_t*>(scratch); }
inline float* scratch_xexs(uint8_t* scratch, size_t m_pad, size_t k) {
  return reinterpret_cast<float*>(scratch + (m_pad * k + 255) / 256 * 256);
}

int quantize(const float* lhs, uint32_t m, uint32_t k, uint32_t m_pad, int sub, uint8_t* scratch,
             hipStream_t s) {
  const size_t qgrid = ((size_t)m_pad * k / 8 + 255) / 256;
  CX_REQUIRE(qgrid < (1ull << 31), "gemm: %zu activation values is too many", (size_t)m_pad * k);
  if (sub == 16)
    hipLaunchKernelGGL(k_quantize_gemm<16>, dim3((unsigned)qgrid), dim3(256), 0, s, lhs, m, k,
                       m_pad, scratch_xq(scratch), scratch_xexs(scratch, m_pad, k));
  else
    hipLaunchKernelGGL(k_quantize_gemm<32>, dim3((unsigned)qgrid), dim3(256), 0, s, lhs, m, k,
                       m_pad, scratch_xq(scratch), scratch_xexs(scratch, m_pad, k));
  CX_HIP(hipGetLastError());
  return CX_OK;
}

// the contraction over rows quantized with a row count m_pad that is a
// multiple of the chosen tile's height
template <int T>
int contract(GemmParams& P, hipStream_t s) {
  gemm_kernel k = nullptr;
  const Config c = config<T>(choose(P.n, P.m), &k);
  CX_REQUIRE(P.m_pad % c.mt == 0 && P.m_pad >= P.m, "gemm: %u padded rows for tiles of %d",
             P.m_pad, c.mt);
  P.xq = scratch_xq(P.scratch);
  P.xexs = scratch_xexs(P.scratch, P.m_pad, P.k);
  P.row_tiles = (P.n + c.tw - 1) / c.tw;
  P.act_tiles = (P.m + c.mt - 1) / c.mt;
  const size_t grid = (size_t)(P.row_tiles + 7) / 8 * 8 * P.act_tiles;
  CX_REQUIRE(grid < (1ull << 31), "gemm: %u x %u is too large", P.n, P.m);
  hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(c.threads), c.lds, s, P);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

template <int T>
int launch(GemmParams& P, hipStream_t s) {
  gemm_kernel k = nullptr;
  const Config c = config<T>(choose(P.n, P.m), &k);
  // activation rows padded to the tile height (zero rows quantize to zero)
  P.m_pad = (P.m + c.mt - 1) / c.mt * c.mt;
  int rc = quantize(P.lhs, P.m, P.k, P.m_pad, 32, P.scratch, s);
  return rc ? rc : contract<T>(P, s);
}

// every tile height (16, 32 or 64 rows) divides 64
inline uint32_t pad64(size_t m) { return (uint32_t)((m + 63) / 64 * 64); }

// the direct-operand contractions (32-value blocks and 16-value sub-blocks)
// over rows quantized in scratch with the type's sub-block size (m_pad set)
bool direct_type(int type) { return cx_is_block32(type) || cx_sub(type) == 16; }
int contract_direct(int type, GemmParams& P, hipStream_t s) {
  P.xq = scratch_xq(P.scratch);
  P.xexs = scratch_xexs(P.scratch, P.m_pad, P.k);
  P.row_tiles = (P.n + 63) / 64;
  P.act_tiles = (P.m + 15) / 16;
  const size_t grid = (size_t)(P.row_tiles + 7) / 8 * 8 * P.act_tiles;
  CX_REQUIRE(grid < (1ull << 31), "gemm: %u x %u is too large", P.n, P.m);
  const dim3 G((unsigned)grid), W(256);
  switch (type) {
    case CX_Q8_0: hipLaunchKernelGGL(k_gemm32<CX_Q8_0>, G, W, 0, s, P); break;
    case CX_Q5_0: hipLaunchKernelGGL(k_gemm32<CX_Q5_0>, G, W, 0, s, P); break;
    case CX_Q2_K: hipLaunchKernelGGL(k_gemm16<CX_Q2_K>, G, W, 0, s, P); break;
    case CX_Q3_K: hipLaunchKernelGGL(k_gemm16<CX_Q3_K>, G, W, 0, s, P); break;
    default: hipLaunchKernelGGL(k_gemm16<CX_Q6_K>, G, W, 0, s, P); break;
  }
  CX_HIP(hipGetLastError());
  return CX_OK;
}

}  // namespace

bool cx_gemm_supported(int type) { return cx_has_gemv(type); }

size_t cx_gemm_scratch_bytes(size_t m, size_t k) {  // xe and xs for sub-blocks of 16
  const size_t m_pad = (m + 63) / 64 * 64;
  return (m_pad * k + 255) / 256 * 256 + m_pad * (k / 16) * 8;
}

int cx_launch_gemm(int type, const uint8_t* w, size_t n, size_t k, const float* lhs, size_t m,
                   float* dst, void* scratch, hipStream_t s) {
  CX_REQUIRE(cx_gemm_supported(type), "gemm: type %d has no MFMA path", type);
  CX_REQUIRE(w && lhs && dst && scratch, "gemm: null pointer");
  const size_t vpb = (size_t)cx_vpb(type);
  CX_REQUIRE(k % vpb == 0 && k > 0, "gemm: k=%zu is not a multiple of %zu", k, vpb);
  CX_REQUIRE(n < (1u << 31) && m < (1u << 24) && k < (1u << 24), "gemm: shape too large");
  CX_REQUIRE(((uintptr_t)w & (direct_type(type) ? 1 : 15)) == 0 && ((uintptr_t)lhs & 15) == 0 &&
                 ((uintptr_t)scratch & 255) == 0,
             "gemm: weights (Q4_K/Q5_K 16-byte, others 2-byte) and activations (16-byte) misaligned");
  if (!n || !m) return CX_OK;
  GemmParams P{};
  P.lhs = lhs;
  P.scratch = reinterpret_cast<uint8_t*>(scratch);
  P.w = w;
  P.dst = dst;
  P.n = (uint32_t)n;
  P.k = (uint32_t)k;
  P.m = (uint32_t)m;
  P.nb = (uint32_t)(k / vpb);
  P.row_bytes = P.nb * cx_bpb(type);
  if (direct_type(type)) {
    P.m_pad = pad64(m);
    const int rc = quantize(lhs, P.m, P.k, P.m_pad, cx_sub(type), P.scratch, s);
    return rc ? rc : contract_direct(type, P, s);
  }
  return type == CX_Q4_K ? launch<CX_Q4_K>(P, s) : launch<CX_Q5_K>(P, s);
}

int cx_gemm_quantize(const float* lhs, size_t m, size_t k, int sub, void* scratch, hipStream_t s) {
  CX_REQUIRE(lhs && scratch, "gemm: null pointer");
  CX_REQUIRE(sub == 16 || sub == 32, "gemm: sub-blocks of 16 or 32, not %d", sub);
  CX_REQUIRE(k % 32 == 0 && k > 0 && k < (1u << 24) && m < (1u << 24), "gemm: %zu x %zu", m, k);
  CX_REQUIRE(((uintptr_t)lhs & 15) == 0 && ((uintptr_t)scratch & 255) == 0,
             "gemm: activations must be 16-byte and scratch 256-byte aligned");
  if (!m) return CX_OK;
  return quantize(lhs, (uint32_t)m, (uint32_t)k, pad64(m), sub, reinterpret_cast<uint8_t*>(scratch),
                  s);
}

int cx_gemm_norm_quantize(const float* x, const float* w, size_t m, size_t k, float eps, int sub,
                          void* scratch, hipStream_t s) {
  CX_REQUIRE(x && w && scratch, "gemm: null pointer");
  CX_REQUIRE(sub == 16 || sub == 32, "gemm: sub-blocks of 16 or 32, not %d", sub);
  CX_REQUIRE(k % 32 == 0 && k > 0 && k < (1u << 24) && m < (1u << 24), "gemm: %zu x %zu", m, k);
  CX_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 &&
                 ((uintptr_t)scratch & 255) == 0,
             "gemm: rows and weights must be 16-byte and scratch 256-byte aligned");
  if (!m) return CX_OK;
  const uint32_t mp = pad64(m);
  uint8_t* sc = reinterpret_cast<uint8_t*>(scratch);
  if (sub == 16)
    hipLaunchKernelGGL(k_norm_quant_gemm<16>, dim3(mp), dim3(256), 0, s, x, w, (uint32_t)m,
                       (uint32_t)k, eps, mp, scratch_xq(sc), scratch_xexs(sc, mp, k));
  else
    hipLaunchKernelGGL(k_norm_quant_gemm<32>, dim3(mp), dim3(256), 0, s, x, w, (uint32_t)m,
                       (uint32_t)k, eps, mp, scratch_xq(sc), scratch_xexs(sc, mp, k));
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_gemm_swiglu_quantize(const float* g, const float* u, size_t m, size_t k, int sub,
                            void* scratch, hipStream_t s) {
  CX_REQUIRE(g && u && scratch, "gemm: null pointer");
  CX_REQUIRE(sub == 16 || sub == 32, "gemm: sub-blocks of 16 or 32, not %d", sub);
  CX_REQUIRE(k % 32 == 0 && k > 0 && k < (1u << 24) && m < (1u << 24), "gemm: %zu x %zu", m, k);
  CX_REQUIRE(((uintptr_t)g & 15) == 0 && ((uintptr_t)u & 15) == 0 &&
                 ((uintptr_t)scratch & 255) == 0,
             "gemm: rows must be 16-byte and scratch 256-byte aligned");
  if (!m) return CX_OK;
  const uint32_t mp = pad64(m);
  uint8_t* sc = reinterpret_cast<uint8_t*>(scratch);
  const size_t grid = ((size_t)mp * k / 8 + 255) / 256;
  CX_REQUIRE(grid < (1ull << 31), "gemm: %zu activation values is too many", (size_t)mp * k);
  if (sub == 16)
    hipLaunchKernelGGL(k_swiglu_quant_gemm<16>, dim3((unsigned)grid), dim3(256), 0, s, g, u,
                       (uint32_t)m, (uint32_t)k, mp, scratch_xq(sc), scratch_xexs(sc, mp, k));
  else
    hipLaunchKernelGGL(k_swiglu_quant_gemm<32>, dim3((unsigned)grid), dim3(256), 0, s, g, u,
                       (uint32_t)m, (uint32_t)k, mp, scratch_xq(sc), scratch_xexs(sc, mp, k));
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_gemm_apply(int type, const uint8_t* w, size_t n, size_t k, size_t m, float* dst,
                  const void* scratch, hipStream_t s) {
  CX_REQUIRE(cx_gemm_supported(type), "gemm: type %d has no MFMA path", type);
  CX_REQUIRE(w && dst && scratch, "gemm: null pointer");
  const size_t vpb = (size_t)cx_vpb(type);
  CX_REQUIRE(k % vpb == 0 && k > 0, "gemm: k=%zu is not a multiple of %zu", k, vpb);
  CX_REQUIRE(n < (1u << 31) && m < (1u << 24) && k < (1u << 24), "gemm: shape too large");
  CX_REQUIRE(((uintptr_t)w & (direct_type(type) ? 1 : 15)) == 0 && ((uintptr_t)scratch & 255) == 0,
             "gemm: weights (Q4_K/Q5_K 16-byte, others 2-byte) or scratch (256-byte) misaligned");
  if (!n || !m) return CX_OK;
  GemmParams P{};
  P.scratch = const_cast<uint8_t*>(reinterpret_cast<const uint8_t*>(scratch));
  P.w = w;
  P.dst = dst;
  P.n = (uint32_t)n;
  P.k = (uint32_t)k;
  P.m = (uint32_t)m;
  P.m_pad = pad64(m);
  P.nb = (uint32_t)(k / vpb);
  P.row_bytes = P.nb * cx_bpb(type);
  if (direct_type(type)) return contract_direct(type, P, s);
  return type == CX_Q4_K ? contract<CX_Q4_K>(P, s) : contract<CX_Q5_K>(P, s);
}

bool cx_gemm_multi_fits(int type, const uint32_t* n, uint32_t count, size_t m) {
  if (!n || count < 1 || count > CX_GEMM_SEGS || !m || m >= (1u << 24) ||
      !cx_gemm_supported(type) || direct_type(type))
    return false;
  uint32_t total = 0;
  for (uint32_t i = 0; i < count; i++) total += n[i];
  if (!total) return false;
  gemm_kernel kern = nullptr;
  const Config c = type == CX_Q4_K ? config<CX_Q4_K>(choose(total, (uint32_t)m), &kern)
                                   : config<CX_Q5_K>(choose(total, (uint32_t)m), &kern);
  for (uint32_t i = 0; count > 1 && i < count; i++)
    if (n[i] % c.tw != 0) return false;  // a tile would straddle two matrices
  return true;
}

int cx_gemm_apply_multi(int type, const uint8_t* const* w, const uint32_t* n, uint32_t count,
                        size_t k, size_t m, float* const* dst, const float* const* bias, int accum,
                        const void* scratch, hipStream_t s) {
  CX_REQUIRE(w && dst && cx_gemm_multi_fits(type, n, count, m),
             "gemm: %u matrices of type %d over %zu rows do not fit one launch", count, type, m);
  const size_t vpb = (size_t)cx_vpb(type);
  CX_REQUIRE(k % vpb == 0 && k > 0 && k < (1u << 24), "gemm: k=%zu", k);
  CX_REQUIRE(((uintptr_t)scratch & 255) == 0, "gemm: scratch misaligned");
  GemmParams P{};
  P.scratch = const_cast<uint8_t*>(reinterpret_cast<const uint8_t*>(scratch));
  P.nseg = count;
  for (uint32_t i = 0; i < count; i++) {
    CX_REQUIRE(w[i] && dst[i] && ((uintptr_t)w[i] & 15) == 0,
               "gemm: matrix %u: null or misaligned (16-byte) pointer", i);
    P.sw[i] = w[i];
    P.sd[i] = dst[i];
    P.sbias[i] = bias ? bias[i] : nullptr;
    P.sr[i + 1] = P.sr[i] + n[i];
  }
  P.accum = accum ? 1u : 0u;
  P.w = w[0];
  P.dst = dst[0];
  P.n = P.sr[count];
  P.k = (uint32_t)k;
  P.m = (uint32_t)m;
  P.m_pad = pad64(m);
  P.nb = (uint32_t)(k / vpb);
  P.row_bytes = P.nb * cx_bpb(type);
  return type == CX_Q4_K ? contract<CX_Q4_K>(P, s) : contract<CX_Q5_K>(P, s);
}
