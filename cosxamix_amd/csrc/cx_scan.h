// cx_scan.h — ordered f32 running sums of non-negative terms by one wave,
// with the rounding of one add per position: the softmax sums of
// ops::softmax (`tot += e`, src/ops.rs:1221-1225) and the sampler's running
// sums (src/sampler.rs:93-124, 139-152). Device code for gfx950; the sums'
// terms sit in LDS.
#pragma once

#include "cx_internal.h"

namespace {

// tot + x[0] + x[1] + ... + x[n-1] in position order, one dependent add a
// position (n a multiple of 16, at most 16 NB; x 16-byte aligned). Every
// active lane forms the same sum from broadcast LDS reads: batches of 16
// (four ds_read_b128), two batches read ahead of the adds (past the end the
// last batch again), the batches unrolled so that the compiler's waits count
// exactly the reads a batch needs. A dependent f32 add issues every ~4.5
// clocks on gfx950; the sum through DPP from lanes 0-15 this replaces took
// ~10 a position (a DPP read of an add's result stalls it).
template <uint32_t NB>
__device__ __forceinline__ float seq_add16(const float* x, uint32_t n, float tot) {
  static_assert(NB % 3 == 0, "three batches an iteration");
  const float4* x4 = reinterpret_cast<const float4*>(x);
  const uint32_t nb = n / 16;
  if (nb == 0) return tot;
  float4 a[4], b[4], c[4];
  auto ld = [&](float4 (&v)[4], uint32_t k) {
    k = min(k, nb - 1);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = x4[4 * k + i];
  };
  auto add = [&](const float4 (&v)[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      tot += v[i].x;
      tot += v[i].y;
      tot += v[i].z;
      tot += v[i].w;
    }
  };
  ld(a, 0);
  ld(b, 1);
#pragma unroll
  for (uint32_t k = 0; k < NB; k += 3) {
    ld(c, k + 2);
    __builtin_amdgcn_sched_barrier(0);
    add(a);
    if (k + 1 >= nb) break;
    ld(a, k + 3);
    __builtin_amdgcn_sched_barrier(0);
    add(b);
    if (k + 2 >= nb) break;
    ld(b, k + 4);
    __builtin_amdgcn_sched_barrier(0);
    add(c);
    if (k + 3 >= nb) break;
  }
  return tot;
}

// Inclusive prefix sum over the wave's 64 lanes (rows of 16 by shifts of
// 1, 2, 4 and 8, then row 0's and row 2's sums into rows 1 and 3, then
// lanes 0-31's sum into rows 2 and 3). Exact for non-negative integers
// whose total is below 2^24; above, every sum that reaches 2^24 stays at
// or above it (rounding is monotone).
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_shifted(float v) {  // 0 where no source lane
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false));
}
__device__ __forceinline__ float wave_scan_incl(float v) {
  v += dpp_shifted<0x111, 0xF>(v);  // row_shr:1
  v += dpp_shifted<0x112, 0xF>(v);  // row_shr:2
  v += dpp_shifted<0x114, 0xF>(v);  // row_shr:4
  v += dpp_shifted<0x118, 0xF>(v);  // row_shr:8
  v += dpp_shifted<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
  v += dpp_shifted<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
  return v;
}

// The binade of s >= 0: E with s in [2^E, 2^(E+1)), and E = -126 for s
// below 2^-125 (zero, subnormals and the first normal binade share the
// spacing 2^-149).
__device__ __forceinline__ int binade_of(float s) {
  return max((int)((__float_as_uint(s) >> 23) & 0xFF), 1) - 127;
}

__device__ __forceinline__ uint32_t first_lane(uint64_t m) {
  return m ? (uint32_t)__builtin_ctzll(m) : 64u;
}

// What seq_scan returns besides the sum: SCAN_SUM the sum alone;
// SCAN_EXCEED / SCAN_REACH also the first position whose running sum is
// > target / >= target (the sampler's draw and nucleus cut), the sum then
// ending there.
enum { SCAN_SUM, SCAN_EXCEED, SCAN_REACH };
template <int M>
__device__ __forceinline__ bool scan_passes(float a, float target) {
  return M == SCAN_REACH ? a >= target : a > target;
}

constexpr uint32_t SCAN_HEAD = 256;

// tot + x[0] + x[1] + ... + x[n-1], added in position order with IEEE f32
// rounding after every add (the reference's `tot += e` loop), by the whole
// wave and without one dependent add per position. x[j] >= 0 (or NaN).
//
// While the running sum s stays in one binade [2^E, 2^(E+1)), every float
// there is a multiple of u = 2^(E-23), and fl(s + x) is the multiple of u
// nearest s + x: s + u * rne(x / u), since s is a multiple of u. So in
// units of u the adds are integer adds of r = rne(x / u), which a prefix
// scan forms in any order, exactly. Two kinds of position end such a run
// and are added as one f32 add instead (an event): the one whose add
// reaches 2^(E+1) (the unit doubles), and one whose x / u lies exactly
// halfway between integers (the rounding then goes to the even sum, which
// depends on s). A window is 256 positions, four a lane; after an event the
// next window starts at the position after it, in the new binade. A sum
// from 0 changes binade every time it doubles, so with `head` the first
// SCAN_HEAD positions are added one by one (seq_add16). A
// sum that is not finite (a NaN term, or +inf) is continued one by one.
//
// The searches (M = SCAN_EXCEED, SCAN_REACH): every running sum before a
// window's first event is (s / u + the scan's prefix) * u exactly, so the
// first position that passes target is read off the scan; an event's sum
// is checked as it is added. *at = that position and the sum ends there,
// or *at = n and the sum is the whole one (a NaN sum, which passes no
// target, ends the search at once and is returned as it is).
//
// Reads x up to n + 511 (values past n are never used: the LDS there must
// exist) and, for the head, needs +0.0 from n to the next multiple of 16
// (seq_add16 adds them: +0.0 changes no sum of non-negative terms, which is
// never -0.0). The result is valid in every lane.
template <int M>
__device__ __forceinline__ float seq_scan(const float* x, uint32_t n, float tot, bool head,
                                          float target, uint32_t* at_out) {
  constexpr bool FIND = M != SCAN_SUM;
  const uint32_t l = threadIdx.x & 63;
  uint32_t p = 0;
  // one by one from p with the running sum t (not finite, or a head that
  // holds the crossing)
  auto serial = [&](float t) -> float {
    for (; p < n; p++) {
      if constexpr (FIND) {
        if (t != t) break;
      }
      t += x[p];
      if constexpr (FIND) {
        if (scan_passes<M>(t, target)) {
          *at_out = p;
          return t;
        }
      }
    }
    if constexpr (FIND) *at_out = n;
    return t;
  };
  if (head && n) {
    p = min(n, SCAN_HEAD);
    const float t0 = tot;
    tot = seq_add16<(SCAN_HEAD / 16 + 2) / 3 * 3>(x, (p + 15) / 16 * 16, tot);
    if constexpr (FIND) {
      // the running sum never decreases (NaN aside): the head holds the
      // crossing iff its sum passes, or may if that sum is NaN
      if (scan_passes<M>(tot, target) || tot != tot) {
        float t = t0;
        for (uint32_t j = 0; j < p; j++) {
          t += x[j];
          if (scan_passes<M>(t, target)) {
            *at_out = j;
            return t;
          }
        }
        *at_out = n;  // a NaN sum and no crossing before it: none after it
        return t;
      }
    }
  }
  if (p >= n) {
    if constexpr (FIND) *at_out = n;
    return tot;
  }
  if (!(tot < INFINITY)) return serial(tot);
  int E = binade_of(tot);
  float A = ldexpf(tot, 23 - E);  // s / u, an integer below 2^24
  // volatile LDS reads: kept where they are written (the next window's are
  // issued after this window's arithmetic and waited for a window later)
  typedef __attribute__((address_space(3))) volatile float lds_vf;
  lds_vf* xl = (lds_vf*)(x + 4 * l);
  float v0 = xl[p], v1 = xl[p + 1], v2 = xl[p + 2], v3 = xl[p + 3];
  for (;;) {
    const int k = 23 - E;
    float r0, c1, c2, c3, P, H;
    uint64_t t0, t1, t2, t3;
    // the window at p in (a0..a3), lane l's positions p + 4 l .. + 3; the
    // next window's values read into (b0..b3). True: no event (and, for a
    // search, no crossing), p advanced.
    auto step = [&](float& a0, float& a1, float& a2, float& a3, float& b0, float& b1, float& b2,
                    float& b3) -> bool {
      const float q0 = ldexpf(a0, k), q1 = ldexpf(a1, k), q2 = ldexpf(a2, k), q3 = ldexpf(a3, k);
      r0 = rintf(q0);  // x / u is exact (inf past 2^128: an event)
      const float r1 = rintf(q1), r2 = rintf(q2), r3 = rintf(q3);
      t0 = __builtin_amdgcn_ballot_w64(!(fabsf(q0 - r0) < 0.5f));  // a tie, or not finite
      t1 = __builtin_amdgcn_ballot_w64(!(fabsf(q1 - r1) < 0.5f));
      t2 = __builtin_amdgcn_ballot_w64(!(fabsf(q2 - r2) < 0.5f));
      t3 = __builtin_amdgcn_ballot_w64(!(fabsf(q3 - r3) < 0.5f));
      c1 = r0 + r1;
      c2 = c1 + r2;
      c3 = c2 + r3;
      __builtin_amdgcn_sched_barrier(0);
      b0 = xl[p + 256];
      b1 = xl[p + 257];
      b2 = xl[p + 258];
      b3 = xl[p + 259];
      __builtin_amdgcn_sched_barrier(0);
      P = wave_scan_incl(c3);  // the window's sum through this lane's last
      H = 16777216.0f - A;     // the binade's room: 2^24 - s / u
      uint64_t ev = t0 | t1 | t2 | t3 | __builtin_amdgcn_ballot_w64(P >= H);
      if constexpr (FIND)  // the lane's last running sum, exact where no event precedes it
        ev |= __builtin_amdgcn_ballot_w64(scan_passes<M>(ldexpf(A + P, -k), target));
      if (ev || n - p <= 256) return false;
      A += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(P), 63));
      p += 256;
      return true;
    };
    float w0, w1, w2, w3;
    for (;;) {
      if (!step(v0, v1, v2, v3, w0, w1, w2, w3)) break;
      if (!step(w0, w1, w2, w3, v0, v1, v2, v3)) break;
    }
    // the window's first event (positions 4 l + i, from ballots) or its
    // end; X, the sum before the lane, is exact up to the first lane with
    // an event, as every sum before it is below H <= 2^24
    const float X = dpp_shifted<0x138, 0xF>(P);  // wave_shr:1
    const uint64_t e0 = t0 | __builtin_amdgcn_ballot_w64(X + r0 >= H);
    const uint64_t e1 = t1 | __builtin_amdgcn_ballot_w64(X + c1 >= H);
    const uint64_t e2 = t2 | __builtin_amdgcn_ballot_w64(X + c2 >= H);
    const uint64_t e3 = t3 | __builtin_amdgcn_ballot_w64(X + c3 >= H);
    const uint32_t at = min(min(4 * first_lane(e0), 4 * first_lane(e1) + 1),
                            min(4 * first_lane(e2) + 2, 4 * first_lane(e3) + 3));
    const uint32_t room = n - p, stop = min(at, room);
    if constexpr (FIND) {
      // the first position that passes, valid before the first event
      const uint64_t g0 = __builtin_amdgcn_ballot_w64(scan_passes<M>(ldexpf(A + (X + r0), -k), target));
      const uint64_t g1 = __builtin_amdgcn_ballot_w64(scan_passes<M>(ldexpf(A + (X + c1), -k), target));
      const uint64_t g2 = __builtin_amdgcn_ballot_w64(scan_passes<M>(ldexpf(A + (X + c2), -k), target));
      const uint64_t g3 = __builtin_amdgcn_ballot_w64(scan_passes<M>(ldexpf(A + (X + c3), -k), target));
      const uint32_t pa = min(min(4 * first_lane(g0), 4 * first_lane(g1) + 1),
                              min(4 * first_lane(g2) + 2, 4 * first_lane(g3) + 3));
      if (pa < stop) {
        const uint32_t lj = pa / 4, ij = pa % 4;
        const float s = X + (ij == 0 ? r0 : ij == 1 ? c1 : ij == 2 ? c2 : c3);
        *at_out = p + pa;
        return ldexpf(A + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), (int)lj)), -k);
      }
    }
    if (stop) {  // the window's positions before the event (or all it has)
      const uint32_t j = stop - 1, lj = j / 4, ij = j % 4;
      const float s = X + (ij == 0 ? r0 : ij == 1 ? c1 : ij == 2 ? c2 : c3);
      A += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), (int)lj));
    }
    if (at >= room) {
      if constexpr (FIND) *at_out = n;
      return ldexpf(A, E - 23);
    }
    const float s = ldexpf(A, E - 23) + x[p + at];  // the event's add
    if constexpr (FIND) {
      if (scan_passes<M>(s, target)) {
        *at_out = p + at;
        return s;
      }
    }
    p += at + 1;
    if (!(s < INFINITY)) return serial(s);
    if (p >= n) {
      if constexpr (FIND) *at_out = n;
      return s;
    }
    const float su = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(s)));
    E = binade_of(su);
    A = ldexpf(su, 23 - E);
    v0 = xl[p];
    v1 = xl[p + 1];
    v2 = xl[p + 2];
    v3 = xl[p + 3];
  }
}

__device__ __forceinline__ float seq_sum_scan(const float* x, uint32_t n, float tot, bool head) {
  return seq_scan<SCAN_SUM>(x, n, tot, head, 0.0f, nullptr);
}

}  // namespace
