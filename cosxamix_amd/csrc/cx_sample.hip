// cx_sample.hip — sampler::Muestreador::elegir (src/sampler.rs:61-152) on the
// GPU, for gfx950: temperature and top-p sampling with the reference's
// arithmetic, so that the same logits and seed give the same token.
//
//   u      = (azar.siguiente() >> 40) as f32 / 2^24      (one draw per call)
//   z_i    = logit_i * (1 / temperature)
//   p      = softmax(z) (src/ops.rs:1206-1230): max; non-finite max gives
//            the uniform 1/n; e_i = exp(z_i - max); S = sum e_i sequential
//            from 0; p_i = e_i * (1/S)
//   top_p >= 1: the first i (index order) whose running sum of p exceeds u
//   else:  the tokens by descending p; the nucleus is the shortest prefix
//          whose running sum reaches top_p (the token that crosses enters);
//          total = its sum; the first token of the nucleus whose running
//          sum exceeds u * total (the last one if none does)
//
// The reference takes the 1024 most probable tokens first (the candidates)
// and sorts every token only when their mass falls short of top_p. Both are
// prefixes of one descending order, which is built here for every token by
// a stable device-wide radix sort; the nucleus is then its first 1024 tokens
// or all of them, by the reference's test on the candidates' mass.
// Ties: the reference sorts with an unstable sort, which leaves the order of
// equal probabilities unspecified; here they go by ascending token index.
//
// Kernels of one call, each a fixed launch (no host decision between them,
// so the sequence can sit in a captured graph):
//   k_samp_z     z_i and per-block maxima                      (grid)
//   k_samp_e     e_i = exp(z_i - max), or the uniform 1/n       (grid)
//   k_samp_sum   S sequentially, 1/S, and the draw of u         (1 workgroup)
//   k_samp_p     p_i = e_i * (1/S)                              (grid)
//   k_rs_count, k_rs_scan, k_rs_scatter, four times: the descending order
//                of p (8-bit digits, least significant first); they return
//                at once when top_p >= 1 (no order needed)
//   k_samp_pick  the token                                      (1 workgroup)
// The sequential sums (S, the running sums) are ordered f32 sums that one
// wave forms by binade scans (cx_scan.h), fed from LDS stages that the other
// waves fill with direct-to-LDS loads.
#include "cx_ops.h"
#include "cx_act.h"
#include "cx_scan.h"

namespace {

constexpr uint32_t ZB = 256;         // threads of the grid kernels
constexpr uint32_t ZV = 8;           // values per thread of the grid kernels
constexpr uint32_t CW = 1024;        // threads of the single-workgroup kernels
constexpr uint32_t SEG = 8192;       // floats per chain stage (32 KiB: four KiB per loader wave)
constexpr uint32_t NST = 4;          // chain stages in the LDS ring
constexpr uint32_t CAND = 1024;      // CANDIDATOS (src/sampler.rs): the first nucleus
constexpr uint32_t RS_T = 256;       // threads of a radix-sort workgroup
constexpr uint32_t RS_R = 8;         // rounds of RS_T elements a tile
constexpr uint32_t RS_TILE = RS_T * RS_R;

// the chains' ring, and the 511 floats past its last stage that a scan reads
constexpr size_t RING_LDS = (NST * SEG + 512) * sizeof(float);

// total-order key of a probability (f32::total_cmp): larger key, larger value
__device__ inline uint32_t pkey(float p) {
  const uint32_t b = __float_as_uint(p);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// ---------------------------------------------------------------- grid kernels
__global__ __launch_bounds__(ZB) void k_samp_z(const float* logits, uint32_t n,
                                               const cx_samp_state* sd, float* pb, float* part) {
  __shared__ float red[ZB / 64];
  const float inv = sd->inv;
  const uint32_t i0 = (blockIdx.x * ZB + threadIdx.x) * ZV;
  float m = -INFINITY;
  for (uint32_t j = 0; j < ZV; j++) {
    const uint32_t i = i0 + j;
    if (i < n) {
      const float z = logits[i] * inv;
      pb[i] = z;
      m = fmaxf(m, z);
    }
  }
  m = cx_wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = red[0];
    for (uint32_t w = 1; w < ZB / 64; w++) b = fmaxf(b, red[w]);
    part[blockIdx.x] = b;
  }
}

__global__ __launch_bounds__(ZB) void k_samp_e(float* pb, uint32_t n, const float* part,
                                               uint32_t nparts, cx_samp_state* sd) {
  __shared__ float mx;
  if (threadIdx.x == 0) {  // max over every z, NaN ignored (f32::max), from -inf
    float m = -INFINITY;
    for (uint32_t b = 0; b < nparts; b++) m = fmaxf(m, part[b]);
    mx = m;
    if (blockIdx.x == 0) sd->uniform = isfinite(m) ? 0u : 1u;
  }
  __syncthreads();
  const float m = mx;
  const bool uni = !isfinite(m);
  const float u = 1.0f / (float)n;
  const uint32_t i0 = (blockIdx.x * ZB + threadIdx.x) * ZV;
  for (uint32_t j = 0; j < ZV; j++) {
    const uint32_t i = i0 + j;
    if (i < n) pb[i] = uni ? u : cx_expf(pb[i] - m);
  }
}

__global__ __launch_bounds__(ZB) void k_samp_p(float* pb, uint32_t n, const cx_samp_state* sd) {
  if (sd->uniform) return;  // the uniform probabilities are already in place
  const float inv = sd->inv_s;
  const uint32_t i0 = (blockIdx.x * ZB + threadIdx.x) * ZV;
  for (uint32_t j = 0; j < ZV; j++) {
    const uint32_t i = i0 + j;
    if (i < n) pb[i] = pb[i] * inv;
  }
}

// ---------------------------------------------------------- ordered sums
// A ring of NST stages of SEG floats: loader waves 1..8 each load SEG / 8
// floats of every stage (1 KiB DMA loads); stage s sits in slot s % NST. Wave 0 walks the stages in
// order; after each stage every wave learns whether it stopped.
static_assert(SEG % 2048 == 0, "whole 1 KiB loads for each of the 8 loader waves");
struct Ring {
  float* lds;
  const float* src;
  uint32_t n, nstage, issued;
  uint32_t wave, lane;
  __device__ void issue(uint32_t s) {
    if (wave < 1 || wave > 8) return;
#pragma unroll
    for (uint32_t h = 0; h < SEG / 2048; h++) {
      const uint32_t o = (wave - 1) * (SEG / 8) + 256 * h, i = s * SEG + o + 4 * lane;
      cx_dma16_async(src + (i < n ? i : 0), lds + (s % NST) * SEG + o);
    }
    issued++;
  }
  // loader waves: this wave's loads up to stage s have landed (SEG / 2048 a
  // stage, NST - 1 stages at most after it)
  __device__ void wait(uint32_t s) {
    if (wave < 1 || wave > 8) return;
    constexpr uint32_t L = SEG / 2048;
    const uint32_t after = issued - (s + 1);
    switch (after) {
      case 0: cx_wait_vm<0>(); break;
      case 1: cx_wait_vm<L>(); break;
      case 2: cx_wait_vm<2 * L>(); break;
      case 3: cx_wait_vm<3 * L>(); break;
      default: cx_wait_vm<3 * L>(); break;
    }
  }
};

// Walks x[0..n) in order through the ring: `stage(v, m, base)` runs on wave
// 0 for each stage (with ALL, on every wave) (m values at LDS v, indices
// base..; +0.0 from m to the next multiple of 16) and returns true, the same
// in every lane (with ALL, in every thread), to stop. Every wave leaves with
// every load landed.
template <bool ALL = false, class F>
__device__ inline void chain_walk(const float* x, uint32_t n, float* lds, F stage) {
  __shared__ uint32_t stop;
  const uint32_t tid = threadIdx.x;
  Ring R{lds, x, n, (n + SEG - 1) / SEG, 0,
         (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6)), tid & 63};
  if (tid == 0) stop = 0;
  for (uint32_t s = 0; s < NST && s < R.nstage; s++) R.issue(s);
  for (uint32_t s = 0; s < R.nstage; s++) {
    R.wait(s);
    cx_wait_lds();
    cx_barrier();  // stage s landed; `stop` from the last stage is visible
    if (stop) break;
    if (ALL) {
      float* v = lds + (s % NST) * SEG;
      const uint32_t m = min(SEG, n - s * SEG);
      // (wave 0 pads what only wave 0 reads: the other waves read below m)
      if (R.wave == 0 && R.lane < (16 - m % 16) % 16) v[m + R.lane] = 0.0f;
      if (stage(v, m, s * SEG) && tid == 0) stop = 1;
    } else if (R.wave == 0) {
      float* v = lds + (s % NST) * SEG;
      const uint32_t m = min(SEG, n - s * SEG);
      if (R.lane < (16 - m % 16) % 16) v[m + R.lane] = 0.0f;  // the loads past n hold x[0..]
      if (stage(v, m, s * SEG) && R.lane == 0) stop = 1;
    }
    cx_wait_lds();
    cx_barrier();  // slot s read
    if (s + NST < R.nstage) R.issue(s + NST);
  }
  cx_wait_vm<0>();
  cx_wait_lds();
  __syncthreads();
}

// One chain stage of a running sum (seq_scan's sum or search) by the whole
// workgroup. The waves take the MW_WIN 256-position windows in parallel (two
// a wave: a stage of twice the positions halves the barriers a position), all in
// the binade E of the running sum s where they start (unit u = 2^(E-23)): a
// window's total N_w of rne(x/u), and whether it holds a tie or a term that
// is not finite. While no window has such an event, the running sum reaches
// no 2^(E+1) and, for a search, no window's last running sum passes the
// target, every add of those windows is an exact integer add in units of u
// (seq_scan's argument), so their sums are exactly s + u·(N_0 + N_1 + ...).
// Wave 0 finds the first window where that fails and runs seq_scan over
// that window alone (the event added as one f32 add, the crossing found
// there); the windows after it start again in the new binade. The stage at
// base 0 (the head's one-by-one adds) and a sum that is not finite go to
// seq_scan whole. Every thread returns the sum, and *at = the crossing's
// index in the stage or m.
constexpr uint32_t MW_WIN = SEG / 256;
static_assert(MW_WIN % (CW / 64) == 0 && MW_WIN <= 64, "whole windows a wave, a lane a window's total");
template <int M>
__device__ inline float stage_scan_mw(const float* v, uint32_t m, float tot, bool head,
                                      float target, uint32_t* at) {
  constexpr bool FIND = M != SCAN_SUM;
  __shared__ float sN[MW_WIN];
  __shared__ uint32_t sbad[MW_WIN];
  __shared__ float s_tot;
  __shared__ uint32_t s_at, s_w0;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t nw = (m + 255) / 256;
  float s = tot;
  uint32_t w0 = 0, where = m;
  for (;;) {
    const bool whole = (head && w0 == 0) || !(s < INFINITY);
    const int E = binade_of(s), k = 23 - E;
    if (!whole) {
#pragma unroll
      for (uint32_t wi = wave; wi < MW_WIN; wi += CW / 64) {
        const uint32_t p = 256 * (w0 + wi) + 4 * lane;
        float c = 0.0f;
        bool bad = false;
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
          const float x = p + i < m ? v[p + i] : 0.0f;
          const float q = ldexpf(x, k), r = rintf(q);  // x / u is exact (inf past 2^128)
          bad |= !(fabsf(q - r) < 0.5f);               // a tie, or not finite
          c += r;
        }
        // the window's total: exact below 2^24, and at or above it otherwise
        const float P = wave_scan_incl(c);
        const uint64_t b = __builtin_amdgcn_ballot_w64(bad);
        if (lane == 63) {
          sN[wi] = P;
          sbad[wi] = b != 0;
        }
      }
      cx_wait_lds();
      __syncthreads();
    }
    if (wave == 0) {
      uint32_t from = 256 * w0, to = m, next = nw;
      if (!whole) {
        const float A0 = ldexpf(s, k);  // s / u, an integer below 2^24
        const uint32_t cnt = min(nw - w0, MW_WIN);
        const float N = lane < cnt ? sN[lane] : 0.0f;
        const float P = wave_scan_incl(N);  // the sums through each window
        const bool ev = lane < cnt && (sbad[lane] || A0 + P >= 16777216.0f ||
                                       (FIND && scan_passes<M>(ldexpf(A0 + P, -k), target)));
        const uint32_t j = min(first_lane(__builtin_amdgcn_ballot_w64(ev)), cnt);
        const float before =
            j ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(P), (int)(j - 1))) : 0.0f;
        s = ldexpf(A0 + before, -k);  // exact: every window before j is event-free
        if (j < cnt) {  // window w0 + j by seq_scan, the next round after it
          from = 256 * (w0 + j);
          to = min(m, from + 256);
          next = w0 + j + 1;
        } else {
          from = to = 0;
          next = w0 + cnt;
        }
      }
      if (from < to) {
        uint32_t kr = to - from;
        s = seq_scan<M>(v + from, to - from, s, head && from == 0, target, FIND ? &kr : nullptr);
        if (FIND && kr < to - from) {
          where = from + kr;
          next = nw;
        }
      }
      if (lane == 0) {
        s_tot = s;
        s_at = where;
        s_w0 = next;
      }
    }
    cx_wait_lds();
    __syncthreads();
    s = s_tot;
    where = s_at;
    w0 = s_w0;
    __syncthreads();  // every thread has read them before they are written again
    if (w0 >= nw) break;
  }
  *at = where;
  return s;
}

// The running sum of x[0..n) continued from *acc: the first index where it
// exceeds target (M = SCAN_EXCEED) or reaches it (SCAN_REACH), or n; *acc
// ends as the sum through that index, or through x[n - 1]. x >= 0 (or NaN).
// (*acc in shared memory; every thread sees the result and *acc on return)
template <int M>
__device__ inline uint32_t chain_find(const float* x, uint32_t n, float* lds, float target,
                                      float* acc) {
  __shared__ uint32_t s_at;
  __syncthreads();  // every read of the last call's s_at and *acc is done
  float a = *acc;
  if (threadIdx.x == 0) s_at = n;
  chain_walk<true>(x, n, lds, [&](const float* v, uint32_t m, uint32_t base) {
    uint32_t k;
    a = stage_scan_mw<M>(v, m, a, base == 0, target, &k);
    if (k < m) {
      if (threadIdx.x == 0) s_at = base + k;
      return true;
    }
    return false;
  });
  if (threadIdx.x == 0) *acc = a;
  __syncthreads();
  return s_at;
}

// the first index of x[0..n) whose running sum exceeds target, or n
__device__ inline uint32_t chain_cross(const float* x, uint32_t n, float* lds, float target) {
  __shared__ float acc;
  __syncthreads();  // no thread still reads the last call's acc
  if (threadIdx.x == 0) acc = 0.0f;
  return chain_find<SCAN_EXCEED>(x, n, lds, target, &acc);
}

// S = e_0 + e_1 + ... sequentially from 0, then 1/S; and the draw of u
__global__ __launch_bounds__(CW) void k_samp_sum(const float* pb, uint32_t n, cx_samp_state* sd) {
  extern __shared__ __align__(16) float ring[];
  if (threadIdx.x == 0) {  // Azar::siguiente (src/daiss.rs:330-337), then uniforme (src/sampler.rs:55-58)
    uint64_t x = sd->azar;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    sd->azar = x;
    sd->u = (float)((x * 0x2545F4914F6CDD1Dull) >> 40) / 16777216.0f;
  }
  if (sd->uniform) return;
  float tot = 0.0f;
  chain_walk<true>(pb, n, ring, [&](const float* v, uint32_t m, uint32_t base) {
    uint32_t k;
    tot = stage_scan_mw<SCAN_SUM>(v, m, tot, base == 0, 0.0f, &k);
    return false;
  });
  if (threadIdx.x == 0) sd->inv_s = 1.0f / tot;
}

// ------------------------------------------------- the descending order
// A stable LSD radix sort of (key, index) with key = ~total-order key of p:
// ascending keys are descending probabilities (f32::total_cmp), and equal
// ones keep ascending index. Four passes of 8-bit digits; a pass counts the
// digits of each tile of RS_TILE elements, scans the counts (digit-major,
// then tile), and scatters each tile in index order. Pass 0 reads p itself;
// the last pass writes the order (ord) and the sorted probabilities (ordp).
__device__ inline uint32_t rs_key(float p) { return ~pkey(p); }
__device__ inline float rs_p(uint32_t key) {  // the probability back from its key
  const uint32_t k = ~key;
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

template <int D>
__global__ __launch_bounds__(RS_T) void k_rs_count(const float* pb, const uint32_t* kin, uint32_t n,
                                                   const cx_samp_state* sd, uint32_t* cnt,
                                                   uint32_t G) {
  if (sd->top_p >= 1.0f) return;
  __shared__ uint32_t h[256];
  const uint32_t tid = threadIdx.x, base = blockIdx.x * RS_TILE;
  h[tid] = 0;
  // every round's key loaded before the first is counted (an index past n
  // reads element n - 1 and is not counted); a load a round waited for
  // each in turn
  uint32_t key[RS_R];
#pragma unroll
  for (uint32_t r = 0; r < RS_R; r++) {
    const uint32_t i = min(base + r * RS_T + tid, n - 1);
    key[r] = D == 0 ? rs_key(pb[i]) : kin[i];
  }
  __syncthreads();
#pragma unroll
  for (uint32_t r = 0; r < RS_R; r++)
    if (base + r * RS_T + tid < n) atomicAdd(&h[(key[r] >> (8 * D)) & 255u], 1u);
  __syncthreads();
  cnt[tid * G + blockIdx.x] = h[tid];
}

// exclusive prefix sum of cnt[0..e) in place, one workgroup of CW threads.
// With LDS (e <= RS_SCAN_LDS words) the counts are staged there by coalesced
// loads, each thread scans a contiguous chunk, and the result goes back
// coalesced; otherwise the chunks are read from global memory.
constexpr uint32_t RS_SCAN_LDS = 32768;
template <bool LDS>
__global__ __launch_bounds__(CW) void k_rs_scan(uint32_t* cnt, uint32_t e, const cx_samp_state* sd) {
  if (sd->top_p >= 1.0f) return;
  extern __shared__ uint32_t stage[];
  __shared__ uint32_t part[CW];
  const uint32_t tid = threadIdx.x, per = (e + CW - 1) / CW;
  const uint32_t lo = min(e, tid * per), hi = min(e, lo + per);
  uint32_t* c = LDS ? stage : cnt;
  if (LDS) {  // eight loads in flight a thread (a loop of one waited for each)
    for (uint32_t i0 = tid; i0 < e; i0 += 8 * CW) {
      uint32_t v[8];
#pragma unroll
      for (uint32_t u = 0; u < 8; u++) v[u] = cnt[min(i0 + u * CW, e - 1)];
#pragma unroll
      for (uint32_t u = 0; u < 8; u++)
        if (i0 + u * CW < e) stage[i0 + u * CW] = v[u];
    }
    __syncthreads();
  }
  uint32_t sum = 0;
  for (uint32_t i = lo; i < hi; i++) sum += c[i];
  part[tid] = sum;
  __syncthreads();
  for (uint32_t off = 1; off < CW; off <<= 1) {  // inclusive scan of the parts
    const uint32_t v = tid >= off ? part[tid - off] : 0u;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  uint32_t run = part[tid] - sum;
  for (uint32_t i = lo; i < hi; i++) {
    const uint32_t x = c[i];
    c[i] = run;
    run += x;
  }
  if (LDS) {
    __syncthreads();
    for (uint32_t i = tid; i < e; i += CW) cnt[i] = stage[i];
  }
}

template <int D>
__global__ __launch_bounds__(RS_T) void k_rs_scatter(const float* pb, const uint32_t* kin,
                                                     const uint32_t* iin, uint32_t n,
                                                     const cx_samp_state* sd, const uint32_t* off,
                                                     uint32_t G, uint32_t* kout, uint32_t* iout,
                                                     float* pout) {
  if (sd->top_p >= 1.0f) return;
  __shared__ uint32_t run[256];     // next position of each digit in this tile
  __shared__ uint32_t wc[4][256];   // digit counts of each wave in this round
  const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, base = blockIdx.x * RS_TILE;
  const uint64_t below = (1ull << lane) - 1;
  run[tid] = off[tid * G + blockIdx.x];
  // every round's key and index loaded before the first round (an index
  // past n reads element n - 1, never used)
  uint32_t keys[RS_R], idxs[RS_R];
#pragma unroll
  for (uint32_t r = 0; r < RS_R; r++) {
    const uint32_t i = min(base + r * RS_T + tid, n - 1);
    keys[r] = D == 0 ? rs_key(pb[i]) : kin[i];
    idxs[r] = D == 0 ? i : iin[i];
  }
#pragma unroll
  for (uint32_t r = 0; r < RS_R; r++) {
    const uint32_t i = base + r * RS_T + tid;
    const bool valid = i < n;
    const uint32_t key = valid ? keys[r] : 0u;
    const uint32_t idx = valid ? idxs[r] : 0u;
    const uint32_t dig = (key >> (8 * D)) & 255u;
    // the lanes of this wave with the same digit
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int bt = 0; bt < 8; bt++) {
      const uint64_t bb = __ballot((dig >> bt) & 1u);
      m &= ((dig >> bt) & 1u) ? bb : ~bb;
    }
    __syncthreads();  // the last round's reads of wc[] and updates of run[] are done
    for (uint32_t d = lane; d < 256; d += 64) wc[w][d] = 0;
    __syncthreads();
    if (valid && (m & below) == 0) wc[w][dig] = (uint32_t)__popcll(m);
    __syncthreads();
    if (valid) {
      uint32_t pos = run[dig] + (uint32_t)__popcll(m & below);
      for (uint32_t v = 0; v < w; v++) pos += wc[v][dig];
      if (kout) kout[pos] = key;
      iout[pos] = idx;
      if (pout) pout[pos] = rs_p(key);
    }
    __syncthreads();  // every read of run[] is done
    run[tid] += wc[0][tid] + wc[1][tid] + wc[2][tid] + wc[3][tid];
  }
}

// --------------------------------------------------------------------- pick
// The token (src/sampler.rs:83-125, 139-152), written to *out and, in the
// token loop, to hist[pos + 1] with the position advanced as the greedy
// argmax does.
__global__ __launch_bounds__(CW) void k_samp_pick(const float* pb, uint32_t n, cx_samp_state* sd,
                                                  const uint32_t* ord, const float* ordp,
                                                  uint32_t* out, cx_dstate* st, uint32_t* hist,
                                                  uint32_t* hist_host) {
  extern __shared__ __align__(16) float ring[];
  __shared__ float s_acc;
  const uint32_t tid = threadIdx.x;
  const float u = sd->u, top_p = sd->top_p;
  uint32_t tok = 0;
  if (top_p >= 1.0f) {  // muestrear_acumulando over 0..n with u
    const uint32_t at = chain_cross(pb, n, ring, u);
    tok = at < n ? at : n - 1;
  } else {
    // the candidates' running sum to top_p (the crossing token enters)
    const uint32_t k = min(CAND, n);
    if (tid == 0) s_acc = 0.0f;
    __syncthreads();
    uint32_t at = chain_find<SCAN_REACH>(ordp, k, ring, top_p, &s_acc);
    uint32_t cut;
    if (at < k) {
      cut = at + 1;
    } else if (s_acc < top_p && k < n) {
      // their mass falls short: the nucleus comes from every token's order
      at = chain_find<SCAN_REACH>(ordp + k, n - k, ring, top_p, &s_acc);
      cut = at < n - k ? k + at + 1 : n;
    } else {
      cut = k;  // a NaN top_p: the candidates, whole
    }
    __syncthreads();
    // total = the nucleus's sum (the running sum where it stopped); then the
    // first token of the nucleus whose running sum exceeds u * total (the
    // last one of the nucleus if none does)
    const float total = s_acc;
    at = chain_cross(ordp, cut, ring, u * total);
    tok = ord[at < cut ? at : cut - 1];
  }
  if (tid == 0) {
    if (out) *out = tok;
    sd->token = tok;
    if (st) {
      const uint32_t nxt = st->pos + 1;
      if (nxt >= st->prompt_end && nxt <= st->cap) {  // hist has cap+1 slots
        hist[nxt] = tok;
        if (hist_host) hist_host[nxt] = tok;
      }
      st->pos = nxt;
    }
  }
}

// the layout of `part`: the per-block maxima, then the sort's keys and
// indices (two buffers of each but the final indices, which are ord) and the
// digit counts
struct SortScratch {
  uint32_t nparts, n4, tiles;
  size_t words() const { return (size_t)(nparts + 63) / 64 * 64 + 3 * (size_t)n4 + 256 * (size_t)tiles; }
};
inline SortScratch sort_scratch(size_t n) {
  SortScratch S;
  S.nparts = (uint32_t)((n + ZB * ZV - 1) / (ZB * ZV));
  S.n4 = (uint32_t)((n + 63) / 64 * 64);
  S.tiles = (uint32_t)((n + RS_TILE - 1) / RS_TILE);
  return S;
}

}  // namespace

size_t cx_sample_parts(size_t n) { return sort_scratch(n).words(); }

int cx_launch_sample(const float* logits, size_t n, cx_samp_state* sd, float* pb, float* part,
                     uint32_t* ord, float* ordp, uint32_t* out, cx_dstate* st, uint32_t* hist,
                     uint32_t* hist_host, hipStream_t s) {
  CX_REQUIRE(logits && sd && pb && part && ord && ordp && n > 0 && n < (1u << 31),
             "sample: bad arguments (n=%zu)", n);
  CX_REQUIRE(((uintptr_t)pb & 15) == 0 && ((uintptr_t)ordp & 15) == 0,
             "sample: the probability buffers must be 16-byte aligned");
  const SortScratch S = sort_scratch(n);
  const unsigned g = S.nparts, G = S.tiles;
  const uint32_t N = (uint32_t)n;
  uint32_t* kA = reinterpret_cast<uint32_t*>(part) + (S.nparts + 63) / 64 * 64;
  uint32_t* iA = kA + S.n4;
  uint32_t* kB = iA + S.n4;
  uint32_t* cnt = kB + S.n4;
  hipLaunchKernelGGL(k_samp_z, dim3(g), dim3(ZB), 0, s, logits, N, sd, pb, part);
  CX_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_samp_e, dim3(g), dim3(ZB), 0, s, pb, N, part, g, sd);
  CX_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_samp_sum, dim3(1), dim3(CW), RING_LDS, s, pb, N, sd);
  CX_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_samp_p, dim3(g), dim3(ZB), 0, s, pb, N, sd);
  CX_HIP(hipGetLastError());
  // the descending order: pb -> (kA, iA) -> (kB, ord) -> (kA, iA) -> ord, ordp
  const uint32_t E = 256 * G;
  auto pass = [&](auto count, auto scatter, const uint32_t* ki, const uint32_t* ii, uint32_t* ko,
                  uint32_t* io, float* po) -> int {
    hipLaunchKernelGGL(count, dim3(G), dim3(RS_T), 0, s, pb, ki, N, sd, cnt, G);
    CX_HIP(hipGetLastError());
    if (E <= RS_SCAN_LDS)
      hipLaunchKernelGGL(k_rs_scan<true>, dim3(1), dim3(CW), E * 4, s, cnt, E, sd);
    else
      hipLaunchKernelGGL(k_rs_scan<false>, dim3(1), dim3(CW), 0, s, cnt, E, sd);
    CX_HIP(hipGetLastError());
    hipLaunchKernelGGL(scatter, dim3(G), dim3(RS_T), 0, s, pb, ki, ii, N, sd, cnt, G, ko, io, po);
    CX_HIP(hipGetLastError());
    return CX_OK;
  };
  int rc;
  if ((rc = pass(k_rs_count<0>, k_rs_scatter<0>, nullptr, nullptr, kA, iA, nullptr)) ||
      (rc = pass(k_rs_count<1>, k_rs_scatter<1>, kA, iA, kB, ord, nullptr)) ||
      (rc = pass(k_rs_count<2>, k_rs_scatter<2>, kB, ord, kA, iA, nullptr)) ||
      (rc = pass(k_rs_count<3>, k_rs_scatter<3>, kA, iA, nullptr, ord, ordp)))
    return rc;
  hipLaunchKernelGGL(k_samp_pick, dim3(1), dim3(CW), RING_LDS, s, pb, N, sd, ord, ordp, out, st,
                     hist, hist_host);
  CX_HIP(hipGetLastError());
  return CX_OK;
}
