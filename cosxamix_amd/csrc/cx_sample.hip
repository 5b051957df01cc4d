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
// The reference takes the 1024 most probable tokens first and sorts all of
// them only when those fall short of top_p; both give the prefix of the
// descending order, which is what is built here: 1024 tokens, then blocks of
// 16384 for the flat distributions that need more.
// Ties: the reference sorts with an unstable sort, which leaves the order of
// equal probabilities unspecified; here they go by ascending token index.
//
// Kernels of one call, each a fixed launch (no host decision between them,
// so the sequence can sit in a captured graph):
//   k_samp_z    z_i and per-block maxima                      (grid)
//   k_samp_e    e_i = exp(z_i - max), or the uniform 1/n       (grid)
//   k_samp_sum  S sequentially, 1/S, and the draw of u         (1 workgroup)
//   k_samp_p    p_i = e_i * (1/S)                              (grid)
//   k_samp_pick the token                                      (1 workgroup)
// The sequential sums (S, the running sums) are single-lane chains fed from
// LDS stages that the other waves fill with direct-to-LDS loads.
#include "cx_ops.h"
#include "cx_act.h"

namespace {

constexpr uint32_t ZB = 256;         // threads of the grid kernels
constexpr uint32_t ZV = 8;           // values per thread of the grid kernels
constexpr uint32_t CW = 1024;        // threads of the single-workgroup kernels
constexpr uint32_t SEG = 2048;       // floats per chain stage (8 KiB: one KiB per loader wave)
constexpr uint32_t NST = 8;          // chain stages in the LDS ring
constexpr uint32_t TOPK0 = 1024;     // tokens of the first block of the descending order
constexpr uint32_t TOPK = 16384;     // tokens of a later block (128 KiB of keys)

constexpr size_t PICK_LDS = TOPK * sizeof(uint64_t);  // the keys, or the chains' ring
static_assert(PICK_LDS >= NST * SEG * sizeof(float), "the ring fits in the keys' LDS");

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

// ------------------------------------------------------ single-lane chains
// A ring of NST stages of SEG floats: loader waves 1..8 each load one KiB of
// every stage; stage s sits in slot s % NST. The chain (thread 0) walks the
// stages in order; after each stage every wave learns whether it stopped.
struct Ring {
  float* lds;
  const float* src;
  uint32_t n, nstage, issued;
  uint32_t wave, lane;
  __device__ void issue(uint32_t s) {
    if (wave < 1 || wave > 8) return;
    const uint32_t i = s * SEG + (wave - 1) * 256 + 4 * lane;
    cx_dma16_async(src + (i < n ? i : 0), lds + (s % NST) * SEG + (wave - 1) * 256);
    issued++;
  }
  // loader waves: this wave's loads up to stage s have landed (one a stage)
  __device__ void wait(uint32_t s) {
    if (wave < 1 || wave > 8) return;
    const uint32_t after = issued - (s + 1);
    switch (after) {
      case 0: cx_wait_vm<0>(); break;
      case 1: cx_wait_vm<1>(); break;
      case 2: cx_wait_vm<2>(); break;
      case 3: cx_wait_vm<3>(); break;
      case 4: cx_wait_vm<4>(); break;
      case 5: cx_wait_vm<5>(); break;
      case 6: cx_wait_vm<6>(); break;
      default: cx_wait_vm<7>(); break;
    }
  }
};

// Walks x[0..n) in order through the ring: `stage(v, m, base)` runs on
// thread 0 for each stage (m values at LDS v, indices base..) and returns
// true to stop. Every wave leaves with every load landed.
template <class F>
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
    if (tid == 0 && stage(lds + (s % NST) * SEG, min(SEG, n - s * SEG), s * SEG)) stop = 1;
    cx_wait_lds();
    cx_barrier();  // slot s read
    if (s + NST < R.nstage) R.issue(s + NST);
  }
  cx_wait_vm<0>();
  cx_wait_lds();
  __syncthreads();
}

// tot += v[0] + ... + v[m) in order; 32 values a batch, the next batch read
// before the current is added (v holds whole batches: reads past m stay in
// the stage)
__device__ inline void stage_sum(float& tot, const float* v, uint32_t m) {
  const float4* v4 = reinterpret_cast<const float4*>(v);
  float4 A[8], B[8];
#pragma unroll
  for (int i = 0; i < 8; i++) A[i] = v4[i];
  uint32_t j = 0;
  for (; j + 32 <= m; j += 32) {
    if (j + 32 < SEG) {
#pragma unroll
      for (int i = 0; i < 8; i++) B[i] = v4[j / 4 + 8 + i];
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      tot += A[i].x;
      tot += A[i].y;
      tot += A[i].z;
      tot += A[i].w;
    }
#pragma unroll
    for (int i = 0; i < 8; i++) A[i] = B[i];
  }
  for (; j < m; j++) tot += v[j];
}

// The running sum acc += v[j] in order, stopping at the first j with
// acc > target (returns j, or m). The sums of a batch of 32 are formed first
// and checked once: acc never decreases (v >= 0), so the batch crosses iff
// its last sum does; a NaN sum takes the one-by-one check.
__device__ inline uint32_t stage_cross(float& acc, const float* v, uint32_t m, float target) {
  const float4* v4 = reinterpret_cast<const float4*>(v);
  float4 A[8], B[8];
#pragma unroll
  for (int i = 0; i < 8; i++) A[i] = v4[i];
  uint32_t j = 0;
  for (; j + 32 <= m; j += 32) {
    if (j + 32 < SEG) {
#pragma unroll
      for (int i = 0; i < 8; i++) B[i] = v4[j / 4 + 8 + i];
    }
    float r[32];
    float a = acc;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      a += A[i].x;
      r[4 * i] = a;
      a += A[i].y;
      r[4 * i + 1] = a;
      a += A[i].z;
      r[4 * i + 2] = a;
      a += A[i].w;
      r[4 * i + 3] = a;
    }
    if (a > target || a != a) {
#pragma unroll
      for (int k = 0; k < 32; k++)
        if (r[k] > target) {
          acc = r[k];
          return j + k;
        }
    }
    acc = a;
#pragma unroll
    for (int i = 0; i < 8; i++) A[i] = B[i];
  }
  for (; j < m; j++) {
    acc += v[j];
    if (acc > target) return j;
  }
  return m;
}

// the first index of x[0..n) whose running sum exceeds target, or n
__device__ inline uint32_t chain_cross(const float* x, uint32_t n, float* lds, float target) {
  __shared__ uint32_t s_at;
  float acc = 0.0f;
  if (threadIdx.x == 0) s_at = n;
  chain_walk(x, n, lds, [&](const float* v, uint32_t m, uint32_t base) {
    const uint32_t k = stage_cross(acc, v, m, target);
    if (k < m) {
      s_at = base + k;
      return true;
    }
    return false;
  });
  return s_at;
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
  chain_walk(pb, n, ring, [&](const float* v, uint32_t m, uint32_t) {
    stage_sum(tot, v, m);
    return false;
  });
  if (threadIdx.x == 0) sd->inv_s = 1.0f / tot;
}

// ------------------------------------------------------------------- pick
// The token (src/sampler.rs:83-125, 139-152), written to *out and, in the
// token loop, to hist[pos + 1] with the position advanced as the greedy
// argmax does.
__device__ inline uint64_t ckey(uint32_t key, uint32_t idx) {  // descending p, then ascending index
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

__device__ inline float key_p(uint64_t c) {  // the probability back from a composite key
  const uint32_t k = (uint32_t)(c >> 32);
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__global__ __launch_bounds__(CW) void k_samp_pick(const float* pb, uint32_t n, cx_samp_state* sd,
                                                  uint32_t* ord, float* ordp, uint32_t* out,
                                                  cx_dstate* st, uint32_t* hist) {
  extern __shared__ __align__(16) float ring[];
  // a block's keys share the LDS of the chains' ring, used after the blocks
  uint64_t* keys = reinterpret_cast<uint64_t*>(ring);
  __shared__ uint32_t hw[CW / 64][256];  // per-wave digit histograms
  __shared__ uint32_t hist8[256];
  __shared__ uint32_t wsum[CW / 64];
  __shared__ uint32_t s_prefix, s_need, s_ngt, s_cut, s_done;
  __shared__ float s_acc;
  const uint32_t tid = threadIdx.x;
  const float u = sd->u, top_p = sd->top_p;
  uint32_t tok = 0;
  if (top_p >= 1.0f) {  // muestrear_acumulando over 0..n with u
    const uint32_t at = chain_cross(pb, n, ring, u);
    tok = at < n ? at : n - 1;
  } else {
    // the descending order, TOPK tokens at a time, until the running sum of
    // p reaches top_p; ord[] receives the order
    if (tid == 0) {
      s_acc = 0.0f;
      s_done = 0;
      s_cut = n;
    }
    uint64_t bound = ~0ull;  // strictly below this composite key
    uint32_t m = 0;
    __syncthreads();
    while (!s_done) {
      const uint32_t kk = min(m == 0 ? TOPK0 : TOPK, n - m);
      const uint32_t sortn = kk <= TOPK0 ? TOPK0 : TOPK;  // a power of two
      // radix select of the kk-th largest 32-bit key among the eligible,
      // most significant byte first
      if (tid == 0) {
        s_prefix = 0;
        s_need = kk;
      }
      __syncthreads();
      uint32_t mask = 0;
      const uint32_t wv = tid >> 6;
      for (int d = 3; d >= 0; d--) {
        for (uint32_t b = tid; b < (CW / 64) * 256; b += CW) (&hw[0][0])[b] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix;
        for (uint32_t i = tid; i < n; i += CW) {
          const uint32_t k = pkey(pb[i]);
          if (ckey(k, i) < bound && (k & mask) == prefix) atomicAdd(&hw[wv][(k >> (8 * d)) & 255], 1u);
        }
        __syncthreads();
        for (uint32_t b = tid; b < 256; b += CW) {
          uint32_t c = 0;
          for (uint32_t w = 0; w < CW / 64; w++) c += hw[w][b];
          hist8[b] = c;
        }
        __syncthreads();
        if (tid == 0) {
          uint32_t need = s_need, above = 0;
          int D = 255;
          for (; D > 0; D--) {
            if (above + hist8[D] >= need) break;
            above += hist8[D];
          }
          s_need = need - above;
          s_prefix = prefix | ((uint32_t)D << (8 * d));
        }
        mask |= 255u << (8 * d);
        __syncthreads();
      }
      // the kk tokens: every eligible key above T, then the first `need` keys
      // equal to T in index order. Wave w owns a contiguous range of indices
      // and reads it 64 at a time (coalesced); a tie's rank is the ties
      // before it: earlier waves, earlier reads, lower lanes.
      const uint32_t T = s_prefix, need = s_need;
      if (tid == 0) s_ngt = 0;
      const uint32_t lane = tid & 63;
      const uint32_t span = ((n + CW / 64 - 1) / (CW / 64) + 63) / 64 * 64;
      const uint32_t w0 = min(n, wv * span), w1 = min(n, w0 + span);
      const uint64_t below = (1ull << lane) - 1;
      uint32_t ties = 0;
      for (uint32_t b0 = w0; b0 < w1; b0 += 64) {
        const uint32_t i = b0 + lane;
        bool tie = false;
        if (i < w1) {
          const uint32_t k = pkey(pb[i]);
          tie = k == T && ckey(k, i) < bound;
        }
        ties += __popcll(__ballot(tie));
      }
      if (lane == 0) wsum[wv] = ties;
      __syncthreads();
      uint32_t run = 0;
      for (uint32_t w = 0; w < wv; w++) run += wsum[w];
      const uint32_t ngt = kk - need;  // keys above T, all taken
      for (uint32_t b0 = w0; b0 < w1; b0 += 64) {
        const uint32_t i = b0 + lane;
        bool tie = false;
        uint64_t c = 0;
        if (i < w1) {
          const uint32_t k = pkey(pb[i]);
          c = ckey(k, i);
          if (c < bound) {
            if (k > T) keys[atomicAdd(&s_ngt, 1u)] = c;
            tie = k == T;
          }
        }
        const uint64_t tm = __ballot(tie);
        const uint32_t r = run + __popcll(tm & below);
        if (tie && r < need) keys[ngt + r] = c;
        run += __popcll(tm);
      }
      for (uint32_t j = kk + tid; j < sortn; j += CW) keys[j] = 0;  // sorts last
      __syncthreads();
      // bitonic sort, descending
      for (uint32_t size = 2; size <= sortn; size <<= 1)
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
          for (uint32_t i = tid; i < sortn; i += CW) {
            const uint32_t j = i ^ stride;
            if (j > i) {
              const bool desc = (i & size) == 0;
              const uint64_t a = keys[i], b = keys[j];
              if ((a < b) == desc) {
                keys[i] = b;
                keys[j] = a;
              }
            }
          }
          __syncthreads();
        }
      for (uint32_t j = tid; j < kk; j += CW) {
        ord[m + j] = 0xFFFFFFFFu - (uint32_t)keys[j];
        ordp[m + j] = key_p(keys[j]);
      }
      __threadfence();  // ord/ordp are read back through other waves' loads
      // the running sum over this block, in order, 32 sums at a time (it
      // never decreases: a batch reaches top_p iff its last sum does)
      if (tid == 0) {
        float acc = s_acc;
        for (uint32_t j = 0; j < kk && !s_done; j += 32) {
          float r[32];
          float a = acc;
          const uint32_t nb = min(32u, kk - j);
#pragma unroll
          for (uint32_t k = 0; k < 32; k++) {
            if (k < nb) a += key_p(keys[j + k]);
            r[k] = a;
          }
          if (a >= top_p || a != a) {
            for (uint32_t k = 0; k < nb; k++)
              if (r[k] >= top_p) {
                s_cut = m + j + k + 1;
                s_done = 1;
                a = r[k];
                break;
              }
          }
          acc = a;
        }
        s_acc = acc;
        if (m + kk == n) s_done = 1;  // never reached: the nucleus is every token
      }
      bound = keys[kk - 1];
      m += kk;
      __syncthreads();
    }
    // total = the nucleus's sum (the running sum where it stopped); then the
    // first token of the nucleus whose running sum exceeds u * total (the
    // last one of the nucleus if none does)
    const uint32_t cut = s_cut;
    const uint32_t at = chain_cross(ordp, cut, ring, u * s_acc);
    tok = ord[at < cut ? at : cut - 1];
  }
  if (tid == 0) {
    if (out) *out = tok;
    sd->token = tok;
    if (st) {
      const uint32_t nxt = st->pos + 1;
      if (nxt >= st->prompt_end && nxt <= st->cap) hist[nxt] = tok;  // hist has cap+1 slots
      st->pos = nxt;
    }
  }
}

}  // namespace

size_t cx_sample_parts(size_t n) { return (n + ZB * ZV - 1) / (ZB * ZV); }

int cx_launch_sample(const float* logits, size_t n, cx_samp_state* sd, float* pb, float* part,
                     uint32_t* ord, float* ordp, uint32_t* out, cx_dstate* st, uint32_t* hist,
                     hipStream_t s) {
  CX_REQUIRE(logits && sd && pb && part && ord && ordp && n > 0 && n < (1u << 31),
             "sample: bad arguments (n=%zu)", n);
  CX_REQUIRE(((uintptr_t)pb & 15) == 0 && ((uintptr_t)ordp & 15) == 0,
             "sample: the probability buffers must be 16-byte aligned");
  const unsigned g = (unsigned)cx_sample_parts(n);
  const size_t ring = (size_t)NST * SEG * sizeof(float);
  hipLaunchKernelGGL(k_samp_z, dim3(g), dim3(ZB), 0, s, logits, (uint32_t)n, sd, pb, part);
  CX_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_samp_e, dim3(g), dim3(ZB), 0, s, pb, (uint32_t)n, part, g, sd);
  CX_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_samp_sum, dim3(1), dim3(CW), ring, s, pb, (uint32_t)n, sd);
  CX_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_samp_p, dim3(g), dim3(ZB), 0, s, pb, (uint32_t)n, sd);
  CX_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_samp_pick, dim3(1), dim3(CW), PICK_LDS, s, pb, (uint32_t)n, sd, ord, ordp, out,
                     st, hist);
  CX_HIP(hipGetLastError());
  return CX_OK;
}
