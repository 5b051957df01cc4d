// cx_ops.hip — the per-token ops around the GEMV, for gfx950.
//
//   embedding row lookup         src/forward.rs:391-405 (descuantizar_filas of one row)
//   RoPE (split halves) + KV     src/ops.rs:1150-1193, src/forward.rs:440-456
//   decode attention (split-K)   src/ops.rs:1258-1325 at tokens = 1
//   causal GQA attention         src/ops.rs:1258-1325
//   softmax                      src/ops.rs:1206-1230
//   silu                         src/kernels/scalar.rs:63-67
//   argmax + token loop state    src/sampler.rs:129-137, src/forward.rs:544-557
#include "cx_ops.h"
#include "cx_act.h"
#include "cx_dequant.h"
#include "cx_scan.h"

namespace {

// ---------------------------------------------------------- embedding
// the token's row of an embedding table of any GGUF type, dequantized
// (quant::descuantizar_filas, src/quant.rs:172-205), 8 values a lane;
// workgroup r makes the row of position st->pos + r into x[r]
template <int T>
__global__ __launch_bounds__(256) void k_embed(const uint8_t* embd, uint32_t dim,
                                               const cx_dstate* st, const uint32_t* hist,
                                               float* x) {
  constexpr int VPB = T == CX_F32 || T == CX_F16 ? 1 : (T == CX_Q8_0 || T == CX_Q5_0 ? 32 : 256);
  constexpr int BPB = T == CX_F32 ? 4 : T == CX_F16 ? 2 : T == CX_Q8_0 ? 34 : T == CX_Q5_0 ? 22
                    : T == CX_Q2_K ? 84 : T == CX_Q3_K ? 110 : T == CX_Q4_K ? 144
                    : T == CX_Q5_K ? 176 : 210;
  const uint32_t tok = hist[st->pos + blockIdx.x];
  const uint8_t* row = embd + (size_t)tok * (dim / VPB) * BPB;
  x += (size_t)blockIdx.x * dim;
  for (uint32_t i = 8 * threadIdx.x; i < dim; i += 2048) {
    float v[8];
    cxq::dequant8<T>(row + i / VPB * BPB, i % VPB, v);
#pragma unroll
    for (int j = 0; j < 8; j++) x[i + j] = v[j];
  }
}

// ------------------------------------------------------ rope + KV append
// Token r (workgroup r) at position st->pos + r: q (H heads) rotated in
// place, k (Hkv heads) rotated and written to K[pos], v copied to V[pos].
// Rotation as src/ops.rs:1185-1188: a' = a*c - b*s, b' = a*s + b*c (no FMA).
__global__ __launch_bounds__(256) void k_rope_kv(float* q, const float* k, const float* v,
                                                 float* kc, float* vc, const float* cos_t,
                                                 const float* sin_t, uint32_t heads,
                                                 uint32_t kvh, uint32_t hd,
                                                 const cx_dstate* st) {
  const uint32_t pos = st->pos + blockIdx.x, half = hd / 2, kvd = kvh * hd;
  q += (size_t)blockIdx.x * heads * hd;
  k += (size_t)blockIdx.x * kvd;
  v += (size_t)blockIdx.x * kvd;
  const float* c = cos_t + (size_t)pos * half;
  const float* s = sin_t + (size_t)pos * half;
  float* kd = kc + (size_t)pos * kvd;
  float* vd = vc + (size_t)pos * kvd;
  for (uint32_t i = threadIdx.x; i < heads * half; i += 256) {
    const uint32_t h = i / half, j = i % half;
    float* lo = q + h * hd + j;
    const float x0 = lo[0], x1 = lo[half];
    lo[0] = x0 * c[j] - x1 * s[j];
    lo[half] = x0 * s[j] + x1 * c[j];
  }
  for (uint32_t i = threadIdx.x; i < kvh * half; i += 256) {
    const uint32_t h = i / half, j = i % half;
    const float x0 = k[h * hd + j], x1 = k[h * hd + j + half];
    kd[h * hd + j] = x0 * c[j] - x1 * s[j];
    kd[h * hd + j + half] = x0 * s[j] + x1 * c[j];
  }
  for (uint32_t i = threadIdx.x; i < kvd; i += 256) vd[i] = v[i];
}

// ------------------------------------------------- decode attention
// Split-K over cached positions ("flash decoding"). Workgroup (split, g)
// handles positions [split*P, +P) for all H/Hkv query heads of KV group g:
// K and V rows of the split are staged in LDS once and shared by the group's
// heads. Scores use the reference's sequential dot order
// (src/kernels/scalar.rs:16-23) times 1/sqrt(hd); each split keeps its own
// max m, sum l = sum exp(s - m) and unnormalised output o = sum e * v.
constexpr int ATT_P = 64;     // positions per split
constexpr int ATT_MAXG = 16;  // query heads per KV group supported

__global__ __launch_bounds__(256) void k_attn_split(const float* q, const float* kc,
                                                    const float* vc, uint32_t heads,
                                                    uint32_t kvh, uint32_t hd,
                                                    const cx_dstate* st, float scale,
                                                    float* pm, float* pl, float* po,
                                                    uint32_t max_splits) {
  extern __shared__ __align__(16) float sh[];
  // query token z (blockIdx.z) sits at position st->pos + z
  const uint32_t z = blockIdx.z, total = st->pos + z + 1;
  q += (size_t)z * heads * hd;
  pm += (size_t)z * max_splits * heads;
  pl += (size_t)z * max_splits * heads;
  po += (size_t)z * max_splits * heads * hd;
  const uint32_t split = blockIdx.x, g = blockIdx.y, per = heads / kvh;
  const uint32_t p0 = split * ATT_P;
  if (p0 >= total) return;
  const uint32_t np = min((uint32_t)ATT_P, total - p0);
  const uint32_t kvd = kvh * hd, ld = hd + 1;
  float* sq = sh;                       // per x hd
  float* skv = sq + per * hd;           // ATT_P x (hd+1)
  float* ssc = skv + ATT_P * ld;        // per x ATT_P
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  for (uint32_t i = tid; i < per * hd; i += 256) sq[i] = q[(g * per) * hd + i];
  for (uint32_t i = tid; i < np * hd; i += 256) {
    const uint32_t p = i / hd, d = i % hd;
    skv[p * ld + d] = kc[(size_t)(p0 + p) * kvd + g * hd + d];
  }
  __syncthreads();
  for (uint32_t i = tid; i < per * np; i += 256) {
    const uint32_t h = i / np, p = i % np;
    const float* a = sq + h * hd;
    const float* b = skv + p * ld;
    float s = 0.0f;
    for (uint32_t d = 0; d < hd; d++) s += a[d] * b[d];
    ssc[h * ATT_P + p] = s * scale;
  }
  __syncthreads();
  for (uint32_t h = wave; h < per; h += 4) {
    const float s = lane < (int)np ? ssc[h * ATT_P + lane] : -INFINITY;
    const float m = cx_wave_max(s);
    const float e = lane < (int)np ? cx_expf(s - m) : 0.0f;
    const float l = cx_wave_sum(e);
    if (lane < (int)np) ssc[h * ATT_P + lane] = e;
    if (lane == 0) {
      const size_t o = ((size_t)split * heads + g * per + h);
      pm[o] = m;
      pl[o] = l;
    }
  }
  __syncthreads();
  for (uint32_t i = tid; i < np * hd; i += 256) {
    const uint32_t p = i / hd, d = i % hd;
    skv[p * ld + d] = vc[(size_t)(p0 + p) * kvd + g * hd + d];
  }
  __syncthreads();
  for (uint32_t i = tid; i < per * hd; i += 256) {
    const uint32_t h = i / hd, d = i % hd;
    float o = 0.0f;
    for (uint32_t p = 0; p < np; p++) o += ssc[h * ATT_P + p] * skv[p * ld + d];
    po[((size_t)split * heads + g * per + h) * hd + d] = o;
  }
}

// Merge the splits of every head: M = max m_s, w_s = exp(m_s - M),
// out = (sum w_s o_s) * (1 / sum w_s l_s).
__global__ void k_attn_combine(const float* pm, const float* pl, const float* po,
                               uint32_t heads, uint32_t hd, const cx_dstate* st,
                               float* out, uint32_t max_splits) {
  const uint32_t z = blockIdx.z, total = st->pos + z + 1, ns = (total + ATT_P - 1) / ATT_P;
  pm += (size_t)z * max_splits * heads;
  pl += (size_t)z * max_splits * heads;
  po += (size_t)z * max_splits * heads * hd;
  out += (size_t)z * heads * hd;
  const uint32_t h = blockIdx.x;
  float M = -INFINITY;
  for (uint32_t s = 0; s < ns; s++) M = fmaxf(M, pm[(size_t)s * heads + h]);
  float L = 0.0f;
  for (uint32_t s = 0; s < ns; s++) L += pl[(size_t)s * heads + h] * cx_expf(pm[(size_t)s * heads + h] - M);
  const float inv = 1.0f / L;
  for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
    float o = 0.0f;
    for (uint32_t s = 0; s < ns; s++)
      o += po[((size_t)s * heads + h) * hd + d] * cx_expf(pm[(size_t)s * heads + h] - M);
    out[h * hd + d] = o * inv;
  }
}

// softmax of one row x[0..n) whose max is mx, in place, in the reference's
// order (src/ops.rs:1211-1229): non-finite max -> uniform; e = exp(x - max);
// the sum accumulated sequentially from 0; x = e * (1 / sum). 256 threads.
__device__ void seq_softmax_inplace(float* x, uint32_t n, float mx, float* red) {
  const int tid = threadIdx.x;
  if (!isfinite(mx)) {
    const float pr = 1.0f / (float)n;
    for (uint32_t p = tid; p < n; p += 256) x[p] = pr;
    __syncthreads();
    return;
  }
  for (uint32_t p = tid; p < n; p += 256) x[p] = cx_expf(x[p] - mx);
  __syncthreads();
  if (tid == 0) {
    float tot = 0.0f;
#pragma unroll 8
    for (uint32_t p = 0; p < n; p++) tot += x[p];
    red[0] = 1.0f / tot;
  }
  __syncthreads();
  const float inv = red[0];
  for (uint32_t p = tid; p < n; p += 256) x[p] = x[p] * inv;
  __syncthreads();
}

// ---------------------------------------------- general causal attention
// One workgroup per (head, token). Scores in the reference's order (sequential
// dot, times 1/sqrt(hd)), softmax over the visible positions (max, exp, sum,
// times 1/sum), output accumulated position by position like
// src/ops.rs:1316-1321. Scores live in LDS (total <= CX_ATT_MAX_TOTAL).
__global__ __launch_bounds__(256) void k_attention(const float* q, const float* k,
                                                   const float* v, uint32_t tokens,
                                                   uint32_t total, uint32_t heads,
                                                   uint32_t kvh, uint32_t hd, float scale,
                                                   float* out) {
  extern __shared__ __align__(16) float sc[];
  __shared__ float red[4];
  const uint32_t h = blockIdx.x, t = blockIdx.y;
  const uint32_t vis = total - tokens + t + 1, per = heads / kvh, g = h / per;
  const uint32_t wq = heads * hd, wkv = kvh * hd;
  const float* qh = q + (size_t)t * wq + h * hd;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float mx = -INFINITY;
  for (uint32_t p = tid; p < vis; p += 256) {
    const float* kp = k + (size_t)p * wkv + g * hd;
    float s = 0.0f;
    for (uint32_t d = 0; d < hd; d++) s += qh[d] * kp[d];
    s = s * scale;
    sc[p] = s;
    mx = fmaxf(mx, s);
  }
  mx = cx_wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  seq_softmax_inplace(sc, vis, mx, red);
  for (uint32_t d = tid; d < hd; d += 256) {
    float o = 0.0f;
    for (uint32_t p = 0; p < vis; p++) o += sc[p] * v[(size_t)p * wkv + g * hd + d];
    out[(size_t)t * wq + h * hd + d] = o;
  }
}

// ------------------------------------------- order-exact decode attention
// The decode step's attention in the reference's own order, for contexts up
// to CX_ATT_LDS_MAX, in two kernels. The scores kernel stages its K rows in
// LDS with direct-to-LDS loads, so a wave keeps up to 63 KiB of the cache
// in flight instead of waiting on one row at a time.
//
// k_attn_scores, one workgroup per (64 positions, head h): the 64 K rows of
// the head's group are copied into LDS by its four waves (rows padded by 16 bytes against bank
// conflicts), then lane p forms the sequential dot of
// src/kernels/scalar.rs:16-23 times 1/sqrt(hd) and writes sc[h][p]. With
// rope tables it first rotates q and this step's key (src/ops.rs:1185-1188:
// a' = a*c - b*s, b' = a*s + b*c, no FMA); the first head of each KV group
// appends the rotated key and the value to the cache at st->pos
// (src/forward.rs:454-455). The score at st->pos uses the rotated key from
// LDS, so no result depends on a cache row written in the same launch.
//
// k_attn_seq, one workgroup per (head, 32 head dims): the head's scores are
// copied in, then the softmax in the reference's order: exact max (from the
// scores kernel's chunk maxima), e = exp(s - max) (glibc's expf), the sum in
// position order from 0 (one add a position, or for long caches the first
// 256 so and the rest by binade scan), p = e * (1/sum) (src/ops.rs:
// 1211-1229). Meanwhile waves 1-3 stream the V slice into registers; they
// form each stage's products p * v[d] and wave 0's lane d adds them into
// out[d] in position order (src/ops.rs:1316-1321). The output is then
// quantized for the output projection (32 values are whole sub-blocks).
// Bit-identical to the scalar reference.
constexpr uint32_t SC_P = 64;     // positions per scores wave

// Waits until at most `later` stages' loads (IPW each) of this wave are
// outstanding, or fewer.
template <uint32_t IPW, uint32_t MAXL>
__device__ inline void wait_stages(uint32_t later) {
  if constexpr (MAXL == 0) {
    (void)later;
    cx_wait_vm<0>();
  } else {
    if (later >= MAXL) cx_wait_vm<MAXL * IPW>();
    else wait_stages<IPW, MAXL - 1>(later);
  }
}


__host__ __device__ constexpr uint32_t sc_stride(uint32_t cap) { return (cap + 3) / 4 * 4; }
// LDS floats for a head's scores: whole 1 KiB loads
__host__ __device__ constexpr uint32_t sc_lds(uint32_t cap) { return (cap + 255) / 256 * 256; }

template <int HD>
__global__ __launch_bounds__(256) void k_attn_scores(const float* q, const float* knew,
                                                    const float* vnew, float* kc, float* vc,
                                                    const float* cos_t, const float* sin_t,
                                                    uint32_t heads, uint32_t kvh,
                                                    const cx_dstate* st, float scale,
                                                    float* sc, float* cm, uint32_t cap) {
  constexpr uint32_t ROWB = HD * 4, PADB = ROWB + 16, PADF = PADB / 4;
  constexpr uint32_t NCH = (SC_P * PADB + 1023) / 1024;
  extern __shared__ __align__(16) uint8_t sm[];
  float* kl = reinterpret_cast<float*>(sm);
  float* qr = reinterpret_cast<float*>(sm + NCH * 1024);
  float* kr = qr + HD;
  constexpr uint32_t half = HD / 2;
  const uint32_t chunk = blockIdx.x, h = blockIdx.y;
  const uint32_t pos = st->pos, total = pos + 1;
  const uint32_t p0 = chunk * SC_P, per = heads / kvh, g = h / per;
  if (p0 >= total) return;
  const uint32_t np = min(SC_P, total - p0), kvd = kvh * HD;
  const uint32_t nck = (cap + SC_P - 1) / SC_P;
  const int tid = threadIdx.x, t = tid & 63, w = tid >> 6;
  // the scale is read here, with the other arguments: read where it is
  // used, its scalar load would make the dots' LDS reads wait for it
  asm volatile("" ::"s"(scale));
  // 1. the K rows [p0, p0 + np) into LDS, a quarter of the loads by each
  //    wave (a wave issues such loads at a bounded rate: four issue them in
  //    a quarter of the time); pad bytes and rows past the end load a valid
  //    dummy that is never read
  const float* kb = kc + (size_t)p0 * kvd + g * HD;
  for (uint32_t c = w; c < NCH; c += 4) {
    const uint32_t o = c * 1024 + 16 * t;
    uint32_t r = o / PADB, b = o % PADB;
    if (r >= np || b >= ROWB) r = 0, b = 0;
    cx_dma16(reinterpret_cast<const uint8_t*>(kb + (size_t)r * kvd) + b, sm + c * 1024);
  }
  // 2. rope while the rows arrive. Every load is issued before the first
  //    wait: q, the tables, this step's key (loaded by every workgroup,
  //    used by the last chunk's) and the value the append stores in step 4
  //    (each a round trip of its own after the dots when loaded where used)
  const bool rot = cos_t != nullptr, has_new = rot && pos < p0 + SC_P;
  const bool append = has_new && h % per == 0;
  float vv[HD / 64];
  if (append && w == 0) {
#pragma unroll
    for (int i = 0; i < HD / 64; i++) vv[i] = vnew[g * HD + t + 64 * i];
  }
  if (rot) {
    const float* c = cos_t + (size_t)pos * half;
    const float* s = sin_t + (size_t)pos * half;
    for (uint32_t j = tid; j < half; j += 256) {
      float x0 = q[h * HD + j], x1 = q[h * HD + j + half];
      float k0 = knew[g * HD + j], k1 = knew[g * HD + j + half];
      float cj = c[j], sj = s[j];
      // (one wait for all six: left alone, the compiler sinks the key's
      // loads into the branch below, after a wait for the others)
      asm volatile("" : "+v"(x0), "+v"(x1), "+v"(k0), "+v"(k1), "+v"(cj), "+v"(sj));
      qr[j] = x0 * cj - x1 * sj;
      qr[j + half] = x0 * sj + x1 * cj;
      if (has_new) {
        const float a = k0 * cj - k1 * sj, b = k0 * sj + k1 * cj;
        kr[j] = a;
        kr[j + half] = b;
      }
    }
  } else {
    for (uint32_t j = tid; j < HD; j += 256) qr[j] = q[h * HD + j];
  }
  cx_wait_vm<0>();
  __syncthreads();
  if (w != 0) return;
  // 3. wave 0, lane t: position p0 + t; the chunk's maximum (fmaxf: a NaN score
  //    is passed over, as in the softmax's own maximum)
  float v = -INFINITY;
  if ((uint32_t)t < np) {
    const uint32_t p = p0 + t;
    const float4* a4 = reinterpret_cast<const float4*>(qr);
    const float4* b4 = reinterpret_cast<const float4*>((has_new && p == pos) ? kr : kl + t * PADF);
    const float s = cx_dot_seq<HD / 4>(a4, b4);
    v = s * scale;
    sc[(size_t)h * sc_stride(cap) + p] = v;
  }
  v = cx_wave_max(v);
  if (t == 0) cm[(size_t)h * nck + chunk] = v;
  // 4. one workgroup of the KV group appends the rotated key (from LDS) and
  //    the value at st->pos for later tokens (src/forward.rs:454-455):
  //    stored after the dots, since a wave waits for its stores as for its
  //    loads, and nothing here reads them
  if (append) {
    float* kd = kc + (size_t)pos * kvd + g * HD;
    float* vd = vc + (size_t)pos * kvd + g * HD;
#pragma unroll
    for (int i = 0; i < HD / 64; i++) {
      kd[t + 64 * i] = kr[t + 64 * i];
      vd[t + 64 * i] = vv[i];
    }
  }
}

// tot += the 32 values of a, in order
__device__ inline void add32(float& tot, const float4 (&a)[8]) {
#pragma unroll
  for (int i = 0; i < 8; i++) {
    tot += a[i].x;
    tot += a[i].y;
    tot += a[i].z;
    tot += a[i].w;
  }
}

constexpr uint32_t SCAN_STAGE = 2048;  // positions a stage of the long softmax

// o += p[j] * v[j] for 8 positions in order. The 8 products are formed
// first, pinned there by an empty asm that takes them as operands: left to
// itself the compiler interleaves each multiply with its add, and the chain
// then waits for a multiply and an add per position instead of one add.
__device__ inline void pv8(float& o, const float4 (&p)[2], const float (&v)[8]) {
  float t0 = p[0].x * v[0], t1 = p[0].y * v[1], t2 = p[0].z * v[2], t3 = p[0].w * v[3];
  float t4 = p[1].x * v[4], t5 = p[1].y * v[5], t6 = p[1].z * v[6], t7 = p[1].w * v[7];
  asm volatile("" : "+v"(t0), "+v"(t1), "+v"(t2), "+v"(t3), "+v"(t4), "+v"(t5), "+v"(t6),
               "+v"(t7));
  o += t0;
  o += t1;
  o += t2;
  o += t3;
  o += t4;
  o += t5;
  o += t6;
  o += t7;
}

// The P.V stage: PV_STP positions of a 32-dim slice in blocks of 4
// positions x 4 dims (block b: positions 4 (b / 8) .. +3, dims 4 (b % 8)
// .. +3). The helpers (waves 1-4) split every stage's blocks, lane l of
// helper h taking blocks 256 k + 64 h + l. A helper loads its
// blocks' V rows straight into registers three stages ahead (no V passes
// through LDS), forms the products p_j * v_j[d] (p_j = e_j * (1/sum), or
// 1/total when uniform; +0.0 past total) and writes them transposed,
// [dim][position], into one of two LDS buffers, while wave 0's chain adds
// the previous stage's products from the other; one barrier a stage, and
// wave 0 issues no load. A buffer row is PV_STP floats, 16-byte chunk c of
// row d stored at chunk c ^ (d % 8), so that the helpers' writes and the
// chain's reads (lane d: four positions of row d a read) spread over the
// 32 banks. Measured and dropped: the ring of direct-to-LDS stages (a
// stage's 16 loads shared by all four waves; ~2100 clocks a stage at config
// 5 against the chain's ~1100, wave 0's refills and the stage coupling);
// each helper a whole stage in turn, loaded into LDS slots of its own and
// transposed in place (a helper's 16 direct-to-LDS loads took ~1450 clocks
// to issue and its transposition ~2000: 2470 a stage); three helpers with
// two blocks a lane (~1600 clocks a stage for a helper's share).
// The kernel's shape, PV_STP positions a stage and PV_NT threads: 128 and
// 320 (four helpers, one block a lane) for caches up to PV_LONG_CAP
// positions, else 256 and 576 (eight helpers): measured on MI355X, the 3B
// decode at ~600 positions 732 tok/s with 128-position stages against 719
// with 256 (the pipeline's fill and drain are a larger share of three
// stages), config 5 at 8200 positions 282.9 tok/s against 273.8.
constexpr uint32_t PV_LONG_CAP = 2048;
__host__ __device__ constexpr uint32_t pv_lds_floats(uint32_t cap, uint32_t stp) {
  return sc_lds(cap) + 2 * stp * 32;  // the scores, then two product buffers of stp x 32
}
// Softmax sums of up to SUM_PLAIN_MAX positions add one position at a time
// (seq_add16); longer ones take the binade scan.
constexpr uint32_t SUM_PLAIN_MAX = 768;
constexpr uint32_t CML_MAX = 256;  // chunk maxima of one head: 16384 positions

// A workgroup's waves go to the CU's four SIMDs in turn, so wave 4 of the
// short shape (five waves) would share SIMD 0 with wave 0's chain, whose
// adds are bound by that SIMD's issue: the short shape launches six waves
// and wave 4 leaves at once (3B decode 741.5 -> 745.3 tok/s). The long
// shape keeps nine (eleven with waves 4 and 8 leaving measured 282.1 ->
// 278.4 tok/s at config 5).
__host__ __device__ constexpr uint32_t pv_lt(uint32_t nt) { return nt == 320 ? 384 : nt; }

// PV_NT active threads (of pv_lt(PV_NT) launched): wave 0's lanes run the
// order-exact accumulation, the others stream V. Rows of the grid past
// HD / 32 are prefetch workgroups (pf).
template <int HD, int SUB, uint32_t PV_STP, uint32_t PV_NT>
__global__ __launch_bounds__(pv_lt(PV_NT)) void k_attn_seq(const float* vc, const float* sc_all,
                                                  const float* cm_all, uint32_t heads,
                                                  uint32_t kvh, const cx_dstate* st, uint32_t cap,
                                                  float* out, int8_t* xq, float* xe, float* xs,
                                                  cx_l2_prefetch pf) {
  constexpr uint32_t DS = 32;  // head dims a workgroup (32 give twice the workgroups of 64,
                               // so the softmax and chains run on more CUs at once)
  constexpr uint32_t PV_BUF = PV_STP * 32;                       // floats of a product buffer
  constexpr uint32_t PV_BPL = PV_STP * 8 / 4 / (PV_NT - 64);     // blocks a helper lane a stage
  static_assert(PV_BPL * (PV_NT - 64) * 4 == PV_STP * 8, "whole blocks a lane");
  if (blockIdx.y >= HD / DS) {
    const uint32_t first = gridDim.x * (HD / DS);
    cx_l2_prefetch_run(pf, blockIdx.x + gridDim.x * blockIdx.y - first, first);
    return;
  }
  extern __shared__ __align__(16) float e[];  // sc_lds(cap) scores, then two product buffers
  float* pbuf = e + sc_lds(cap);
  __shared__ uint64_t etab[32];  // exp's table in LDS: no global load after the prefetch
  __shared__ float red[4];
  __shared__ float osum[DS];  // the output, for its quantization
  __shared__ __align__(16) float cml[CML_MAX];  // the head's chunk maxima
  // The workgroups of a (KV group, dims slice) pair
  // take linear ids i, i + 8, i + 16, ...: workgroups are dispatched to the
  // 8 XCDs round-robin, so the heads of a group that read the same V slice
  // share one XCD's L2, and each V line is fetched from memory once.
  uint32_t h = blockIdx.x, y = blockIdx.y;
  {
    constexpr uint32_t NY = HD / DS;
    const uint32_t n = heads * NY, per = heads / kvh;
    if (n % 8 == 0) {
      const uint32_t L = blockIdx.x + gridDim.x * blockIdx.y, J = (L % 8) * (n / 8) + L / 8;
      y = J / per % NY;
      h = J / per / NY * per + J % per;
    }
  }
  const int wl = threadIdx.x >> 6;  // the launched wave
  if (pv_lt(PV_NT) != PV_NT && wl == 4) return;
  const uint32_t total = st->pos + 1, g = h / (heads / kvh);
  const uint32_t d0 = y * DS, kvd = kvh * HD;
  // the active wave and thread (the short shape's wave 5 is active wave 4)
  const int t = threadIdx.x & 63, w = pv_lt(PV_NT) != PV_NT ? wl - wl / 4 : wl, tid = 64 * w + t;
  // 1. the head's scores as untracked direct-to-LDS loads; with one query
  //    token wave 0 first fetches the chunk maxima the scores kernel wrote
  //    (64 positions a chunk, at most CML_MAX chunks). Both cover the
  //    whole cache (positions past the token's are loaded and never used),
  //    so that they are issued before the position state arrives.
  const uint32_t nckc = (cap + SC_P - 1) / SC_P;
  if (w == 0) {  // lane t: chunks t, t + 64, ... (past the chunks: chunk 0)
    const float* crow = cm_all + (size_t)h * nckc;
    for (uint32_t i = 0; 64 * i < nckc; i++)
      cx_dma4_async(crow + (64 * i + t < nckc ? 64 * i + t : 0), cml + 64 * i);
  }
  const float* srow = sc_all + (size_t)h * sc_stride(cap);
  const uint32_t nsc = (cap + 255) / 256;  // 1 KiB per load
  for (uint32_t c = w; c < nsc; c += PV_NT / 64) {
    const uint32_t i = c * 256 + 4 * t;
    cx_dma16_async(srow + (i < cap ? i : 0), e + c * 256);
  }
  const uint32_t nck = (total + SC_P - 1) / SC_P;
  if (tid == 0) {  // while the scores arrive; uniform indices: scalar loads
    const uint64_t tab[32] = CX_EXP2_TAB;
    for (int i = 0; i < 32; i++) etab[i] = tab[i];
  }
  const uint32_t nstage = (total + PV_STP - 1) / PV_STP;
  // a helper lane's blocks: b = (PV_NT - 64) k + 64 (w - 1) + l, position
  // quad b / 8, dim quad b % 8 (the same for every k)
  const uint32_t b0 = 64 * (w - 1) + t;
  const float* vb = vc + g * HD + d0 + 4 * (b0 % 8);
  struct Vb {
    float4 a[PV_BPL][4];  // block k's four positions (dims 4 (b0 % 8) .. +3)
  };
  auto load = [&](Vb& R, uint32_t s) {  // stage s's rows (past total: position 0's)
#pragma unroll
    for (uint32_t k = 0; k < PV_BPL; k++)
#pragma unroll
      for (uint32_t i = 0; i < 4; i++) {
        uint32_t p = s * PV_STP + 4 * ((b0 + (PV_NT - 64) * k) / 8) + i;
        if (p >= total) p = 0;
        R.a[k][i] = *reinterpret_cast<const float4*>(vb + (size_t)p * kvd);
      }
  };
  // The scores land before the V loads are issued (issued together, every
  // workgroup's V burst would queue ahead of the scores the softmax needs
  // first); a helper's first three stages then load during the softmax.
  cx_wait_vm<0>();
  Vb r0, r1, r2;
  if (w != 0) {  // (a stage past the last loads rows of position 0, never used)
    load(r0, 0);
    load(r1, 1);
    load(r2, 2);
  }
  cx_wait_lds();
  cx_barrier();  // every wave's scores (and chunk maxima) and the exp table are in LDS
  float o = 0.0f;
  // 2. softmax over positions [0, total): the maximum of the chunk maxima
  //    (the same in every wave), e = exp(s - max) of the first PV_NT
  //    positions by every thread, then of the rest by the helpers while
  //    wave 0 adds the ones formed: the sum is the f32 sum in position
  //    order from 0 (src/ops.rs:1211-1229): one add a position up to
  //    SUM_PLAIN_MAX positions, else the first 256 one by one and the rest
  //    by seq_sum_scan. The division by the sum is folded into the
  //    products below.
  float mx = -INFINITY;
#pragma unroll
  for (uint32_t i = 0; i < CML_MAX / 64; i++)
    if (64 * i + t < nck) mx = fmaxf(mx, cml[64 * i + t]);
  mx = cx_wave_max(mx);
  const bool uniform = !isfinite(mx);  // all -inf, or a NaN (src/ops.rs:1214-1219)
  const float pu = 1.0f / (float)total;
  const uint32_t r64 = (total + 63) / 64 * 64;  // +0.0 from total to r64 (seq_add16)
  if ((uint32_t)tid < total)
    e[tid] = uniform ? pu : cx_expf_tab(e[tid] - mx, etab);
  else if ((uint32_t)tid < r64)
    e[tid] = 0.0f;
  cx_wait_lds();
  cx_barrier();
  float tot = 0.0f;
  if (total <= SUM_PLAIN_MAX) {
    // the helpers form the other exps at once while wave 0 adds the first
    // 256, then wave 0 adds the rest
    if (w != 0) {
      for (uint32_t p = PV_NT + tid - 64; p < r64; p += PV_NT - 64)
        e[p] = p >= total ? 0.0f : uniform ? pu : cx_expf_tab(e[p] - mx, etab);
    } else if (!uniform) {
      tot = seq_add16<18>(e, (min(total, 256u) + 15) / 16 * 16, 0.0f);
    }
    if (total > 256) {
      cx_wait_lds();
      cx_barrier();  // the rest of the exps are in LDS
      // one add a position (~4.5 clocks): at these lengths faster than the
      // binade scan, whose windows and events cost more than they save
      // (1.7 us at 388 positions, against ~0.9)
      if (w == 0 && !uniform)
        tot = seq_add16<(SUM_PLAIN_MAX / 16 + 2) / 3 * 3>(e + 256, (total - 256 + 15) / 16 * 16, tot);
    }
  } else {
    // a longer cache: stages of SCAN_STAGE positions, the first stage's
    // exps by every thread, then the helpers forming stage s + 1's while
    // wave 0 adds stage s's
    for (uint32_t p = PV_NT + tid; p < min(SCAN_STAGE, r64); p += PV_NT)
      e[p] = p >= total ? 0.0f : uniform ? pu : cx_expf_tab(e[p] - mx, etab);
    cx_wait_lds();
    cx_barrier();
    const uint32_t nss = (total + SCAN_STAGE - 1) / SCAN_STAGE;
    for (uint32_t s = 0; s < nss; s++) {
      if (w != 0) {
        const uint32_t b = SCAN_STAGE * (s + 1), end = min(b + SCAN_STAGE, r64);
        for (uint32_t p = b + tid - 64; p < end; p += PV_NT - 64)
          e[p] = p >= total ? 0.0f : uniform ? pu : cx_expf_tab(e[p] - mx, etab);
      } else if (!uniform) {
        tot = seq_sum_scan(e + SCAN_STAGE * s, min(SCAN_STAGE, total - SCAN_STAGE * s), tot, s == 0);
      }
      if (s + 1 < nss) {
        cx_wait_lds();
        cx_barrier();  // stage s + 1's exps are in LDS
      }
    }
  }
  if (tid == 15) red[0] = 1.0f / tot;
  cx_wait_lds();
  cx_barrier();
  const float inv = red[0];
  // 3. out[d0 + t], the sum over positions of p * v[d0 + t] in position
  //    order (wave 0's lane t), a stage behind the helper that forms the
  //    stage's products
  // stage s's products into buffer s % 2, then stage s + 3 into the
  // registers (always: past the last stage, rows of position 0)
  auto make = [&](Vb& R, uint32_t s) {
    float* pb = pbuf + (s & 1) * PV_BUF;
#pragma unroll
    for (uint32_t k = 0; k < PV_BPL; k++) {
      const uint32_t b = b0 + (PV_NT - 64) * k, q = b / 8, r = b % 8, p0 = s * PV_STP + 4 * q;
      const float4 e4 = *reinterpret_cast<const float4*>(e + p0);
      float pp[4] = {e4.x, e4.y, e4.z, e4.w};
      if (!uniform)
#pragma unroll
        for (int i = 0; i < 4; i++) pp[i] = pp[i] * inv;
      float m[4][4];  // [dim j][position i]
#pragma unroll
      for (uint32_t i = 0; i < 4; i++) {
        const bool live = p0 + i < total;
        m[0][i] = live ? pp[i] * R.a[k][i].x : 0.0f;
        m[1][i] = live ? pp[i] * R.a[k][i].y : 0.0f;
        m[2][i] = live ? pp[i] * R.a[k][i].z : 0.0f;
        m[3][i] = live ? pp[i] * R.a[k][i].w : 0.0f;
      }
#pragma unroll
      for (uint32_t j = 0; j < 4; j++) {
        const uint32_t d = 4 * r + j;
        *reinterpret_cast<float4*>(pb + d * PV_STP + 4 * (q ^ (d & 7))) =
            make_float4(m[j][0], m[j][1], m[j][2], m[j][3]);
      }
    }
    load(R, s + 3);
  };
  // The helpers and wave 0 run loops of their own, one barrier a stage,
  // s = 0 .. nstage. A helper forms stage s's products into buffer s % 2
  // from the registers its loads went to three stages before, then loads
  // stage s + 3 into them (past the last stage too: rows of position 0),
  // every step unconditional and three stages a pass, so that r0, r1 and r2
  // keep their registers and the compiler's wait for a stage's loads leaves
  // the next two stages' in flight.
  if (w != 0) {
    for (uint32_t base = 0;; base += 3) {
      make(r0, base);
      cx_wait_lds();
      cx_barrier();  // stage s's products are formed; stage s - 1's are read
      if (base + 1 > nstage) break;
      make(r1, base + 1);
      cx_wait_lds();
      cx_barrier();
      if (base + 2 > nstage) break;
      make(r2, base + 2);
      cx_wait_lds();
      cx_barrier();
      if (base + 3 > nstage) break;
    }
    cx_wait_vm<0>();  // the last, unused loads
    return;
  }
  for (uint32_t s = 0; s <= nstage; s++) {
    if (s >= 1 && t < (int)DS) {
      // stage s - 1: 32 positions a batch, the next batch's reads ahead of
      // the adds; the stage's last batch ends past total with products of
      // +0.0 (adding +0.0 changes no sum that starts at +0.0)
      const uint32_t sp = s - 1;
      const float* pr = pbuf + (sp & 1) * PV_BUF + t * PV_STP;
      const uint32_t sw = (uint32_t)t & 7;
      constexpr uint32_t NQ = PV_STP / 32;  // batches a stage
      const uint32_t nq = min(NQ, (total - sp * PV_STP + 31) / 32);
      auto rd = [&](float4 (&a)[8], uint32_t b) {
#pragma unroll
        for (uint32_t i = 0; i < 8; i++)
          a[i] = *reinterpret_cast<const float4*>(pr + 4 * ((8 * b + i) ^ sw));
      };
      float4 a[8], b[8];
      rd(a, 0);
      rd(b, 1);
#pragma unroll
      for (uint32_t k = 0; k < NQ; k += 2) {
        __builtin_amdgcn_sched_barrier(0);
        add32(o, a);
        if (k + 1 >= nq) break;
        if (k + 2 < NQ) rd(a, k + 2);
        __builtin_amdgcn_sched_barrier(0);
        add32(o, b);
        if (k + 2 >= nq) break;
        if (k + 3 < NQ) rd(b, k + 3);
      }
    }
    cx_wait_lds();
    cx_barrier();
  }
  if (t >= (int)DS) return;
  out[h * HD + d0 + t] = o;
  if (!xq) return;
  osum[t] = o;
  cx_wait_lds();
  if (t < (int)(DS / 8)) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = osum[8 * t + j];
    cx_quant8<SUB>(v, (size_t)h * HD + d0 + 8 * t, xq, xe, xs);
  }
}

// ------------------------------------ order-exact attention, many queries
// The batched prefill's attention (several query tokens; q rotated and the
// caches filled by the chunk's rope/KV launch) in the reference's order:
// every query token's scores, softmax and P·V exactly as k_attn_scores and
// k_attn_seq form them for one, but MT_Q tokens a workgroup, one a wave.
// The K chunk (scores) or the V stages (softmax-V) are loaded once for the
// MT_Q tokens, and their chains run at once, one per SIMD.
constexpr uint32_t MT_Q = 4;

// k_attn_scores_mt, one workgroup per (64 positions, head h, MT_Q tokens):
// the chunk's K rows into LDS (rows padded by 16 bytes against bank
// conflicts) and the tokens' q rows; wave w's lane t forms token
// (MT_Q zg + w)'s score at position p0 + t, the sequential dot of
// src/kernels/scalar.rs:16-23 times 1/sqrt(hd), where the token sees it.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_scores_mt(const float* q, const float* kc,
                                                       uint32_t heads, uint32_t kvh,
                                                       const cx_dstate* st, float scale, float* sc,
                                                       uint32_t cap, uint32_t T) {
  constexpr uint32_t ROWB = HD * 4, PADB = ROWB + 16, PADF = PADB / 4;
  constexpr uint32_t NCH = (SC_P * PADB + 1023) / 1024;
  extern __shared__ __align__(16) uint8_t sm[];
  const float* kl = reinterpret_cast<const float*>(sm);
  float* qs = reinterpret_cast<float*>(sm + NCH * 1024);  // MT_Q rows of HD
  const uint32_t chunk = blockIdx.x, h = blockIdx.y, z0 = blockIdx.z * MT_Q;
  const uint32_t pos = st->pos, p0 = chunk * SC_P, zn = min(MT_Q, T - z0);
  const uint32_t tmax = pos + z0 + zn;  // the largest count of positions a token sees
  if (p0 >= tmax) return;
  const uint32_t np = min(SC_P, tmax - p0), g = h / (heads / kvh), kvd = kvh * HD;
  const int tid = threadIdx.x, t = tid & 63, w = tid >> 6;
  asm volatile("" ::"s"(scale));  // read with the arguments, not by the dots
  const float* kb = kc + (size_t)p0 * kvd + g * HD;
  for (uint32_t c = w; c < NCH; c += 4) {
    const uint32_t o = c * 1024 + 16 * t;
    uint32_t r = o / PADB, b = o % PADB;
    if (r >= np || b >= ROWB) r = 0, b = 0;  // a valid dummy, never read
    cx_dma16(reinterpret_cast<const uint8_t*>(kb + (size_t)r * kvd) + b, sm + c * 1024);
  }
  for (uint32_t j = tid; j < zn * HD; j += 256)
    qs[j] = q[((size_t)(z0 + j / HD) * heads + h) * HD + j % HD];
  cx_wait_vm<0>();
  __syncthreads();
  if ((uint32_t)w >= zn) return;
  const uint32_t z = z0 + w, total = pos + z + 1;
  if (p0 + t < total && (uint32_t)t < np) {
    const float s = cx_dot_seq<HD / 4>(reinterpret_cast<const float4*>(qs + w * HD),
                                       reinterpret_cast<const float4*>(kl + t * PADF));
    sc[((size_t)z * heads + h) * sc_stride(cap) + p0 + t] = s * scale;
  }
}

// k_attn_seq_mt, one workgroup per (head h, MT_DS head dims, MT_Q tokens):
// wave w takes token z = MT_Q zg + w and its total = pos + z + 1 positions.
// Its scores row into LDS; the softmax in the reference's order (exact
// max; e = exp(s - max), glibc's expf; the sum in position order from 0,
// its first 256 adds one by one and the rest by binade scan; p = e * (1/sum);
// a max that is not finite gives 1/total: src/ops.rs:1211-1229); then lane
// t accumulates out[d0 + t] = sum over positions of p * v[d0 + t] in
// position order (src/ops.rs:1316-1321). The V slice streams through a ring
// of MT_NST stages of MT_STP positions, each loaded a quarter by each wave
// and read by every wave's chain.
constexpr uint32_t MT_DS = 64, MT_STP = 64, MT_NST = 4;  // a 64 KiB ring
constexpr uint32_t MT_SLOT = MT_STP * MT_DS;             // floats a stage
__host__ __device__ constexpr uint32_t mt_lds_floats(uint32_t cap) {
  return MT_Q * sc_lds(cap) + MT_NST * MT_SLOT;
}
template <int HD>
__global__ __launch_bounds__(256) void k_attn_seq_mt(const float* vc, const float* sc_all,
                                                    uint32_t heads, uint32_t kvh,
                                                    const cx_dstate* st, uint32_t cap, uint32_t T,
                                                    float* out) {
  constexpr uint32_t IPW = MT_SLOT * 4 / 1024 / 4;  // 1 KiB loads a stage, per wave
  constexpr uint32_t LPP = MT_DS / 4;                // lanes per position in a load
  static_assert(IPW >= 1 && 4 + MT_NST * IPW <= 63, "loads a wave keeps in flight");
  extern __shared__ __align__(16) float e[];  // MT_Q scores rows of sc_lds(cap), then the ring
  __shared__ uint64_t etab[32];
  const uint32_t scl = sc_lds(cap);
  float* ring = e + MT_Q * scl;
  const uint32_t h = blockIdx.x, d0 = blockIdx.y * MT_DS, z0 = blockIdx.z * MT_Q;
  const uint32_t zn = min(MT_Q, T - z0), pos = st->pos, tmax = pos + z0 + zn;
  const int tid = threadIdx.x, t = tid & 63, w = tid >> 6;
  const uint32_t g = h / (heads / kvh), kvd = kvh * HD;
  const bool mine = (uint32_t)w < zn;  // this wave has a token
  const uint32_t z = z0 + w, total = pos + z + 1;
  float* ew = e + w * scl;
  // 1. the token's scores (whole 1 KiB loads over the cache), then the
  //    first MT_NST stages of V (positions past tmax load position 0 and
  //    are never read): a wave's loads complete in issue order, so waiting
  //    for all but its V loads waits for its scores
  if (mine) {
    const float* srow = sc_all + ((size_t)z * heads + h) * sc_stride(cap);
    for (uint32_t c = 0; c * 256 < cap; c++) {
      const uint32_t i = c * 256 + 4 * t;
      cx_dma16_async(srow + (i < cap ? i : 0), ew + c * 256);
    }
  }
  const float* vb = vc + g * HD + d0;
  auto issue = [&](uint32_t s) {  // wave w's loads of stage s: 4 positions each
    float* dst = ring + (s % MT_NST) * MT_SLOT;
    for (uint32_t j = 0; j < IPW; j++) {
      const uint32_t i = w + 4 * j;
      uint32_t p = s * MT_STP + i * (64 / LPP) + t / LPP;
      if (p >= tmax) p = 0;
      cx_dma16_async(reinterpret_cast<const uint8_t*>(vb + (size_t)p * kvd) + (t % LPP) * 16,
                     dst + i * 256);
    }
  };
  for (uint32_t s = 0; s < MT_NST; s++) issue(s);
  if (tid == 0) {
    const uint64_t tab[32] = CX_EXP2_TAB;
    for (int i = 0; i < 32; i++) etab[i] = tab[i];
  }
  cx_wait_vm<MT_NST * IPW>();
  cx_wait_lds();
  cx_barrier();  // the scores and the exp table are in LDS
  float o = 0.0f;
  if (mine) {
    // 2. the softmax of this token's row (one wave; its LDS accesses are in order)
    float mx = -INFINITY;
    for (uint32_t p = t; p < total; p += 64) mx = fmaxf(mx, ew[p]);
    mx = cx_wave_max(mx);
    const bool uniform = !isfinite(mx);  // all -inf, or a NaN (src/ops.rs:1214-1219)
    const float pu = 1.0f / (float)total;
    const uint32_t r64 = (total + 63) / 64 * 64;  // +0.0 from total to r64 (the scan's head)
    for (uint32_t p = t; p < r64; p += 64)
      ew[p] = p >= total ? 0.0f : uniform ? pu : cx_expf_tab(ew[p] - mx, etab);
    if (!uniform) {
      const float inv = 1.0f / seq_sum_scan(ew, total, 0.0f, true);
      for (uint32_t p = t; p < total; p += 64) ew[p] = ew[p] * inv;
    }
  }
  // 3. P·V, stage s in slot s % MT_NST; MT_NST stages were issued, and
  //    stage s + MT_NST is issued once stage s is read
  const uint32_t nstage = (tmax + MT_STP - 1) / MT_STP;
  const uint32_t refills = nstage > MT_NST ? nstage - MT_NST : 0u;
  for (uint32_t s = 0; s < nstage; s++) {
    const uint32_t issued = MT_NST + min(s, refills);
    wait_stages<IPW, MT_NST - 1>(issued - s - 1);
    cx_wait_lds();
    cx_barrier();  // stage s has landed, from every wave
    if (mine && s * MT_STP < total) {
      const float* vs = ring + (s % MT_NST) * MT_SLOT + t;
      const float* ps = ew + s * MT_STP;
      if ((s + 1) * MT_STP <= total) {
        // two batches of 32 positions: the second's reads are issued before
        // the first's arithmetic
        const float4* p4 = reinterpret_cast<const float4*>(ps);
        float va[32], vb2[32];
        float4 pa[8], pb[8];
#pragma unroll
        for (int j = 0; j < 32; j++) va[j] = vs[j * MT_DS];
#pragma unroll
        for (int i = 0; i < 8; i++) pa[i] = p4[i];
#pragma unroll
        for (int j = 0; j < 32; j++) vb2[j] = vs[(32 + j) * MT_DS];
#pragma unroll
        for (int i = 0; i < 8; i++) pb[i] = p4[8 + i];
        static_assert(MT_STP == 64, "two batches of 32 a stage");
#pragma unroll
        for (int k = 0; k < 4; k++)
          pv8(o, *reinterpret_cast<const float4(*)[2]>(pa + 2 * k),
              *reinterpret_cast<const float(*)[8]>(va + 8 * k));
#pragma unroll
        for (int k = 0; k < 4; k++)
          pv8(o, *reinterpret_cast<const float4(*)[2]>(pb + 2 * k),
              *reinterpret_cast<const float(*)[8]>(vb2 + 8 * k));
      } else {
        for (uint32_t j = 0; s * MT_STP + j < total; j++) o += ps[j] * vs[j * MT_DS];
      }
    }
    cx_wait_lds();
    cx_barrier();  // every chain has read the slot: refill it
    if (s + MT_NST < nstage) issue(s + MT_NST);
  }
  cx_wait_vm<0>();  // the loads of stages past the last one have landed
  if (mine) out[((size_t)z * heads + h) * HD + d0 + t] = o;
}

// -------------------------------------------------------------- softmax
__global__ __launch_bounds__(256) void k_softmax(float* x, uint32_t width) {
  __shared__ float red[4];
  float* row = x + (size_t)blockIdx.x * width;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float mx = -INFINITY;
  for (uint32_t i = tid; i < width; i += 256) mx = fmaxf(mx, row[i]);
  mx = cx_wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  if (!isfinite(mx)) {  // all -inf, or a NaN: uniform (src/ops.rs:1214-1219)
    const float p = 1.0f / (float)width;
    for (uint32_t i = tid; i < width; i += 256) row[i] = p;
    return;
  }
  float tot = 0.0f;
  for (uint32_t i = tid; i < width; i += 256) {
    const float e = cx_expf(row[i] - mx);
    row[i] = e;
    tot += e;
  }
  tot = cx_wave_sum(tot);
  if (lane == 0) red[wave] = tot;
  __syncthreads();
  tot = ((red[0] + red[1]) + red[2]) + red[3];
  const float inv = 1.0f / tot;
  for (uint32_t i = tid; i < width; i += 256) row[i] = row[i] * inv;
}

__global__ void k_silu(float* out, const float* in, size_t n) {
  for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const float x = in[i];
    out[i] = cx_silu1(x);
  }
}

// -------------------------------------------------------------- argmax
// (value, index) pairs; a beats b if larger, or equal with a lower index.
// NaN entries never win; index 0 wins when v[0] is NaN (strict '>' scan of
// src/sampler.rs:129-137 never leaves index 0 then).
constexpr uint32_t ARG_CHUNK = 4096;

__global__ __launch_bounds__(256) void k_argmax_part(const float* v, uint32_t n, float* pv,
                                                     uint32_t* pi) {
  __shared__ VI red[4];
  const uint32_t b0 = blockIdx.x * ARG_CHUNK, b1 = min(n, b0 + ARG_CHUNK);
  VI best{-INFINITY, 0xFFFFFFFFu};
  for (uint32_t i = b0 + threadIdx.x; i < b1; i += 256) {
    const float x = v[i];
    if (!(x != x)) best = vi_best(best, VI{x, i});
  }
  best = vi_wave(best);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    VI r = vi_best(vi_best(red[0], red[1]), vi_best(red[2], red[3]));
    pv[blockIdx.x] = r.v;
    pi[blockIdx.x] = r.i;
  }
}

// Final reduction. With `st` (the model's token loop), also advances the
// loop: hist[pos+1] = argmax when position pos+1 is past the prompt (and the
// same slot of the pinned host copy hist_host, when given), then pos += 1.
__global__ __launch_bounds__(256) void k_argmax_final(const float* v, const float* pv,
                                                      const uint32_t* pi, uint32_t nparts,
                                                      uint32_t* out, cx_dstate* st,
                                                      uint32_t* hist, uint32_t* hist_host) {
  constexpr uint32_t PPT = 16;  // pairs a thread a round
  __shared__ VI red[4];
  // every load before the first wait: the token state and v[0] (thread 0's
  // tail uses them), then a round's pairs, an index past the end reading
  // the last pair again (a repeated pair leaves the maximum as it is). A
  // loop of one pair a thread waited for each pair in turn.
  float x[PPT];
  uint32_t ix[PPT];
  auto load = [&](uint32_t b) {
#pragma unroll
    for (uint32_t u = 0; u < PPT; u++) {
      const uint32_t i = min(b + threadIdx.x + 256 * u, nparts - 1);
      x[u] = pv[i];
      ix[u] = pi[i];
    }
  };
  load(0);
  uint32_t pos = 0, pend = 0, cap = 0;
  if (st) {
    pos = st->pos;
    pend = st->prompt_end;
    cap = st->cap;
  }
  const float v0 = v[0];
  VI best{-INFINITY, 0xFFFFFFFFu};
  for (uint32_t b = 0;;) {
#pragma unroll
    for (uint32_t u = 0; u < PPT; u++) best = vi_best(best, VI{x[u], ix[u]});
    b += 256 * PPT;
    if (b >= nparts) break;
    load(b);
  }
  best = vi_wave(best);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    VI r = vi_best(vi_best(red[0], red[1]), vi_best(red[2], red[3]));
    uint32_t tok = r.i;
    if (v0 != v0 || tok == 0xFFFFFFFFu) tok = 0;
    if (out) *out = tok;
    if (st) {
      const uint32_t nxt = pos + 1;
      if (nxt >= pend && nxt <= cap) {  // hist has cap+1 slots
        hist[nxt] = tok;
        if (hist_host) hist_host[nxt] = tok;
      }
      st->pos = nxt;
    }
  }
}

// single-workgroup argmax for the operator entry point (no partial buffers)
__global__ __launch_bounds__(1024) void k_argmax_one(const float* v, uint32_t n, uint32_t* out) {
  __shared__ VI red[16];
  VI best{-INFINITY, 0xFFFFFFFFu};
  for (uint32_t i = threadIdx.x; i < n; i += 1024) {
    const float x = v[i];
    if (!(x != x)) best = vi_best(best, VI{x, i});
  }
  best = vi_wave(best);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    VI r = red[0];
    for (int w = 1; w < 16; w++) r = vi_best(r, red[w]);
    const float v0 = v[0];
    *out = (v0 != v0 || r.i == 0xFFFFFFFFu) ? 0u : r.i;
  }
}

// General RoPE for the operator entry point: tokens at positions pos.. .
__global__ __launch_bounds__(256) void k_rope(float* x, uint32_t tokens, uint32_t heads,
                                              uint32_t hd, const float* cos_t,
                                              const float* sin_t, uint32_t pos) {
  const uint32_t half = hd / 2, per_tok = heads * half;
  const size_t total = (size_t)tokens * per_tok;
  for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    const uint32_t t = (uint32_t)(i / per_tok), r = (uint32_t)(i % per_tok);
    const uint32_t h = r / half, j = r % half;
    const float c = cos_t[(size_t)(pos + t) * half + j], s = sin_t[(size_t)(pos + t) * half + j];
    float* lo = x + (size_t)t * heads * hd + h * hd + j;
    const float x0 = lo[0], x1 = lo[half];
    lo[0] = x0 * c - x1 * s;
    lo[half] = x0 * s + x1 * c;
  }
}

}  // namespace

// the token loop's device state, set in stream order
__global__ void k_set_state(cx_dstate* st, uint32_t pos, uint32_t prompt_end, uint32_t cap) {
  if (threadIdx.x == 0) *st = cx_dstate{pos, prompt_end, cap, 0};
}

// ================================================================ launchers
int cx_launch_set_state(cx_dstate* st, uint32_t pos, uint32_t prompt_end, uint32_t cap,
                        hipStream_t s) {
  hipLaunchKernelGGL(k_set_state, dim3(1), dim3(64), 0, s, st, pos, prompt_end, cap);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_argmax_one(const float* v, size_t n, uint32_t* out, hipStream_t s) {
  CX_REQUIRE(v && out && n > 0 && n < 0xFFFFFFFFull, "argmax: bad arguments (n=%zu)", n);
  hipLaunchKernelGGL(k_argmax_one, dim3(1), dim3(1024), 0, s, v, (uint32_t)n, out);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_rope(float* x, size_t tokens, size_t heads, size_t hd, const float* cos_t,
                   const float* sin_t, size_t pos, hipStream_t s) {
  const size_t total = tokens * heads * (hd / 2);
  if (!total) return CX_OK;
  const unsigned grid = (unsigned)((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
  hipLaunchKernelGGL(k_rope, dim3(grid), dim3(256), 0, s, x, (uint32_t)tokens, (uint32_t)heads,
                     (uint32_t)hd, cos_t, sin_t, (uint32_t)pos);
  CX_HIP(hipGetLastError());
  return CX_OK;
}
int cx_launch_embed(int type, const uint8_t* embd, uint32_t dim, const cx_dstate* st,
                    const uint32_t* hist, float* x, uint32_t rows, hipStream_t s) {
  CX_REQUIRE(dim % 8 == 0 && dim % (uint32_t)cx_vpb(type) == 0,
             "embedding: a row of %u values is not whole blocks of type %d", dim, type);
  CX_REQUIRE(rows >= 1, "embedding: no rows");
  const dim3 g(rows), wg(256);
  switch (type) {
    case CX_F32: hipLaunchKernelGGL(k_embed<CX_F32>, g, wg, 0, s, embd, dim, st, hist, x); break;
    case CX_F16: hipLaunchKernelGGL(k_embed<CX_F16>, g, wg, 0, s, embd, dim, st, hist, x); break;
    case CX_Q8_0: hipLaunchKernelGGL(k_embed<CX_Q8_0>, g, wg, 0, s, embd, dim, st, hist, x); break;
    case CX_Q5_0: hipLaunchKernelGGL(k_embed<CX_Q5_0>, g, wg, 0, s, embd, dim, st, hist, x); break;
    case CX_Q2_K: hipLaunchKernelGGL(k_embed<CX_Q2_K>, g, wg, 0, s, embd, dim, st, hist, x); break;
    case CX_Q3_K: hipLaunchKernelGGL(k_embed<CX_Q3_K>, g, wg, 0, s, embd, dim, st, hist, x); break;
    case CX_Q4_K: hipLaunchKernelGGL(k_embed<CX_Q4_K>, g, wg, 0, s, embd, dim, st, hist, x); break;
    case CX_Q5_K: hipLaunchKernelGGL(k_embed<CX_Q5_K>, g, wg, 0, s, embd, dim, st, hist, x); break;
    case CX_Q6_K: hipLaunchKernelGGL(k_embed<CX_Q6_K>, g, wg, 0, s, embd, dim, st, hist, x); break;
    default: cx_set_error("embedding: type %d has no dequantizer", type); return CX_EINVAL;
  }
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_rope_kv(float* q, const float* k, const float* v, float* kc, float* vc,
                      const float* cos_t, const float* sin_t, uint32_t heads, uint32_t kvh,
                      uint32_t hd, const cx_dstate* st, uint32_t rows, hipStream_t s) {
  CX_REQUIRE(rows >= 1, "rope: no rows");
  hipLaunchKernelGGL(k_rope_kv, dim3(rows), dim3(256), 0, s, q, k, v, kc, vc, cos_t, sin_t, heads,
                     kvh, hd, st);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

size_t cx_attn_splits(size_t cap) { return (cap + ATT_P - 1) / ATT_P; }


namespace {
// One query token: the softmax-V kernel with helper-made products, 32 dims
// a workgroup (a ring of RING floats), plus rows of prefetch workgroups.
template <int HD, uint32_t STP, uint32_t NT>
int launch_seq_shape(const cx_attn_args& a, hipStream_t s) {
  const size_t lds = pv_lds_floats(a.cap, STP) * sizeof(float);
  CX_REQUIRE(lds <= 158 * 1024 && (a.cap + SC_P - 1) / SC_P <= CML_MAX,
             "attention: %u cached positions need %zu bytes of LDS", a.cap, lds);
  const uint32_t rows = HD / 32, np = cx_l2_prefetch_groups(a.pf, a.heads * rows);
  const dim3 grid(a.heads, rows + (np + a.heads - 1) / a.heads, 1);
  if (a.sub == 16)
    hipLaunchKernelGGL((k_attn_seq<HD, 16, STP, NT>), grid, dim3(pv_lt(NT)), lds, s, a.vc, a.sc, a.cm,
                       a.heads, a.kvh, a.st, a.cap, a.out, a.xq, a.xe, a.xs, a.pf);
  else
    hipLaunchKernelGGL((k_attn_seq<HD, 32, STP, NT>), grid, dim3(pv_lt(NT)), lds, s, a.vc, a.sc, a.cm,
                       a.heads, a.kvh, a.st, a.cap, a.out, a.xq, a.xe, a.xs, a.pf);
  CX_HIP(hipGetLastError());
  return CX_OK;
}
template <int HD>
int launch_seq_one(const cx_attn_args& a, hipStream_t s) {
  return a.cap <= PV_LONG_CAP ? launch_seq_shape<HD, 128, 320>(a, s)
                              : launch_seq_shape<HD, 256, 576>(a, s);
}

template <int HD>
int launch_exact(const cx_attn_args& a, float scale, hipStream_t s) {
  constexpr size_t sc_bytes = (SC_P * (HD * 4 + 16) + 1023) / 1024 * 1024 + 2 * HD * 4;
  const uint32_t T = a.tokens ? a.tokens : 1;
  if (T > 1) {  // many query tokens: MT_Q a workgroup, f32 output only
    const uint32_t G = (T + MT_Q - 1) / MT_Q;
    constexpr size_t sc_mt = (SC_P * (HD * 4 + 16) + 1023) / 1024 * 1024 + MT_Q * HD * 4;
    hipLaunchKernelGGL(k_attn_scores_mt<HD>, dim3((a.cap + SC_P - 1) / SC_P, a.heads, G),
                       dim3(256), sc_mt, s, a.q, a.kc, a.heads, a.kvh, a.st, scale, a.sc, a.cap, T);
    CX_HIP(hipGetLastError());
    const size_t lds = mt_lds_floats(a.cap) * sizeof(float);
    CX_REQUIRE(lds <= 158 * 1024, "attention: %u cached positions need %zu bytes of LDS", a.cap,
               lds);
    hipLaunchKernelGGL(k_attn_seq_mt<HD>, dim3(a.heads, HD / MT_DS, G), dim3(256), lds, s, a.vc,
                       a.sc, a.heads, a.kvh, a.st, a.cap, T, a.out);
    CX_HIP(hipGetLastError());
    return CX_OK;
  }
  CX_REQUIRE(a.cm, "attention: the chunk maxima buffer");
  hipLaunchKernelGGL(k_attn_scores<HD>, dim3((a.cap + SC_P - 1) / SC_P, a.heads), dim3(256),
                     sc_bytes, s, a.q, a.knew, a.vnew, a.kc, a.vc, a.cos_t, a.sin_t, a.heads,
                     a.kvh, a.st, scale, a.sc, a.cm, a.cap);
  CX_HIP(hipGetLastError());
  return launch_seq_one<HD>(a, s);  // one token: 32 dims a workgroup
}

// One query token over a longer cache: the scores of all heads of a KV group
// from one kernel (cx_attn.hip's k_att_qk, the same sc/cm layout), then the
// same softmax-V kernel with a smaller V ring.
template <int HD>
int launch_long(const cx_attn_args& a, float scale, hipStream_t s) {
  CX_REQUIRE(a.cm, "attention: the chunk maxima buffer");
  int rc = cx_launch_att_scores(a, scale, s);
  if (rc) return rc;
  return launch_seq_one<HD>(a, s);
}
}  // namespace

int cx_launch_attn_decode(const cx_attn_args& a, hipStream_t s) {
  const uint32_t heads = a.heads, kvh = a.kvh, hd = a.hd;
  CX_REQUIRE(kvh && heads % kvh == 0, "attention: %u heads / %u groups", heads, kvh);
  CX_REQUIRE(a.mode != 2 || heads / kvh <= ATT_MAXG,
             "attention: split-K takes at most %d query heads per KV group", ATT_MAXG);
  CX_REQUIRE(hd == 64 || hd == 128, "attention: head_dim %u (64 or 128 supported)", hd);
  CX_REQUIRE(!a.xq || ((a.sub == 16 || a.sub == 32) && a.xe && a.xs),
             "attention: quantized output needs sub 16 or 32");
  CX_REQUIRE(!a.cos_t || (a.knew && a.vnew && a.sin_t), "attention: rope needs the new k/v");
  const uint32_t T = a.tokens ? a.tokens : 1;
  CX_REQUIRE(T == 1 || (!a.cos_t && !a.xq),
             "attention: several query tokens take rotated q and filled caches, f32 output");
  CX_REQUIRE(a.st && T <= 65535, "attention: %u query tokens", T);
  const float scale = 1.0f / sqrtf((float)hd);
  if (a.mode != 2) {
    // two order-exact designs: the cache's scores held in LDS (short
    // caches: fewer, lighter stages), or streamed (any length)
    if (a.cap <= CX_ATT_LDS_MAX && heads / kvh <= ATT_MAXG)
      return hd == 64 ? launch_exact<64>(a, scale, s) : launch_exact<128>(a, scale, s);
    if (T == 1 && a.cap <= CX_ATT_LONG_MAX && heads / kvh <= ATT_MAXG)
      return hd == 64 ? launch_long<64>(a, scale, s) : launch_long<128>(a, scale, s);
    return cx_launch_attn_exact(a, scale, s);
  }
  int rc;
  if (a.cos_t && (rc = cx_launch_rope_kv(a.q, a.knew, a.vnew, a.kc, a.vc, a.cos_t, a.sin_t, heads,
                                         kvh, hd, a.st, 1, s)))
    return rc;
  const uint32_t ns = (uint32_t)cx_attn_splits(a.cap), per = heads / kvh;
  const size_t lds = sizeof(float) * (per * hd + ATT_P * (hd + 1) + per * ATT_P);
  hipLaunchKernelGGL(k_attn_split, dim3(ns, kvh, T), dim3(256), lds, s, a.q, a.kc, a.vc, heads,
                     kvh, hd, a.st, scale, a.pm, a.pl, a.po, ns);
  CX_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_attn_combine, dim3(heads, 1, T), dim3(128), 0, s, a.pm, a.pl, a.po, heads,
                     hd, a.st, a.out, ns);
  CX_HIP(hipGetLastError());
  if (a.xq) return cx_launch_quantize(a.out, 1, (size_t)heads * hd, a.sub, a.xq, a.xe, a.xs, s);
  return CX_OK;
}

int cx_launch_attention(const float* q, const float* k, const float* v, size_t tokens,
                        size_t total, size_t heads, size_t kvh, size_t hd, float* out,
                        hipStream_t s) {
  CX_REQUIRE(kvh && heads % kvh == 0, "attention: %zu heads do not split in %zu groups", heads, kvh);
  CX_REQUIRE(tokens <= total, "attention: %zu new tokens and only %zu in total", tokens, total);
  CX_REQUIRE(total <= CX_ATT_MAX_TOTAL, "attention: total %zu above %d", total, CX_ATT_MAX_TOTAL);
  if (!tokens) return CX_OK;
  const float scale = 1.0f / sqrtf((float)hd);
  hipLaunchKernelGGL(k_attention, dim3((unsigned)heads, (unsigned)tokens), dim3(256),
                     total * sizeof(float), s, q, k, v, (uint32_t)tokens, (uint32_t)total,
                     (uint32_t)heads, (uint32_t)kvh, (uint32_t)hd, scale, out);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_softmax(float* x, size_t len, size_t width, hipStream_t s) {
  CX_REQUIRE(width && len % width == 0, "softmax: %zu values are not rows of %zu", len, width);
  if (!len) return CX_OK;
  hipLaunchKernelGGL(k_softmax, dim3((unsigned)(len / width)), dim3(256), 0, s, x, (uint32_t)width);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_silu(float* out, const float* in, size_t n, hipStream_t s) {
  if (!n) return CX_OK;
  const unsigned grid = (unsigned)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
  hipLaunchKernelGGL(k_silu, dim3(grid), dim3(256), 0, s, out, in, n);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

size_t cx_argmax_parts(size_t n) { return (n + ARG_CHUNK - 1) / ARG_CHUNK; }

// The argmax's second step alone, over nparts pairs another launch wrote
// (the lm_head's epilogue, cx_launch_gemv_argmax)
int cx_launch_argmax_final(const float* v, const float* pv, const uint32_t* pi, uint32_t nparts,
                           uint32_t* out, cx_dstate* st, uint32_t* hist, uint32_t* hist_host,
                           hipStream_t s) {
  CX_REQUIRE(v && pv && pi && nparts > 0, "argmax: bad arguments");
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, v, pv, pi, nparts, out, st, hist,
                     hist_host);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_argmax(const float* v, size_t n, float* pv, uint32_t* pi, uint32_t* out,
                     cx_dstate* st, uint32_t* hist, uint32_t* hist_host, hipStream_t s) {
  CX_REQUIRE(n > 0 && n < 0xFFFFFFFFull, "argmax: length %zu", n);
  const uint32_t parts = (uint32_t)cx_argmax_parts(n);
  hipLaunchKernelGGL(k_argmax_part, dim3(parts), dim3(256), 0, s, v, (uint32_t)n, pv, pi);
  CX_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, v, pv, pi, parts, out, st, hist,
                     hist_host);
  CX_HIP(hipGetLastError());
  return CX_OK;
}
