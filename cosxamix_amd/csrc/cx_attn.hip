// cx_attn.hip — order-exact GQA decode attention for any cache length, gfx950.
//
// ops::atencion at one query token (src/ops.rs:1258-1325), in the
// reference's arithmetic order, bit for bit:
//   s_p    = (sum_i q_i * k_p,i, sequential from 0) * (1 / sqrt(hd))
//   m      = max_p s_p; a non-finite m gives the uniform 1/total
//            (src/ops.rs:1214-1219)
//   e_p    = exp(s_p - m)                     (glibc's expf, cx_expf.h)
//   S      = sum_p e_p, sequential from 0 in position order
//   prob_p = e_p * (1 / S)
//   out_d  = sum_p prob_p * v_p,d, sequential from 0 in position order
//
// k_att_qk, one workgroup per (64 positions, KV group): the chunk's K rows
// go to LDS once for all query heads of the group; lane p of wave w forms
// the sequential dot of position p for heads w, w+4, ...; the scores go to
// `sc` and each head's maximum over the chunk to `cm`. With rope tables it
// also rotates the queries and this step's key, and the workgroup whose
// chunk holds st->pos appends the key and value to the cache.
//
// k_att_sv, one workgroup per (KV group, 32 head dims): two passes over the
// positions, each a pipeline of LDS stages filled by direct-to-LDS loads.
//   pass S: wave 0's lane h runs head h's sum chain while the other waves
//           compute the next stage's exponentials;
//   pass P: lane (h, d) of the chain waves runs out[h][d]'s chain over
//           prob_p * v_p,d while the helper waves compute the next stage's
//           probabilities.
// Every step off the chains (dots, maxima, exponentials, products of the
// probability) runs in parallel; the chains cost ~4 clocks (S) and ~8 (P)
// per position, so the step grows linearly with the cache length.
#include "cx_ops.h"
#include "cx_act.h"

namespace {

constexpr uint32_t QK_P = 64;   // positions per scores workgroup
constexpr uint32_t SV_DS = 32;  // head dims per softmax-V workgroup
constexpr uint32_t S_SP = 256;  // positions per pass-S stage (one KiB per head)
constexpr uint32_t S_PAD = S_SP + 36;  // 292 floats: 36 mod 64 banks apart
constexpr uint32_t P_SP = 256;  // positions per pass-P stage
constexpr uint32_t P_PAD = P_SP + 4;
constexpr uint32_t P_VCH = P_SP * SV_DS * 4 / 1024;  // the stage's V: 1 KiB chunks
constexpr uint32_t NSTS = 6;    // pass-S ring stages
constexpr uint32_t MAXG = 64;   // query heads per KV group

__host__ __device__ constexpr uint32_t sc_stride(uint32_t cap) { return (cap + 3) / 4 * 4; }
__host__ __device__ constexpr uint32_t att_chunks(uint32_t cap) { return (cap + QK_P - 1) / QK_P; }
// pass-P stage: V [P_SP][SV_DS] floats (32 KiB), then the scores [per][P_SP]
// (one KiB a head)
__host__ __device__ constexpr uint32_t p_chunks(uint32_t per) { return P_VCH + per * P_SP / 256; }
__host__ __device__ constexpr uint32_t chain_waves(uint32_t per) { return (per + 1) / 2; }

// s_waitcnt vmcnt(n) for a wave-uniform n: at most n of this wave's vector
// memory operations still outstanding. Exact for every n below 63 (waiting
// for fewer would expose the latency of the loads issued last); vmcnt(63)
// above, which is as strong as the hardware counter allows.
__device__ inline void wait_vm_le(uint32_t n) {
#define CX_W(k) \
  case k:       \
    cx_wait_vm<k>(); \
    break;
  switch (n) {
    CX_W(0) CX_W(1) CX_W(2) CX_W(3) CX_W(4) CX_W(5) CX_W(6) CX_W(7) CX_W(8) CX_W(9) CX_W(10) CX_W(11) CX_W(12) CX_W(13) CX_W(14) CX_W(15) CX_W(16) CX_W(17) CX_W(18) CX_W(19) CX_W(20) CX_W(21) CX_W(22) CX_W(23) CX_W(24) CX_W(25) CX_W(26) CX_W(27) CX_W(28) CX_W(29) CX_W(30) CX_W(31) CX_W(32) CX_W(33) CX_W(34) CX_W(35) CX_W(36) CX_W(37) CX_W(38) CX_W(39) CX_W(40) CX_W(41) CX_W(42) CX_W(43) CX_W(44) CX_W(45) CX_W(46) CX_W(47) CX_W(48) CX_W(49) CX_W(50) CX_W(51) CX_W(52) CX_W(53) CX_W(54) CX_W(55) CX_W(56) CX_W(57) CX_W(58) CX_W(59) CX_W(60) CX_W(61) CX_W(62)
    default:
      cx_wait_vm<63>();
  }
#undef CX_W
}

// ------------------------------------------------------------- scores
template <int HD>
__global__ __launch_bounds__(256) void k_att_qk(const float* q, const float* knew,
                                                const float* vnew, float* kc, float* vc,
                                                const float* cos_t, const float* sin_t,
                                                uint32_t kvh, uint32_t per, const cx_dstate* st,
                                                float scale, float* sc, float* cm, uint32_t cap) {
  constexpr uint32_t ROWB = HD * 4, PADB = ROWB + 16, PADF = PADB / 4;
  constexpr uint32_t NCH = (QK_P * PADB + 1023) / 1024;
  constexpr uint32_t half = HD / 2;
  extern __shared__ __align__(16) uint8_t sm[];
  float* kl = reinterpret_cast<float*>(sm);                // QK_P rows of PADF floats
  float* qr = reinterpret_cast<float*>(sm + NCH * 1024);   // per x HD queries
  float* kr = qr + per * HD;                               // this step's key, rotated
  // query token z (blockIdx.z) sits at position st->pos + z
  const uint32_t z = blockIdx.z, pos = st->pos + z, total = pos + 1;
  const uint32_t c = blockIdx.x, p0 = c * QK_P, g = blockIdx.y;
  if (p0 >= total) return;
  const uint32_t np = min(QK_P, total - p0), kvd = kvh * HD, heads = kvh * per;
  const uint32_t stride = sc_stride(cap), nck = att_chunks(cap);
  q += ((size_t)z * heads + (size_t)g * per) * HD;
  sc += ((size_t)z * heads + (size_t)g * per) * stride;
  cm += ((size_t)z * heads + (size_t)g * per) * nck;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // 1. the chunk's K rows into LDS (padded by 16 bytes); pad bytes and rows
  //    past the end load a valid dummy that is never read
  const float* kb = kc + (size_t)p0 * kvd + g * HD;
  for (uint32_t ch = wave; ch < NCH; ch += 4) {
    const uint32_t o = ch * 1024 + 16 * lane;
    uint32_t r = o / PADB, b = o % PADB;
    if (r >= np || b >= ROWB) r = 0, b = 0;
    cx_dma16(reinterpret_cast<const uint8_t*>(kb + (size_t)r * kvd) + b, sm + ch * 1024);
  }
  // 2. rope while the rows arrive (src/ops.rs:1185-1188: a' = a*c - b*s,
  //    b' = a*s + b*c, no FMA); the chunk holding st->pos scores that
  //    position with the rotated key from LDS and appends the key and value
  //    at the end (src/forward.rs:454-455), so no result depends on a row
  //    written here
  //    Every load is issued before the first wait: the queries, the
  //    tables, this step's key (with query head 0's pairs: j < half) and
  //    the value the append stores in step 4 (each a round trip of its own
  //    after the others when loaded where used).
  const bool rot = cos_t != nullptr, has_new = rot && pos < p0 + QK_P;
  float vv = 0.0f;
  if (has_new && (uint32_t)tid < (uint32_t)HD) vv = vnew[(size_t)z * kvd + g * HD + tid];
  if (rot) {
    const float* cc = cos_t + (size_t)pos * half;
    const float* ss = sin_t + (size_t)pos * half;
    const float* kn = knew + (size_t)z * kvd + g * HD;
    for (uint32_t i = tid; i < per * half; i += 256) {
      const uint32_t hl = i / half, j = i % half;
      const bool key = has_new && i < half;
      float x0 = q[hl * HD + j], x1 = q[hl * HD + j + half];
      float cj = cc[j], sj = ss[j], k0 = 0.0f, k1 = 0.0f;
      if (key) k0 = kn[j], k1 = kn[j + half];
      asm volatile("" : "+v"(x0), "+v"(x1), "+v"(cj), "+v"(sj), "+v"(k0), "+v"(k1));
      qr[hl * HD + j] = x0 * cj - x1 * sj;
      qr[hl * HD + j + half] = x0 * sj + x1 * cj;
      if (key) {
        const float a = k0 * cj - k1 * sj, b = k0 * sj + k1 * cj;
        kr[j] = a;
        kr[j + half] = b;
      }
    }
  } else {
    for (uint32_t i = tid; i < per * HD; i += 256) qr[i] = q[i];
  }
  cx_wait_vm<0>();
  __syncthreads();
  // 3. lane p of wave w: position p0 + p of heads w, w + 4, ...; the
  //    sequential dot of src/kernels/scalar.rs:16-23, then the chunk maximum
  const uint32_t p = lane;
  const float4* b4 = reinterpret_cast<const float4*>((has_new && p0 + p == pos) ? kr : kl + p * PADF);
  for (uint32_t hl = wave; hl < per; hl += 4) {
    float s = -INFINITY;
    if (p < np) {
      const float4* a4 = reinterpret_cast<const float4*>(qr + hl * HD);
      s = cx_dot_seq<HD / 4>(a4, b4) * scale;
      sc[(size_t)hl * stride + p0 + p] = s;
    }
    const float m = cx_wave_max(s);
    if (lane == 0) cm[(size_t)hl * nck + c] = m;
  }
  // 4. the appended key (rotated, from LDS) and value: stored after the
  //    dots, since a wave waits for its stores as for its loads
  if (has_new && (uint32_t)tid < (uint32_t)HD) {
    float* kd = kc + (size_t)pos * kvd + g * HD;
    float* vd = vc + (size_t)pos * kvd + g * HD;
    kd[tid] = kr[tid];
    vd[tid] = vv;
  }
}

// ----------------------------------------------- softmax sums and PV chains
// A workgroup takes up to HB query heads of one KV group (nh of them) and
// SV_DS head dims: ceil(nh / 2) chain waves (32 lanes per head) and twice as
// many helper waves. LDS: the pass-P ring (nstp stages of p_chunks(nh) KiB) and
// the probabilities; pass S's ring and exponentials alias the ring's last
// slots, so only its first `ka` stages can be filled while pass S runs.
constexpr uint32_t HB = 8;  // query heads per workgroup
struct SvLayout {
  uint32_t nstp, ka;
  uint32_t ring_p, pbuf, ring_s, ebuf, bytes;
};
constexpr uint32_t LDS_BUDGET = 158 * 1024;  // dynamic LDS, below the CU's 160 KiB
constexpr uint32_t NSTP_MAX = 12;
__host__ __device__ inline SvLayout sv_layout(uint32_t nh) {
  SvLayout L;
  const uint32_t pch = p_chunks(nh), nhp = 2 * chain_waves(nh);
  const uint32_t lp_max = (pch + nhp - 1) / nhp;  // pass-P loads per helper wave per stage
  const uint32_t s_bytes = NSTS * nh * 1024 + 2 * nh * S_PAD * 4;  // pass S's region
  const uint32_t pb_bytes = 2 * nh * P_PAD * 4;
  uint32_t n = (LDS_BUDGET - pb_bytes) / (pch * 1024);
  n = n < NSTP_MAX ? n : NSTP_MAX;
  const uint32_t vm = 56 / lp_max;  // loads in flight per wave stay below vmcnt's 63
  n = n < vm ? n : vm;
  L.nstp = n;
  L.ring_p = 0;
  L.pbuf = n * pch * 1024;
  const uint32_t ring_bytes = L.pbuf, end_p = L.pbuf + pb_bytes;
  if (ring_bytes >= s_bytes) {  // pass S at the end of the ring
    const uint32_t s_at = (ring_bytes - s_bytes) / 1024 * 1024;
    L.ka = s_at / (pch * 1024);
    L.ring_s = s_at;
    L.bytes = end_p;
  } else {  // past the probabilities
    L.ka = n;
    L.ring_s = end_p;
    L.bytes = end_p + s_bytes;
  }
  L.ebuf = L.ring_s + NSTS * nh * 1024;
  return L;
}

// tot += x[0] + ... + x[n) in order, n a multiple of 32; the reads of the
// next 32 values are issued before the adds of the current 32
__device__ inline void add32(float& tot, const float4 (&a)[8]) {
#pragma unroll
  for (int i = 0; i < 8; i++) {
    tot += a[i].x;
    tot += a[i].y;
    tot += a[i].z;
    tot += a[i].w;
  }
}
__device__ inline void seq_add(float& tot, const float* x, uint32_t n) {
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float4 A[8], B[8];
#pragma unroll
  for (int i = 0; i < 8; i++) A[i] = x4[i];
  for (uint32_t b = 0; b < n / 4; b += 16) {
    const bool more = b + 8 < n / 4;
#pragma unroll
    for (int i = 0; i < 8; i++) B[i] = more ? x4[b + 8 + i] : A[i];
    add32(tot, A);
    if (!more) break;
    const bool more2 = b + 16 < n / 4;
#pragma unroll
    for (int i = 0; i < 8; i++) A[i] = more2 ? x4[b + 16 + i] : B[i];
    add32(tot, B);
    if (!more2) break;
  }
}

// o += p[j] * v[j] for 8 positions in order: the 8 products are formed first
// (pinned before the adds), so the chain waits on one add per position
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
// a stage of 64 positions in batches of 16, the next batch's reads issued
// before the current batch's arithmetic
struct PvBatch {
  float v[16];
  float4 p[4];
};
__device__ inline void pv_load(PvBatch& b, const float4* p4, const float* vs, uint32_t j0) {
#pragma unroll
  for (int j = 0; j < 16; j++) b.v[j] = vs[(j0 + j) * SV_DS];
#pragma unroll
  for (int i = 0; i < 4; i++) b.p[i] = p4[j0 / 4 + i];
}
__device__ inline void pv_apply(float& o, const PvBatch& b) {
  const float4 p0[2] = {b.p[0], b.p[1]}, p1[2] = {b.p[2], b.p[3]};
  const float v0[8] = {b.v[0], b.v[1], b.v[2], b.v[3], b.v[4], b.v[5], b.v[6], b.v[7]};
  const float v1[8] = {b.v[8], b.v[9], b.v[10], b.v[11], b.v[12], b.v[13], b.v[14], b.v[15]};
  pv8(o, p0, v0);
  pv8(o, p1, v1);
}
__device__ inline void pv_stage64(float& o, const float* pb, const float* vs) {
  const float4* p4 = reinterpret_cast<const float4*>(pb);
  PvBatch a, b;
  pv_load(a, p4, vs, 0);
  pv_load(b, p4, vs, 16);
  pv_apply(o, a);
  pv_load(a, p4, vs, 32);
  pv_apply(o, b);
  pv_load(b, p4, vs, 48);
  pv_apply(o, a);
  pv_apply(o, b);
}

// four exponentials exp(x - m), independent, in flight together
__device__ inline float4 exp4(float4 x, float m, const uint64_t* etab) {
  return make_float4(cx_expf_tab(x.x - m, etab), cx_expf_tab(x.y - m, etab),
                     cx_expf_tab(x.z - m, etab), cx_expf_tab(x.w - m, etab));
}

template <int SUB>
__global__ __launch_bounds__(768) void k_att_sv(const float* vc, const float* sc, const float* cm,
                                                uint32_t kvh, uint32_t per, uint32_t hd,
                                                const cx_dstate* st, uint32_t cap, float* out,
                                                int8_t* xq, float* xe, float* xs) {
  extern __shared__ __align__(16) uint8_t sm[];
  __shared__ uint64_t etab[32];
  __shared__ float Ms[HB], invs[HB];
  __shared__ int unif[HB];
  // workgroup (g * nhb + hb, y, z): heads hb*HB .. + nh of KV group g,
  // dims d0 .. d0 + SV_DS, query token z at position st->pos + z
  const uint32_t nhb = (per + HB - 1) / HB, g = blockIdx.x / nhb, hb = blockIdx.x % nhb;
  const uint32_t nh = min(HB, per - hb * HB), h0 = g * per + hb * HB;
  const SvLayout LY = sv_layout(nh);
  float* ring_s = reinterpret_cast<float*>(sm + LY.ring_s);
  float* ebuf = reinterpret_cast<float*>(sm + LY.ebuf);
  float* ring_p = reinterpret_cast<float*>(sm + LY.ring_p);
  float* pbuf = reinterpret_cast<float*>(sm + LY.pbuf);
  const uint32_t ncw = chain_waves(nh), nhp = 2 * ncw, nw = ncw + nhp, pch = p_chunks(nh);
  const uint32_t nstp = LY.nstp;
  const uint32_t z = blockIdx.z, total = st->pos + z + 1;
  const uint32_t d0 = blockIdx.y * SV_DS, kvd = kvh * hd, heads = kvh * per;
  const uint32_t stride = sc_stride(cap), nck = att_chunks(cap), nc = (total + QK_P - 1) / QK_P;
  sc += ((size_t)z * heads + h0) * stride;
  cm += ((size_t)z * heads + h0) * nck;
  out += ((size_t)z * heads + h0) * hd + d0;
  const float* vb = vc + g * hd + d0;
  const int tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t nss = (total + S_SP - 1) / S_SP, nsp = (total + P_SP - 1) / P_SP;
  // a workgroup of fewer heads than the launch's largest leaves waves
  // nw.. idle: they only take part in the barriers
  const bool active = wave < nw;

  // Loads are issued by helper waves only, so the chains never wait on an
  // issue. Pass S: chunk h (head h's 256 positions) by wave 1 + h % (nw - 1);
  // pass P: chunk ch of the stage by wave ncw + ch % nhp.
  const uint32_t nhw = nw - 1;
  const uint32_t ls = active && wave >= 1 && wave - 1 < nh ? (nh - 1 - (wave - 1)) / nhw + 1 : 0;
  const uint32_t lp =
      active && wave >= ncw && wave - ncw < pch ? (pch - 1 - (wave - ncw)) / nhp + 1 : 0;
  uint32_t issued = 0;
  auto issue_s = [&](uint32_t s) {
    if (wave == 0 || !active) return;
    for (uint32_t h = wave - 1; h < nh; h += nhw) {
      const uint32_t p = s * S_SP + 4 * lane;
      cx_dma16_async(sc + (size_t)h * stride + (p < total ? p : 0),
                     ring_s + ((s % NSTS) * nh + h) * 256);
      issued++;
    }
  };
  auto issue_p = [&](uint32_t s) {
    if (wave < ncw || !active) return;
    float* base = ring_p + (s % nstp) * pch * 256;
    for (uint32_t ch = wave - ncw; ch < pch; ch += nhp) {
      const uint32_t j = ch * 64 + lane;  // 16-byte slot of the stage
      const float* src = sc;              // dummy: any valid address
      if (ch < P_VCH) {                   // V[p][0..32) of 8 positions per chunk
        const uint32_t p = s * P_SP + j / 8;
        if (p < total) src = vb + (size_t)p * kvd + 4 * (j % 8);
      } else {                            // scores[h][p]
        const uint32_t k = j - P_VCH * 64, h = k / (P_SP / 4), p = s * P_SP + 4 * (k % (P_SP / 4));
        if (h < nh && p < total) src = sc + (size_t)h * stride + p;
      }
      cx_dma16_async(src, base + ch * 256);
      issued++;
    }
  };
  // Issue order: pass S's first stages; pass P's first ka stages; pass S's
  // later stages (its loop, stage s at iteration s - NSTS + 1); pass P's
  // stages ka..nstp-1 (after pass S); pass P's later stages (its loop, stage
  // s at iteration s - nstp + 2). done_*(s): this wave's load count once the
  // loads of that stage were issued.
  const uint32_t as = min(NSTS, nss), ap = min(nstp, nsp), pa = min(LY.ka, ap);
  const uint32_t more_s = nss > NSTS ? nss - NSTS : 0;
  auto done_s = [&](uint32_t s) {
    return s < as ? (s + 1) * ls : as * ls + pa * lp + (s - NSTS + 1) * ls;
  };
  auto done_p = [&](uint32_t s) {
    return s < pa   ? as * ls + (s + 1) * lp
           : s < ap ? as * ls + pa * lp + more_s * ls + (s - pa + 1) * lp
                    : as * ls + ap * lp + more_s * ls + (s - nstp + 1) * lp;
  };

  // 1. pass S's first stages; each head's maximum from the chunk maxima
  //    (fmaxf from -inf, as over the scores themselves: the compiler's wait
  //    for these plain loads also waits for the stages before them); then
  //    the pass-P stages that do not share LDS with pass S
  for (uint32_t s = 0; s < as; s++) issue_s(s);
  if (tid == 0) {
    const uint64_t tab[32] = CX_EXP2_TAB;
    for (int i = 0; i < 32; i++) etab[i] = tab[i];
  }
  for (uint32_t h = wave; h < nh; h += nw) {
    float m = -INFINITY;
    for (uint32_t c = lane; c < nc; c += 64) m = fmaxf(m, cm[(size_t)h * nck + c]);
    m = cx_wave_max(m);
    if (lane == 0) {
      Ms[h] = m;
      unif[h] = !isfinite(m);
    }
  }
  for (uint32_t s = 0; s < pa; s++) issue_p(s);

  // 2. pass S: wave 0's lane h sums head h's exponentials in position order
  //    while waves 1.. compute the next stage's, four positions a lane. Past
  //    the end of the cache a stage holds +0.0 exponentials: adding them
  //    leaves the sum's bits as they are, so the chain runs whole stages.
  float tot = 0.0f;
  const bool sum_lane = wave == 0 && (uint32_t)lane < nh;
  for (uint32_t s = 0; s <= nss; s++) {
    if (s < nss) wait_vm_le(issued - done_s(s));
    cx_wait_lds();
    cx_barrier();  // stage s in LDS; the exponentials of stage s - 1 written
    // refill the slot the helpers read in the last iteration (so the issue
    // runs beside the chain instead of between its stages)
    if (s >= 1 && s - 1 + NSTS < nss) issue_s(s - 1 + NSTS);
    if (wave > 0 && active && s < nss) {
      const float* rs = ring_s + (s % NSTS) * nh * 256;
      float* eb = ebuf + (s & 1) * nh * S_PAD;
      for (uint32_t G = tid - 64; G < nh * (S_SP / 4); G += 64 * nhw) {
        const uint32_t h = G / (S_SP / 4), p = 4 * (G % (S_SP / 4)), P = s * S_SP + p;
        float4 e = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (P < total && !unif[h]) {
          e = exp4(*reinterpret_cast<const float4*>(rs + h * 256 + p), Ms[h], etab);
          if (P + 3 >= total) {  // the cache ends inside these four
            if (P + 1 >= total) e.y = 0.0f;
            if (P + 2 >= total) e.z = 0.0f;
            e.w = 0.0f;
          }
        }
        *reinterpret_cast<float4*>(eb + h * S_PAD + p) = e;
      }
    }
    if (sum_lane && s >= 1) seq_add(tot, ebuf + ((s - 1) & 1) * nh * S_PAD + lane * S_PAD, S_SP);
    cx_wait_lds();
    cx_barrier();  // slot s % NSTS and the exponentials of stage s - 1 read
  }
  if (sum_lane) invs[lane] = 1.0f / tot;
  for (uint32_t s = pa; s < ap; s++) issue_p(s);  // pass S's LDS is free
  cx_wait_lds();
  cx_barrier();

  // 3. pass P: lane (h, d) of waves 0..ncw-1 accumulates prob_p * v_p,d in
  //    position order while the other waves compute the next stage's
  //    probabilities prob_p = exp(s_p - m) * (1/S) (uniform: 1/total)
  const uint32_t hl = tid / SV_DS, dd = tid % SV_DS;
  const bool chain = wave < ncw && hl < nh;
  float o = 0.0f;
  const float u = 1.0f / (float)total;
  for (uint32_t s = 0; s <= nsp; s++) {
    if (s < nsp) wait_vm_le(issued - done_p(s));
    cx_wait_lds();
    cx_barrier();  // stage s in LDS; the probabilities of stage s - 1 written
    // refill the slot the chains read in the last iteration
    if (s >= 2 && s - 2 + nstp < nsp) issue_p(s - 2 + nstp);
    if (wave >= ncw && active && s < nsp) {
      const float* rs = ring_p + (s % nstp) * pch * 256 + P_VCH * 256;
      float* pb = pbuf + (s & 1) * nh * P_PAD;
      // the stage's probabilities over the helper lanes (up to four a lane)
      for (uint32_t i = tid - 64 * ncw; i < nh * P_SP; i += 64 * nhp) {
        const uint32_t h = i / P_SP, p = i % P_SP;
        float pr = 0.0f;
        if (s * P_SP + p < total)
          pr = unif[h] ? u : cx_expf_tab(rs[h * P_SP + p] - Ms[h], etab) * invs[h];
        pb[h * P_PAD + p] = pr;
      }
    }
    if (chain && s >= 1) {
      const float* pb = pbuf + ((s - 1) & 1) * nh * P_PAD + hl * P_PAD;
      const float* vs = ring_p + ((s - 1) % nstp) * pch * 256 + dd;
      const uint32_t n = min(P_SP, total - (s - 1) * P_SP);
      if (n == P_SP) {
#pragma unroll 1
        for (uint32_t b = 0; b < P_SP; b += 64) pv_stage64(o, pb + b, vs + b * SV_DS);
      } else {
        for (uint32_t p = 0; p < n; p++) o += pb[p] * vs[p * SV_DS];
      }
    }
    cx_wait_lds();
    cx_barrier();  // slot (s - 1) % nstp and the probabilities of stage s - 1 read
  }

  // 4. the output, and its quantization for the output projection (SUB
  //    consecutive dims of one head are whole sub-blocks of this slice)
  if (chain) out[(size_t)hl * hd + dd] = o;
  if (!xq) return;
  float* os = pbuf;  // every read of it is done
  if (chain) os[tid] = o;
  cx_wait_lds();
  __syncthreads();
  if ((uint32_t)tid < nh * SV_DS / 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = os[8 * tid + j];
    const uint32_t h = 8 * tid / SV_DS, d = 8 * tid % SV_DS;
    cx_quant8<SUB>(v, ((size_t)h0 + h) * hd + d0 + d, xq, xe, xs);
  }
}

}  // namespace

size_t cx_attn_chunk_floats(size_t heads, size_t cap) { return heads * att_chunks((uint32_t)cap); }

int cx_launch_att_scores(const cx_attn_args& a, float scale, hipStream_t s) {
  const uint32_t per = a.heads / a.kvh, T = a.tokens ? a.tokens : 1;
  CX_REQUIRE(per >= 1 && per <= MAXG, "attention: %u query heads per KV group (at most %u)", per,
             MAXG);  // k_att_qk keeps a group's queries in LDS
  CX_REQUIRE(a.hd % SV_DS == 0 && (a.hd == 64 || a.hd == 128), "attention: head_dim %u", a.hd);
  CX_REQUIRE(a.sc && a.cm, "attention: scores and chunk maxima buffers");
  CX_REQUIRE(((uintptr_t)a.sc & 15) == 0, "attention: the scores must be 16-byte aligned");
  const size_t qk_lds = (QK_P * (a.hd * 4 + 16) + 1023) / 1024 * 1024 + (per + 1) * a.hd * 4;
  const dim3 qk_grid(att_chunks(a.cap), a.kvh, T);
  if (a.hd == 64)
    hipLaunchKernelGGL(k_att_qk<64>, qk_grid, dim3(256), qk_lds, s, a.q, a.knew, a.vnew, a.kc,
                       a.vc, a.cos_t, a.sin_t, a.kvh, per, a.st, scale, a.sc, a.cm, a.cap);
  else
    hipLaunchKernelGGL(k_att_qk<128>, qk_grid, dim3(256), qk_lds, s, a.q, a.knew, a.vnew, a.kc,
                       a.vc, a.cos_t, a.sin_t, a.kvh, per, a.st, scale, a.sc, a.cm, a.cap);
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_attn_exact(const cx_attn_args& a, float scale, hipStream_t s) {
  const uint32_t per = a.heads / a.kvh, T = a.tokens ? a.tokens : 1;
  int rc = cx_launch_att_scores(a, scale, s);
  if (rc) return rc;
  const uint32_t nhb = (per + HB - 1) / HB, nh = per < HB ? per : HB;
  const SvLayout LY = sv_layout(nh);  // the largest workgroup's
  CX_REQUIRE(LY.nstp >= 3 && LY.bytes <= LDS_BUDGET,
             "attention: %u heads per workgroup need %u bytes of LDS", nh, LY.bytes);
  const dim3 sv_grid(a.kvh * nhb, a.hd / SV_DS, T), sv_wg(192 * chain_waves(nh));
  if (a.xq && a.sub == 16)
    hipLaunchKernelGGL(k_att_sv<16>, sv_grid, sv_wg, LY.bytes, s, a.vc, a.sc, a.cm, a.kvh, per,
                       a.hd, a.st, a.cap, a.out, a.xq, a.xe, a.xs);
  else
    hipLaunchKernelGGL(k_att_sv<32>, sv_grid, sv_wg, LY.bytes, s, a.vc, a.sc, a.cm, a.kvh, per,
                       a.hd, a.st, a.cap, a.out, a.xq, a.xe, a.xs);
  CX_HIP(hipGetLastError());
  return CX_OK;
}
