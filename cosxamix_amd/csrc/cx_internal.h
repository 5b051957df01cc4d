// cx_internal.h — launch-level interfaces shared between translation units.
#pragma once

#include <cstdio>
#include <string>
#include <vector>

#include "cx_common.h"

// An L2 prefetch run by extra workgroups of a launch that leaves most CUs
// and most of HBM's bandwidth idle (the one-token attention). Job i reads
// `tiles` tiles of `tile` bytes of p0 (and of p1 if set), tile t on XCD
// t % 8, where the next launches' workgroup t reads it (workgroups go to
// XCDs by index, round robin); a job with no tiles is skipped.
struct cx_l2_job {
  const uint8_t *p0, *p1;
  size_t bytes;  // of each of p0, p1
  uint32_t tile, tiles;
};
constexpr int CX_L2_JOBS = 7;
struct cx_l2_prefetch {
  cx_l2_job job[CX_L2_JOBS];
};

// Reads bytes [o, o + len) of p0 and of p1 (either may be null; clipped to
// total), 16-byte loads, sixteen in flight per lane over both ranges (a
// gate/up tile's two halves are one round trip); the values feed an empty
// asm statement, which keeps the loads and stores nothing.
__device__ inline void cx_l2_touch(const uint8_t* p0, const uint8_t* p1, size_t o, uint32_t len,
                                   size_t total) {
  if (o >= total) return;
  const uint32_t n = (uint32_t)(((o + len < total ? o + len : total) - o) / 16);  // chunks per range
  const uint32_t n0 = p0 ? n : 0, nt = n0 + (p1 ? n : 0);
  uint32_t acc = 0;
  for (uint32_t c0 = threadIdx.x; c0 < nt; c0 += 16 * blockDim.x) {
    uint4 v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const uint32_t c = c0 + (uint32_t)j * blockDim.x;
      v[j] = uint4{0, 0, 0, 0};
      if (c < nt)
        v[j] = *reinterpret_cast<const uint4*>((c < n0 ? p0 + o + 16 * (size_t)c
                                                        : p1 + o + 16 * (size_t)(c - n0)));
    }
#pragma unroll
    for (int j = 0; j < 16; j++) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  asm volatile("" : : "v"(acc));
}

// Prefetch workgroup j of a launch whose first `first` workgroups (in
// dispatch order) do other work: skips to the next multiple of 8 so that
// tile t runs on XCD t % 8, then the jobs' tiles in order, each job from a
// multiple of 8.
__device__ inline void cx_l2_prefetch_run(const cx_l2_prefetch& pf, uint32_t j, uint32_t first) {
  const uint32_t skip = (8 - first % 8) % 8;
  if (j < skip) return;
  uint32_t t = j - skip;
  for (int i = 0; i < CX_L2_JOBS; i++) {
    const cx_l2_job& b = pf.job[i];
    if (t < b.tiles) {
      cx_l2_touch(b.p0, b.p1, (size_t)t * b.tile, b.tile, b.bytes);
      return;
    }
    t -= (b.tiles + 7) / 8 * 8;
  }
}

// The workgroups a prefetch adds to a launch of `first` workgroups
inline uint32_t cx_l2_prefetch_groups(const cx_l2_prefetch& pf, uint32_t first) {
  uint32_t n = 0;
  for (int i = 0; i < CX_L2_JOBS; i++) n += (pf.job[i].tiles + 7) / 8 * 8;
  return n ? (8 - first % 8) % 8 + n : 0;
}

// One matrix of a (possibly multi-matrix) GEMV launch. All segments of one
// launch share the activation, the row width k and the weight type.
struct cx_seg {
  const uint8_t* w;     // rows x row_bytes, GGUF raw
  float* y;             // rows
  const float* bias;    // rows or nullptr (Qwen2 q/k/v bias, src/forward.rs:360-366)
  uint32_t rows;
};

// The i8 activation of a GEMV (ops::cuantizar_i8_en, src/ops.rs:178-198,
// with the per-sub-block sums of src/ops.rs:472-483): xq[k] (16-byte
// aligned), xe[k/sub], xs[k/sub] in device memory.
struct cx_qact {
  const int8_t* xq;
  const float* xe;
  const float* xs;
};

enum cx_epi { CX_EPI_STORE = 0, CX_EPI_ACCUM = 1 };

// GEMV over `nseg` segments: seg[i].y[r] (=|+=) row r of seg[i].w . act.
// `dbg` (single segment only) receives the integer sub-block sums.
int cx_launch_gemv(int type, const cx_seg* segs, int nseg, uint32_t k, const cx_qact& act,
                   int epi, int32_t* dbg, hipStream_t s);
// The lm_head with the argmax's first step in its epilogue: the per-tile
// (largest output, row) pairs in apv/api, *nparts of them (0, and nothing
// launched, where the row kernel does not take the matrix).
uint32_t cx_gemv_argmax_parts(int type, uint32_t n, uint32_t k);
int cx_launch_gemv_argmax(int type, const cx_seg& seg, uint32_t k, const cx_qact& act, float* apv,
                          uint32_t* api, uint32_t* nparts, hipStream_t s);
// The same GEMV with its activation made by every workgroup from f32 x:
// rmsnorm(x, w, eps) (kernels/mod.rs:511) then quantization (ops.rs:178), in
// the shadow of the weight loads. For launches of a few hundred workgroups;
// x and w are 16-byte aligned.
int cx_launch_gemv_norm(int type, const cx_seg* segs, int nseg, uint32_t k, const float* x,
                        const float* w, float eps, int epi, hipStream_t s);

// The decode step's gate/up projections and SwiGLU in one launch
// (src/forward.rs:472-487) for gate and up of one type at row width k
// (cx_glu_fits): rmsnorm(x, w) quantized per workgroup, gate and up rows
// [32t, 32t+32) in workgroup t, then silu(gate) * up quantized in sub-blocks
// of `sub` (the down projection's) into xq/xe/xs. Bit-identical to
// cx_launch_gemv_norm over gate and up followed by cx_launch_swiglu_quant.
// I % 32 == 0. cx_glu_supported: the k-quant types (Q4_K, Q5_K), whose
// tiles the attention's L2 prefetch also knows; cx_glu_fits adds Q8_0 and
// Q5_0 where both 32-row tiles fit in LDS.
bool cx_glu_supported(int type);
bool cx_glu_fits(int type, uint32_t k);
int cx_launch_gemv_glu(int type, const uint8_t* wg, const uint8_t* wu, uint32_t I, uint32_t k,
                       const float* x, const float* w, float eps, int sub, int8_t* xq, float* xe,
                       float* xs, hipStream_t s);

// A prefetch job of the tiles of the plain GEMV of w (n x k; Q4_K, Q5_K,
// Q8_0, Q5_0) or of the gate/up launch of wg and wu (I x k), each into the
// L2 it is read from; false (and no job) where the launch has no such
// tiling.
bool cx_gemv_prefetch_plan(int type, const uint8_t* w, uint32_t n, uint32_t k, cx_l2_job* job);
bool cx_glu_prefetch_plan(int type, const uint8_t* wg, const uint8_t* wu, uint32_t I, uint32_t k,
                          cx_l2_job* job);

// Producers of the i8 activation, one value per lane:
//   quantize   : rows x k values of x                           (ops.rs:178)
//   swiglu     : silu(g) * u, n values                          (forward.rs:483-487)
//   norm       : rmsnorm(x, w, eps) of one row of n values     (kernels/mod.rs:511)
int cx_launch_quantize(const float* x, size_t rows, size_t k, int sub, int8_t* xq, float* xe,
                       float* xs, hipStream_t s);
int cx_launch_swiglu_quant(const float* g, const float* u, size_t n, int sub, int8_t* xq,
                           float* xe, float* xs, hipStream_t s);
int cx_launch_norm_quant(const float* x, const float* w, size_t n, float eps, int sub,
                         int8_t* xq, float* xe, float* xs, hipStream_t s);
int cx_launch_rmsnorm(float* out, const float* in, const float* w, size_t rows, size_t n,
                      float eps, hipStream_t s);
// Row forms of the decode step's ops, for the batched prefill: rmsnorm of
// rows in the fused GEMV prologue's f64 tree (bit-identical to it); SwiGLU;
// y[r] += a[r % a_rows] (residual: a_rows = rows; bias: a_rows = 1)
int cx_launch_norm_rows(const float* x, const float* w, size_t rows, size_t k, float eps,
                        float* out, hipStream_t s);
int cx_launch_swiglu_rows(const float* g, const float* u, size_t n, float* out, hipStream_t s);
int cx_launch_add_rows(float* y, const float* a, size_t rows, size_t n, size_t a_rows,
                       hipStream_t s);

// m activation rows at once on int8 MFMA (every GEMV type): lhs[m][k] f32
// is quantized into `scratch` (cx_gemm_scratch_bytes, 256-byte aligned),
// then dst[m][n] is formed, every value bit-identical to the per-row GEMV.
bool cx_gemm_supported(int type);
size_t cx_gemm_scratch_bytes(size_t m, size_t k);
int cx_launch_gemm(int type, const uint8_t* w, size_t n, size_t k, const float* lhs, size_t m,
                   float* dst, void* scratch, hipStream_t s);
// The same in two steps, for several matrices over one activation: quantize
// lhs once into scratch in sub-blocks of `sub` (cx_sub of the types to come),
// then contract any number of matrices of width k and that sub-block size
// against it (scratch of cx_gemm_scratch_bytes(m, k)).
int cx_gemm_quantize(const float* lhs, size_t m, size_t k, int sub, void* scratch, hipStream_t s);
// cx_gemm_quantize of rmsnorm(x) * w (cx_launch_norm_rows' values), and of
// silu(g) * u (cx_launch_swiglu_rows'), without the f32 rows in between
int cx_gemm_norm_quantize(const float* x, const float* w, size_t m, size_t k, float eps, int sub,
                          void* scratch, hipStream_t s);
int cx_gemm_swiglu_quantize(const float* g, const float* u, size_t m, size_t k, int sub,
                            void* scratch, hipStream_t s);
int cx_gemm_apply(int type, const uint8_t* w, size_t n, size_t k, size_t m, float* dst,
                  const void* scratch, hipStream_t s);
// cx_gemm_apply of `count` matrices of one type and width k (up to
// CX_GEMM_SEGS: q/k/v, gate/up) in one launch, matrix i (n[i] rows, weights
// w[i]) into dst[i] (m x n[i]), with optional per-matrix biases (dst =
// acc + bias[r]) and, with accum, added into dst (dst = dst + ...); every
// value as cx_gemm_apply (and the separate adds) give it. Only where
// cx_gemm_multi_fits: Q4_K/Q5_K, and with several matrices every n[i] a
// multiple of the tile's rows.
#define CX_GEMM_SEGS 3
bool cx_gemm_multi_fits(int type, const uint32_t* n, uint32_t count, size_t m);
int cx_gemm_apply_multi(int type, const uint8_t* const* w, const uint32_t* n, uint32_t count,
                        size_t k, size_t m, float* const* dst, const float* const* bias, int accum,
                        const void* scratch, hipStream_t s);

// Format conversion (cx_quant.hip): bit-identical to quant::descuantizar,
// descuantizar_filas and desempaquetar_i8; rows[] are device indices.
int cx_launch_dequantize(int type, const uint8_t* b, size_t n, float* y, hipStream_t s);
int cx_launch_dequantize_rows(int type, const uint8_t* b, uint32_t width, const uint32_t* rows,
                              size_t nrows, float* y, hipStream_t s);
int cx_launch_unpack_i8(int type, const uint8_t* b, size_t n, int8_t* q, float* esc, float* off,
                        hipStream_t s);
// dst[m][n] = x[m][k] . W^T for F32/F16 weight rows (ops::matmul's
// unquantized path, src/ops.rs:87-156)
int cx_launch_matmul_f(int type, const uint8_t* w, size_t n, size_t k, const float* x, size_t m,
                       float* dst, hipStream_t s);

// GGUF (cx_gguf.hip)
int cx_gguf_read(const char* path, cx_gguf** out);
void cx_gguf_release(cx_gguf* g);
const cx_gguf_tensor* cx_gguf_tensors(const cx_gguf* g, size_t* n);
// [data_start + offset, + bytes) checked against overflow and the file size
int cx_gguf_range(const cx_gguf* g, const cx_gguf_tensor& t, uint64_t* from);
int cx_gguf_read_bytes(const cx_gguf* g, uint64_t from, void* host, size_t n, FILE* f);
// one metadata entry to write: type 4 (u32: u), 10 (u64: u), 6 (f32: f), 8 (string: s)
struct cx_gguf_meta {
  std::string key;
  uint32_t type;
  uint64_t u;
  double f;
  std::string s;
};
int cx_gguf_write(const char* path, const std::vector<cx_gguf_meta>& meta,
                  const std::vector<cx_gguf_tensor>& tensors,
                  const std::vector<const void*>& host_data);
