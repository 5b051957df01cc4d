// cx_quant.hip — format conversion on the GPU and the unquantized matmul:
//   quant::descuantizar        (src/quant.rs:124-162)  -> cx_launch_dequantize
//   quant::descuantizar_filas  (src/quant.rs:172-205)  -> cx_launch_dequantize_rows
//   quant::desempaquetar_i8    (src/quant.rs:238-468)  -> cx_launch_unpack_i8
//   ops::matmul for F32/F16    (src/ops.rs:87-156)     -> cx_launch_matmul_f
// Every value of the first three is bit-identical to the reference's (the
// per-type expressions are in cx_dequant.h). Eight values per lane, block by
// block; bytes are read with byte loads, so any alignment of the source works.

#include "cx_dequant.h"
#include "cx_internal.h"

namespace {

template <int T>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* b, size_t n, float* y) {
  const size_t i = 8 * (blockIdx.x * 256ull + threadIdx.x);
  if (i >= n) return;
  constexpr int VPB = T == CX_F32 || T == CX_F16 ? 1 : (T == CX_Q8_0 || T == CX_Q5_0 ? 32 : 256);
  constexpr int BPB = T == CX_F32 ? 4 : T == CX_F16 ? 2 : T == CX_Q8_0 ? 34 : T == CX_Q5_0 ? 22
                    : T == CX_Q2_K ? 84 : T == CX_Q3_K ? 110 : T == CX_Q4_K ? 144
                    : T == CX_Q5_K ? 176 : 210;
  float v[8];
  if (VPB == 1 && i + 8 > n) {  // the tail of an unquantized vector
    for (size_t j = i; j < n; j++)
      y[j] = T == CX_F32 ? reinterpret_cast<const float*>(b)[j] : cxq::f16_at(b + 2 * j);
    return;
  }
  cxq::dequant8<T>(b + i / VPB * BPB, (uint32_t)(i % VPB), v);
  reinterpret_cast<float4*>(y + i)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(y + i)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// rows[r] of a row-major matrix of `width` values per row into y[r][width]
template <int T>
__global__ __launch_bounds__(256) void k_dequant_rows(const uint8_t* b, uint32_t width,
                                                      const uint32_t* rows, size_t nrows,
                                                      float* y) {
  const size_t i = 8 * (blockIdx.x * 256ull + threadIdx.x);
  if (i >= nrows * width) return;
  constexpr int VPB = T == CX_F32 || T == CX_F16 ? 1 : (T == CX_Q8_0 || T == CX_Q5_0 ? 32 : 256);
  constexpr int BPB = T == CX_F32 ? 4 : T == CX_F16 ? 2 : T == CX_Q8_0 ? 34 : T == CX_Q5_0 ? 22
                    : T == CX_Q2_K ? 84 : T == CX_Q3_K ? 110 : T == CX_Q4_K ? 144
                    : T == CX_Q5_K ? 176 : 210;
  const size_t r = i / width, col = i % width;
  const size_t row_bytes = (size_t)width / VPB * BPB;
  float v[8];
  cxq::dequant8<T>(b + rows[r] * row_bytes + col / VPB * BPB, (uint32_t)(col % VPB), v);
  reinterpret_cast<float4*>(y + i)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(y + i)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

template <int T>
__global__ __launch_bounds__(256) void k_unpack(const uint8_t* b, size_t n, int8_t* q, float* esc,
                                                float* off) {
  const size_t i = 8 * (blockIdx.x * 256ull + threadIdx.x);
  if (i >= n) return;
  constexpr int VPB = T == CX_Q8_0 || T == CX_Q5_0 ? 32 : 256;
  constexpr int BPB = T == CX_Q8_0 ? 34 : T == CX_Q5_0 ? 22 : T == CX_Q2_K ? 84
                    : T == CX_Q3_K ? 110 : T == CX_Q4_K ? 144 : T == CX_Q5_K ? 176 : 210;
  constexpr int SUB = T == CX_Q2_K || T == CX_Q3_K || T == CX_Q6_K ? 16 : 32;
  int8_t v[8];
  float e, o;
  cxq::unpack8<T>(b + i / VPB * BPB, (uint32_t)(i % VPB), v, e, o);
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    lo |= (uint32_t)(uint8_t)v[j] << (8 * j);
    hi |= (uint32_t)(uint8_t)v[4 + j] << (8 * j);
  }
  *reinterpret_cast<uint2*>(q + i) = make_uint2(lo, hi);
  if (i % SUB == 0) {
    esc[i / SUB] = e;
    off[i / SUB] = o;
  }
}

// dst[a][r] = sum_i lhs[a][i] * w[r][i] for F32/F16 rows (the f16 widening is
// exact, src/quant.rs:38-60). One wave per weight row, 4 values a lane per
// step, up to 8 activation rows per pass; f32 FMA partial sums, then a
// butterfly over the wave. The reference's kernels::dot adds in another
// order (8-lane FMA, src/kernels/x86.rs:25-71): equal within f32 rounding.
template <int T>
__global__ __launch_bounds__(256) void k_matmul_f(const uint8_t* w, uint32_t n, uint32_t k,
                                                  const float* x, uint32_t m, float* dst) {
  const uint32_t lane = threadIdx.x & 63, r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= n) return;  // whole wave: no barrier below
  const size_t rb = (size_t)k * (T == CX_F32 ? 4 : 2);
  const uint8_t* row = w + (size_t)r * rb;
  for (uint32_t a0 = 0; a0 < m; a0 += 8) {
    const uint32_t na = m - a0 < 8 ? m - a0 : 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t i = 4 * lane; i < k; i += 256) {
      float wv[4];
      if (T == CX_F32) {
        const float4 f = *reinterpret_cast<const float4*>(row + 4 * (size_t)i);
        wv[0] = f.x; wv[1] = f.y; wv[2] = f.z; wv[3] = f.w;
      } else {
        const uint2 h = *reinterpret_cast<const uint2*>(row + 2 * (size_t)i);
        wv[0] = cx_h2f(h.x & 0xFFFF); wv[1] = cx_h2f(h.x >> 16);
        wv[2] = cx_h2f(h.y & 0xFFFF); wv[3] = cx_h2f(h.y >> 16);
      }
#pragma unroll
      for (uint32_t a = 0; a < 8; a++) {
        if (a < na) {
          const float4 xv = *reinterpret_cast<const float4*>(x + (size_t)(a0 + a) * k + i);
          acc[a] = fmaf(xv.x, wv[0], acc[a]);
          acc[a] = fmaf(xv.y, wv[1], acc[a]);
          acc[a] = fmaf(xv.z, wv[2], acc[a]);
          acc[a] = fmaf(xv.w, wv[3], acc[a]);
        }
      }
    }
#pragma unroll
    for (uint32_t a = 0; a < 8; a++) {
      if (a < na) {
        float v = acc[a];
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) v += __shfl_xor(v, s, 64);
        if (lane == 0) dst[(size_t)(a0 + a) * n + r] = v;
      }
    }
  }
}

bool dequant_type(int t) {
  return t == CX_F32 || t == CX_F16 || t == CX_Q8_0 || t == CX_Q5_0 || cx_is_kquant(t);
}

}  // namespace

int cx_launch_dequantize(int type, const uint8_t* b, size_t n, float* y, hipStream_t s) {
  CX_REQUIRE(dequant_type(type), "dequantize: type %d has no dequantizer", type);
  CX_REQUIRE(n % (size_t)cx_vpb(type) == 0,
             "dequantize: %zu values are not whole blocks of %d", n, cx_vpb(type));
  CX_REQUIRE(b && y, "dequantize: null pointer");
  CX_REQUIRE(((uintptr_t)y & 15) == 0 && (type != CX_F32 || ((uintptr_t)b & 3) == 0),
             "dequantize: the output must be 16-byte aligned (and F32 input 4-byte aligned)");
  if (!n) return CX_OK;
  const size_t grid = (n + 2047) / 2048;
  CX_REQUIRE(grid < (1ull << 31), "dequantize: %zu values is too many", n);
  const dim3 g((unsigned)grid), wg(256);
  switch (type) {
    case CX_F32: hipLaunchKernelGGL(k_dequant<CX_F32>, g, wg, 0, s, b, n, y); break;
    case CX_F16: hipLaunchKernelGGL(k_dequant<CX_F16>, g, wg, 0, s, b, n, y); break;
    case CX_Q8_0: hipLaunchKernelGGL(k_dequant<CX_Q8_0>, g, wg, 0, s, b, n, y); break;
    case CX_Q5_0: hipLaunchKernelGGL(k_dequant<CX_Q5_0>, g, wg, 0, s, b, n, y); break;
    case CX_Q2_K: hipLaunchKernelGGL(k_dequant<CX_Q2_K>, g, wg, 0, s, b, n, y); break;
    case CX_Q3_K: hipLaunchKernelGGL(k_dequant<CX_Q3_K>, g, wg, 0, s, b, n, y); break;
    case CX_Q4_K: hipLaunchKernelGGL(k_dequant<CX_Q4_K>, g, wg, 0, s, b, n, y); break;
    case CX_Q5_K: hipLaunchKernelGGL(k_dequant<CX_Q5_K>, g, wg, 0, s, b, n, y); break;
    default: hipLaunchKernelGGL(k_dequant<CX_Q6_K>, g, wg, 0, s, b, n, y); break;
  }
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_dequantize_rows(int type, const uint8_t* b, uint32_t width, const uint32_t* rows,
                              size_t nrows, float* y, hipStream_t s) {
  CX_REQUIRE(dequant_type(type), "dequantize rows: type %d has no dequantizer", type);
  CX_REQUIRE(width % 8 == 0 && width % (uint32_t)cx_vpb(type) == 0,
             "dequantize rows: a row of %u values is not whole blocks", width);
  CX_REQUIRE(b && rows && y && ((uintptr_t)y & 15) == 0,
             "dequantize rows: null pointer or unaligned output");
  if (!nrows || !width) return CX_OK;
  const size_t grid = (nrows * width / 8 + 255) / 256;
  CX_REQUIRE(grid < (1ull << 31), "dequantize rows: too many values");
  const dim3 g((unsigned)grid), wg(256);
  switch (type) {
    case CX_F32: hipLaunchKernelGGL(k_dequant_rows<CX_F32>, g, wg, 0, s, b, width, rows, nrows, y); break;
    case CX_F16: hipLaunchKernelGGL(k_dequant_rows<CX_F16>, g, wg, 0, s, b, width, rows, nrows, y); break;
    case CX_Q8_0: hipLaunchKernelGGL(k_dequant_rows<CX_Q8_0>, g, wg, 0, s, b, width, rows, nrows, y); break;
    case CX_Q5_0: hipLaunchKernelGGL(k_dequant_rows<CX_Q5_0>, g, wg, 0, s, b, width, rows, nrows, y); break;
    case CX_Q2_K: hipLaunchKernelGGL(k_dequant_rows<CX_Q2_K>, g, wg, 0, s, b, width, rows, nrows, y); break;
    case CX_Q3_K: hipLaunchKernelGGL(k_dequant_rows<CX_Q3_K>, g, wg, 0, s, b, width, rows, nrows, y); break;
    case CX_Q4_K: hipLaunchKernelGGL(k_dequant_rows<CX_Q4_K>, g, wg, 0, s, b, width, rows, nrows, y); break;
    case CX_Q5_K: hipLaunchKernelGGL(k_dequant_rows<CX_Q5_K>, g, wg, 0, s, b, width, rows, nrows, y); break;
    default: hipLaunchKernelGGL(k_dequant_rows<CX_Q6_K>, g, wg, 0, s, b, width, rows, nrows, y); break;
  }
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_unpack_i8(int type, const uint8_t* b, size_t n, int8_t* q, float* esc, float* off,
                        hipStream_t s) {
  CX_REQUIRE(cx_sub(type) > 0, "unpack: type %d has no direct unpacking to i8", type);
  CX_REQUIRE(n % (size_t)cx_vpb(type) == 0, "unpack: %zu values are not whole blocks", n);
  CX_REQUIRE(b && q && esc && off && ((uintptr_t)q & 7) == 0,
             "unpack: null pointer or q not 8-byte aligned");
  if (!n) return CX_OK;
  const size_t grid = (n + 2047) / 2048;
  CX_REQUIRE(grid < (1ull << 31), "unpack: %zu values is too many", n);
  const dim3 g((unsigned)grid), wg(256);
  switch (type) {
    case CX_Q8_0: hipLaunchKernelGGL(k_unpack<CX_Q8_0>, g, wg, 0, s, b, n, q, esc, off); break;
    case CX_Q5_0: hipLaunchKernelGGL(k_unpack<CX_Q5_0>, g, wg, 0, s, b, n, q, esc, off); break;
    case CX_Q2_K: hipLaunchKernelGGL(k_unpack<CX_Q2_K>, g, wg, 0, s, b, n, q, esc, off); break;
    case CX_Q3_K: hipLaunchKernelGGL(k_unpack<CX_Q3_K>, g, wg, 0, s, b, n, q, esc, off); break;
    case CX_Q4_K: hipLaunchKernelGGL(k_unpack<CX_Q4_K>, g, wg, 0, s, b, n, q, esc, off); break;
    case CX_Q5_K: hipLaunchKernelGGL(k_unpack<CX_Q5_K>, g, wg, 0, s, b, n, q, esc, off); break;
    default: hipLaunchKernelGGL(k_unpack<CX_Q6_K>, g, wg, 0, s, b, n, q, esc, off); break;
  }
  CX_HIP(hipGetLastError());
  return CX_OK;
}

int cx_launch_matmul_f(int type, const uint8_t* w, size_t n, size_t k, const float* x, size_t m,
                       float* dst, hipStream_t s) {
  CX_REQUIRE(type == CX_F32 || type == CX_F16, "matmul: type %d is not F32/F16", type);
  CX_REQUIRE(w && x && dst, "matmul: null pointer");
  CX_REQUIRE(k % 4 == 0 && n < (1u << 31) && k < (1u << 31) && m < (1u << 31),
             "matmul: k=%zu must be a multiple of 4", k);
  CX_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0,
             "matmul: weights and activations must be 16-byte aligned");
  if (!n || !m) return CX_OK;
  const dim3 g((unsigned)((n + 3) / 4)), wg(256);
  if (type == CX_F32)
    hipLaunchKernelGGL(k_matmul_f<CX_F32>, g, wg, 0, s, w, (uint32_t)n, (uint32_t)k, x, (uint32_t)m, dst);
  else
    hipLaunchKernelGGL(k_matmul_f<CX_F16>, g, wg, 0, s, w, (uint32_t)n, (uint32_t)k, x, (uint32_t)m, dst);
  CX_HIP(hipGetLastError());
  return CX_OK;
}
