// cx_probe.hip — a measurement kernel, not part of the decode path: a
// streaming read of a buffer at the rate HBM (or the Infinity Cache, for
// buffers that fit in it) delivers to a grid of 16-byte loads. It gives the
// roofline a measured read peak next to the nominal 8 TB/s, and the read
// rate a launch of a given size reaches (the GEMV's own bytes), with no
// arithmetic after the loads.
#include "cx_common.h"

namespace {

// Every 16-byte word of p[0, n16) is loaded once and folded into an xor:
// a workgroup reads chunks of 32 KB in turn (chunk c, c + grid, ...), each
// thread eight 16-byte words 4 KB apart within the chunk, so that a wave's
// loads are contiguous 1 KB runs; the fold is stored only when it equals a
// value no buffer here produces, so that the loads stay. Non-temporal loads
// (NT) read 1 GB at ~6.8 TB/s on MI355X, plain ones at ~6.1 (grids of 512
// to 16384 workgroups measured the same within 2%).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__global__ __launch_bounds__(256) void k_stream_read(const uint4* p, size_t n16, uint32_t* sink) {
  constexpr size_t CH = 256 * 8;  // 16-byte words a chunk
  const size_t nfull = n16 / CH;
  uint32_t acc = 0;
  for (size_t c = blockIdx.x; c < nfull; c += gridDim.x) {
    const u32x4* q = reinterpret_cast<const u32x4*>(p) + c * CH + threadIdx.x;
    u32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = NT ? __builtin_nontemporal_load(q + j * 256) : q[j * 256];
#pragma unroll
    for (int j = 0; j < 8; j++) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  for (size_t i = nfull * CH + (size_t)blockIdx.x * 256 + threadIdx.x; i < n16;
       i += (size_t)gridDim.x * 256) {
    const uint4 v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace

extern "C" int cx_stream_read(const void* p, size_t bytes, uint32_t* sink, void* stream) {
  CX_REQUIRE(p && sink, "stream_read: null pointer");
  CX_REQUIRE(((uintptr_t)p & 15) == 0 && bytes % 16 == 0, "stream_read: p and bytes must be 16-byte multiples");
  const size_t n16 = bytes / 16;
  if (!n16) return CX_OK;
  // at most eight workgroups a CU, each thread at least eight loads
  size_t grid = (n16 + 2047) / 2048;
  if (grid > 2048) grid = 2048;
  hipLaunchKernelGGL(k_stream_read<true>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint4*)p, n16, sink);
  CX_HIP(hipGetLastError());
  return CX_OK;
}
