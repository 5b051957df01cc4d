// cx_common.h — shared device/host helpers for the gfx950 decode path.
//
// Everything in this library is compiled with -ffp-contract=off: an f32
// expression rounds exactly where it is written, the way the reference's Rust
// does. Where a fused multiply-add is wanted it is spelled out (fmaf).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/cosxamix_hip.h"

#define CX_WAVE 64

// ------------------------------------------------------------------ errors
void cx_set_error(const char* fmt, ...);
#define CX_HIP(call)                                                          \
  do {                                                                        \
    hipError_t e_ = (call);                                                   \
    if (e_ != hipSuccess) {                                                   \
      cx_set_error("%s:%d: %s: %s", __FILE__, __LINE__, #call,                \
                   hipGetErrorString(e_));                                    \
      return CX_EHIP;                                                         \
    }                                                                         \
  } while (0)
#define CX_REQUIRE(cond, ...)                                                 \
  do {                                                                        \
    if (!(cond)) {                                                            \
      cx_set_error(__VA_ARGS__);                                              \
      return CX_EINVAL;                                                       \
    }                                                                         \
  } while (0)

// ------------------------------------------------------- format geometry
// src/gguf.rs:83-111 and src/quant.rs:213-219
__host__ __device__ inline int cx_bpb(int t) {
  switch (t) {
    case CX_F32: return 4;
    case CX_F16: return 2;
    case CX_Q8_0: return 34;
    case CX_Q5_0: return 22;
    case CX_Q2_K: return 84;
    case CX_Q3_K: return 110;
    case CX_Q4_K: return 144;
    case CX_Q5_K: return 176;
    case CX_Q6_K: return 210;
    default: return 0;
  }
}
__host__ __device__ inline int cx_vpb(int t) {
  switch (t) {
    case CX_F32: case CX_F16: return 1;
    case CX_Q8_0: case CX_Q5_0: return 32;
    case CX_Q2_K: case CX_Q3_K: case CX_Q4_K: case CX_Q5_K: case CX_Q6_K: return 256;
    default: return 0;
  }
}
__host__ __device__ inline int cx_sub(int t) {
  switch (t) {
    case CX_Q8_0: case CX_Q5_0: case CX_Q4_K: case CX_Q5_K: return 32;
    case CX_Q2_K: case CX_Q3_K: case CX_Q6_K: return 16;
    default: return 0;
  }
}
inline bool cx_is_kquant(int t) {
  return t == CX_Q2_K || t == CX_Q3_K || t == CX_Q4_K || t == CX_Q5_K || t == CX_Q6_K;
}
// the 32-value block formats without a minimum (Q8_0, Q5_0): GGUF's choice
// for matrices whose width is not a multiple of 256 (src/gguf.rs:80-82)
inline bool cx_is_block32(int t) { return t == CX_Q8_0 || t == CX_Q5_0; }
// every format the GEMV reads: the k-quants and the 32-value blocks
inline bool cx_has_gemv(int t) { return cx_is_kquant(t) || cx_is_block32(t); }

// ------------------------------------------------------ device helpers
__device__ inline float cx_h2f(uint32_t h16) {
  // v_cvt_f32_f16: exact for every finite half, subnormals included (f16
  // denormals are not flushed in this build). Matches quant.rs:38-60.
  _Float16 h;
  uint16_t b = (uint16_t)h16;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}

// lane i <- lane i^1, inside a quad (DPP quad_perm [1,0,3,2])
__device__ inline int cx_xor1(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
}
// lane i <- lane i^2, inside a quad (DPP quad_perm [2,3,0,1])
__device__ inline int cx_xor2(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
}
__device__ inline float cx_xor1f(float v) {
  return __int_as_float(cx_xor1(__float_as_int(v)));
}
__device__ inline float cx_xor2f(float v) {
  return __int_as_float(cx_xor2(__float_as_int(v)));
}

// Deterministic wave64 sum: butterfly, every lane ends with the same value.
__device__ inline float cx_wave_sum(float v) {
  v += __shfl_xor(v, 1, CX_WAVE);
  v += __shfl_xor(v, 2, CX_WAVE);
  v += __shfl_xor(v, 4, CX_WAVE);
  v += __shfl_xor(v, 8, CX_WAVE);
  v += __shfl_xor(v, 16, CX_WAVE);
  v += __shfl_xor(v, 32, CX_WAVE);
  return v;
}
// A lane's value from the lane a DPP control selects (every lane valid:
// quad permutes and row mirrors)
template <int CTRL>
__device__ inline uint32_t cx_dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ inline double cx_dpp_d(double v) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint64_t lo = cx_dpp<CTRL>((uint32_t)u), hi = cx_dpp<CTRL>((uint32_t)(u >> 32));
  return __longlong_as_double((long long)(lo | (hi << 32)));
}
constexpr int CX_DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int CX_DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int CX_DPP_HALF_MIRROR = 0x141;  // lane i of 8 <- 7 - i
constexpr int CX_DPP_MIRROR = 0x140;       // lane i of 16 <- 15 - i

// The xor butterfly v += v[lane ^ o], o = 1, 2, ..., 32: every lane ends
// with the same tree's sum. Levels 4 and 8 read lane i ^ 7 and i ^ 15 (the
// row mirrors), which after the levels before hold the same value as
// i ^ 4 and i ^ 8; an f32/f64 add is commutative, so the result is the
// butterfly's bit for bit. The first four levels are DPP moves, the last
// two cross rows through the LDS crossbar.
__device__ inline double cx_wave_sum_d(double v) {
  v += cx_dpp_d<CX_DPP_XOR1>(v);
  v += cx_dpp_d<CX_DPP_XOR2>(v);
  v += cx_dpp_d<CX_DPP_HALF_MIRROR>(v);
  v += cx_dpp_d<CX_DPP_MIRROR>(v);
  v += __shfl_xor(v, 16, CX_WAVE);
  v += __shfl_xor(v, 32, CX_WAVE);
  return v;
}
__device__ inline float cx_wave_max(float v) {
  v = fmaxf(v, __uint_as_float(cx_dpp<CX_DPP_XOR1>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(cx_dpp<CX_DPP_XOR2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(cx_dpp<CX_DPP_HALF_MIRROR>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(cx_dpp<CX_DPP_MIRROR>(__float_as_uint(v))));
  v = fmaxf(v, __shfl_xor(v, 16, CX_WAVE));
  v = fmaxf(v, __shfl_xor(v, 32, CX_WAVE));
  return v;
}

// argmax pairs (src/sampler.rs:129-137): the larger value, the lower index
// among equal values; callers leave NaN out (a NaN never wins)
struct VI {
  float v;
  uint32_t i;
};
__device__ inline VI vi_best(VI a, VI b) {
  return (a.v > b.v || (a.v == b.v && a.i < b.i)) ? a : b;
}
__device__ inline VI vi_wave(VI a) {
  for (int o = 1; o < 64; o <<= 1) {
    VI b{__shfl_xor(a.v, o, 64), (uint32_t)__shfl_xor((int)a.i, o, 64)};
    a = vi_best(a, b);
  }
  return a;
}

// Pipelines of direct-to-LDS loads (global_load_lds) need partial waits:
// __syncthreads() carries a workgroup fence after which the compiler waits
// for every outstanding vector load (vmcnt(0)), draining the pipeline. These
// wait exactly as asked; their "memory" clobbers keep the compiler from
// moving memory accesses across them.
typedef __attribute__((address_space(3))) void* cx_lds_ptr;
template <int N>
__device__ inline void cx_wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ inline void cx_wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
__device__ inline void cx_barrier() { asm volatile("s_barrier" ::: "memory"); }
// 16 bytes from global `g` into LDS at (wave-uniform) `l` + 16 * lane
__device__ inline void cx_dma16(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds(g, (cx_lds_ptr)l, 16, 0, 0);
}
// The same load hidden from the compiler: it then inserts no wait of its own
// before later LDS reads (it would wait for every load, since it cannot tell
// which LDS bytes are in flight). The caller orders the data with
// cx_wait_vm<N>() — loads complete in issue order — and must not leave the
// kernel with such a load outstanding.
// `l` must be the same for every lane of the wave; M0 (the LDS address of
// the load) is saved and restored around it.
__device__ inline void cx_dma16_async(const void* g, void* l) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(cx_lds_ptr)l);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %2, off\n\ts_nop 0\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(la), "v"(g)
      : "memory");
}

// The same for 4 bytes a lane: LDS `l` + 4 * lane.
__device__ inline void cx_dma4_async(const void* g, void* l) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(cx_lds_ptr)l);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
      "global_load_lds_dword %2, off\n\ts_nop 0\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(la), "v"(g)
      : "memory");
}

// s = 0; s += a[i] * b[i] for i = 0, 1, ... in order (the sequential f32
// dot of src/kernels/scalar.rs:16-23) over N4 float4s (LDS or global). The
// operands stream in batches of 16 values, two batches ahead of the adds;
// a batch's 16 products are formed first and pinned by empty asms that take
// them as operands: left to itself the compiler interleaves each multiply
// with its add, and the chain then waits for a multiply and an add per term
// instead of one add.
template <int N4>
__device__ inline float cx_dot_seq(const float4* a, const float4* b) {
  static_assert(N4 % 4 == 0, "batches of four float4");
  constexpr int NB = N4 / 4;
  float4 x[2][4], y[2][4];
#pragma unroll
  for (int k = 0; k < 2 && k < NB; k++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      x[k][j] = a[4 * k + j];
      y[k][j] = b[4 * k + j];
    }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NB; i++) {
    const int k = i & 1;
    float t[16];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      t[4 * j] = x[k][j].x * y[k][j].x;
      t[4 * j + 1] = x[k][j].y * y[k][j].y;
      t[4 * j + 2] = x[k][j].z * y[k][j].z;
      t[4 * j + 3] = x[k][j].w * y[k][j].w;
    }
    asm volatile("" : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]), "+v"(t[4]), "+v"(t[5]),
                 "+v"(t[6]), "+v"(t[7]));
    asm volatile("" : "+v"(t[8]), "+v"(t[9]), "+v"(t[10]), "+v"(t[11]), "+v"(t[12]),
                 "+v"(t[13]), "+v"(t[14]), "+v"(t[15]));
    if (i + 2 < NB)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        x[k][j] = a[4 * (i + 2) + j];
        y[k][j] = b[4 * (i + 2) + j];
      }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 16; j++) s += t[j];
  }
  return s;
}

// Rust `f32 as i32` (saturating, NaN -> 0) then `as i8` (low 8 bits),
// without branches: r clamped to [-2^31, 2147483520] (the largest f32 below
// 2^31) converts exactly as the in-range cast, then r >= 2^31 and NaN are
// selected.
__device__ inline int8_t cx_rust_i8(float r) {
  const float c = fminf(fmaxf(r, -2147483648.0f), 2147483520.0f);
  int32_t v = (int32_t)c;
  v = r >= 2147483648.0f ? 2147483647 : v;
  v = r != r ? 0 : v;
  return (int8_t)(uint8_t)(uint32_t)v;
}

// ------------------------------------------------- library state
// A host thread's context on one device: the stream of the host-pointer
// entry points and the device scratch of the operators. Each host thread
// holds its own (taken from a per-device pool at its first call, returned
// when the thread ends), so calls from different threads never share a
// scratch buffer at the same time: every use of a context's scratch is
// stream-ordered after the previous one (the `used` event), whichever
// stream or thread made it.
struct cx_lib {
  int device;
  hipStream_t stream;   // library stream for host-pointer entry points
  void* scratch;        // device scratch of this thread's calls
  size_t scratch_bytes;
  hipEvent_t used;      // recorded after the last enqueued work on the scratch
  bool used_valid;
};
cx_lib* cx_lib_get();   // the calling thread's context on its current device
// The calling thread's scratch of at least `bytes` for work about to be
// enqueued on stream s; s first waits for every earlier use of it.
int cx_scratch_acquire(size_t bytes, hipStream_t s, void** out);
// Marks the end of the enqueued work on s that uses the scratch.
void cx_scratch_release(hipStream_t s);

// One call's use of the calling thread's scratch on one stream: get() waits
// (in stream order) for the earlier uses, the destructor records the end of
// this call's work, on every return path.
class cx_scratch {
 public:
  explicit cx_scratch(hipStream_t s) : s_(s) {}
  cx_scratch(const cx_scratch&) = delete;
  cx_scratch& operator=(const cx_scratch&) = delete;
  int get(size_t bytes, void** out) {
    const int rc = cx_scratch_acquire(bytes, s_, out);
    held_ = held_ || rc == CX_OK;
    return rc;
  }
  ~cx_scratch() {
    if (held_) cx_scratch_release(s_);
  }

 private:
  hipStream_t s_;
  bool held_ = false;
};
