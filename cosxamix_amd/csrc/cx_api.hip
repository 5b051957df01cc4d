// cx_api.hip — the C ABI (include/cosxamix_hip.h): kernel contract,
// operators, and the Qwen2 model with its cache and captured decode step.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <math.h>

#include <functional>
#include <mutex>
#include <string>
#include <vector>

#include "cx_ops.h"

// =================================================================== errors
static thread_local char g_err[512];
void cx_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}
extern "C" const char* cx_last_error(void) { return g_err; }

// ================================================================ state
// The device of the calling thread's host-pointer entry points and models.
static thread_local int g_device = 0;

// Per-device pools of thread contexts. A thread takes a context at its first
// call on a device and gives it back when it ends; a context is never freed,
// so no thread can see its stream released under it, and its scratch is
// stream-ordered: the next thread's first use waits (on the device, in
// stream order) for the work the previous holder left queued. The pool only
// grows to the largest number of threads that ran at once.
static std::mutex g_pool_mu;
static std::vector<cx_lib*> g_pool[64];

namespace {
struct ThreadContexts {
  cx_lib* ctx[64] = {};
  ~ThreadContexts() {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    for (int d = 0; d < 64; d++)
      if (ctx[d]) g_pool[d].push_back(ctx[d]);
  }
};
}  // namespace
static thread_local ThreadContexts t_ctx;

cx_lib* cx_lib_get() {
  const int dev = g_device;
  if (dev < 0 || dev >= 64) return nullptr;
  if (cx_lib* L = t_ctx.ctx[dev]) return L;
  cx_lib* L = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    if (!g_pool[dev].empty()) {
      L = g_pool[dev].back();
      g_pool[dev].pop_back();
    }
  }
  if (!L) {
    if (hipSetDevice(dev) != hipSuccess) return nullptr;
    hipStream_t s = nullptr;
    hipEvent_t ev = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
      (void)hipStreamDestroy(s);
      return nullptr;
    }
    L = new cx_lib{dev, s, nullptr, 0, ev, false};
  }
  t_ctx.ctx[dev] = L;
  return L;
}

static bool capturing(hipStream_t s) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// The calling thread's scratch of at least `bytes`, for work about to be
// enqueued on stream s. s first waits for the `used` event, which follows
// every earlier use of the scratch on any stream (each use waited for the
// one before it), by this thread or by the thread that held the context
// before. Growing frees the old buffer and allocates the new one in s's
// order (hipFreeAsync/hipMallocAsync) after those uses, so no other stream
// or thread is waited for. Under stream capture the scratch cannot grow and
// the captured work is not ordered after earlier uses: the caller orders its
// graph's launches, as for any captured work.
int cx_scratch_acquire(size_t bytes, hipStream_t s, void** out) {
  cx_lib* L = cx_lib_get();
  if (!L) {
    cx_set_error("no HIP device %d", g_device);
    return CX_EHIP;
  }
  const bool cap = capturing(s);
  if (!cap && L->used_valid) CX_HIP(hipStreamWaitEvent(s, L->used, 0));
  if (L->scratch_bytes < bytes) {
    CX_REQUIRE(!cap,
               "the calling thread's scratch must grow to %zu bytes while the stream is being "
               "captured: make the same call once before the capture, or use "
               "cx_matmul_auto_noalloc",
               bytes);
    CX_HIP(hipSetDevice(L->device));
    if (L->scratch) CX_HIP(hipFreeAsync(L->scratch, s));
    L->scratch = nullptr;
    L->scratch_bytes = 0;
    CX_HIP(hipMallocAsync(&L->scratch, bytes, s));
    L->scratch_bytes = bytes;
  }
  *out = L->scratch;
  return CX_OK;
}

void cx_scratch_release(hipStream_t s) {
  cx_lib* L = cx_lib_get();
  if (!L || capturing(s)) return;
  if (hipEventRecord(L->used, s) == hipSuccess) {
    L->used_valid = true;
    return;
  }
  // without the event the next use could not be ordered: finish the work
  (void)hipStreamSynchronize(s);
  L->used_valid = false;
}

static int noalloc_scratch(int dev, void** out);

extern "C" int cx_init(int device) {
  int n = 0;
  CX_HIP(hipGetDeviceCount(&n));
  CX_REQUIRE(device >= 0 && device < n && device < 64, "cx_init: device %d of %d", device, n);
  g_device = device;
  CX_HIP(hipSetDevice(device));
  // the allocation-free entry point's array is looked up here; a failure
  // is not cx_init's: that entry point tries again and reports it
  void* sp = nullptr;
  (void)noalloc_scratch(device, &sp);
  if (!cx_lib_get()) {
    cx_set_error("cx_init: no stream on device %d", device);
    return CX_EHIP;
  }
  return CX_OK;
}

extern "C" size_t cx_row_bytes(int type, size_t k) {
  const int vpb = cx_vpb(type);
  if (!vpb || k % (size_t)vpb) return 0;
  return k / vpb * cx_bpb(type);
}
extern "C" int cx_sub_block(int type) { return cx_sub(type); }

// ================================================== 1. kernel contract
static float dot_host(int type, const uint8_t* b, const int8_t* xq, const float* xe,
                      const float* xs, size_t nb) {
  if (!b || !xq || !xe || !xs || !nb) {
    cx_set_error("dot: null pointer or zero blocks");
    return NAN;
  }
  cx_lib* L = cx_lib_get();
  if (!L) {
    cx_set_error("no HIP device");
    return NAN;
  }
  const size_t k = nb * 256, nsub = k / cx_sub(type), rb = nb * cx_bpb(type);
  const size_t o_x = (rb + 255) / 256 * 256, o_e = o_x + k, o_s = o_e + nsub * 4,
               o_y = o_s + nsub * 4, total = o_y + 256;
  hipStream_t s = L->stream;
  void* sp = nullptr;
  cx_scratch scr(s);
  if (scr.get(total, &sp)) return NAN;
  uint8_t* d = (uint8_t*)sp;
  if (hipMemcpyAsync(d, b, rb, hipMemcpyHostToDevice, s) != hipSuccess ||
      hipMemcpyAsync(d + o_x, xq, k, hipMemcpyHostToDevice, s) != hipSuccess ||
      hipMemcpyAsync(d + o_e, xe, nsub * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
      hipMemcpyAsync(d + o_s, xs, nsub * 4, hipMemcpyHostToDevice, s) != hipSuccess) {
    cx_set_error("dot: copy to device failed");
    return NAN;
  }
  cx_seg seg{d, (float*)(d + o_y), nullptr, 1};
  cx_qact act{(const int8_t*)(d + o_x), (const float*)(d + o_e), (const float*)(d + o_s)};
  if (cx_launch_gemv(type, &seg, 1, (uint32_t)k, act, CX_EPI_STORE, nullptr, s)) return NAN;
  float y = NAN;
  if (hipMemcpyAsync(&y, d + o_y, 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess) {
    cx_set_error("dot: copy back failed");
    return NAN;
  }
  return y;
}
extern "C" float cx_dot_q2k_i8(const uint8_t* b, const int8_t* q, const float* e, const float* s, size_t n) {
  return dot_host(CX_Q2_K, b, q, e, s, n);
}
extern "C" float cx_dot_q3k_i8(const uint8_t* b, const int8_t* q, const float* e, const float* s, size_t n) {
  return dot_host(CX_Q3_K, b, q, e, s, n);
}
extern "C" float cx_dot_q4k_i8(const uint8_t* b, const int8_t* q, const float* e, const float* s, size_t n) {
  return dot_host(CX_Q4_K, b, q, e, s, n);
}
extern "C" float cx_dot_q5k_i8(const uint8_t* b, const int8_t* q, const float* e, const float* s, size_t n) {
  return dot_host(CX_Q5_K, b, q, e, s, n);
}
extern "C" float cx_dot_q6k_i8(const uint8_t* b, const int8_t* q, const float* e, const float* s, size_t n) {
  return dot_host(CX_Q6_K, b, q, e, s, n);
}

// ============================================================ 2. operators
#define STREAM(s) ((hipStream_t)(s))

extern "C" int cx_quantize_act(const float* x, size_t rows, size_t k, int sub, int8_t* xq,
                               float* xe, float* xs, void* stream) {
  return cx_launch_quantize(x, rows, k, sub, xq, xe, xs, STREAM(stream));
}

static int gemv_quantized(int type, const uint8_t* w, size_t n, size_t k, const int8_t* xq,
                          const float* xe, const float* xs, float* y, int32_t* dbg,
                          hipStream_t s) {
  CX_REQUIRE(n < (1u << 31) && k < (1u << 31), "gemv: shape too large");
  cx_seg seg{w, y, nullptr, (uint32_t)n};
  cx_qact act{xq, xe, xs};
  return cx_launch_gemv(type, &seg, 1, (uint32_t)k, act, CX_EPI_STORE, dbg, s);
}

extern "C" int cx_gemv(int type, const uint8_t* w, size_t n, size_t k, const int8_t* xq,
                       const float* xe, const float* xs, float* y, void* stream) {
  return gemv_quantized(type, w, n, k, xq, xe, xs, y, nullptr, STREAM(stream));
}

extern "C" int cx_gemv_subsums(int type, const uint8_t* w, size_t n, size_t k, const int8_t* xq,
                               const float* xe, const float* xs, int32_t* out, void* stream) {
  void* sp = nullptr;
  cx_scratch scr(STREAM(stream));
  int rc = scr.get(n * sizeof(float) + 256, &sp);
  if (rc) return rc;
  return gemv_quantized(type, w, n, k, xq, xe, xs, (float*)sp, out, STREAM(stream));
}

extern "C" int cx_quantize_blocks(int type, const float* x, size_t n, uint8_t* out, void* stream) {
  CX_REQUIRE(x && out, "quantize_blocks: null pointer");
  return cx_quantize_blocks_dev(type, x, n, out, STREAM(stream));
}

// The i8 activation of `rows` rows of k values in the library's scratch:
// xq (rows*k bytes), xe and xs (rows*k/sub floats each), for each sub-block
// size asked for, in the calling thread's scratch (held by `scr` for the
// call's work).
namespace {
struct QuantScratch {
  int8_t* xq = nullptr;
  float* xe = nullptr;
  float* xs = nullptr;
  cx_qact row(size_t f, size_t k, int sub) const {
    const size_t ns = k / sub;
    return cx_qact{xq + f * k, xe + f * ns, xs + f * ns};
  }
};
}  // namespace

static int quant_scratch(cx_scratch& scr, size_t rows, size_t k, QuantScratch* q16,
                         QuantScratch* q32) {
  auto up = [](size_t b) { return (b + 255) / 256 * 256; };
  const size_t xq_b = up(rows * k);
  auto part = [&](int sub) { return xq_b + 2 * up(rows * (k / sub) * 4); };
  void* sp = nullptr;
  int rc = scr.get((q16 ? part(16) : 0) + (q32 ? part(32) : 0), &sp);
  if (rc) return rc;
  uint8_t* p = (uint8_t*)sp;
  auto carve = [&](QuantScratch* q, int sub) {
    const size_t eb = up(rows * (k / sub) * 4);
    q->xq = (int8_t*)p;
    q->xe = (float*)(p + xq_b);
    q->xs = (float*)(p + xq_b + eb);
    p += part(sub);
  };
  if (q16) carve(q16, 16);
  if (q32) carve(q32, 32);
  return CX_OK;
}

extern "C" int cx_dequantize(int type, const uint8_t* bytes, size_t n, float* y, void* stream) {
  return cx_launch_dequantize(type, bytes, n, y, STREAM(stream));
}

extern "C" int cx_dequantize_rows(int type, const uint8_t* data, size_t width, size_t total_rows,
                                  const size_t* rows, size_t n_rows, float* y, void* stream) {
  CX_REQUIRE(rows || !n_rows, "dequantize rows: null row list");
  CX_REQUIRE(width < (1u << 31) && total_rows < (1ull << 32), "dequantize rows: shape too large");
  std::vector<uint32_t> ids(n_rows);
  for (size_t i = 0; i < n_rows; i++) {
    // src/quant.rs:194-197: a row past the data is an error, not a read
    CX_REQUIRE(rows[i] < total_rows, "dequantize rows: row %zu is past the %zu rows of the data",
               rows[i], total_rows);
    ids[i] = (uint32_t)rows[i];
  }
  if (!n_rows) return CX_OK;
  void* sp = nullptr;
  cx_scratch scr(STREAM(stream));
  int rc = scr.get(n_rows * 4, &sp);
  if (rc) return rc;
  CX_HIP(hipMemcpyAsync(sp, ids.data(), n_rows * 4, hipMemcpyHostToDevice, STREAM(stream)));
  rc = cx_launch_dequantize_rows(type, data, (uint32_t)width, (const uint32_t*)sp, n_rows, y,
                                 STREAM(stream));
  // the host copy of the indices must outlive the (possibly asynchronous) upload
  if (!rc) CX_HIP(hipStreamSynchronize(STREAM(stream)));
  return rc;
}

extern "C" int cx_unpack_i8(int type, const uint8_t* bytes, size_t n, int8_t* q, float* esc,
                            float* off, int* sub, void* stream) {
  int rc = cx_launch_unpack_i8(type, bytes, n, q, esc, off, STREAM(stream));
  if (!rc && sub) *sub = cx_sub(type);
  return rc;
}

// The argument checks of cx_matmul_auto and cx_matmul_auto_noalloc, made
// before any scratch is sized or taken.
static int matmul_auto_check(size_t k, size_t n, const float* lhs, const uint8_t* w, int type,
                             float* dst) {
  CX_REQUIRE(lhs && w && dst, "matmul_auto: null pointer");
  // src/ops.rs:1064-1071: the unquantized formats take the f32 path
  if (type == CX_F32 || type == CX_F16) return CX_OK;
  CX_REQUIRE(cx_has_gemv(type), "matmul_auto: type %d has no quantized path here", type);
  CX_REQUIRE(k % (size_t)cx_vpb(type) == 0, "matmul_auto: a row of %zu is not a multiple of the block of %d",
             k, cx_vpb(type));
  CX_REQUIRE(n < (1u << 31) && k < (1u << 31), "matmul_auto: shape too large");
  return CX_OK;
}

// Scratch bytes cx_matmul_auto needs for m rows of k values of `type` (a
// type matmul_auto_check accepts): the MFMA contraction's padded rows for
// m > 1, the rows' i8 quantization for the row-by-row GEMV, nothing for
// F32/F16.
static size_t matmul_auto_scratch(size_t m, size_t k, int type) {
  if (type == CX_F32 || type == CX_F16 || !m || !cx_sub(type)) return 0;
  if (m > 1 && cx_gemm_supported(type)) return cx_gemm_scratch_bytes(m, k);
  auto up = [](size_t b) { return (b + 255) / 256 * 256; };
  return up(m * k) + 2 * up(m * (k / cx_sub(type)) * 4);
}

// cx_matmul_auto, after matmul_auto_check, on a given scratch (at least
// matmul_auto_scratch bytes, 256-byte aligned), or on the calling thread's
// own scratch when `scratch` is NULL
static int matmul_auto_on(size_t m, size_t k, size_t n, const float* lhs, const uint8_t* w,
                          int type, float* dst, void* scratch, hipStream_t s) {
  if (type == CX_F32 || type == CX_F16) return cx_launch_matmul_f(type, w, n, k, lhs, m, dst, s);
  if (!m || !n) return CX_OK;
  cx_scratch scr(s);
  if (!scratch) {
    int rc = scr.get(matmul_auto_scratch(m, k, type), &scratch);
    if (rc) return rc;
  }
  // Several rows: all at once on int8 MFMA, each output bit-identical to the
  // row-by-row GEMV below.
  if (m > 1 && cx_gemm_supported(type))
    return cx_launch_gemm(type, w, n, k, lhs, m, dst, scratch, s);
  // Every input row is quantized once (ops.rs:469-483), then each output row
  // is the fused GEMV of its own input row: row by row is exactly the
  // reference's "one row equals a batch" (ops.rs:1364-1393).
  auto up = [](size_t b) { return (b + 255) / 256 * 256; };
  const int sub = cx_sub(type);
  uint8_t* p = (uint8_t*)scratch;
  QuantScratch q;
  q.xq = (int8_t*)p;
  q.xe = (float*)(p + up(m * k));
  q.xs = (float*)(p + up(m * k) + up(m * (k / sub) * 4));
  int rc = cx_launch_quantize(lhs, m, k, sub, q.xq, q.xe, q.xs, s);
  if (rc) return rc;
  for (size_t f = 0; f < m; f++) {
    cx_seg seg{w, dst + f * n, nullptr, (uint32_t)n};
    rc = cx_launch_gemv(type, &seg, 1, (uint32_t)k, q.row(f, k, sub), CX_EPI_STORE, nullptr, s);
    if (rc) return rc;
  }
  return CX_OK;
}

extern "C" int cx_matmul_auto(size_t m, size_t k, size_t n, const float* lhs, const uint8_t* w,
                              int type, float* dst, void* stream) {
  int rc = matmul_auto_check(k, n, lhs, w, type, dst);
  if (rc) return rc;
  return matmul_auto_on(m, k, n, lhs, w, type, dst, nullptr, STREAM(stream));
}

// ------------------------------------------- the allocation-free variant
// cx_matmul_auto for callers that cannot allocate: its scratch is this
// fixed array, one copy per GPU, held until the process ends. Every call on
// a GPU shares that GPU's copy, so calls that overlap on one GPU (from any
// thread or stream) race; nothing in it needs to start at zero (the
// quantization writes every byte the contraction reads).
static __device__ __align__(256) uint8_t scratch[CX_NOALLOC_SCRATCH_BYTES];

// The array's device address on each GPU, looked up with that device
// current (the host-side name is not a device address). Only a successful
// lookup is kept; a failed one is tried again by the next call.
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];

static int noalloc_scratch(int dev, void** out) {
  CX_REQUIRE(dev >= 0 && dev < 64, "no HIP device %d", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int prev = 0;
    void* p = nullptr;
    hipError_t e = hipGetDevice(&prev);
    if (e == hipSuccess) e = hipSetDevice(dev);
    if (e == hipSuccess) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      const hipError_t r = hipSetDevice(prev);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess || !p) {
      cx_set_error("matmul_auto_noalloc: the scratch of device %d has no address: %s", dev,
                   hipGetErrorString(e));
      return CX_EHIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CX_OK;
}

extern "C" int cx_matmul_auto_noalloc(size_t m, size_t k, size_t n, const float* lhs,
                                      const uint8_t* w, int type, float* dst, void* stream) {
  int rc = matmul_auto_check(k, n, lhs, w, type, dst);
  if (rc) return rc;
  const size_t need = matmul_auto_scratch(m, k, type);
  CX_REQUIRE(need <= CX_NOALLOC_SCRATCH_BYTES,
             "matmul_auto_noalloc: %zu x %zu rows need %zu bytes of scratch, past its %d", m, k,
             need, CX_NOALLOC_SCRATCH_BYTES);
  int dev = 0;
  CX_HIP(hipGetDevice(&dev));
  void* sp = nullptr;
  if ((rc = noalloc_scratch(dev, &sp))) return rc;
  return matmul_auto_on(m, k, n, lhs, w, type, dst, sp, STREAM(stream));
}

extern "C" int cx_matmul_multi_1row(const float* x, size_t k, size_t count,
                                    const uint8_t* const* w, const int* types, const size_t* ns,
                                    float* const* dsts, void* stream) {
  CX_REQUIRE(x && w && types && ns && dsts, "multi: null pointer");
  // the row quantized once per sub-block size in use (16 and/or 32)
  bool need16 = false, need32 = false;
  for (size_t i = 0; i < count; i++) {
    CX_REQUIRE(cx_has_gemv(types[i]), "multi: type %d has no quantized path here", types[i]);
    CX_REQUIRE(k % (size_t)cx_vpb(types[i]) == 0, "multi: a row of %zu is not whole blocks of type %d",
               k, types[i]);
    (cx_sub(types[i]) == 16 ? need16 : need32) = true;
  }
  QuantScratch q16, q32;
  cx_scratch scr(STREAM(stream));
  int rc = quant_scratch(scr, 1, k, need16 ? &q16 : nullptr, need32 ? &q32 : nullptr);
  if (rc) return rc;
  if (need16 && (rc = cx_launch_quantize(x, 1, k, 16, q16.xq, q16.xe, q16.xs, STREAM(stream))))
    return rc;
  if (need32 && (rc = cx_launch_quantize(x, 1, k, 32, q32.xq, q32.xe, q32.xs, STREAM(stream))))
    return rc;
  std::vector<bool> done(count, false);
  for (size_t i = 0; i < count; i++) {
    if (done[i]) continue;
    cx_seg segs[4];
    int nseg = 0;
    for (size_t j = i; j < count && nseg < 4; j++) {
      if (done[j] || types[j] != types[i]) continue;
      segs[nseg++] = cx_seg{w[j], dsts[j], nullptr, (uint32_t)ns[j]};
      done[j] = true;
    }
    const QuantScratch& q = cx_sub(types[i]) == 16 ? q16 : q32;
    rc = cx_launch_gemv(types[i], segs, nseg, (uint32_t)k, q.row(0, k, cx_sub(types[i])),
                        CX_EPI_STORE, nullptr, STREAM(stream));
    if (rc) return rc;
  }
  return CX_OK;
}

extern "C" int cx_rmsnorm(float* out, const float* in, const float* w, size_t rows, size_t n,
                          float eps, void* stream) {
  return cx_launch_rmsnorm(out, in, w, rows, n, eps, STREAM(stream));
}
extern "C" int cx_silu(float* out, const float* in, size_t n, void* stream) {
  CX_REQUIRE(out && in, "silu: null pointer");
  return cx_launch_silu(out, in, n, STREAM(stream));
}

// src/ops.rs:1108-1129: f32 powf frequency, f64 angle, f64 cos/sin, f32 store
extern "C" int cx_rope_tables(size_t hd, float base, size_t ctx, float* c, float* s) {
  CX_REQUIRE(hd % 2 == 0 && c && s, "rope_tables: head_dim %zu must be even", hd);
  const size_t half = hd / 2;
  for (size_t j = 0; j < half; j++) {
    const float freq = 1.0f / powf(base, 2.0f * (float)j / (float)hd);
    for (size_t p = 0; p < ctx; p++) {
      const double ang = (double)p * (double)freq;
      c[p * half + j] = (float)cos(ang);
      s[p * half + j] = (float)sin(ang);
    }
  }
  return CX_OK;
}

extern "C" int cx_rope(float* x, size_t tokens, size_t heads, size_t hd, const float* cos_t,
                       const float* sin_t, size_t ctx, size_t pos, void* stream) {
  CX_REQUIRE(hd % 2 == 0, "rope: head_dim %zu must be even", hd);
  CX_REQUIRE(pos + tokens <= ctx, "rope: positions %zu..%zu past the table of %zu", pos,
             pos + tokens, ctx);
  CX_REQUIRE(x && cos_t && sin_t, "rope: null pointer");
  return cx_launch_rope(x, tokens, heads, hd, cos_t, sin_t, pos, STREAM(stream));
}

extern "C" int cx_softmax(float* x, size_t len, size_t width, void* stream) {
  CX_REQUIRE(x, "softmax: null pointer");
  return cx_launch_softmax(x, len, width, STREAM(stream));
}

extern "C" int cx_attention(const float* q, const float* k, const float* v, size_t tokens,
                            size_t total, size_t heads, size_t kv_heads, size_t hd, float* out,
                            void* stream) {
  CX_REQUIRE(q && k && v && out, "attention: null pointer");
  return cx_launch_attention(q, k, v, tokens, total, heads, kv_heads, hd, out, STREAM(stream));
}

extern "C" int cx_attention_decode(const float* q, const float* k, const float* v, size_t total,
                                   size_t heads, size_t kvh, size_t hd, int mode, float* out,
                                   void* stream) {
  CX_REQUIRE(q && k && v && out && total > 0, "attention_decode: bad arguments");
  CX_REQUIRE(mode >= 0 && mode <= 2, "attention_decode: mode %d", mode);
  const size_t cap = total;
  const size_t ns = cx_attn_splits(cap);
  auto up = [](size_t n) { return (n + 255) / 256 * 256; };
  const size_t o_pm = 256, o_pl = o_pm + up(ns * heads * 4), o_po = o_pl + up(ns * heads * 4),
               o_sc = o_po + up(ns * heads * hd * 4),
               o_cm = o_sc + up(cx_attn_score_floats(heads, cap) * 4),
               bytes = o_cm + up(cx_attn_chunk_floats(heads, cap) * 4);
  void* sp = nullptr;
  cx_scratch scr(STREAM(stream));
  int rc = scr.get(bytes, &sp);
  if (rc) return rc;
  uint8_t* b = (uint8_t*)sp;
  cx_dstate* st = (cx_dstate*)b;
  float* pm = (float*)(b + o_pm);
  float* pl = (float*)(b + o_pl);
  float* po = (float*)(b + o_po);
  float* sc = (float*)(b + o_sc);
  float* cm = (float*)(b + o_cm);
  hipStream_t s = STREAM(stream);
  // the kernels read the position from device state: pos = total - 1
  cx_dstate h{(uint32_t)(total - 1), 0u, (uint32_t)cap, 0u};
  CX_HIP(hipMemcpyAsync(st, &h, sizeof h, hipMemcpyHostToDevice, s));
  cx_attn_args a{};
  a.q = (float*)q;  // not written: no rope tables
  a.kc = (float*)k;
  a.vc = (float*)v;
  a.heads = (uint32_t)heads;
  a.kvh = (uint32_t)kvh;
  a.hd = (uint32_t)hd;
  a.cap = (uint32_t)cap;
  a.st = st;
  a.pm = pm;
  a.pl = pl;
  a.po = po;
  a.sc = sc;
  a.cm = cm;
  a.out = out;
  a.mode = mode;
  rc = cx_launch_attn_decode(a, s);
  if (rc) return rc;
  CX_HIP(hipStreamSynchronize(s));  // the state lives in shared scratch
  return CX_OK;
}

extern "C" int cx_argmax(const float* v, size_t n, uint32_t* out, void* stream) {
  return cx_launch_argmax_one(v, n, out, STREAM(stream));
}

// Muestreador::nuevo (src/sampler.rs:38-47): Azar::con_semilla (a zero seed
// is remapped, src/daiss.rs:322-328), 1/temperature, top_p clamped to [0, 1]
// (a NaN stays NaN, as f32::clamp leaves it)
static cx_samp_state sampler_state(uint64_t seed, float temperature, float top_p) {
  cx_samp_state h{};
  h.azar = seed ? seed : 0x9E3779B97F4A7C15ull;
  h.inv = 1.0f / temperature;
  h.top_p = top_p < 0.0f ? 0.0f : (top_p > 1.0f ? 1.0f : top_p);
  return h;
}

// Muestreador::elegir (src/sampler.rs:61-125) on device logits; the
// generator's state is the caller's (host), advanced by one draw when
// temperature > 0. Returns when *out (host) holds the token.
extern "C" int cx_sample(const float* logits, size_t n, float temperature, float top_p,
                         uint64_t* state, uint32_t* out, void* stream) {
  CX_REQUIRE(state && out, "sample: null state or output");
  if (n == 0) {  // src/sampler.rs:62-64
    *out = 0;
    return CX_OK;
  }
  CX_REQUIRE(logits && n < (1u << 31), "sample: bad logits (n=%zu)", n);
  hipStream_t s = STREAM(stream);
  auto up = [](size_t b) { return (b + 255) / 256 * 256; };
  // (the chains' 16-byte loads may reach 3 floats past the last value)
  const size_t o_pb = 256, o_part = o_pb + up((n + 4) * 4),
               o_ord = o_part + up(cx_sample_parts(n) * 4), o_ordp = o_ord + up(n * 4),
               o_tok = o_ordp + up((n + 4) * 4), bytes = o_tok + 256;
  void* sp = nullptr;
  cx_scratch scr(s);
  int rc = scr.get(bytes, &sp);
  if (rc) return rc;
  uint8_t* b = (uint8_t*)sp;
  uint32_t* tok = (uint32_t*)(b + o_tok);
  if (temperature <= 0.0f) {  // greedy: the argmax, no draw
    if ((rc = cx_launch_argmax_one(logits, n, tok, s))) return rc;
    CX_HIP(hipMemcpyAsync(out, tok, 4, hipMemcpyDeviceToHost, s));
    CX_HIP(hipStreamSynchronize(s));
    return CX_OK;
  }
  cx_samp_state h = sampler_state(1, temperature, top_p);
  h.azar = *state;  // the caller's generator, as it stands
  cx_samp_state* sd = (cx_samp_state*)b;
  CX_HIP(hipMemcpyAsync(sd, &h, sizeof h, hipMemcpyHostToDevice, s));
  if ((rc = cx_launch_sample(logits, n, sd, (float*)(b + o_pb), (float*)(b + o_part),
                             (uint32_t*)(b + o_ord), (float*)(b + o_ordp), tok, nullptr, nullptr,
                             nullptr, s)))
    return rc;
  CX_HIP(hipMemcpyAsync(&h, sd, sizeof h, hipMemcpyDeviceToHost, s));
  CX_HIP(hipStreamSynchronize(s));
  *state = h.azar;
  *out = h.token;
  return CX_OK;
}

// ================================================================ 3. model
namespace {
struct Tensor {
  std::string name;
  int type;
  uint64_t dims[2];  // width, rows (1 for a vector)
  uint32_t n_dims;   // as stored in GGUF
  size_t bytes;
  size_t offset;     // in the model's pool
};
// one layer (src/forward.rs:139-156, Capa): every matrix with its own type, as
// in real GGUF files (Q4_K_M keeps some attn_v / ffn_down in Q6_K); biases
// may be absent (architectures without them)
struct Layer {
  const float *attn_norm, *q_bias, *k_bias, *v_bias, *ffn_norm;
  const uint8_t *q, *k, *v, *o, *gate, *up, *down;
  int t_q, t_k, t_v, t_o, t_gate, t_up, t_down;
};
}  // namespace

struct cx_model {
  cx_config cfg;
  int device;
  // caches made from this model and not yet freed; a model freed while some
  // remain is released by the last cx_cache_free (they use its stream and
  // buffers)
  int n_caches;
  bool closed;
  int t_embd, t_out;
  bool tied;  // no output.weight: the lm_head is token_embd (src/forward.rs:218-227)
  hipStream_t stream;
  uint8_t* pool;
  size_t pool_bytes;
  std::vector<Tensor> tensors;
  std::vector<Layer> layers;
  const uint8_t* embd;
  const float* out_norm;
  const uint8_t* out;
  float *cos_t, *sin_t;
  // per-step activations
  float *x, *q, *k, *v, *att, *g, *u, *logits, *apv;
  uint32_t* api;
  uint32_t* amax_out;
  // the i8 activation of the next GEMV: max(dim, ffn) values, sub >= 16
  int8_t* xq;
  float *xe, *xs;
};

// The batched prefill's buffers: T tokens of every activation, the
// contraction's quantized rows, and T query tokens of attention scratch.
// Made at a cache's first multi-token forward.
struct cx_prefill {
  uint32_t T;
  float *x, *nrm, *q, *k, *v, *att, *g, *u, *tmp;  // nrm also holds the SwiGLU rows
  float *sc, *cm;
  void* scratch;
};

struct cx_cache {
  cx_model* m;
  size_t cap, len;
  float* kv;        // [layers][2][cap][kvd]
  uint32_t* hist;   // tokens by position, cap + 1
  uint32_t* htok;   // the generated tokens by position, pinned host memory, cap + 1
  uint32_t* htok_dev;  // its device address (written by the token loop's last kernel)
  cx_dstate* st;
  float *pm, *pl, *po;  // split-K partials
  float* sc;            // scores of the order-exact attention, heads x cap
  float* cm;            // and their maxima per chunk of positions
  hipGraphExec_t exec;    // the captured step (greedy tail)
  bool have_graph;
  hipGraphExec_t exec_s;  // the captured step with the sampler's tail
  bool have_graph_s;
  bool sampling;          // steps and prefills take the sampler's tail
  // the sampler's state and scratch, made at the first sampled generation
  cx_samp_state* sd;
  float *spb, *spart, *sordp;
  uint32_t* sord;
  cx_prefill pf;
};

static void* pool_at(cx_model* m, size_t off) { return m->pool + off; }

static void model_destroy(cx_model* m) {
  (void)hipSetDevice(m->device);
  (void)hipStreamSynchronize(m->stream);
  float* bufs[] = {m->x,      m->q,   m->k,     m->v,     m->att, m->g, m->u,
                   m->logits, m->apv, m->cos_t, m->sin_t, m->xe,  m->xs};
  for (float* b : bufs)
    if (b) (void)hipFree(b);
  if (m->xq) (void)hipFree(m->xq);
  if (m->api) (void)hipFree(m->api);
  if (m->amax_out) (void)hipFree(m->amax_out);
  if (m->pool) (void)hipFree(m->pool);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
}

extern "C" void cx_model_free(cx_model* m) {
  if (!m) return;
  m->closed = true;
  if (m->n_caches == 0) model_destroy(m);
}

static cx_model* model_new(const cx_config& c) {
  if (hipSetDevice(g_device) != hipSuccess) {
    cx_set_error("model: no HIP device %d", g_device);
    return nullptr;
  }
  cx_model* m = new cx_model();
  m->cfg = c;
  m->device = g_device;
  if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess) {
    m->stream = nullptr;
    cx_model_free(m);
    cx_set_error("model: stream");
    return nullptr;
  }
  return m;
}

static size_t tensor_bytes(int t, uint64_t w, uint64_t r) {
  return (size_t)(w / (uint64_t)cx_vpb(t) * (uint64_t)cx_bpb(t) * r);
}

// Views of the model's tensors by name (src/forward.rs:210-247), with the
// shapes and types this path computes: matrices in a GEMV type (Q2_K..Q6_K
// on widths of whole 256-value blocks, Q8_0/Q5_0 on widths of 32),
// norms and biases F32, token_embd in any type with a dequantizer, the lm_head
// a GEMV type or F32/F16 (tied to token_embd when output.weight is absent).
static int bind_views(cx_model* m) {
  cx_config& c = m->cfg;
  auto find = [&](const std::string& n) -> const Tensor* {
    for (const Tensor& T : m->tensors)
      if (T.name == n) return &T;
    return nullptr;
  };
  const Tensor* E = find("token_embd.weight");
  CX_REQUIRE(E, "model: missing tensor token_embd.weight");
  CX_REQUIRE(E->dims[0] == c.dim, "model: token_embd rows of %llu values, dim is %u",
             (unsigned long long)E->dims[0], c.dim);
  c.vocab = (uint32_t)E->dims[1];
  CX_REQUIRE(c.vocab > 0 && cx_vpb(E->type) > 0, "model: token_embd of type %d", E->type);
  m->t_embd = E->type;
  m->embd = (const uint8_t*)pool_at(m, E->offset);
  CX_REQUIRE(c.heads && c.kv_heads && c.dim % c.heads == 0 && c.heads % c.kv_heads == 0,
             "model: %u heads / %u kv heads do not divide dim %u", c.heads, c.kv_heads, c.dim);
  const uint32_t D = c.dim, hd = D / c.heads, kvd = c.kv_heads * hd;
  CX_REQUIRE(hd == 64 || hd == 128, "model: head_dim %u (the decode attention supports 64 and 128)",
             hd);
  CX_REQUIRE(D % 32 == 0, "model: dim %u is not a multiple of 32", D);
  auto vec = [&](const std::string& n, uint64_t len, bool optional,
                 const float** p) -> int {
    const Tensor* T = find(n);
    if (!T && optional) {
      *p = nullptr;
      return CX_OK;
    }
    CX_REQUIRE(T, "model: missing tensor %s", n.c_str());
    CX_REQUIRE(T->type == CX_F32 && T->dims[0] * T->dims[1] == len,
               "model: %s must be F32 of %llu values", n.c_str(), (unsigned long long)len);
    *p = (const float*)pool_at(m, T->offset);
    return CX_OK;
  };
  auto mat = [&](const std::string& n, uint64_t w, uint64_t r, const uint8_t** p,
                 int* t) -> int {
    const Tensor* T = find(n);
    CX_REQUIRE(T, "model: missing tensor %s", n.c_str());
    CX_REQUIRE(cx_has_gemv(T->type),
               "model: %s is of type %d; the GEMV reads Q2_K..Q6_K, Q8_0 and Q5_0", n.c_str(),
               T->type);
    CX_REQUIRE(w % (uint64_t)cx_vpb(T->type) == 0, "model: %s rows of %llu values are not whole blocks",
               n.c_str(), (unsigned long long)w);
    CX_REQUIRE(T->dims[0] == w && T->dims[1] == r, "model: %s is %llux%llu, expected %llux%llu",
               n.c_str(), (unsigned long long)T->dims[0], (unsigned long long)T->dims[1],
               (unsigned long long)w, (unsigned long long)r);
    *p = (const uint8_t*)pool_at(m, T->offset);
    *t = T->type;
    return CX_OK;
  };
  const Tensor* G0 = find("blk.0.ffn_gate.weight");
  CX_REQUIRE(G0, "model: missing tensor blk.0.ffn_gate.weight");
  c.ffn = (uint32_t)G0->dims[1];
  CX_REQUIRE(c.ffn % 32 == 0, "model: ffn %u is not a multiple of 32", c.ffn);
  const uint32_t I = c.ffn;
  m->layers.clear();
  int rc;
  for (uint32_t i = 0; i < c.layers; i++) {
    const std::string p = "blk." + std::to_string(i) + ".";
    Layer L{};
    if ((rc = vec(p + "attn_norm.weight", D, false, &L.attn_norm)) ||
        (rc = mat(p + "attn_q.weight", D, D, &L.q, &L.t_q)) ||
        (rc = vec(p + "attn_q.bias", D, true, &L.q_bias)) ||
        (rc = mat(p + "attn_k.weight", D, kvd, &L.k, &L.t_k)) ||
        (rc = vec(p + "attn_k.bias", kvd, true, &L.k_bias)) ||
        (rc = mat(p + "attn_v.weight", D, kvd, &L.v, &L.t_v)) ||
        (rc = vec(p + "attn_v.bias", kvd, true, &L.v_bias)) ||
        (rc = mat(p + "attn_output.weight", D, D, &L.o, &L.t_o)) ||
        (rc = vec(p + "ffn_norm.weight", D, false, &L.ffn_norm)) ||
        (rc = mat(p + "ffn_gate.weight", D, I, &L.gate, &L.t_gate)) ||
        (rc = mat(p + "ffn_up.weight", D, I, &L.up, &L.t_up)) ||
        (rc = mat(p + "ffn_down.weight", I, D, &L.down, &L.t_down)))
      return rc;
    m->layers.push_back(L);
  }
  if ((rc = vec("output_norm.weight", D, false, &m->out_norm))) return rc;
  const Tensor* O = find("output.weight");
  m->tied = O == nullptr;
  if (!O) O = E;
  CX_REQUIRE(cx_has_gemv(O->type) || O->type == CX_F32 || O->type == CX_F16,
             "model: the output matrix is of type %d (GEMV types or F32/F16)", O->type);
  CX_REQUIRE(D % (uint32_t)cx_vpb(O->type) == 0, "model: output rows of %u values are not whole blocks",
             D);
  CX_REQUIRE(O->dims[0] == D && O->dims[1] == c.vocab, "model: output.weight shape");
  m->t_out = O->type;
  m->out = (const uint8_t*)pool_at(m, O->offset);
  return CX_OK;
}

// rope tables and the per-step buffers of a model whose views are bound
static int model_finish(cx_model* m) {
  const cx_config& c = m->cfg;
  const uint32_t D = c.dim, hd = D / c.heads, kvd = c.kv_heads * hd, I = c.ffn, V = c.vocab;
  CX_REQUIRE(c.ctx > 0, "model: zero context");
  // rope tables on the host, exactly as src/ops.rs:1108-1129, then uploaded
  const size_t n = (size_t)c.ctx * (hd / 2);
  std::vector<float> hc(n), hs(n);
  cx_rope_tables(hd, c.rope_base, c.ctx, hc.data(), hs.data());
  if (hipMalloc(&m->cos_t, n * 4) != hipSuccess || hipMalloc(&m->sin_t, n * 4) != hipSuccess ||
      hipMemcpy(m->cos_t, hc.data(), n * 4, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(m->sin_t, hs.data(), n * 4, hipMemcpyHostToDevice) != hipSuccess) {
    cx_set_error("model: rope tables");
    return CX_ENOMEM;
  }
  // the argmax's pairs: its own first step's, or the lm_head epilogue's
  const size_t parts = std::max(cx_argmax_parts(V), (size_t)cx_gemv_argmax_parts(m->t_out, V, D));
  if (hipMalloc(&m->x, D * 4) || hipMalloc(&m->q, D * 4) || hipMalloc(&m->k, kvd * 4) ||
      hipMalloc(&m->v, kvd * 4) || hipMalloc(&m->att, D * 4) || hipMalloc(&m->g, I * 4) ||
      hipMalloc(&m->u, I * 4) || hipMalloc(&m->logits, (size_t)V * 4) ||
      hipMalloc(&m->apv, parts * 4) || hipMalloc(&m->api, parts * 4) ||
      hipMalloc(&m->amax_out, 4) || hipMalloc(&m->xq, (D > I ? D : I)) ||
      hipMalloc(&m->xe, (D > I ? D : I) / 16 * 4) || hipMalloc(&m->xs, (D > I ? D : I) / 16 * 4)) {
    cx_set_error("model: activation buffers");
    return CX_ENOMEM;
  }
  return CX_OK;
}

// src/daiss.rs:396-407 (inicio_de)
static float init_sigma(const std::string& n, uint32_t layers, int* kind) {
  auto ends = [&](const char* s) {
    size_t l = strlen(s);
    return n.size() >= l && n.compare(n.size() - l, l, s) == 0;
  };
  if (ends(".bias")) { *kind = 0; return 0.0f; }
  if (ends("_norm.weight")) { *kind = 1; return 1.0f; }
  *kind = 2;
  if (ends("attn_output.weight") || ends("ffn_down.weight"))
    return 0.02f / sqrtf(2.0f * (float)layers);
  return 0.02f;
}

extern "C" int cx_model_create_daiss(const cx_config* cfg, int t_lin, int t_down, int t_out,
                                     uint64_t seed, cx_model** out) {
  CX_REQUIRE(cfg && out, "model: null argument");
  const cx_config c = *cfg;
  CX_REQUIRE(c.layers && c.dim && c.heads && c.kv_heads && c.ffn && c.vocab && c.ctx,
             "model: zero-sized config");
  CX_REQUIRE(c.dim % c.heads == 0 && c.heads % c.kv_heads == 0, "model: heads do not divide");
  CX_REQUIRE(c.dim / c.heads == 64 || c.dim / c.heads == 128,
             "model: head_dim %u (the decode attention supports 64 and 128)", c.dim / c.heads);
  // the quantizers the reference has (src/quant.rs:744-805): Q8_0 on rows of
  // 32 values, Q2_K..Q5_K on rows of 256 (Config::admite_kquants,
  // src/daiss.rs:210-220)
  for (int t : {t_lin, t_down, t_out}) {
    CX_REQUIRE(t == CX_Q8_0 || (cx_is_kquant(t) && t != CX_Q6_K),
               "model: weights must be Q8_0 or Q2_K..Q5_K (the quantizers the reference has)");
    CX_REQUIRE(c.dim % cx_vpb(t) == 0 && c.ffn % cx_vpb(t) == 0,
               "model: dim %u and ffn %u are not whole blocks of type %d", c.dim, c.ffn, t);
  }
  cx_model* m = model_new(c);
  if (!m) return CX_EHIP;
  const uint32_t D = c.dim, hd = D / c.heads, kvd = c.kv_heads * hd, I = c.ffn, V = c.vocab;
  // tensor table in the order of src/daiss.rs:236-303; token_embd F32 (the
  // BASELINE fixtures keep embeddings f32)
  auto add = [&](const std::string& n, int t, uint64_t w, uint64_t r) {
    Tensor T{n, t, {w, r}, r == 1 ? 1u : 2u, tensor_bytes(t, w, r), 0};
    m->tensors.push_back(T);
  };
  add("token_embd.weight", CX_F32, D, V);
  for (uint32_t i = 0; i < c.layers; i++) {
    const std::string p = "blk." + std::to_string(i) + ".";
    add(p + "attn_norm.weight", CX_F32, D, 1);
    add(p + "attn_q.weight", t_lin, D, D);
    add(p + "attn_q.bias", CX_F32, D, 1);
    add(p + "attn_k.weight", t_lin, D, kvd);
    add(p + "attn_k.bias", CX_F32, kvd, 1);
    add(p + "attn_v.weight", t_lin, D, kvd);
    add(p + "attn_v.bias", CX_F32, kvd, 1);
    add(p + "attn_output.weight", t_lin, D, D);
    add(p + "ffn_norm.weight", CX_F32, D, 1);
    add(p + "ffn_gate.weight", t_lin, D, I);
    add(p + "ffn_up.weight", t_lin, D, I);
    add(p + "ffn_down.weight", t_down, I, D);
  }
  add("output_norm.weight", CX_F32, D, 1);
  add("output.weight", t_out, D, V);
  size_t off = 0, biggest = 0;
  for (Tensor& T : m->tensors) {
    T.offset = off;
    off += (T.bytes + 255) / 256 * 256;
    const size_t elems = T.dims[0] * T.dims[1];
    if (T.type != CX_F32 && elems > biggest) biggest = elems;
  }
  m->pool_bytes = off;
  int rc = CX_OK;
  float* tmp = nullptr;
  auto fail = [&](int code) {
    if (tmp) (void)hipFree(tmp);
    cx_model_free(m);
    return code;
  };
  if (hipMalloc(&m->pool, m->pool_bytes) != hipSuccess) {
    cx_set_error("model: cannot allocate %zu bytes of weights", m->pool_bytes);
    return fail(CX_ENOMEM);
  }
  if (hipMalloc(&tmp, biggest * sizeof(float)) != hipSuccess) {
    cx_set_error("model: cannot allocate the generation buffer");
    return fail(CX_ENOMEM);
  }
  for (const Tensor& T : m->tensors) {
    int kind;
    const float sigma = init_sigma(T.name, c.layers, &kind);
    const size_t elems = T.dims[0] * T.dims[1];
    float* dstf = T.type == CX_F32 ? (float*)pool_at(m, T.offset) : tmp;
    if (kind == 2)
      rc = cx_gen_rows_f32(dstf, cx_fnv_name(T.name.c_str()), seed, (uint32_t)T.dims[1],
                           (uint32_t)T.dims[0], sigma, m->stream);
    else
      rc = cx_gen_fill(dstf, elems, sigma, m->stream);
    if (!rc && T.type != CX_F32)
      rc = cx_quantize_blocks_dev(T.type, tmp, elems, (uint8_t*)pool_at(m, T.offset), m->stream);
    if (rc) return fail(rc);
  }
  if (hipStreamSynchronize(m->stream) != hipSuccess) {
    cx_set_error("model: generation failed: %s", hipGetErrorString(hipGetLastError()));
    return fail(CX_EHIP);
  }
  (void)hipFree(tmp);
  tmp = nullptr;
  if ((rc = bind_views(m)) || (rc = model_finish(m))) return fail(rc);
  *out = m;
  return CX_OK;
}

// The tensors of a Qwen2-style model (src/forward.rs:210-247); anything else
// in the file is not loaded
static bool model_tensor_name(const std::string& n) {
  static const char* top[] = {"token_embd.weight", "output_norm.weight", "output.weight"};
  for (const char* t : top)
    if (n == t) return true;
  if (n.compare(0, 4, "blk.") != 0) return false;
  static const char* per[] = {".attn_norm.weight", ".attn_q.weight", ".attn_q.bias",
                              ".attn_k.weight",    ".attn_k.bias",   ".attn_v.weight",
                              ".attn_v.bias",      ".attn_output.weight", ".ffn_norm.weight",
                              ".ffn_gate.weight",  ".ffn_up.weight", ".ffn_down.weight"};
  for (const char* t : per) {
    const size_t l = strlen(t);
    if (n.size() > l && n.compare(n.size() - l, l, t) == 0) return true;
  }
  return false;
}

// Modelo::abrir (src/forward.rs:187-266): config from the <arch>.* metadata
// (the reference reads qwen2.*; general.architecture names the prefix), every
// tensor the forward uses uploaded to one HBM pool unchanged (the kernels
// read GGUF bytes as they are), read through a pinned staging buffer.
extern "C" int cx_model_open(const char* path, cx_model** out) {
  CX_REQUIRE(path && out, "model: null argument");
  *out = nullptr;
  cx_gguf* g = nullptr;
  int rc = cx_gguf_read(path, &g);
  if (rc) return rc;
  struct Closer {
    cx_gguf* g;
    ~Closer() { cx_gguf_release(g); }
  } closer{g};
  char arch[64] = "qwen2";
  size_t alen = 0;
  if (cx_gguf_meta_str(g, "general.architecture", -1, arch, sizeof arch, &alen) != CX_OK)
    snprintf(arch, sizeof arch, "qwen2");
  const std::string A = arch;
  auto meta_u = [&](const char* key, uint32_t* v) -> int {
    uint64_t x;
    int r = cx_gguf_meta_int(g, (A + "." + key).c_str(), &x);
    if (r) return r;
    CX_REQUIRE(x < (1ull << 32), "model: %s.%s = %llu", A.c_str(), key, (unsigned long long)x);
    *v = (uint32_t)x;
    return CX_OK;
  };
  cx_config c{};
  if ((rc = meta_u("block_count", &c.layers)) || (rc = meta_u("embedding_length", &c.dim)) ||
      (rc = meta_u("attention.head_count", &c.heads)) ||
      (rc = meta_u("attention.head_count_kv", &c.kv_heads)) ||
      (rc = meta_u("context_length", &c.ctx)))
    return rc;
  double eps = 1e-6, base = 10000.0;
  (void)cx_gguf_meta_float(g, (A + ".attention.layer_norm_rms_epsilon").c_str(), &eps);
  (void)cx_gguf_meta_float(g, (A + ".rope.freq_base").c_str(), &base);
  c.eps = (float)eps;
  c.rope_base = (float)base;
  CX_REQUIRE(c.layers && c.dim && c.heads && c.kv_heads && c.ctx, "model: zero-sized config");
  cx_model* m = model_new(c);
  if (!m) return CX_EHIP;
  uint8_t* stage = nullptr;
  FILE* f = nullptr;
  auto fail = [&](int code) {
    if (stage) (void)hipHostFree(stage);
    if (f) fclose(f);
    cx_model_free(m);
    return code;
  };
  size_t n = 0;
  const cx_gguf_tensor* gt = cx_gguf_tensors(g, &n);
  std::vector<uint64_t> from;
  size_t off = 0;
  for (size_t i = 0; i < n; i++) {
    const cx_gguf_tensor& t = gt[i];
    if (!model_tensor_name(t.name)) continue;
    if (t.n_dims < 1 || t.n_dims > 2 || cx_vpb(t.type) == 0) {
      cx_set_error("model: %s has %u dims of type %d", t.name, t.n_dims, t.type);
      return fail(CX_EINVAL);
    }
    uint64_t at;
    if ((rc = cx_gguf_range(g, t, &at))) return fail(rc);
    Tensor T{t.name, t.type, {t.dims[0], t.n_dims == 2 ? t.dims[1] : 1}, t.n_dims,
             (size_t)t.bytes, off};
    if (T.dims[0] % (uint64_t)cx_vpb(t.type) != 0) {
      cx_set_error("model: %s rows of %llu values are not whole blocks", t.name,
                   (unsigned long long)T.dims[0]);
      return fail(CX_EINVAL);
    }
    m->tensors.push_back(T);
    from.push_back(at);
    off += (T.bytes + 255) / 256 * 256;
  }
  m->pool_bytes = off;
  if (hipMalloc(&m->pool, off) != hipSuccess) {
    cx_set_error("model: cannot allocate %zu bytes of weights", off);
    return fail(CX_ENOMEM);
  }
  const size_t STAGE = 64u << 20;
  if (hipHostMalloc((void**)&stage, STAGE) != hipSuccess) {
    stage = nullptr;
    cx_set_error("model: cannot allocate the staging buffer");
    return fail(CX_ENOMEM);
  }
  f = fopen(path, "rb");
  if (!f) {
    cx_set_error("model: cannot open %s", path);
    return fail(CX_EINVAL);
  }
  for (size_t i = 0; i < m->tensors.size(); i++) {
    const Tensor& T = m->tensors[i];
    for (size_t done = 0; done < T.bytes; done += STAGE) {
      const size_t len = T.bytes - done < STAGE ? T.bytes - done : STAGE;
      if ((rc = cx_gguf_read_bytes(g, from[i] + done, stage, len, f))) return fail(rc);
      if (hipMemcpy(m->pool + T.offset + done, stage, len, hipMemcpyHostToDevice) != hipSuccess) {
        cx_set_error("model: upload of %s failed", T.name.c_str());
        return fail(CX_EHIP);
      }
    }
  }
  fclose(f);
  f = nullptr;
  (void)hipHostFree(stage);
  stage = nullptr;
  if ((rc = bind_views(m)) || (rc = model_finish(m))) return fail(rc);
  *out = m;
  return CX_OK;
}

// The model as a GGUF file (the daiss writer's metadata, src/daiss.rs:422-468,
// and Escritor::escribir's layout): tensors in table order, bytes as in HBM.
extern "C" int cx_model_save_gguf(const cx_model* m, const char* path) {
  CX_REQUIRE(m && path, "model: null argument");
  const cx_config& c = m->cfg;
  auto u32m = [](const char* k, uint64_t v) { return cx_gguf_meta{k, 4, v, 0.0, ""}; };
  std::vector<cx_gguf_meta> meta = {
      {"general.architecture", 8, 0, 0.0, "qwen2"},
      {"general.name", 8, 0, 0.0, "cosxamix-hip"},
      u32m("qwen2.block_count", c.layers),
      u32m("qwen2.context_length", c.ctx),
      u32m("qwen2.embedding_length", c.dim),
      u32m("qwen2.feed_forward_length", c.ffn),
      u32m("qwen2.attention.head_count", c.heads),
      u32m("qwen2.attention.head_count_kv", c.kv_heads),
      {"qwen2.attention.layer_norm_rms_epsilon", 6, 0, (double)c.eps, ""},
      {"qwen2.rope.freq_base", 6, 0, (double)c.rope_base, ""},
  };
  std::vector<cx_gguf_tensor> ts;
  std::vector<std::vector<uint8_t>> host(m->tensors.size());
  std::vector<const void*> ptrs;
  CX_HIP(hipSetDevice(m->device));
  CX_HIP(hipStreamSynchronize(m->stream));
  for (size_t i = 0; i < m->tensors.size(); i++) {
    const Tensor& T = m->tensors[i];
    cx_gguf_tensor t{};
    snprintf(t.name, sizeof t.name, "%s", T.name.c_str());
    t.type = T.type;
    t.n_dims = T.n_dims;
    t.dims[0] = T.dims[0];
    t.dims[1] = T.n_dims == 2 ? T.dims[1] : 1;
    t.elements = T.dims[0] * T.dims[1];
    t.bytes = T.bytes;
    ts.push_back(t);
    host[i].resize(T.bytes);
    CX_HIP(hipMemcpy(host[i].data(), m->pool + T.offset, T.bytes, hipMemcpyDeviceToHost));
    ptrs.push_back(host[i].data());
  }
  return cx_gguf_write(path, meta, ts, ptrs);
}

extern "C" int cx_model_config(const cx_model* m, cx_config* out) {
  CX_REQUIRE(m && out, "null");
  *out = m->cfg;
  return CX_OK;
}
extern "C" int cx_model_tensor_count(const cx_model* m) { return m ? (int)m->tensors.size() : 0; }
extern "C" int cx_model_tensor_info(const cx_model* m, int idx, char* name, size_t cap, int* type,
                                    uint64_t dims[2], size_t* bytes) {
  CX_REQUIRE(m && idx >= 0 && idx < (int)m->tensors.size(), "tensor index %d", idx);
  const Tensor& T = m->tensors[idx];
  if (name && cap) snprintf(name, cap, "%s", T.name.c_str());
  if (type) *type = T.type;
  if (dims) { dims[0] = T.dims[0]; dims[1] = T.dims[1]; }
  if (bytes) *bytes = T.bytes;
  return CX_OK;
}
extern "C" int cx_model_tensor_copy(const cx_model* m, int idx, void* host, size_t bytes) {
  CX_REQUIRE(m && idx >= 0 && idx < (int)m->tensors.size() && host, "tensor copy: index %d", idx);
  const Tensor& T = m->tensors[idx];
  CX_REQUIRE(bytes >= T.bytes, "tensor copy: %zu bytes for a tensor of %zu", bytes, T.bytes);
  CX_HIP(hipSetDevice(m->device));
  CX_HIP(hipMemcpy(host, m->pool + T.offset, T.bytes, hipMemcpyDeviceToHost));
  return CX_OK;
}
extern "C" const void* cx_model_tensor_data(const cx_model* m, int idx) {
  if (!m || idx < 0 || idx >= (int)m->tensors.size()) {
    cx_set_error("tensor index %d", idx);
    return nullptr;
  }
  return m->pool + m->tensors[idx].offset;
}
extern "C" size_t cx_model_weight_bytes(const cx_model* m) {
  if (!m) return 0;
  size_t b = 0;
  for (const Tensor& T : m->tensors)
    if (T.name != "token_embd.weight") b += T.bytes;
  // one embedding row; a tied lm_head reads the whole table
  const size_t row = tensor_bytes(m->t_embd, m->cfg.dim, 1);
  return b + row + (m->tied ? tensor_bytes(m->t_embd, m->cfg.dim, m->cfg.vocab) : 0);
}

// ------------------------------------------------------------------ cache
extern "C" int cx_cache_new(cx_model* m, size_t cap, cx_cache** out) {
  CX_REQUIRE(m && out && cap > 0, "cache: bad arguments");
  CX_REQUIRE(cap <= m->cfg.ctx, "cache: %zu tokens past the context of %u", cap, m->cfg.ctx);
  CX_HIP(hipSetDevice(m->device));
  const cx_config& c = m->cfg;
  const size_t kvd = (size_t)c.kv_heads * (c.dim / c.heads);
  CX_REQUIRE(!m->closed, "cache: the model was freed");
  cx_cache* C = new cx_cache();
  C->m = m;
  m->n_caches++;
  C->cap = cap;
  C->len = 0;
  const size_t ns = cx_attn_splits(cap);
  if (hipMalloc(&C->kv, (size_t)c.layers * 2 * cap * kvd * 4) || hipMalloc(&C->hist, (cap + 1) * 4) ||
      hipMalloc(&C->st, sizeof(cx_dstate)) || hipMalloc(&C->pm, ns * c.heads * 4) ||
      hipMalloc(&C->pl, ns * c.heads * 4) || hipMalloc(&C->po, ns * c.heads * (c.dim / c.heads) * 4) ||
      hipMalloc(&C->sc, cx_attn_score_floats(c.heads, cap) * 4) ||
      hipMalloc(&C->cm, cx_attn_chunk_floats(c.heads, cap) * 4) ||
      hipHostMalloc((void**)&C->htok, (cap + 1) * 4, hipHostMallocMapped) ||
      hipHostGetDevicePointer((void**)&C->htok_dev, C->htok, 0)) {
    cx_cache_free(C);
    cx_set_error("cache: cannot allocate %zu tokens", cap);
    return CX_ENOMEM;
  }
  *out = C;
  return CX_OK;
}
extern "C" size_t cx_cache_len(const cx_cache* c) { return c ? c->len : 0; }
// src/forward.rs:98-110
extern "C" int cx_cache_truncate(cx_cache* c, size_t n) {
  CX_REQUIRE(c, "null cache");
  if (n < c->len) c->len = n;
  return CX_OK;
}
extern "C" void cx_cache_clear(cx_cache* c) {
  if (c) c->len = 0;
}
// Cache::bytes (src/forward.rs:130-136): the f32 K and V the cache holds,
// len tokens of every layer
extern "C" size_t cx_cache_bytes(const cx_cache* c) {
  if (!c) return 0;
  const cx_config& g = c->m->cfg;
  return c->len * 2 * (size_t)g.layers * g.kv_heads * (g.dim / g.heads) * 4;
}
// Cache::prefijo (src/forward.rs:117-128): a new cache of `cap` tokens (0 =
// the source's capacity) holding a copy of the source's first min(n, len)
// tokens; stream-ordered after the source's work
extern "C" int cx_cache_prefix(const cx_cache* src, size_t n, size_t cap, cx_cache** out) {
  CX_REQUIRE(src && out, "cache prefix: null argument");
  cx_model* m = src->m;
  const size_t keep = n < src->len ? n : src->len;
  if (!cap) cap = src->cap;
  CX_REQUIRE(keep <= cap, "cache prefix: %zu tokens do not fit a cache of %zu", keep, cap);
  cx_cache* C = nullptr;
  int rc = cx_cache_new(m, cap, &C);
  if (rc) return rc;
  const cx_config& g = m->cfg;
  const size_t kvd = (size_t)g.kv_heads * (g.dim / g.heads);
  hipStream_t s = m->stream;
  if (keep) {
    for (uint32_t l = 0; l < g.layers; l++)
      for (int kv = 0; kv < 2; kv++) {
        const float* from = src->kv + ((size_t)l * 2 + kv) * src->cap * kvd;
        float* to = C->kv + ((size_t)l * 2 + kv) * cap * kvd;
        if (hipMemcpyAsync(to, from, keep * kvd * 4, hipMemcpyDeviceToDevice, s) != hipSuccess) {
          cx_cache_free(C);
          cx_set_error("cache prefix: copy failed");
          return CX_EHIP;
        }
      }
    if (hipMemcpyAsync(C->hist, src->hist, keep * 4, hipMemcpyDeviceToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
      cx_cache_free(C);
      cx_set_error("cache prefix: copy failed");
      return CX_EHIP;
    }
  }
  C->len = keep;
  *out = C;
  return CX_OK;
}
extern "C" void cx_cache_free(cx_cache* c) {
  if (!c) return;
  (void)hipSetDevice(c->m->device);
  (void)hipStreamSynchronize(c->m->stream);
  if (c->have_graph) (void)hipGraphExecDestroy(c->exec);
  if (c->have_graph_s) (void)hipGraphExecDestroy(c->exec_s);
  const cx_prefill& P = c->pf;
  void* bufs[] = {c->kv,   c->hist, c->st,   c->pm,    c->pl,    c->po,  c->sc,    c->cm,
                  c->sd,   c->spb,  c->spart, c->sordp, c->sord,  P.x,    P.nrm,    P.q,
                  P.k,     P.v,     P.att,   P.g,      P.u,      P.tmp,  P.sc,     P.cm,
                  P.scratch};
  for (void* b : bufs)
    if (b) (void)hipFree(b);
  if (c->htok) (void)hipHostFree(c->htok);
  cx_model* m = c->m;
  delete c;
  if (--m->n_caches == 0 && m->closed) model_destroy(m);
}

// ------------------------------------------------------- one decode step
// src/forward.rs:420-501 for one token at position st->pos, then argmax and
// the position advance. Every kernel reads the position from the device
// state, so the sequence is captured once per cache and replayed.
// The fused-norm GEMV over matrices that share an input, one launch per
// weight type (proyectar_varias, src/forward.rs:333-368): rmsnorm(x, w) then
// the projections; segments of one launch share the type.
static int gemv_norm_by_type(const int* types, const cx_seg* segs, int n, uint32_t k,
                             const float* x, const float* w, float eps, hipStream_t s) {
  bool done[4] = {false, false, false, false};
  for (int i = 0; i < n; i++) {
    if (done[i]) continue;
    cx_seg group[4];
    int ng = 0;
    for (int j = i; j < n; j++)
      if (!done[j] && types[j] == types[i]) {
        group[ng++] = segs[j];
        done[j] = true;
      }
    int rc = cx_launch_gemv_norm(types[i], group, ng, k, x, w, eps, CX_EPI_STORE, s);
    if (rc) return rc;
  }
  return CX_OK;
}

static int enqueue_tail(cx_cache* C);

static int enqueue_step(cx_cache* C) {
  cx_model* m = C->m;
  const cx_config& c = m->cfg;
  hipStream_t s = m->stream;
  const uint32_t D = c.dim, hd = D / c.heads, kvd = c.kv_heads * hd, I = c.ffn;
  const cx_qact act{m->xq, m->xe, m->xs};
  int rc = cx_launch_embed(m->t_embd, m->embd, D, C->st, C->hist, m->x, 1, s);
  if (rc) return rc;
  for (uint32_t li = 0; li < c.layers; li++) {
    const Layer& L = m->layers[li];
    float* kc = C->kv + (size_t)li * 2 * C->cap * kvd;
    float* vc = kc + C->cap * kvd;
    // src/forward.rs:422-464: rmsnorm, q/k/v with bias, rope, attention
    const cx_seg qkv[3] = {{L.q, m->q, L.q_bias, D}, {L.k, m->k, L.k_bias, kvd},
                           {L.v, m->v, L.v_bias, kvd}};
    const int tqkv[3] = {L.t_q, L.t_k, L.t_v};
    if ((rc = gemv_norm_by_type(tqkv, qkv, 3, D, m->x, L.attn_norm, c.eps, s))) return rc;
    cx_attn_args a{};
    a.q = m->q;
    a.knew = m->k;
    a.vnew = m->v;
    a.kc = kc;
    a.vc = vc;
    a.cos_t = m->cos_t;
    a.sin_t = m->sin_t;
    a.heads = c.heads;
    a.kvh = c.kv_heads;
    a.hd = hd;
    a.cap = (uint32_t)C->cap;
    a.st = C->st;
    a.pm = C->pm;
    a.pl = C->pl;
    a.po = C->po;
    a.sc = C->sc;
    a.cm = C->cm;
    a.out = m->att;
    a.xq = m->xq;  // the output projection's activation
    a.xe = m->xe;
    a.xs = m->xs;
    a.sub = cx_sub(L.t_o);
    const bool glu = L.t_gate == L.t_up && cx_glu_fits(L.t_gate, D) && I % 32 == 0;
    // the attention's spare CUs pull the o-proj's and gate/up's weights into L2
    // (all of them: past L2's 4 MB an XCD the Infinity Cache still holds
    // them; trimming config 5's 75 MB to 28 MB made its token 0.8% slower)
    (void)cx_gemv_prefetch_plan(L.t_o, L.o, D, D, &a.pf.job[0]);
    if (glu) (void)cx_glu_prefetch_plan(L.t_gate, L.gate, L.up, I, D, &a.pf.job[1]);
    // With a cache past the short path (the attention then runs for tens of
    // µs), the down projection's weights too: beyond L2's capacity, they are
    // read back from the Infinity Cache (config 5: +0.6% a token)
    if (a.cap > CX_ATT_LDS_MAX) (void)cx_gemv_prefetch_plan(L.t_down, L.down, D, I, &a.pf.job[2]);
    // and the next layer's K rows, which its scores kernel reads in one
    // burst (config 5 285.1 -> 285.6 tok/s, 3B 742.6 -> 743.3)
    if (li + 1 < c.layers) {
      const size_t kb = C->cap * (size_t)kvd * 4;
      const uint32_t tile = 256u << 10;
      a.pf.job[3] = cx_l2_job{reinterpret_cast<const uint8_t*>(kc + 2 * C->cap * kvd), nullptr, kb,
                              tile, (uint32_t)((kb + tile - 1) / tile)};
      // there also the next layer's q, k and v, read back from the
      // Infinity Cache by its q/k/v launch (config 5 291.3 -> 291.8 tok/s)
      if (a.cap > CX_ATT_LDS_MAX) {
        const Layer& N = m->layers[li + 1];
        const uint8_t* w3[3] = {N.q, N.k, N.v};
        const int t3[3] = {N.t_q, N.t_k, N.t_v};
        const uint32_t n3[3] = {D, kvd, kvd};
        for (int j = 0; j < 3; j++) {
          const size_t b = (size_t)n3[j] * (D / cx_vpb(t3[j])) * cx_bpb(t3[j]);
          a.pf.job[4 + j] = cx_l2_job{w3[j], nullptr, b, tile, (uint32_t)((b + tile - 1) / tile)};
        }
      }
    }
    // At long caches the jobs stream far more than L2 holds: the o-proj's
    // tiles go last, so that they are still in L2 when the o-proj launch,
    // the next one, reads them
    if (a.cap > CX_ATT_LDS_MAX) {
      const cx_l2_job o = a.pf.job[0];
      for (int j = 0; j + 1 < CX_L2_JOBS; j++) a.pf.job[j] = a.pf.job[j + 1];
      a.pf.job[CX_L2_JOBS - 1] = o;
    }
    if ((rc = cx_launch_attn_decode(a, s))) return rc;
    // src/forward.rs:466-469: output projection added to the residual
    cx_seg o{L.o, m->x, nullptr, D};
    if ((rc = cx_launch_gemv(L.t_o, &o, 1, D, act, CX_EPI_ACCUM, nullptr, s))) return rc;
    // src/forward.rs:472-491: rmsnorm, gate/up, SwiGLU, down added to the residual
    if (glu) {
      // gate, up and SwiGLU in one launch, bit-identical to the three below
      if ((rc = cx_launch_gemv_glu(L.t_gate, L.gate, L.up, I, D, m->x, L.ffn_norm, c.eps,
                                   cx_sub(L.t_down), m->xq, m->xe, m->xs, s)))
        return rc;
    } else {
      const cx_seg gu[2] = {{L.gate, m->g, nullptr, I}, {L.up, m->u, nullptr, I}};
      const int tgu[2] = {L.t_gate, L.t_up};
      if ((rc = gemv_norm_by_type(tgu, gu, 2, D, m->x, L.ffn_norm, c.eps, s))) return rc;
      if ((rc = cx_launch_swiglu_quant(m->g, m->u, I, cx_sub(L.t_down), m->xq, m->xe, m->xs, s)))
        return rc;
    }
    cx_seg dn{L.down, m->x, nullptr, D};
    if ((rc = cx_launch_gemv(L.t_down, &dn, 1, I, act, CX_EPI_ACCUM, nullptr, s))) return rc;
  }
  return enqueue_tail(C);
}

// src/forward.rs:495-501: the final rmsnorm and the output projection of the
// residual m->x, then the argmax (or, while sampling, Muestreador::elegir),
// which writes the next token at st->pos + 1 (when past the prompt) and
// advances st->pos
static int enqueue_tail(cx_cache* C) {
  cx_model* m = C->m;
  const cx_config& c = m->cfg;
  hipStream_t s = m->stream;
  const uint32_t D = c.dim;
  const cx_qact act{m->xq, m->xe, m->xs};
  int rc;
  if (cx_has_gemv(m->t_out)) {
    if ((rc = cx_launch_norm_quant(m->x, m->out_norm, D, c.eps, cx_sub(m->t_out), m->xq, m->xe,
                                   m->xs, s)))
      return rc;
    cx_seg lm{m->out, m->logits, nullptr, c.vocab};
    if (!C->sampling) {
      // the lm_head's tiles write the argmax's pairs themselves (one launch
      // fewer: 3B 6.7 us a token) where the row kernel takes the matrix
      uint32_t nparts = 0;
      if ((rc = cx_launch_gemv_argmax(m->t_out, lm, D, act, m->apv, m->api, &nparts, s)))
        return rc;
      if (nparts)
        return cx_launch_argmax_final(m->logits, m->apv, m->api, nparts, m->amax_out, C->st,
                                      C->hist, C->htok_dev, s);
    }
    if ((rc = cx_launch_gemv(m->t_out, &lm, 1, D, act, CX_EPI_STORE, nullptr, s))) return rc;
  } else {  // an unquantized (tied) lm_head: the f32 path (src/ops.rs:1064-1071)
    if ((rc = cx_launch_rmsnorm(m->att, m->x, m->out_norm, 1, D, c.eps, s))) return rc;
    if ((rc = cx_launch_matmul_f(m->t_out, m->out, c.vocab, D, m->att, 1, m->logits, s)))
      return rc;
  }
  if (C->sampling)
    return cx_launch_sample(m->logits, c.vocab, C->sd, C->spb, C->spart, C->sord, C->sordp,
                            m->amax_out, C->st, C->hist, C->htok_dev, s);
  return cx_launch_argmax(m->logits, c.vocab, m->apv, m->api, m->amax_out, C->st, C->hist,
                          C->htok_dev, s);
}

// the step graph of the current tail (greedy or sampling), captured once
static int ensure_graph(cx_cache* C) {
  bool& have = C->sampling ? C->have_graph_s : C->have_graph;
  hipGraphExec_t& exec = C->sampling ? C->exec_s : C->exec;
  if (have) return CX_OK;
  cx_model* m = C->m;
  hipGraph_t g;
  CX_HIP(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
  int rc = enqueue_step(C);
  hipError_t e = hipStreamEndCapture(m->stream, &g);
  if (rc) {
    if (e == hipSuccess) (void)hipGraphDestroy(g);
    return rc;
  }
  CX_HIP(e);
  hipError_t ie = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  CX_HIP(ie);
  have = true;
  return CX_OK;
}

// Runs `steps` decode steps starting at position C->len, with positions
// [C->len, prompt_end) fed from `toks` (already in hist).
static int run_steps(cx_cache* C, size_t prompt_end, size_t steps, float* step_ms) {
  cx_model* m = C->m;
  cx_dstate st{(uint32_t)C->len, (uint32_t)prompt_end, (uint32_t)C->cap, 0};
  CX_HIP(hipMemcpyAsync(C->st, &st, sizeof st, hipMemcpyHostToDevice, m->stream));
  int rc = ensure_graph(C);
  if (rc) return rc;
  std::vector<hipEvent_t> ev;
  if (step_ms) {
    ev.resize(steps + 1);
    for (auto& e : ev) CX_HIP(hipEventCreate(&e));
    CX_HIP(hipEventRecord(ev[0], m->stream));
  }
  hipGraphExec_t exec = C->sampling ? C->exec_s : C->exec;
  for (size_t i = 0; i < steps; i++) {
    CX_HIP(hipGraphLaunch(exec, m->stream));
    if (step_ms) CX_HIP(hipEventRecord(ev[i + 1], m->stream));
  }
  CX_HIP(hipStreamSynchronize(m->stream));
  if (step_ms) {
    for (size_t i = 0; i < steps; i++) CX_HIP(hipEventElapsedTime(&step_ms[i], ev[i], ev[i + 1]));
    for (auto& e : ev) (void)hipEventDestroy(e);
  }
  C->len += steps;
  return CX_OK;
}

// ------------------------------------------------------ batched prefill
// Modelo::forward over several tokens (src/forward.rs:375-505) as one pass
// per layer over a chunk of up to T tokens. The GEMVs become the int8 MFMA
// contraction for Q4_K/Q5_K (other types run the GEMV row by row), and the
// attention runs the decode step's kernels with one query token per grid
// slice. Every value equals what token-by-token decoding computes:
// - the contraction is bit-identical to the GEMV;
// - the rows are normalized in the fused GEMV prologue's tree;
// - the quantization of a row is a function of its values alone;
// - bias and residual adds are the same single f32 adds as the epilogues;
// - the attention kernels and their path (exact or split-K, by capacity)
//   are the decode step's.
// So a prompt gives the same logits, cache and tokens either way.
static const size_t kPrefillMaxT = 256;
static const size_t kPrefillAttnBytes = 256ull << 20;  // attention scratch bound

static int prefill_alloc(cx_cache* C) {
  cx_prefill& P = C->pf;
  if (P.T) return CX_OK;
  const cx_config& c = C->m->cfg;
  const size_t D = c.dim, hd = D / c.heads, kvd = c.kv_heads * hd, I = c.ffn, H = c.heads;
  const size_t per_tok = (cx_attn_score_floats(H, C->cap) + cx_attn_chunk_floats(H, C->cap)) * 4;
  size_t T = kPrefillAttnBytes / per_tok;
  T = T > kPrefillMaxT ? kPrefillMaxT : T < 16 ? 16 : T / 16 * 16;
  if (T > C->cap) T = C->cap;
  const size_t wide = D > I ? D : I;
  struct Want {
    float** p;
    size_t floats;
  } want[] = {{&P.x, T * D},   {&P.nrm, T * wide}, {&P.q, T * D},   {&P.k, T * kvd},
              {&P.v, T * kvd}, {&P.att, T * D},    {&P.g, T * I},   {&P.u, T * I},
              {&P.tmp, T * D}};
  for (const Want& w : want)
    if (hipMalloc(w.p, w.floats * 4) != hipSuccess) goto fail;
  if (hipMalloc(&P.sc, T * cx_attn_score_floats(H, C->cap) * 4) != hipSuccess ||
      hipMalloc(&P.cm, T * cx_attn_chunk_floats(H, C->cap) * 4) != hipSuccess)
    goto fail;
  if (hipMalloc(&P.scratch, cx_gemm_scratch_bytes(T, wide)) != hipSuccess) goto fail;
  P.T = (uint32_t)T;
  return CX_OK;
fail:
  for (void* b : {(void*)P.x, (void*)P.nrm, (void*)P.q, (void*)P.k, (void*)P.v, (void*)P.att,
                  (void*)P.g, (void*)P.u, (void*)P.tmp, (void*)P.sc, (void*)P.cm, P.scratch})
    if (b) (void)hipFree(b);
  P = cx_prefill{};
  cx_set_error("prefill: cannot allocate the buffers of %zu tokens", T);
  return CX_ENOMEM;
}

// out[r] = W . in[r] for `rows` rows of width k: the MFMA contraction,
// quantizing `in` unless *quantized (the sub-block size an earlier call of
// the same input quantized with, or 0) already matches the type's; the GEMV
// row by row on the step's activation buffers otherwise.
static int prefill_matmul(cx_cache* C, int type, const uint8_t* w, uint32_t n, uint32_t k,
                          const float* in, uint32_t rows, float* out, int* quantized) {
  cx_model* m = C->m;
  hipStream_t s = m->stream;
  int rc;
  if (cx_gemm_supported(type)) {
    const int sub = cx_sub(type);
    if (*quantized != sub && (rc = cx_gemm_quantize(in, rows, k, sub, C->pf.scratch, s))) return rc;
    *quantized = sub;
    return cx_gemm_apply(type, w, n, k, rows, out, C->pf.scratch, s);
  }
  const cx_qact act{m->xq, m->xe, m->xs};
  for (uint32_t r = 0; r < rows; r++) {
    if ((rc = cx_launch_quantize(in + (size_t)r * k, 1, k, cx_sub(type), m->xq, m->xe, m->xs, s)))
      return rc;
    cx_seg seg{w, out + (size_t)r * n, nullptr, n};
    if ((rc = cx_launch_gemv(type, &seg, 1, k, act, CX_EPI_STORE, nullptr, s))) return rc;
  }
  return CX_OK;
}

// out[i] = in . w[i]^T (+ bias[i]) for `count` matrices over one input
// (q/k/v, gate/up), or with accum (one matrix) out[0] += in . w[0]^T: on the
// MFMA contraction in one launch with the adds in its epilogue when the
// matrices fit one (cx_gemm_multi_fits), else a launch a matrix and the
// adds as row kernels. The same f32 adds either way: acc + bias, then
// out + that.
// the matrices take one contraction launch (one type, cx_gemm_multi_fits)
static bool prefill_fits(const int* type, const uint32_t* n, uint32_t count, uint32_t rows) {
  for (uint32_t i = 1; i < count; i++)
    if (type[i] != type[0]) return false;
  return cx_gemm_multi_fits(type[0], n, count, rows);
}

// rmsnorm of the residual rows into the input of the matrices that follow:
// straight into their quantized rows when they take one contraction launch
// (*quantized is then their sub-block size), else into P.nrm
static int prefill_norm(cx_cache* C, const float* nw, const int* type, const uint32_t* n,
                        uint32_t count, uint32_t rows, int* quantized) {
  cx_prefill& P = C->pf;
  const cx_config& c = C->m->cfg;
  if (prefill_fits(type, n, count, rows)) {
    *quantized = cx_sub(type[0]);
    return cx_gemm_norm_quantize(P.x, nw, rows, c.dim, c.eps, *quantized, P.scratch, C->m->stream);
  }
  return cx_launch_norm_rows(P.x, nw, rows, c.dim, c.eps, P.nrm, C->m->stream);
}

static int prefill_linear(cx_cache* C, const int* type, const uint8_t* const* w,
                          const uint32_t* n, uint32_t count, uint32_t k, const float* in,
                          uint32_t rows, float* const* out, const float* const* bias, bool accum,
                          int* quantized) {
  CX_REQUIRE(!accum || count == 1, "prefill: an accumulating product takes one matrix");
  hipStream_t s = C->m->stream;
  int rc;
  if (prefill_fits(type, n, count, rows)) {
    const int sub = cx_sub(type[0]);
    if (*quantized != sub && (rc = cx_gemm_quantize(in, rows, k, sub, C->pf.scratch, s))) return rc;
    *quantized = sub;
    return cx_gemm_apply_multi(type[0], w, n, count, k, rows, out, bias, accum, C->pf.scratch, s);
  }
  for (uint32_t i = 0; i < count; i++) {
    float* dst = accum ? C->pf.tmp : out[i];
    if ((rc = prefill_matmul(C, type[i], w[i], n[i], k, in, rows, dst, quantized)) ||
        (bias && bias[i] && (rc = cx_launch_add_rows(dst, bias[i], rows, n[i], 1, s))) ||
        (accum && (rc = cx_launch_add_rows(out[i], dst, rows, n[i], rows, s))))
      return rc;
  }
  return CX_OK;
}

// tokens at positions [st->pos, st->pos + nt), already in hist: the layers
static int enqueue_prefill_chunk(cx_cache* C, uint32_t nt) {
  cx_model* m = C->m;
  cx_prefill& P = C->pf;
  const cx_config& c = m->cfg;
  hipStream_t s = m->stream;
  const uint32_t D = c.dim, hd = D / c.heads, kvd = c.kv_heads * hd, I = c.ffn;
  int rc = cx_launch_embed(m->t_embd, m->embd, D, C->st, C->hist, P.x, nt, s);
  if (rc) return rc;
  for (uint32_t li = 0; li < c.layers; li++) {
    const Layer& L = m->layers[li];
    float* kc = C->kv + (size_t)li * 2 * C->cap * kvd;
    float* vc = kc + C->cap * kvd;
    // src/forward.rs:422-464
    int qd = 0;
    {
      const int t[3] = {L.t_q, L.t_k, L.t_v};
      const uint8_t* w[3] = {L.q, L.k, L.v};
      const uint32_t n[3] = {D, kvd, kvd};
      float* o[3] = {P.q, P.k, P.v};
      const float* b[3] = {L.q_bias, L.k_bias, L.v_bias};
      if ((rc = prefill_norm(C, L.attn_norm, t, n, 3, nt, &qd)) ||
          (rc = prefill_linear(C, t, w, n, 3, D, P.nrm, nt, o, b, false, &qd)))
        return rc;
    }
    if ((rc = cx_launch_rope_kv(P.q, P.k, P.v, kc, vc, m->cos_t, m->sin_t, c.heads, c.kv_heads,
                                hd, C->st, nt, s)))
      return rc;
    cx_attn_args a{};
    a.q = P.q;
    a.kc = kc;
    a.vc = vc;
    a.heads = c.heads;
    a.kvh = c.kv_heads;
    a.hd = hd;
    a.cap = (uint32_t)C->cap;
    a.st = C->st;
    a.sc = P.sc;
    a.cm = P.cm;
    a.out = P.att;
    a.tokens = nt;
    if ((rc = cx_launch_attn_decode(a, s))) return rc;
    // src/forward.rs:466-491
    qd = 0;
    {  // x += att . o^T
      const int t[1] = {L.t_o};
      const uint8_t* w[1] = {L.o};
      const uint32_t n[1] = {D};
      float* o[1] = {P.x};
      if ((rc = prefill_linear(C, t, w, n, 1, D, P.att, nt, o, nullptr, true, &qd))) return rc;
    }
    qd = 0;
    {
      const int t[2] = {L.t_gate, L.t_up};
      const uint8_t* w[2] = {L.gate, L.up};
      const uint32_t n[2] = {I, I};
      float* o[2] = {P.g, P.u};
      if ((rc = prefill_norm(C, L.ffn_norm, t, n, 2, nt, &qd)) ||
          (rc = prefill_linear(C, t, w, n, 2, D, P.nrm, nt, o, nullptr, false, &qd)))
        return rc;
    }
    qd = 0;
    {  // x += swiglu . down^T
      const int t[1] = {L.t_down};
      const uint8_t* w[1] = {L.down};
      const uint32_t n[1] = {D};
      float* o[1] = {P.x};
      if (prefill_fits(t, n, 1, nt)) {  // silu(g) * u straight into the quantized rows
        if ((rc = cx_gemm_swiglu_quantize(P.g, P.u, nt, I, cx_sub(t[0]), P.scratch, s))) return rc;
        qd = cx_sub(t[0]);
      } else if ((rc = cx_launch_swiglu_rows(P.g, P.u, (size_t)nt * I, P.nrm, s))) {
        return rc;
      }
      if ((rc = prefill_linear(C, t, w, n, 1, I, P.nrm, nt, o, nullptr, true, &qd))) return rc;
    }
  }
  return CX_OK;
}

// Positions [C->len, C->len + t) of hist through the model, in chunks; then
// the last token's logits and argmax (the argmax writes hist[len + t]).
static int prefill(cx_cache* C, size_t t) {
  cx_model* m = C->m;
  hipStream_t s = m->stream;
  int rc = prefill_alloc(C);
  if (rc) return rc;
  const cx_prefill& P = C->pf;
  const uint32_t D = m->cfg.dim, end = (uint32_t)(C->len + t), cap = (uint32_t)C->cap;
  uint32_t last = 0;
  for (size_t c0 = 0; c0 < t; c0 += P.T) {
    const uint32_t nt = (uint32_t)(t - c0 < P.T ? t - c0 : P.T);
    if ((rc = cx_launch_set_state(C->st, (uint32_t)(C->len + c0), end, cap, s)) ||
        (rc = enqueue_prefill_chunk(C, nt)))
      return rc;
    last = nt - 1;
  }
  CX_HIP(hipMemcpyAsync(m->x, P.x + (size_t)last * D, (size_t)D * 4, hipMemcpyDeviceToDevice, s));
  if ((rc = cx_launch_set_state(C->st, end - 1, end, cap, s)) || (rc = enqueue_tail(C))) return rc;
  CX_HIP(hipStreamSynchronize(s));
  C->len = end;
  return CX_OK;
}

extern "C" int cx_forward(cx_model* m, cx_cache* C, const uint32_t* toks, size_t t,
                          float* logits_host, uint32_t* argmax_out) {
  CX_REQUIRE(m && C && C->m == m, "forward: model/cache mismatch");
  CX_REQUIRE(toks && t > 0, "forward: no tokens to process");
  CX_REQUIRE(C->len + t <= C->cap, "forward: %zu tokens past the cache of %zu", C->len + t, C->cap);
  for (size_t i = 0; i < t; i++)
    CX_REQUIRE(toks[i] < m->cfg.vocab, "forward: token %u is not in a vocabulary of %u", toks[i],
               m->cfg.vocab);
  CX_HIP(hipSetDevice(m->device));
  CX_HIP(hipMemcpyAsync(C->hist + C->len, toks, t * 4, hipMemcpyHostToDevice, m->stream));
  int rc = t > 1 ? prefill(C, t) : run_steps(C, C->len + t, t, nullptr);
  if (rc) return rc;
  if (logits_host)
    CX_HIP(hipMemcpy(logits_host, m->logits, (size_t)m->cfg.vocab * 4, hipMemcpyDeviceToHost));
  if (argmax_out) CX_HIP(hipMemcpy(argmax_out, m->amax_out, 4, hipMemcpyDeviceToHost));
  return CX_OK;
}

// Modelo::generar (src/forward.rs:533-559), and the token loop of
// MotorPropio (src/engine_own.rs:257-282), on the device token loop:
//   logits = forward(prompt);
//   repeat up to max_new times: t = elegir(logits); stop at a stop token
//   (not returned); push t; al_token(t) == false stops; stop when the cache
//   holds the context; logits = forward([t]).
// The step graph reads each token from device memory and writes the next
// one (to hist and to the pinned host copy htok), so steps are launched up
// to `ahead` tokens before the host has looked at them; the host then reads
// token k once step k-1 has finished and applies the stopping rule. Steps
// launched past the stop only write the cache beyond its length: the cache
// keeps exactly the prompt and the forwarded tokens, as the reference's.
static int generate(cx_model* m, cx_cache* C, const uint32_t* prompt, size_t n, size_t max_new,
                    const uint32_t* stops, size_t n_stops, cx_token_fn fn, void* user,
                    uint32_t* out, size_t* n_out, float* step_ms) {
  CX_REQUIRE(m && C && C->m == m && n_out, "generate: bad arguments");
  CX_REQUIRE(prompt && n > 0, "generate: empty prompt");
  CX_REQUIRE(stops || !n_stops, "generate: null stop list");
  *n_out = 0;
  const size_t start = C->len, ctx = m->cfg.ctx;
  CX_REQUIRE(start + n <= C->cap, "generate: the prompt needs %zu tokens of a cache of %zu",
             start + n, C->cap);
  for (size_t i = 0; i < n; i++)
    CX_REQUIRE(prompt[i] < m->cfg.vocab, "generate: token %u is not in the vocabulary", prompt[i]);
  CX_HIP(hipSetDevice(m->device));
  CX_HIP(hipMemcpyAsync(C->hist + start, prompt, n * 4, hipMemcpyHostToDevice, m->stream));
  int rc = n > 1 ? prefill(C, n) : run_steps(C, start + n, n, nullptr);
  if (rc) return rc;
  if (!max_new) return CX_OK;
  // generated token k is at position pos0 + k; step k forwards it
  const size_t pos0 = start + n;
  size_t can = max_new < ctx - pos0 ? max_new : ctx - pos0;  // steps the reference may take
  if (can > C->cap - pos0) can = C->cap - pos0;               // steps the cache holds
  const size_t ahead = fn ? 2 : 8;
  cx_dstate st{(uint32_t)pos0, (uint32_t)pos0, (uint32_t)C->cap, 0};
  CX_HIP(hipMemcpyAsync(C->st, &st, sizeof st, hipMemcpyHostToDevice, m->stream));
  if ((rc = ensure_graph(C))) return rc;
  const hipGraphExec_t exec = C->sampling ? C->exec_s : C->exec;
  // ev[i + 1] follows step i; ev[0] precedes step 0 (a ring when not timing)
  const size_t nev = step_ms ? can + 1 : ahead + 2;
  std::vector<hipEvent_t> ev(nev);
  for (auto& e : ev) CX_HIP(hipEventCreate(&e));
  auto event = [&](size_t i) { return ev[i % nev]; };
  rc = CX_OK;
  hipError_t he = hipEventRecord(event(0), m->stream);
  size_t launched = 0, made = 0, forwarded = 0;
  for (size_t k = 0; he == hipSuccess; k++) {
    while (he == hipSuccess && launched < can && launched < k + ahead) {
      he = hipGraphLaunch(exec, m->stream);
      if (he == hipSuccess) he = hipEventRecord(event(launched + 1), m->stream);
      launched++;
    }
    if (he != hipSuccess) break;
    // token 0 came with the prompt's forward (synchronous); token k > 0 with step k - 1
    if (k > 0 && (he = hipEventSynchronize(event(k))) != hipSuccess) break;
    const uint32_t t = C->htok[pos0 + k];
    bool stop = false;
    for (size_t i = 0; i < n_stops; i++) stop |= t == stops[i];
    if (stop) break;
    if (out) out[made] = t;
    made++;
    if (fn && !fn(t, user)) break;
    if (pos0 + k >= ctx) break;  // the cache holds the context: t is not forwarded
    if (k >= can) {              // the reference forwards t; this cache has no room for it
      cx_set_error("generate: the cache of %zu tokens is full before generation ends", C->cap);
      rc = CX_ENOMEM;
      break;
    }
    forwarded = k + 1;
    if (made == max_new) break;
  }
  const hipError_t se = hipStreamSynchronize(m->stream);  // steps launched past the stop
  if (he == hipSuccess) he = se;
  // only the steps that forwarded a returned token are timed: steps
  // launched past the stop made tokens that are thrown away
  if (he == hipSuccess && step_ms)
    for (size_t i = 0; i < forwarded && he == hipSuccess; i++)
      he = hipEventElapsedTime(&step_ms[i], ev[i], ev[i + 1]);
  for (auto& e : ev) (void)hipEventDestroy(e);
  CX_HIP(he);
  C->len = pos0 + forwarded;
  *n_out = made;
  return rc;
}

static int generate_eos(cx_model* m, cx_cache* C, const uint32_t* prompt, size_t n,
                        size_t max_new, uint32_t eos, uint32_t* out, size_t* n_out,
                        float* step_ms) {
  return generate(m, C, prompt, n, max_new, &eos, eos == UINT32_MAX ? 0 : 1, nullptr, nullptr,
                  out, n_out, step_ms);
}

extern "C" int cx_generate(cx_model* m, cx_cache* C, const uint32_t* prompt, size_t n,
                           size_t max_new, uint32_t eos, uint32_t* out, size_t* n_out,
                           float* step_ms) {
  return generate_eos(m, C, prompt, n, max_new, eos, out, n_out, step_ms);
}

static int sampler_buffers(cx_cache* C) {
  if (C->sd) return CX_OK;
  const size_t V = C->m->cfg.vocab;
  // the chains' 16-byte loads may reach 3 floats past the last value
  if (hipMalloc(&C->sd, sizeof(cx_samp_state)) != hipSuccess ||
      hipMalloc(&C->spb, (V + 4) * 4) != hipSuccess ||
      hipMalloc(&C->spart, cx_sample_parts(V) * 4) != hipSuccess ||
      hipMalloc(&C->sord, V * 4) != hipSuccess || hipMalloc(&C->sordp, (V + 4) * 4) != hipSuccess) {
    cx_set_error("sample: cannot allocate the sampler's buffers");
    return CX_ENOMEM;
  }
  return CX_OK;
}

// Muestreador::nuevo(seed, temperature, top_p) (src/sampler.rs:38-47) for
// the generation that follows; temperature <= 0 is greedy, with no draw
// (src/sampler.rs:65-66)
static int sampled(cx_model* m, cx_cache* C, uint64_t seed, float temperature, float top_p,
                   const std::function<int()>& run) {
  if (temperature <= 0.0f) return run();
  CX_REQUIRE(m && C && C->m == m, "generate: bad arguments");
  CX_HIP(hipSetDevice(m->device));
  int rc = sampler_buffers(C);
  if (rc) return rc;
  const cx_samp_state h = sampler_state(seed, temperature, top_p);
  CX_HIP(hipMemcpyAsync(C->sd, &h, sizeof h, hipMemcpyHostToDevice, m->stream));
  C->sampling = true;
  rc = run();
  C->sampling = false;
  return rc;
}

extern "C" int cx_generate_sampled(cx_model* m, cx_cache* C, const uint32_t* prompt, size_t n,
                                   size_t max_new, uint32_t eos, uint64_t seed, float temperature,
                                   float top_p, uint32_t* out, size_t* n_out, float* step_ms) {
  return sampled(m, C, seed, temperature, top_p, [&] {
    return generate_eos(m, C, prompt, n, max_new, eos, out, n_out, step_ms);
  });
}

extern "C" int cx_generate_stream(cx_model* m, cx_cache* C, const uint32_t* prompt, size_t n,
                                  size_t max_new, const uint32_t* stops, size_t n_stops,
                                  uint64_t seed, float temperature, float top_p, cx_token_fn fn,
                                  void* user, uint32_t* out, size_t* n_out) {
  return sampled(m, C, seed, temperature, top_p, [&] {
    return generate(m, C, prompt, n, max_new, stops, n_stops, fn, user, out, n_out, nullptr);
  });
}

