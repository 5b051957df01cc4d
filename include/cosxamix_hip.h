/*
 * cosxamix_hip.h — C ABI of the MI355X (gfx950) decode path.
 *
 * Drop-in boundary for the reference crate Brashkie/Cosxamix's batch-1 decode
 * token loop. Three levels, mirroring the reference's own nesting:
 *
 *   1. kernel contract   — the reference's `type Kernel` FFI
 *                          (src/kernels/q2k.rs:153, src/kernels/q5k.rs:35);
 *   2. operators         — ops::matmul_auto / matmul_varias_una_fila /
 *                          cuantizar_i8_en / rope / atencion / softmax,
 *                          kernels::rmsnorm / silu, sampler::argmax;
 *   3. model             — forward::Modelo::{forward, generar} and
 *                          forward::Cache.
 *
 * Conventions
 *   - Return value: CX_OK (0) or a negative CX_E* code; cx_last_error()
 *     gives the message (replaces the reference's Result<_, String>).
 *     Level-1 functions return the f32 like the reference and report an
 *     error as NaN plus cx_last_error().
 *   - Level-1 pointers are HOST pointers (same as the reference contract).
 *     Level-2 pointers are DEVICE pointers (hipMalloc'd or torch tensors);
 *     `stream` is a hipStream_t (NULL = the HIP null stream) and the call is
 *     asynchronous on it. Level-3 objects own their device memory.
 *   - Types are GGML type ids (src/gguf.rs:39-54).
 *   - Threads. Level-1 functions are reentrant and thread-safe, like the
 *     reference's pure `type Kernel` that rayon calls from many threads at
 *     once (src/ops.rs:487-500): each host thread has its own stream and
 *     device scratch. Level-2 functions may run on several threads at once.
 *     The calls that use a thread's scratch (cx_matmul_auto,
 *     cx_matmul_multi_1row, cx_gemv_subsums, cx_dequantize_rows,
 *     cx_attention_decode, cx_sample) are ordered on the device after that
 *     scratch's previous use, whatever stream it was on, also when a thread
 *     ends with work still queued and another thread takes its scratch; the
 *     host is not blocked, and a growing scratch is reallocated in stream
 *     order. Under stream capture the scratch cannot grow (CX_EINVAL: make
 *     the call once before capturing) and the caller orders the graph's
 *     launches. A cx_model and its caches are used by one thread at a time;
 *     the reference serialises generation behind a Mutex
 *     (src/engine_own.rs:62,185).
 */
#ifndef COSXAMIX_HIP_H
#define COSXAMIX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids — src/gguf.rs:39-54 */
enum {
  CX_F32 = 0, CX_F16 = 1, CX_Q5_0 = 6, CX_Q8_0 = 8,
  CX_Q2_K = 10, CX_Q3_K = 11, CX_Q4_K = 12, CX_Q5_K = 13, CX_Q6_K = 14
};

/* status codes */
enum { CX_OK = 0, CX_EINVAL = -1, CX_EHIP = -2, CX_ENOMEM = -3, CX_ENOTSUP = -4 };

/* Last error message of the calling thread ("" if none). */
const char *cx_last_error(void);

/* Select the device used by host-pointer entry points and by models created
 * afterwards on this thread. Optional: device 0 is used by default. */
int cx_init(int device);

/* Bytes of one row of `k` values of `type` (src/ops.rs:462:
 * k / valores_por_bloque * bytes_por_bloque). 0 if the type is unknown or k
 * is not a multiple of the block. */
size_t cx_row_bytes(int type, size_t k);
/* Sub-block the activation is quantized with for `type`
 * (src/quant.rs:213-219); 0 = none. */
int cx_sub_block(int type);

/* ===================================================== 1. kernel contract
 * float kernel(const u8 *bloques, const i8 *xq, const f32 *xe, const f32 *xs,
 *              size_t n_bloques)
 * One row of n_bloques super-blocks against an i8 activation with one f32
 * scale xe and one f32 sum xs per sub-block. HOST pointers; runs the same
 * GEMV kernel as cx_gemv on one row. Replace, one for one:
 *   cx_dot_q2k_i8 <- cosxamix_q2k_{asm,c,zig} / q2k::dot (src/kernels/q2k.rs:153-185,262-292)
 *   cx_dot_q3k_i8 <- cosxamix_q3k_{c,completo} / kernels::dot_q3k_i8 (src/kernels/mod.rs:416-446)
 *   cx_dot_q4k_i8 <- kernels::dot_q4k_i8 (src/kernels/mod.rs:347-400); the asm
 *                    cosxamix_q4k_completo contract with acc[16] is
 *                    subsumed: this returns the reduced f32.
 *   cx_dot_q5k_i8 <- cosxamix_q5k_{asm,c,zig} / kernels::dot_q5k_i8 (src/kernels/q5k.rs:35, mod.rs:480-493)
 *   cx_dot_q6k_i8 <- kernels::dot_q6k_i8 (src/kernels/mod.rs:453-473)
 */
float cx_dot_q2k_i8(const uint8_t *bloques, const int8_t *xq, const float *xe,
                    const float *xs, size_t n_bloques);
float cx_dot_q3k_i8(const uint8_t *bloques, const int8_t *xq, const float *xe,
                    const float *xs, size_t n_bloques);
float cx_dot_q4k_i8(const uint8_t *bloques, const int8_t *xq, const float *xe,
                    const float *xs, size_t n_bloques);
float cx_dot_q5k_i8(const uint8_t *bloques, const int8_t *xq, const float *xe,
                    const float *xs, size_t n_bloques);
float cx_dot_q6k_i8(const uint8_t *bloques, const int8_t *xq, const float *xe,
                    const float *xs, size_t n_bloques);

/* ============================================================ 2. operators
 * All pointers are DEVICE pointers. */

/* ops::cuantizar_i8_en + the per-sub-block sums (src/ops.rs:178-198,
 * 472-483), applied to `rows` rows of `k` values: xq[rows*k],
 * xe/xs[rows*k/sub]. Bit-exact with the reference. */
int cx_quantize_act(const float *x, size_t rows, size_t k, int sub,
                    int8_t *xq, float *xe, float *xs, void *stream);

/* y[r] = row r of W (n rows, GGUF raw bytes) . activation, for r < n.
 * The per-row fused dot of ops::matmul_i8_fusionado with m = 1
 * (src/ops.rs:435-522) for Q2_K, Q3_K, Q4_K, Q5_K, Q6_K (k % 256 == 0);
 * for Q8_0 and Q5_0 (k % 32 == 0) the buffer path of
 * ops::matmul_i8_directo (src/ops.rs:310-414: desempaquetar_i8, then
 * kernels::dot_i8_escalado's block-order sum, scalar.rs:95-109). xq 16-byte
 * aligned; xe/xs 16-byte (k-quants) or 4-byte (Q8_0/Q5_0) aligned. */
int cx_gemv(int type, const uint8_t *w, size_t n, size_t k, const int8_t *xq,
            const float *xe, const float *xs, float *y, void *stream);

/* Test hook on the GEMV kernel: writes the integer per-sub-block sums that
 * the kernel's lanes form (out[n][k/sub]) — the E_j of
 * src/kernels/scalar.rs:147-166 (Q3_K: the +4-biased sum, scalar.rs:262-270;
 * Q6_K: unsigned 0..63). No counterpart in the reference. */
int cx_gemv_subsums(int type, const uint8_t *w, size_t n, size_t k,
                    const int8_t *xq, const float *xe, const float *xs,
                    int32_t *out, void *stream);

/* quant::cuantizar_bloques (src/quant.rs:744-805 ->
 * src/quant_kquants.rs:160-399): n f32 values (whole blocks) -> GGUF blocks,
 * one GPU thread per block. Q8_0, Q2_K, Q3_K, Q4_K, Q5_K. The same bytes as
 * the reference's quantizers for the same input. */
int cx_quantize_blocks(int type, const float *x, size_t n, uint8_t *out,
                       void *stream);

/* quant::descuantizar (src/quant.rs:124-162; formats 501-679): n values
 * (whole blocks) of GGUF bytes of `type` to f32. F32, F16, Q8_0, Q5_0,
 * Q2_K..Q6_K. Bit-identical to the reference. `y` 16-byte aligned. */
int cx_dequantize(int type, const uint8_t *bytes, size_t n, float *y,
                  void *stream);

/* quant::descuantizar_filas (src/quant.rs:172-205): rows[i] (HOST array of
 * n_rows indices below total_rows) of a row-major matrix of `width` values
 * per row, into y[n_rows][width] (device). Same types as cx_dequantize. */
int cx_dequantize_rows(int type, const uint8_t *data, size_t width,
                       size_t total_rows, const size_t *rows, size_t n_rows,
                       float *y, void *stream);

/* quant::desempaquetar_i8 (src/quant.rs:238-468): n values of `type` to
 * i8 q[n] and per sub-block scale esc[n/sub] and offset off[n/sub]
 * (value = esc*q + off; off = 0 for the formats without a minimum). *sub
 * (host) receives the sub-block size (src/quant.rs:213-219). Q8_0, Q5_0,
 * Q2_K..Q6_K. Bit-identical to the reference. */
int cx_unpack_i8(int type, const uint8_t *bytes, size_t n, int8_t *q,
                 float *esc, float *off, int *sub, void *stream);

/* ops::matmul_auto (src/ops.rs:1056-1093): dst[m,n] = lhs[m,k] . W[n,k]^T,
 * lhs/dst f32 row-major, W GGUF raw rows. k-quants (k % 256 == 0) and
 * Q8_0/Q5_0 (k % 32 == 0, the buffer path of matmul_i8_directo): quantizes
 * lhs internally; m = 1 is the GEMV, m > 1 the int8 MFMA contraction, both
 * bit-identical to the row-by-row dot. F32/F16
 * (ops::matmul, src/ops.rs:87-156): f32 dot of each lhs row with the
 * widened weight row, equal to the reference within f32 rounding; k % 4 == 0. */
int cx_matmul_auto(size_t m, size_t k, size_t n, const float *lhs,
                   const uint8_t *w, int type, float *dst, void *stream);

/* cx_matmul_auto without allocating: no counterpart in the reference. For
 * callers that cannot call hipMalloc (code under HIP graph capture, serving
 * loops, harnesses that forbid allocation). Same arguments and results as
 * cx_matmul_auto (bit-identical), but its scratch is a fixed device array of
 * CX_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends: a call
 * needing more (about m * k bytes plus m * k / 2 for m > 1, m * k * 1.5 for
 * m = 1) fails with CX_EINVAL. Every call on a GPU shares that array, so
 * calls that overlap on one GPU (any thread, any stream) race: order them.
 * cx_init looks the array's address up; if that fails, every call tries
 * again until the lookup succeeds. Arguments are checked (CX_EINVAL) before
 * the scratch is sized. */
#define CX_NOALLOC_SCRATCH_BYTES (32 << 20)
int cx_matmul_auto_noalloc(size_t m, size_t k, size_t n, const float *lhs,
                           const uint8_t *w, int type, float *dst,
                           void *stream);

/* ops::matmul_varias_una_fila (src/ops.rs:895-1009): dsts[i] = x . W_i^T for
 * `count` matrices sharing one activation vector of length k; one
 * quantization per sub size and one launch per type. Bit-identical to
 * `count` separate cx_matmul_auto(1, ...) calls (src/ops.rs:1614-1670).
 * The arrays are host arrays of device pointers. */
int cx_matmul_multi_1row(const float *x, size_t k, size_t count,
                         const uint8_t *const *w, const int *types,
                         const size_t *ns, float *const *dsts, void *stream);

/* kernels::rmsnorm (src/kernels/mod.rs:511-536; spec scalar.rs:36-54, f64
 * accumulation), over `rows` rows of n. */
int cx_rmsnorm(float *out, const float *in, const float *w, size_t rows,
               size_t n, float eps, void *stream);

/* kernels::silu (src/kernels/mod.rs:495-509): out = x / (1 + exp(-x)). */
int cx_silu(float *out, const float *in, size_t n, void *stream);

/* ops::frecuencias_rope (src/ops.rs:1108-1129) — HOST arrays of ctx*hd/2. */
int cx_rope_tables(size_t head_dim, float base, size_t ctx, float *cos_host,
                   float *sin_host);

/* ops::rope (src/ops.rs:1150-1193), split-half rotation in place.
 * x[tokens][heads*head_dim]; cos_t/sin_t device tables of ctx*head_dim/2. */
int cx_rope(float *x, size_t tokens, size_t heads, size_t head_dim,
            const float *cos_t, const float *sin_t, size_t ctx, size_t pos,
            void *stream);

/* ops::softmax (src/ops.rs:1206-1230), rows of `width` in place. */
int cx_softmax(float *x, size_t len, size_t width, void *stream);

/* ops::atencion (src/ops.rs:1258-1325): causal GQA. q[tokens][H*hd],
 * k/v[total][Hkv*hd], out[tokens][H*hd]. */
int cx_attention(const float *q, const float *k, const float *v, size_t tokens,
                 size_t total, size_t heads, size_t kv_heads, size_t head_dim,
                 float *out, void *stream);

/* ops::atencion at tokens = 1 (src/ops.rs:1258-1325) with the decode-step
 * kernels of the model: q[H*hd] of the token at position total-1 against
 * k/v[total][Hkv*hd]. mode 0 or 1: order-exact, bit-identical to the
 * reference's scalar order at any length (what the model runs); 2: split-K
 * (partial softmaxes combined: equal within f32 rounding). */
int cx_attention_decode(const float *q, const float *k, const float *v,
                        size_t total, size_t heads, size_t kv_heads,
                        size_t head_dim, int mode, float *out, void *stream);

/* sampler::argmax (src/sampler.rs:129-137): first index of the max;
 * *out is a DEVICE uint32. */
int cx_argmax(const float *v, size_t n, uint32_t *out, void *stream);

/* A measurement probe with no counterpart in the reference: reads
 * bytes (a multiple of 16) from the 16-byte aligned device buffer p once,
 * with no arithmetic after the loads (sink: a device uint32 the kernel
 * only writes for one improbable fold of the data). The bench times it to
 * report a measured read peak beside the nominal 8 TB/s. */
int cx_stream_read(const void *p, size_t bytes, uint32_t *sink, void *stream);

/* sampler::Muestreador::elegir (src/sampler.rs:61-152) on device logits[n]:
 * temperature <= 0 is the argmax with no draw; otherwise one draw of the
 * xorshift64* generator whose state *state (HOST) holds (Azar::siguiente,
 * src/daiss.rs:330-337; seed it as Azar::con_semilla does: a zero seed is
 * 0x9E3779B97F4A7C15), the softmax of logits/temperature, and top-p (clamped
 * to [0, 1]; >= 1 samples the whole vocabulary in index order). *out (HOST)
 * receives the token. Equal probabilities are ordered by ascending index
 * (the reference's unstable sort leaves that order unspecified). */
int cx_sample(const float *logits, size_t n, float temperature, float top_p,
              uint64_t *state, uint32_t *out, void *stream);

/* ============================================================ GGUF files
 * Host-only (no device work). Gguf::abrir and Pesos (src/gguf.rs:119-436). */

typedef struct cx_gguf cx_gguf;

/* InfoTensor (src/gguf.rs:172-194): dims as stored (fastest-varying first:
 * a weight matrix is [row width, rows]); offset from the data section;
 * bytes = elements / values_per_block * bytes_per_block. */
typedef struct {
  char name[128];
  int type;
  uint32_t n_dims;
  uint64_t dims[4];
  uint64_t offset;
  uint64_t elements;
  uint64_t bytes;
} cx_gguf_tensor;

/* Gguf::abrir (src/gguf.rs:274-342): header, metadata and tensor table of a
 * GGUF v2/v3 file; the weights are not read. Errors as the reference: not a
 * GGUF, unknown version, a truncated header, > 4 dims, an unknown type. */
int cx_gguf_open(const char *path, cx_gguf **out);
void cx_gguf_free(cx_gguf *g);
/* version, counts, the aligned start of the data section and the alignment
 * (general.alignment, default 32) */
int cx_gguf_header(const cx_gguf *g, uint32_t *version, uint64_t *n_tensors,
                   uint64_t *n_meta, uint64_t *data_start, uint64_t *alignment);
/* Gguf::meta_entero / meta_decimal (src/gguf.rs:348-355; Valor::entero,
 * decimal at 143-163): CX_EINVAL when the key is missing or not a number. */
int cx_gguf_meta_int(const cx_gguf *g, const char *key, uint64_t *out);
int cx_gguf_meta_float(const cx_gguf *g, const char *key, double *out);
/* Valor::texto: a string value (index < 0) or element `index` of a list of
 * strings; *len gets its length, buf (cap bytes) a NUL-terminated copy. */
int cx_gguf_meta_str(const cx_gguf *g, const char *key, long index, char *buf,
                     size_t cap, size_t *len);
/* GGUF value type (0..12) of a key and its element count if a list (else 1) */
int cx_gguf_meta_type(const cx_gguf *g, const char *key, uint32_t *type,
                      uint64_t *count);
/* Gguf::tensor (src/gguf.rs:344-346): index of the named tensor or -1 */
int cx_gguf_find(const cx_gguf *g, const char *name);
int cx_gguf_tensor_info(const cx_gguf *g, int idx, cx_gguf_tensor *out);
/* Gguf::datos_de / Pesos::de (src/gguf.rs:357-436): the tensor's bytes into
 * a host buffer of `cap` bytes; a tensor reaching past the end of the file
 * (every offset sum checked for overflow) is an error, not a read. */
int cx_gguf_tensor_read(const cx_gguf *g, const cx_gguf_tensor *t, void *host,
                        size_t cap);

/* ================================================================ 3. model */

/* forward::Config (src/forward.rs:36-55) */
typedef struct {
  uint32_t layers, dim, heads, kv_heads, ffn, vocab, ctx;
  float eps, rope_base;
} cx_config;

typedef struct cx_model cx_model;
typedef struct cx_cache cx_cache;

/* A Qwen2-architecture model with daiss-style seeded random weights
 * (src/daiss.rs:236-303 tensors, 317-379 RNG, 396-407 init, 494-586 write),
 * generated directly in HBM. Linear weights in `linear_type`, ffn_down in
 * `down_type`, output.weight in `out_type`; token_embd, norms and q/k/v
 * biases F32. The reference writes a GGUF and opens it with Modelo::abrir
 * (src/forward.rs:187-266); here the tensors are made where they are used. */
int cx_model_create_daiss(const cx_config *cfg, int linear_type, int down_type,
                          int out_type, uint64_t seed, cx_model **out);
/* Modelo::abrir (src/forward.rs:187-266): a Qwen2-architecture GGUF file
 * into HBM. Config from <general.architecture>.* metadata (block_count,
 * embedding_length, attention.head_count[_kv], context_length,
 * layer_norm_rms_epsilon = 1e-6 and rope.freq_base = 10000 if absent);
 * vocab and ffn from the tensors. Per-tensor types: matrices Q2_K..Q6_K
 * (mixed per tensor, as Q*_K_M files are), norms and biases F32 (biases may
 * be absent), token_embd any type cx_dequantize reads, output.weight a
 * matrix type or F32/F16 and tied to token_embd when absent
 * (src/forward.rs:218-227). The bytes are uploaded unchanged. */
int cx_model_open(const char *path, cx_model **out);
/* The model as a GGUF file: the reference daiss writer's metadata
 * (src/daiss.rs:422-468) and Escritor::escribir's layout (src/gguf_write.rs),
 * tensors in table order with their bytes as held in HBM. */
int cx_model_save_gguf(const cx_model *m, const char *path);
void cx_model_free(cx_model *m);
int cx_model_config(const cx_model *m, cx_config *out);

/* Tensor table, for mirroring the model on the host: names as in GGUF
 * (src/daiss.rs:236-303), dims[0] = row width, dims[1] = rows. */
int cx_model_tensor_count(const cx_model *m);
int cx_model_tensor_info(const cx_model *m, int idx, char *name,
                         size_t name_cap, int *type, uint64_t dims[2],
                         size_t *bytes);
int cx_model_tensor_copy(const cx_model *m, int idx, void *host, size_t bytes);
/* Device address of a tensor's bytes (read-only view, owned by the model). */
const void *cx_model_tensor_data(const cx_model *m, int idx);
/* Bytes of weights streamed per decode token (all matrices + one embedding
 * row); the algorithmic traffic of one token without the KV reads. */
size_t cx_model_weight_bytes(const cx_model *m);

/* forward::Cache (src/forward.rs:62-137), with room for `cap` tokens. A
 * cache belongs to its model: cx_model_free on a model with live caches
 * releases the model when its last cache is freed (caches can be freed
 * before or after their model). */
int cx_cache_new(cx_model *m, size_t cap, cx_cache **out);
size_t cx_cache_len(const cx_cache *c);
int cx_cache_truncate(cx_cache *c, size_t n);
void cx_cache_clear(cx_cache *c);
void cx_cache_free(cx_cache *c);
/* Cache::bytes (src/forward.rs:130-136): bytes of K and V the cache holds
 * (len tokens x layers x 2 x kv_heads*head_dim f32), not its capacity. */
size_t cx_cache_bytes(const cx_cache *c);
/* Cache::prefijo (src/forward.rs:117-128): a new cache of the same model
 * with room for `cap` tokens (0 = the source's capacity) holding a copy of
 * the source's first min(n, len) tokens, as MotorPropio borrows another
 * session's prefix (src/engine_own.rs:227-245). */
int cx_cache_prefix(const cx_cache *src, size_t n, size_t cap, cx_cache **out);

/* Modelo::forward (src/forward.rs:375-505): appends `t` tokens to the cache
 * and gives the logits of the last one (HOST buffer of vocab floats, may be
 * NULL) and its argmax (may be NULL). */
int cx_forward(cx_model *m, cx_cache *c, const uint32_t *toks, size_t t,
               float *logits_host, uint32_t *argmax_out);

/* Modelo::generar (src/forward.rs:533-559) with a greedy sampler
 * (src/sampler.rs:65-66): prefill `prompt`, then up to max_new tokens.
 * `eos` stops generation like Modelo::fin (pass UINT32_MAX for none): the
 * stop token is not returned or forwarded, and the device stops within a
 * few steps of it. out[] gets the tokens, *n_out how many; the cache then
 * holds the prompt and the forwarded tokens, as the reference's. The cache
 * needs room for the positions generation reaches (CX_ENOMEM, with the
 * tokens made so far in out/n_out, when it fills first). If step_ms is not
 * NULL (room for max_new values) it gets the decode time (ms, HIP events)
 * of each step that forwarded a returned token, in order: their number is
 * the cache's growth past the prompt, cx_cache_len after the call minus
 * (cx_cache_len before it + n), at most *n_out; the rest of step_ms is
 * left as it was. */
int cx_generate(cx_model *m, cx_cache *c, const uint32_t *prompt, size_t n,
                size_t max_new, uint32_t eos, uint32_t *out, size_t *n_out,
                float *step_ms);
/* Modelo::generar with Muestreador::nuevo(seed, temperature, top_p)
 * (src/forward.rs:533-559, src/sampler.rs:38-47): as cx_generate, each
 * token drawn by the sampler on the GPU inside the captured step. */
int cx_generate_sampled(cx_model *m, cx_cache *c, const uint32_t *prompt,
                        size_t n, size_t max_new, uint32_t eos, uint64_t seed,
                        float temperature, float top_p, uint32_t *out,
                        size_t *n_out, float *step_ms);

/* The `al_token` of Modelo::generar (src/forward.rs:538-553): called on the
 * calling thread with each token as it is pushed; returning 0 stops
 * generation at once (that token is returned, not forwarded). */
typedef int (*cx_token_fn)(uint32_t token, void *user);
/* Modelo::generar with its per-token callback, and MotorPropio's token loop
 * (src/engine_own.rs:257-282): any of the n_stops tokens in `stops` ends
 * generation unreturned (the reference stops at Modelo::fin and at the
 * chat's end-of-turn token); temperature <= 0 is greedy, otherwise
 * Muestreador::nuevo(seed, temperature, top_p) draws on the GPU. The
 * callback sees each token while the next steps already run on the device;
 * otherwise as cx_generate. `fn` may be NULL. */
int cx_generate_stream(cx_model *m, cx_cache *c, const uint32_t *prompt,
                       size_t n, size_t max_new, const uint32_t *stops,
                       size_t n_stops, uint64_t seed, float temperature,
                       float top_p, cx_token_fn fn, void *user, uint32_t *out,
                       size_t *n_out);

#ifdef __cplusplus
}
#endif
#endif
