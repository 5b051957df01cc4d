/*
 * cx_oracle.h — CPU oracle for the decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP product
 * path is compared against. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it. The product library never links,
 * loads or calls anything here.
 *
 * Every function restates, in plain C with IEEE f32 semantics (no FMA
 * contraction, no fast-math), one function of the reference crate
 * Brashkie/Cosxamix; the reference file:line is given beside each one.
 *
 * Parity pinning (what checks each part; see tests/test_oracle_*.py):
 *   - row dots Q2_K..Q5_K: the reference's own compiled native kernels
 *     (oracle/_ref, built from /root/reference/kernels) + golden fixtures,
 *     and brute-force integer sub-block sums;
 *   - f16<->f32: exhaustive over all 65536 halves vs the CPU's F16C;
 *   - activation quantizer: closed-form invariants of ops.rs:1431-1457;
 *   - unpack/dequant: exact-reconstruction identity (quant.rs:892-928);
 *     Q6_K: one-hot bytes against the reference's layout table
 *     (kernels/scalar.rs:276-291) through dequant, unpack and the row dot;
 *   - RoPE: one-hot rotations and the float64 rotation (direction pinned);
 *     attention: the float64 softmax(q.k/sqrt(Dh)).v closed form (scale
 *     pinned);
 *   - seeds: FNV-1a published vectors; Azar normals: Box-Muller in float64
 *     on the exact xorshift uniforms, to a few f32 ulps;
 *   - quantizers Q2_K..Q5_K: byte for byte on exact-grid blocks whose bytes
 *     follow from the format alone, plus the reference invariants
 *     (quant_kquants.rs:427-503). On general inputs their exact bytes rest
 *     on the line-by-line restatement (a Rust build of the reference would
 *     pin them; GEMV parity does not depend on them: GPU and CPU read the
 *     same bytes).
 * tests/test_oracle_mutants.py shows each pin fails on a plausible slip.
 */
#ifndef CX_ORACLE_H
#define CX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids — src/gguf.rs:39-54 */
enum {
  ORC_F32 = 0, ORC_F16 = 1, ORC_Q5_0 = 6, ORC_Q8_0 = 8,
  ORC_Q2_K = 10, ORC_Q3_K = 11, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14
};

/* src/gguf.rs:83-111 */
size_t orc_values_per_block(int type);
size_t orc_bytes_per_block(int type);
/* src/quant.rs:213-219 ; returns 0 for "None" */
int orc_sub_block(int type);

/* src/quant.rs:38-60, 691-731 */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float x);

/* src/quant.rs:108-117 (escala_y_minimo) */
void orc_scale_min_k4(int j, const uint8_t *q12, uint8_t *sc, uint8_t *mn);
/* src/quant.rs:87-106 (escalas_q3k), `blk` points at the 110-byte block */
void orc_scales_q3k(const uint8_t *blk, int8_t out[16]);

/* src/quant.rs:124-162 and 501-679 (descuantizar). n = values. 0 ok, -1 err */
int orc_dequantize(int type, const uint8_t *src, float *dst, size_t n);
/* src/quant.rs:238-468 (desempaquetar_i8). Returns sub size or -1 */
int orc_unpack_i8(int type, const uint8_t *src, size_t n, int8_t *q,
                  float *scales, float *offsets);
/* src/quant.rs:744-805 + src/quant_kquants.rs. Returns bytes written or -1 */
long orc_quantize_blocks(int type, const float *x, size_t n, uint8_t *out);
/* Test hook: the per-sub-block search of one 256-value block of Q2_K, Q3_K,
 * Q4_K or Q5_K as the quantizers run it (scales, -mins, 256 codes).
 * Returns the number of sub-blocks, or -1. */
int orc_kquant_search(int type, const float *x, float *scales, float *neg_mins, int32_t *l);

/* src/daiss.rs:317-357 (Azar) and 364-379 (semilla_de) */
typedef struct { uint64_t state; } orc_azar;
void orc_azar_seed(orc_azar *a, uint64_t s);
uint64_t orc_azar_next(orc_azar *a);
void orc_azar_normals(orc_azar *a, float sigma, float *z0, float *z1);
uint64_t orc_seed_of(uint64_t model_seed, const char *name, uint64_t row);
/* src/daiss.rs:539-564 — one row of `width` normals from its per-row seed */
void orc_daiss_row(uint64_t model_seed, const char *name, uint64_t row,
                   float sigma, float *out, size_t width);

/* src/daiss.rs:539-571: `rows` rows of `width` normals, each from its
 * per-row seed, quantized row by row to `type` into out (rows * row bytes).
 * Rows are independent, so the result does not depend on `threads`. */
int orc_daiss_matrix(uint64_t model_seed, const char *name, size_t rows,
                     size_t width, float sigma, int type, uint8_t *out,
                     int threads);

/* src/ops.rs:178-198 (cuantizar_i8_en) + sums xs (src/ops.rs:472-483) */
void orc_quantize_act(const float *x, size_t k, int sub, int8_t *xq,
                      float *xe, float *xs);

/* Row dots, scalar spec — src/kernels/scalar.rs:132-324, q2k.rs:41-69.
 * Signature = the reference's `Kernel` C ABI (q2k.rs:153). */
typedef float (*orc_row_kernel)(const uint8_t *blocks, const int8_t *xq,
                                const float *xe, const float *xs,
                                size_t n_blocks);
float orc_dot_q2k(const uint8_t *b, const int8_t *xq, const float *xe,
                  const float *xs, size_t nb);
float orc_dot_q3k(const uint8_t *b, const int8_t *xq, const float *xe,
                  const float *xs, size_t nb);
float orc_dot_q4k(const uint8_t *b, const int8_t *xq, const float *xe,
                  const float *xs, size_t nb);
float orc_dot_q5k(const uint8_t *b, const int8_t *xq, const float *xe,
                  const float *xs, size_t nb);
float orc_dot_q6k(const uint8_t *b, const int8_t *xq, const float *xe,
                  const float *xs, size_t nb);
orc_row_kernel orc_row_kernel_for(int type);
/* Per-sub-block integer sums E_s that the scalar spec forms before scaling
 * (Q3_K: the +4-biased sum of scalar.rs:262-270; Q6_K: unsigned 0..63). */
int orc_subsums(int type, const uint8_t *b, const int8_t *xq, size_t nb,
                int32_t *out);

/* src/kernels/scalar.rs:16-23, 36-54, 63-67 */
float orc_dot_f32(const float *a, const float *b, size_t n);
void orc_rmsnorm(float *out, const float *in, const float *w, size_t n,
                 float eps);
void orc_silu(float *out, const float *in, size_t n);
/* src/sampler.rs:129-137 */
uint32_t orc_argmax(const float *v, size_t n);

/* src/ops.rs:1108-1129, 1150-1193, 1206-1230, 1258-1325 */
void orc_rope_tables(size_t head_dim, float base, size_t ctx, float *cos_t,
                     float *sin_t);
int orc_rope(float *x, size_t tokens, size_t heads, size_t head_dim,
             const float *cos_t, const float *sin_t, size_t ctx, size_t pos);
int orc_softmax(float *x, size_t len, size_t width);
int orc_attention(const float *q, const float *k, const float *v,
                  size_t tokens, size_t total, size_t heads, size_t kv_heads,
                  size_t head_dim, float *out);

/* src/ops.rs:435-522 (matmul_i8_fusionado): dst[m,n] = lhs[m,k] . W[n,k]^T.
 * `kern` NULL = the scalar spec for `type`. `threads` >= 1: rows of output
 * are split in chunks of 32 (ops.rs:43) across a pthread pool; `prefetch`
 * rows ahead are touched with __builtin_prefetch (ops.rs:52-79). */
int orc_matmul_fused(size_t m, size_t k, size_t n, const float *lhs,
                     const uint8_t *w, int type, float *dst,
                     orc_row_kernel kern, int threads, int prefetch);
/* src/ops.rs:895-1009 (matmul_varias_una_fila) */
float orc_dot_i8_scaled(const int8_t *a, const int8_t *b, const float *esc_a,
                        const float *esc_b, size_t n, int block);
int orc_matmul_direct(size_t m, size_t k, size_t n, const float *lhs, const uint8_t *w,
                      int type, float *dst, int threads);
int orc_matmul_multi_1row(const float *x, size_t k, size_t count,
                          const uint8_t *const *ws, const int *types,
                          const size_t *ns, float *const *dsts, int threads);

/* ---- Qwen2 forward on host memory: src/forward.rs:36-137, 375-505 ---- */
typedef struct {
  size_t layers, dim, heads, kv_heads, ffn, vocab, ctx;
  float eps, rope_base;
} orc_config;

typedef struct {
  const float *attn_norm, *q_bias, *k_bias, *v_bias, *ffn_norm;
  const uint8_t *q, *k, *v, *o, *gate, *up, *down;
  int t_q, t_k, t_v, t_o, t_gate, t_up, t_down;
} orc_layer;

typedef struct {
  orc_config cfg;
  const float *embd;            /* F32 [vocab][dim] */
  const float *out_norm;        /* [dim] */
  const uint8_t *out;           /* [vocab] rows of dim, type t_out */
  int t_out;
  const orc_layer *layers;      /* cfg.layers entries */
  float *cos_t, *sin_t;         /* ctx x head_dim/2, owned */
  orc_row_kernel kern_override; /* NULL = scalar spec */
  int threads;
  /* 0: the reference's attention order. A test hook otherwise: the sums
   * split over chunks of attn_chunk positions (orc_attention_split) */
  int attn_chunk;
} orc_model;

typedef struct {
  size_t len, cap;   /* tokens */
  float **k, **v;    /* per layer: cap x kv_dim */
} orc_cache;

int orc_model_init(orc_model *m, const orc_config *cfg, const float *embd,
                   const float *out_norm, const uint8_t *out, int t_out,
                   const orc_layer *layers, int threads);
void orc_model_release(orc_model *m);
int orc_cache_init(orc_cache *c, const orc_config *cfg, size_t cap);
void orc_cache_release(orc_cache *c, const orc_config *cfg);
void orc_cache_truncate(orc_cache *c, size_t n);
/* Test hook, not the reference's order: attention whose softmax and P.V
 * sums are split over chunks of `chunk` positions, each chunk's (max, sum of
 * exps, unnormalized P.V) formed in order, then combined with the factors
 * exp(m_i - M) -- the order of a split-K kernel. */
int orc_attention_split(const float *q, const float *k, const float *v, size_t tokens,
                        size_t total, size_t heads, size_t kvh, size_t hd, size_t chunk,
                        float *out);
/* logits of the last token into `logits` (vocab floats) */
int orc_forward(const orc_model *m, const uint32_t *toks, size_t t,
                orc_cache *c, float *logits);
/* src/forward.rs:533-559 with a greedy sampler and no EOS */
int orc_generate(const orc_model *m, const uint32_t *prompt, size_t n,
                 size_t max_new, orc_cache *c, uint32_t *out, size_t *n_out);

/* sampler::Muestreador (src/sampler.rs:27-152): temperature and top-p
 * sampling with Azar. Equal probabilities are ordered by ascending index
 * (the reference's unstable sort leaves their order unspecified). */
typedef struct {
  orc_azar azar;
  float temp, top_p;
} orc_sampler;
void orc_sampler_init(orc_sampler *s, uint64_t seed, float temp, float top_p);
uint32_t orc_sample(orc_sampler *s, const float *logits, size_t n);
/* Modelo::generar (src/forward.rs:533-559) with the sampler and an end
 * token (UINT32_MAX: none) */
int orc_generate_sampled(const orc_model *m, const uint32_t *prompt, size_t n,
                         size_t max_new, orc_sampler *s, uint32_t eos,
                         orc_cache *c, uint32_t *out, size_t *n_out);

const char *orc_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
