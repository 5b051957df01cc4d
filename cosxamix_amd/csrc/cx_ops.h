// cx_ops.h — launchers of the per-token ops (cx_ops.hip).
#pragma once

#include "cx_internal.h"

// Device-side state of one cache's token loop. Kernels of a captured decode
// step read the position from here, so one graph serves every position.
struct cx_dstate {
  uint32_t pos;         // tokens already in the cache = position of this step
  uint32_t prompt_end;  // positions below this come from the prompt
  uint32_t cap;         // cache capacity (tokens)
  uint32_t pad;
};

int cx_launch_set_state(cx_dstate* st, uint32_t pos, uint32_t prompt_end, uint32_t cap,
                        hipStream_t s);

// Device state of the sampler (cx_sample.hip): the Azar state, 1/temperature
// and top_p set by the host; u, 1/S and the uniform flag written per call.
struct cx_samp_state {
  uint64_t azar;
  float inv, top_p;
  float u, inv_s;
  uint32_t uniform, token;
};
// 4-byte words of the sampler's `part` scratch for a vocabulary of n (the
// per-block maxima and the descending-order sort's keys, indices, counts)
size_t cx_sample_parts(size_t n);
// One Muestreador::elegir with temperature on device logits[n]: pb (n
// floats), part (cx_sample_parts(n) words), ord (n), ordp (n floats) are scratch;
// the token goes to *out (device, optional) and, with st, to hist[pos + 1]
// (and hist_host[pos + 1], pinned host memory, when given) with the position
// advanced (the token loop's argmax step).
int cx_launch_sample(const float* logits, size_t n, cx_samp_state* sd, float* pb, float* part,
                     uint32_t* ord, float* ordp, uint32_t* out, cx_dstate* st, uint32_t* hist,
                     uint32_t* hist_host, hipStream_t s);

#define CX_ATT_MAX_TOTAL 16000  // general attention keeps scores in LDS
// Decode attention holds a head's scores in LDS for caches up to this many
// tokens (cx_ops.hip) and streams them above it (cx_attn.hip); both paths
// are order-exact.
#define CX_ATT_LDS_MAX 4096
// one query token: the same softmax-V kernel up to this many cached
// positions (a smaller V ring leaves LDS for the scores), with k_att_qk's
// scores; k_att_sv above
#define CX_ATT_LONG_MAX 11520

// x[r] = row hist[st->pos + r] of the embedding table (GGUF bytes of
// `type`), dequantized, for r < rows
int cx_launch_embed(int type, const uint8_t* embd, uint32_t dim, const cx_dstate* st,
                    const uint32_t* hist, float* x, uint32_t rows, hipStream_t s);
// rows tokens at positions st->pos + r: q[r] rotated in place, k[r] rotated
// into K[pos], v[r] into V[pos]
int cx_launch_rope_kv(float* q, const float* k, const float* v, float* kc, float* vc,
                      const float* cos_t, const float* sin_t, uint32_t heads, uint32_t kvh,
                      uint32_t hd, const cx_dstate* st, uint32_t rows, hipStream_t s);
size_t cx_attn_splits(size_t cap);
// floats of the exact path's score buffer (rows padded to 4 floats; the
// buffer must start 16-byte aligned) and of its per-chunk maxima
inline size_t cx_attn_score_floats(size_t heads, size_t cap) { return heads * ((cap + 3) / 4 * 4); }
size_t cx_attn_chunk_floats(size_t heads, size_t cap);

// One decode step's attention (src/ops.rs:1258-1325 at tokens = 1). The
// order-exact path (modes 0 and 1, cx_attn.hip) is bit-identical to the
// reference for any cache length; split-K (mode 2) combines partial
// softmaxes in another order.
struct cx_attn_args {
  float* q;                    // heads*hd; rotated in place by the split-K path
  const float* knew;           // this step's k and v (kvh*hd), used with rope
  const float* vnew;
  float* kc;                   // caches [cap][kvh*hd]
  float* vc;
  const float* cos_t;          // rope tables; null: q is final and the caches
  const float* sin_t;          //   already hold position st->pos
  uint32_t heads, kvh, hd, cap;
  const cx_dstate* st;
  float *pm, *pl, *po;         // split-K partials
  float *sc, *cm;              // exact path: scores, per-chunk maxima
  float* out;                  // heads*hd
  int8_t* xq;                  // optional: out quantized for the next GEMV
  float *xe, *xs;
  int sub;
  int mode;                    // 0 or 1: order-exact, 2: split-K
  // query tokens (0 or 1: one). T > 1: token z at position st->pos + z,
  // q/out rows of heads*hd, sc and the split partials T times their
  // one-token size; q already rotated and the caches already filled
  // (cos_t null), no quantized output.
  uint32_t tokens;
  cx_l2_prefetch pf;           // optional (a and b0 null: none); one token only
};
int cx_launch_attn_decode(const cx_attn_args& a, hipStream_t s);
int cx_launch_attn_exact(const cx_attn_args& a, float scale, hipStream_t s);
// k_att_qk alone: the scores sc[h][p] (times the scale) and the chunk maxima
// cm[h][chunk] of every head, any cache length (rope and the KV append
// as k_attn_scores)
int cx_launch_att_scores(const cx_attn_args& a, float scale, hipStream_t s);
int cx_launch_attention(const float* q, const float* k, const float* v, size_t tokens,
                        size_t total, size_t heads, size_t kvh, size_t hd, float* out,
                        hipStream_t s);
int cx_launch_softmax(float* x, size_t len, size_t width, hipStream_t s);
int cx_launch_silu(float* out, const float* in, size_t n, hipStream_t s);
size_t cx_argmax_parts(size_t n);
int cx_launch_argmax_final(const float* v, const float* pv, const uint32_t* pi, uint32_t nparts,
                           uint32_t* out, cx_dstate* st, uint32_t* hist, uint32_t* hist_host,
                           hipStream_t s);
int cx_launch_argmax(const float* v, size_t n, float* pv, uint32_t* pi, uint32_t* out,
                     cx_dstate* st, uint32_t* hist, uint32_t* hist_host, hipStream_t s);

int cx_launch_argmax_one(const float* v, size_t n, uint32_t* out, hipStream_t s);
int cx_launch_rope(float* x, size_t tokens, size_t heads, size_t hd, const float* cos_t,
                   const float* sin_t, size_t pos, hipStream_t s);

// cx_gen.hip: daiss-style seeded weights generated in HBM
int cx_gen_rows_f32(float* out, uint64_t name_hash, uint64_t seed, uint32_t rows, uint32_t width,
                    float sigma, hipStream_t s);
int cx_gen_fill(float* out, size_t n, float value, hipStream_t s);
int cx_quantize_blocks_dev(int type, const float* x, size_t n, uint8_t* out, hipStream_t s);
uint64_t cx_fnv_name(const char* name);
