/*
 * ref_shim.c — TEST INFRASTRUCTURE ONLY (linked into oracle/_ref only).
 *
 * Adapts the reference's hand-written Q4_K assembly contract
 *   void cosxamix_q4k_completo(blocks, xq, xe, xs, n_blocks, float acc[16])
 * (src/kernels/q4k_asm.rs:171-203) to the 5-argument row-kernel ABI used by
 * every other reference kernel (src/kernels/q2k.rs:153), finishing with the
 * same horizontal reduction the reference uses, reducir_f32
 * (src/kernels/x86.rs:92-99): ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)), and the
 * final `sum(acc[0..8]) - sum(acc[8..16])` of q4k_asm.rs:214-235.
 */
#include <stddef.h>
#include <stdint.h>

void cosxamix_q4k_completo(const uint8_t *, const int8_t *, const float *,
                           const float *, size_t, float *);

static float reduce8(const float *a) {
  float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
  float t0 = s0 + s2, t1 = s1 + s3;
  return t0 + t1;
}

float cxref_q4k_row(const uint8_t *b, const int8_t *xq, const float *xe,
                    const float *xs, size_t nb) {
  float acc[16] = {0};
  cosxamix_q4k_completo(b, xq, xe, xs, nb, acc);
  return reduce8(acc) - reduce8(acc + 8);
}
