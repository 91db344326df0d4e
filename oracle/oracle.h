/*
 * oracle.h -- CPU restatement of the reference's INT8 group-quantized matmul
 * path (test infrastructure only).
 *
 * THIS IS A CHECKER, NOT PRODUCT CODE. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it. The HIP library never calls it.
 *
 * Every function restates the reference's algorithm from its source, cited as
 * path:line relative to the reference repository root. It is plain scalar C,
 * built with -ffp-contract=off so that every fp32 operation is the one written
 * here (fused multiply-adds are spelled fmaf explicitly where the reference
 * fuses them).
 *
 * Pinning (see tests/test_oracle.py):
 *   - q16 / a_s / int32 group sums / M=1 fp32 output / general-path fp32 output:
 *     bit-exact against oracle/_ref (the reference sources compiled here) on the
 *     committed golden vectors, plus known-answer cases (constant group, one
 *     spike, all-zero group, round-half-even ties) and an int64 brute force.
 *   - argmax: brute force and the tie / NaN / -inf cases of greedy_decode.
 *   - swiglu: against the compiled reference swiglu() (libm expf).
 */
#ifndef Q3VL_ORACLE_H
#define Q3VL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* a7: per-row, per-group RMS int16 activation quantizer.
 * A [M,K] fp32 -> q [M,K] int16, a_s [M,K/gs] fp32. */
void orc_quantize_rows(const float *A, size_t M, size_t K, size_t gs,
                       int16_t *q, float *a_s);

/* a5/a6: M=1 lane-ordered GEMV. G (optional) receives [N,K/gs] int32 sums. */
void orc_gemv_lanes(const float *x, const int8_t *W, const float *S, float *y,
                    int32_t *G, size_t N, size_t K, size_t gs);

/* a4: general path. contract!=0 evaluates acc = fma(G*a_s, w_s, acc);
 * contract==0 evaluates acc = acc + (G*a_s)*w_s with three roundings. */
void orc_linear_general(const float *A, const int8_t *W, const float *S,
                        float *C, int32_t *G, size_t M, size_t N, size_t K,
                        size_t gs, int contract);

/* a4 dispatch: lane path when M==1 && N>=1024 && K>=1024, else general. */
int orc_uses_lane_path(size_t M, size_t N, size_t K);
void orc_linear_i8(const float *A, const int8_t *W, const float *S, float *C,
                   int32_t *G, size_t M, size_t N, size_t K, size_t gs);

/* a9: gate[i] = (g / (1 + expf(-g))) * up[i], in place on gate. */
void orc_swiglu(float *gate, const float *up, size_t n);

/* a11: greedy_decode argmax over each of M rows of V logits. */
int32_t orc_argmax(const float *logits, size_t V);
void orc_argmax_rows(const float *logits, size_t M, size_t V, int32_t *ids);

#ifdef __cplusplus
}
#endif

#endif
