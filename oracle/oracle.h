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
 *   - quantize_groupwise: closed forms -- groups whose maximum is 127 (g + 1)
 *     have scale g + 1 exactly and x = k (g + 1) maps to k (so the group
 *     indexing and sign are pinned), an all-zero group has scale
 *     fp32(1e-8) / 127 and zeros, and x / s = n + 1/2 rounds to even -- plus the
 *     bound |q s - x| <= s / 2 on random data.
 */
#ifndef Q3VL_ORACLE_H
#define Q3VL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-row, per-group RMS int16 activation quantizer
 * (matmul/src/cpu_f32a_i8f32sb_f32c_avx2.cpp:135-177).
 * A [M,K] fp32 -> q [M,K] int16, a_s [M,K/gs] fp32. */
void orc_quantize_rows(const float *A, size_t M, size_t K, size_t gs,
                       int16_t *q, float *a_s);

/* M=1 lane-ordered GEMV (cpu_f32a_i8f32sb_f32c_avx2.cpp:122-224). G (optional) receives [N,K/gs] int32 sums. */
void orc_gemv_lanes(const float *x, const int8_t *W, const float *S, float *y,
                    int32_t *G, size_t N, size_t K, size_t gs);

/* General path (cpu_f32a_i8f32sb_f32c_avx2.cpp:477-662). contract!=0 evaluates acc = fma(G*a_s, w_s, acc);
 * contract==0 evaluates acc = acc + (G*a_s)*w_s with three roundings. */
void orc_linear_general(const float *A, const int8_t *W, const float *S,
                        float *C, int32_t *G, size_t M, size_t N, size_t K,
                        size_t gs, int contract);

/* Dispatch (matmul/src/cpu_wrapper.cpp:339-348): lane path when M==1 && N>=1024 && K>=1024, else general. */
int orc_uses_lane_path(size_t M, size_t N, size_t K);
void orc_linear_i8(const float *A, const int8_t *W, const float *S, float *C,
                   int32_t *G, size_t M, size_t N, size_t K, size_t gs);

/* swiglu (layers/src/text_layer.cpp:420-434): gate[i] = (g / (1 + expf(-g))) * up[i], in place on gate. */
void orc_swiglu(float *gate, const float *up, size_t n);

/* greedy_decode (tokenizer/src/utils.cpp:34-44): argmax over each of M rows of V logits. */
int32_t orc_argmax(const float *logits, size_t V);
void orc_argmax_rows(const float *logits, size_t M, size_t V, int32_t *ids);

/* The checkpoint exporter's weight quantizer, quantize_groupwise of
 * export_bin/export_qwen_bin.py:260-275 (numpy fp32): m = max|x| + 1e-8,
 * s = m / 127, q = round-half-even(x / s) clipped to [-127, 127].
 * x [count] -> q [count], scales [count / group]. */
void orc_quantize_groupwise(const float *x, size_t count, size_t group, int8_t *q,
                            float *scales);

/* ---- decode step (decode_oracle.c): the int8 path's caller, forward_text */
typedef struct orc_model {
    int vocab, hidden, inter, layers, heads, kv_heads, head_dim, max_seq, gs;
    float eps;
    const int8_t *emb_w;   const float *emb_s;    /* [vocab, hidden], tied lm_head */
    const int8_t *fnorm_w; const float *fnorm_s;  /* [hidden] final norm */
    const int8_t *anorm_w; const float *anorm_s;  /* [L, hidden] pre-attention norm */
    const int8_t *mnorm_w; const float *mnorm_s;  /* [L, hidden] pre-MLP norm */
    const int8_t *qnorm_w; const float *qnorm_s;  /* [L, head_dim] */
    const int8_t *knorm_w; const float *knorm_s;  /* [L, head_dim] */
    const int8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;  /* [L, N, K] each */
    const float *sq, *sk, *sv, *so, *sg, *su, *sd;   /* [L, N, K/gs] */
    const float *rope_cos, *rope_sin;                /* [max_seq, head_dim/2] */
} orc_model;

float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);
float orc_sumsq(const float *x, size_t n);
void orc_embed(const int8_t *emb_w, const float *emb_s, size_t hidden, size_t gs,
               int32_t token, float *out);
void orc_rms_norm_i8(const float *x, const int8_t *w, const float *ws, size_t n, size_t gs,
                     float eps, float *out);
void orc_rms_norm_inplace_i8(float *x, const int8_t *w, const float *ws, size_t n, size_t gs,
                             float eps, size_t batches);
void orc_rope(float *x, const float *cos_row, const float *sin_row, size_t heads, size_t hd);
float orc_exp256(float x);
void orc_softmax(float *x, size_t n);
void orc_attention(const float *q, const float *kc, const float *vc, size_t heads,
                   size_t kv_heads, size_t hd, size_t max_seq, size_t pos, float *att,
                   float *out);
void orc_attention_chunked(const float *q, const float *kc, const float *vc, size_t heads,
                           size_t kv_heads, size_t hd, size_t max_seq, size_t pos, float *att,
                           float *out);
#define ORC_KV_FP16 1
#define ORC_ATTN_CHUNKED 2
int32_t orc_decode_step(const orc_model *m, void *k_cache, void *v_cache, int flags,
                        int32_t token, size_t pos, float *logits);

#ifdef __cplusplus
}
#endif

#endif
