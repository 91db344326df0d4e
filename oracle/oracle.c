/*
 * oracle.c -- scalar C restatement of the reference INT8 matmul path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library, never the thing
 * measured or shipped (only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it). Built with -O2 -ffp-contract=off so the fp32
 * operation sequence is exactly the one written below.
 *
 * Reference file: matmul/src/cpu_f32a_i8f32sb_f32c_avx2.cpp (cited as "i8:")
 * and matmul/include/simd_utils.hpp (cited as "simd:").
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* simd:5-19 add_reduce_mm_256: 128-bit halves added lane-wise, then two
 * horizontal adds: ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)). */
static float tree8(const float v[8]) {
    float s0 = v[0] + v[4], s1 = v[1] + v[5];
    float s2 = v[2] + v[6], s3 = v[3] + v[7];
    return (s0 + s1) + (s2 + s3);
}

/* x86 cvtps2dq under the default MXCSR (round-to-nearest-even): NaN and
 * out-of-range inputs give INT32_MIN ("integer indefinite"). */
static int32_t cvt_rne_i32(float p) {
    if (!(p >= -2147483648.0f && p < 2147483648.0f)) return INT32_MIN;
    return (int32_t)nearbyintf(p);
}

/* packs_epi32: signed saturation to int16. */
static int16_t sat16(int32_t v) {
    if (v > 32767) return 32767;
    if (v < -32768) return -32768;
    return (int16_t)v;
}

/* One row of the activation quantizer, i8:135-177 (same logic at i8:348-390
 * and i8:488-530). */
static void quantize_row(const float *a, size_t K, size_t gs, int16_t *q,
                         float *a_s) {
    const float inv_gs = 1.0f / (float)gs;   /* i8:129 */
    const float inv_127 = 1.0f / 127.0f;     /* i8:130 */
    for (size_t kk = 0; kk < K; kk += gs) {
        /* i8:136-145: two 8-lane FMA chains over 16-element steps. */
        float p0[8] = {0}, p1[8] = {0};
        for (size_t k = kk; k < kk + gs; k += 16) {
            for (int i = 0; i < 8; ++i) {
                p0[i] = fmaf(a[k + i], a[k + i], p0[i]);
                p1[i] = fmaf(a[k + 8 + i], a[k + 8 + i], p1[i]);
            }
        }
        /* i8:148: add the two chains lane-wise, then the fixed tree. */
        float v[8];
        for (int i = 0; i < 8; ++i) v[i] = p0[i] + p1[i];
        const float sumsq = tree8(v);
        /* i8:151-152. gs is a power of two, so sumsq*inv_gs is exact and a
         * contracted or uncontracted "+1e-6f" round identically. */
        const float rms = sqrtf(sumsq * inv_gs + 1e-6f);
        const float s_val = rms * inv_127;
        a_s[kk / gs] = s_val;                 /* i8:154 */
        const float inv = 1.0f / s_val;       /* i8:156 */
        /* i8:158-176: multiply, cvtps2dq, packs_epi32 (order restored by
         * the 0xD8 permute, which only undoes the pack interleave). */
        for (size_t k = kk; k < kk + gs; ++k) q[k] = sat16(cvt_rne_i32(a[k] * inv));
    }
}

void orc_quantize_rows(const float *A, size_t M, size_t K, size_t gs,
                       int16_t *q, float *a_s) {
    const size_t Kg = K / gs;
    for (size_t m = 0; m < M; ++m) quantize_row(A + m * K, K, gs, q + m * K, a_s + m * Kg);
}

/* a5 gemv_lg_N_lg_K_transpose (i8:122-224) and a6 ..._decode (i8:327-455):
 * identical arithmetic; the second only chunks rows and prefetches. */
void orc_gemv_lanes(const float *x, const int8_t *W, const float *S, float *y,
                    int32_t *G, size_t N, size_t K, size_t gs) {
    const size_t Kg = K / gs;
    int16_t *q = (int16_t *)malloc(K * sizeof(int16_t));
    float *as = (float *)malloc(Kg * sizeof(float));
    quantize_row(x, K, gs, q, as);
    for (size_t n = 0; n < N; ++n) {
        const int8_t *w = W + n * K;
        float c[8] = {0};
        for (size_t g = 0; g < Kg; ++g) {
            /* i8:202-209: madd_epi16 lane j = q[2j]w[2j] + q[2j+1]w[2j+1],
             * added over the group's 16-element steps. */
            int32_t L[8] = {0};
            for (size_t k = g * gs; k < (g + 1) * gs; k += 16)
                for (int j = 0; j < 8; ++j)
                    L[j] += (int32_t)q[k + 2 * j] * w[k + 2 * j] +
                            (int32_t)q[k + 2 * j + 1] * w[k + 2 * j + 1];
            if (G) {
                int32_t t = 0;
                for (int j = 0; j < 8; ++j) t += L[j];
                G[n * Kg + g] = t;
            }
            /* i8:211-216: activation scale times weight scale, then one FMA
             * per lane, groups in order. */
            const float sc = as[g] * S[n * Kg + g];
            for (int j = 0; j < 8; ++j) c[j] = fmaf((float)L[j], sc, c[j]);
        }
        y[n] = tree8(c); /* i8:219-222 */
    }
    free(q);
    free(as);
}

/* a4 general path linear_int8_fp32s_int32acc_transpose (i8:477-662): per row
 * quantization, then for each output groups in ascending order (TK=256 tiles
 * are visited in order and each holds whole groups for gs<=256):
 *   acc += float(G) * a_s * w_s     (i8:613-617, 652)
 * evaluated left to right; GCC contracts the final multiply-add into an FMA
 * under its default -ffp-contract=fast, which the golden vectors confirm. */
void orc_linear_general(const float *A, const int8_t *W, const float *S,
                        float *C, int32_t *G, size_t M, size_t N, size_t K,
                        size_t gs, int contract) {
    const size_t Kg = K / gs;
    int16_t *q = (int16_t *)malloc((K ? K : 1) * sizeof(int16_t));
    float *as = (float *)malloc((Kg ? Kg : 1) * sizeof(float));
    for (size_t m = 0; m < M; ++m) {
        quantize_row(A + m * K, K, gs, q, as);
        for (size_t n = 0; n < N; ++n) {
            const int8_t *w = W + n * K;
            float acc = 0.0f;
            for (size_t g = 0; g < Kg; ++g) {
                int32_t t = 0;
                for (size_t k = g * gs; k < (g + 1) * gs; ++k) t += (int32_t)q[k] * w[k];
                if (G) G[(m * N + n) * Kg + g] = t;
                const float ga = (float)t * as[g];
                const float ws = S[(n * K) / gs + g];
                if (contract) acc = fmaf(ga, ws, acc);
                else acc = acc + ga * ws;
            }
            C[m * N + n] = acc;
        }
    }
    free(q);
    free(as);
}

/* i8:464-475 shape dispatch. */
int orc_uses_lane_path(size_t M, size_t N, size_t K) {
    return M == 1 && N >= 1024 && K >= 1024;
}

void orc_linear_i8(const float *A, const int8_t *W, const float *S, float *C,
                   int32_t *G, size_t M, size_t N, size_t K, size_t gs) {
    if (orc_uses_lane_path(M, N, K)) orc_gemv_lanes(A, W, S, C, G, N, K, gs);
    else orc_linear_general(A, W, S, C, G, M, N, K, gs, 1);
}

/* layers/src/text_layer.cpp:420-434 swiglu. */
void orc_swiglu(float *gate, const float *up, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float x = gate[i];
        const float silu = x / (1.0f + expf(-x));
        gate[i] = silu * up[i];
    }
}

/* tokenizer/src/utils.cpp:34-44 greedy_decode: first index of the strict
 * maximum starting from -FLT_MAX; NaN never wins; nothing above -FLT_MAX -> 0. */
int32_t orc_argmax(const float *logits, size_t V) {
    float best = -FLT_MAX;
    int32_t idx = 0;
    for (size_t i = 0; i < V; ++i) {
        if (logits[i] > best) {
            best = logits[i];
            idx = (int32_t)i;
        }
    }
    return idx;
}

void orc_argmax_rows(const float *logits, size_t M, size_t V, int32_t *ids) {
    for (size_t m = 0; m < M; ++m) ids[m] = orc_argmax(logits + m * V, V);
}

/* export_bin/export_qwen_bin.py:260-275. numpy evaluates every step in
 * float32 (the array dtype; the Python scalars 1e-8 and 127 are cast to it):
 * np.max(np.abs(x)) + 1e-8, maxv / qmax, np.round(x / scales) (half to even,
 * rintf under the default rounding mode), then np.clip. */
void orc_quantize_groupwise(const float *x, size_t count, size_t group, int8_t *q,
                            float *scales) {
    for (size_t g = 0; g * group < count; ++g) {
        const float *xg = x + g * group;
        float m = 0.0f;
        for (size_t i = 0; i < group; ++i) {
            const float a = fabsf(xg[i]);
            if (a > m) m = a;
        }
        const float s = (m + 1e-8f) / 127.0f;
        scales[g] = s;
        for (size_t i = 0; i < group; ++i) {
            float r = rintf(xg[i] / s);
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            q[g * group + i] = (int8_t)r;
        }
    }
}
