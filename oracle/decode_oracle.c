/*
 * decode_oracle.c -- scalar C restatement of the reference's text decode step
 * (model/src/forward.cpp:458-720) on an int8 model: the caller of the int8
 * matmul path. TEST INFRASTRUCTURE ONLY (checker for the GPU decode step and
 * cpu_baseline material), built with -ffp-contract=off.
 *
 * Reference files: layers/src/text_layer.cpp ("tl:"), layers/include/
 * simd_utils.hpp ("ls:"), model/src/load_model.cpp ("lm:").
 *
 * Where the reference leaves the order to the compiler (`#pragma omp simd
 * reduction`), the tail attention positions (tl:626-633) follow GCC's AVX2
 * vectorization (identified against the compiled reference), and the RMS sum
 * of squares (tl:120-124, 248-252) uses this build's fixed order (pinned to a
 * tolerance). Everything else follows the reference's explicit order.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* ------------------------------------------------------------ fp16 helpers */
float orc_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalize */
            int e = -1;
            do {
                man <<= 1;
                ++e;
            } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* IEEE round-to-nearest-even float -> half. */
uint16_t orc_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u);
    if (ax >= 0x477FF000u) return sign | 0x7C00u; /* rounds to >= 65520: inf */
    if (ax < 0x38800000u) {                        /* below 2^-14: subnormal */
        if (ax < 0x33000000u) return sign;         /* < 2^-25: rounds to 0 */
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126 - e; /* 14..24 */
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1);
        const uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (r & 1u))) ++r;
        return sign | (uint16_t)r;
    }
    uint32_t r = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return sign | (uint16_t)r;
}

/* ---------------------------------------------------------- building blocks */

/* Sum of squares in the order the reference's `omp simd reduction(+:ss)`
 * loops take (tl:121-124, tl:247-250, compiled for 8-wide AVX2): lane l
 * accumulates x[j]*x[j] for j = l (mod 8) with one FMA per term, then the
 * lanes are folded left to right, ((c0 + c1) + c2) + ... + c7. Terms past the
 * last multiple of 8 are added after the fold, one FMA each. */
float orc_sumsq(const float *x, size_t n) {
    float c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const size_t n8 = n & ~(size_t)7;
    for (size_t j = 0; j < n8; j += 8)
        for (int l = 0; l < 8; ++l) c[l] = fmaf(x[j + l], x[j + l], c[l]);
    float s = c[0];
    for (int l = 1; l < 8; ++l) s = s + c[l];
    for (size_t j = n8; j < n; ++j) s = fmaf(x[j], x[j], s);
    return s;
}

/* tl:3-49 embedding_lookup, int8 group-quantized branch. */
void orc_embed(const int8_t *emb_w, const float *emb_s, size_t hidden, size_t gs,
               int32_t token, float *out) {
    const int8_t *w = emb_w + (size_t)token * hidden;
    const float *s = emb_s + (size_t)token * hidden / gs;
    for (size_t i = 0; i < hidden; ++i) out[i] = (float)w[i] * s[i / gs];
}

/* tl:110-147 rms_norm, int8 group-quantized weight, one row. The argument of
 * sqrt is a float, so the float overload is taken: inv = (float)(1.0 /
 * (double)sqrtf(ss/n + eps)), out = w * ((s_g * inv) * x). */
void orc_rms_norm_i8(const float *x, const int8_t *w, const float *ws, size_t n, size_t gs,
                     float eps, float *out) {
    const float ss = orc_sumsq(x, n);
    const float inv_hs = 1.0f / (float)n;
    const float inv = (float)(1.0 / (double)sqrtf(ss * inv_hs + eps));
    for (size_t g = 0; g < n; g += gs) {
        const float combined = ws[g / gs] * inv;
        for (size_t j = g; j < g + gs; ++j) out[j] = (float)w[j] * (combined * x[j]);
    }
}

/* tl:234-270 rms_norm_inplace, int8 group-quantized weight, `batches` rows of
 * n: inv = 1.0f / sqrtf(ss/n + eps) in fp32, x = w * ((s_g * inv) * x). */
void orc_rms_norm_inplace_i8(float *x, const int8_t *w, const float *ws, size_t n, size_t gs,
                             float eps, size_t batches) {
    const float inv_hs = 1.0f / (float)n;
    for (size_t b = 0; b < batches; ++b) {
        float *xr = x + b * n;
        const float ss = orc_sumsq(xr, n);
        const float inv = 1.0f / sqrtf(ss * inv_hs + eps);
        for (size_t g = 0; g < n; g += gs) {
            const float combined = ws[g / gs] * inv;
            for (size_t j = g; j < g + gs; ++j) xr[j] = (float)w[j] * (combined * xr[j]);
        }
    }
}

/* tl:712-760 apply_rotary (and the rotation of tl:767-824): per head, with
 * half = hd/2: y1 = fma(x1, c, -(x2*s)), y2 = fma(x1, s, x2*c). */
void orc_rope(float *x, const float *cos_row, const float *sin_row, size_t heads, size_t hd) {
    const size_t half = hd / 2;
    for (size_t h = 0; h < heads; ++h) {
        float *x1 = x + h * hd, *x2 = x1 + half;
        for (size_t i = 0; i < half; ++i) {
            const float a = x1[i], b = x2[i], c = cos_row[i], s = sin_row[i];
            x1[i] = fmaf(a, c, -(b * s));
            x2[i] = fmaf(a, s, b * c);
        }
    }
}

/* ls:7-47 exp256_ps, one lane: clamp, n = floor(x*log2e), g = x - n*ln2 (one
 * rounding), degree-4 Taylor by FMAs, times 2^n built from the exponent
 * bits. Note 2^n is -inf for n = -128 (x below about -88.03), as in the
 * reference. */
float orc_exp256(float x) {
    x = fminf(x, 88.3762626647949f);
    x = fmaxf(x, -88.3762626647949f);
    const float ln2 = 0.69314718056f, inv_ln2 = 1.44269504089f;
    const float fx = floorf(x * inv_ln2);
    const int32_t n = (int32_t)fx;
    const float g = fmaf(-fx, ln2, x);
    float y = fmaf(g, 1.0f, 1.0f);
    const float g2 = g * g;
    y = fmaf(g2, 0.5f, y);
    const float g3 = g2 * g;
    y = fmaf(g3, 1.0f / 6.0f, y);
    const float g4 = g3 * g;
    y = fmaf(g4, 1.0f / 24.0f, y);
    const uint32_t bits = (uint32_t)(n + 127) << 23;
    float p;
    memcpy(&p, &bits, 4);
    return y * p;
}

/* tl:436-535 softmax (AVX2 branch) over x[0..n). */
void orc_softmax(float *x, size_t n) {
    if (n == 0) return;
    const size_t nb = n / 8 * 8;
    float lane_max[8];
    for (int l = 0; l < 8; ++l) lane_max[l] = -INFINITY;
    for (size_t i = 0; i < nb; ++i) {
        const float v = x[i];
        const int l = (int)(i % 8);
        /* _mm256_max_ps(vmax, v): returns v when vmax is not greater */
        lane_max[l] = lane_max[l] > v ? lane_max[l] : v;
    }
    float mx = lane_max[0];
    for (int k = 1; k < 8; ++k) mx = fmaxf(mx, lane_max[k]);
    for (size_t i = nb; i < n; ++i) mx = fmaxf(mx, x[i]);
    if (!isfinite(mx)) {
        memset(x, 0, n * sizeof(float));
        return;
    }
    float lane_sum[8] = {0};
    for (size_t i = 0; i < nb; ++i) {
        const float v = x[i];
        const float e = v > -INFINITY ? orc_exp256(v - mx) : 0.0f;
        x[i] = e;
        lane_sum[i % 8] = lane_sum[i % 8] + e;
    }
    double sum = 0.0;
    for (int k = 0; k < 8; ++k) sum += lane_sum[k];
    for (size_t i = nb; i < n; ++i) {
        if (x[i] == -INFINITY) {
            x[i] = 0.0f;
            continue;
        }
        x[i] = orc_exp256(x[i] - mx);
        sum += x[i];
    }
    if (!(sum > 0.0) || !isfinite(sum)) {
        memset(x, 0, n * sizeof(float));
        return;
    }
    const float inv_sum = (float)(1.0 / sum);
    for (size_t i = 0; i < n; ++i) x[i] *= inv_sum;
}

/* 8 FMA lane chains over the head dimension then the fixed 8-lane tree
 * (tl:598-620 with add_reduce_mm_256_layer). */
static float dot_lanes(const float *q, const float *k, size_t hd) {
    float c[8] = {0};
    for (size_t i = 0; i < hd; i += 8)
        for (int l = 0; l < 8; ++l) c[l] = fmaf(q[i + l], k[i + l], c[l]);
    const float s0 = c[0] + c[4], s1 = c[1] + c[5], s2 = c[2] + c[6], s3 = c[3] + c[7];
    return (s0 + s1) + (s2 + s3);
}

/* Tail positions (tl:626-633): `#pragma omp simd reduction(+:score)` over
 * score += q[i]*k[i], restated as GCC's AVX2 vectorization of it: the same 8
 * FMA lane chains, then the lanes added in order l0 + l1 + ... + l7
 * (identified against the compiled reference on all-tail probes). */
static float dot_tail(const float *q, const float *k, size_t hd) {
    float c[8] = {0};
    for (size_t i = 0; i < hd; i += 8)
        for (int l = 0; l < 8; ++l) c[l] = fmaf(q[i + l], k[i + l], c[l]);
    float s = c[0];
    for (int l = 1; l < 8; ++l) s = s + c[l];
    return s;
}

/* tl:575-650 attn_scores_all_heads + softmax, and tl:655-710
 * attn_weighted_sum_all_heads, for one layer. kc/vc: that layer's cache rows
 * as fp32 [kv_heads][max_seq][hd] (an fp16 cache is widened by the caller).
 * q [heads][hd] -> out [heads][hd]; att scratch [pos+1]. */
void orc_attention(const float *q, const float *kc, const float *vc, size_t heads,
                   size_t kv_heads, size_t hd, size_t max_seq, size_t pos, float *att,
                   float *out) {
    const size_t kv_mul = heads / kv_heads;
    const float inv_sqrt_d = 1.0f / sqrtf((float)hd);
    for (size_t h = 0; h < heads; ++h) {
        const float *qh = q + h * hd;
        const float *kh = kc + (h / kv_mul) * max_seq * hd;
        const float *vh = vc + (h / kv_mul) * max_seq * hd;
        /* main loop: blocks of 8 positions with t + 8 <= pos (tl:593-622);
         * the tail loop then recomputes t in [pos/8*8, pos] (tl:626-634) */
        for (size_t t = 0; t <= pos; ++t) att[t] = dot_lanes(qh, kh + t * hd, hd) * inv_sqrt_d;
        for (size_t t = pos / 8 * 8; t <= pos; ++t)
            att[t] = dot_tail(qh, kh + t * hd, hd) * inv_sqrt_d;
        orc_softmax(att, pos + 1);
        float *oh = out + h * hd;
        for (size_t d = 0; d < hd; ++d) {
            float acc = 0.0f;
            for (size_t t = 0; t <= pos; ++t) acc = fmaf(att[t], vh[t * hd + d], acc);
            oh[d] = acc;
        }
    }
}

/* The chunked attention order (no counterpart in the reference; the GPU's
 * Q3VL_ATTN_CHUNKED): scores as orc_attention computes them, then per query
 * head and 64-position chunk c (positions t of the chunk below pos + 1):
 *   m_c = max of the chunk's scores (fmaxf from -inf),
 *   e_t = exp256(s_t - m_c), 0 for s_t = -inf or m_c not finite, and 0 for
 *         the chunk's slots past the context,
 *   l_c = xor butterfly over the chunk's 64 slots: for offsets 32, 16, 8, 4,
 *         2, 1 every slot i becomes slot i + slot (i ^ offset); slot 0,
 *   o_c[d] = fmaf chain over the chunk's t ascending of e_t * v_t[d];
 * then, over the chunks ascending: M = max_c m_c, w_c = exp256(m_c - M) (0
 * for m_c = -inf or M not finite), L and O[d] fmaf chains of w_c * l_c and
 * w_c * o_c[d], out[d] = O[d] * (1.0f / L) when L is finite and positive,
 * else 0. The whole head is 0 when M is finite and exp256(min_c - M) is -inf
 * for some chunk, min_c being the chunk's smallest score above -inf: the
 * reference's softmax has a -inf term exactly then (exp256 is -inf on a
 * half-line, fl(s - M) is monotone in s) and zeroes the head
 * (text_layer.cpp:512-515). */
void orc_attention_chunked(const float *q, const float *kc, const float *vc, size_t heads,
                           size_t kv_heads, size_t hd, size_t max_seq, size_t pos, float *att,
                           float *out) {
    const size_t kv_mul = heads / kv_heads, n = pos + 1, nch = (n + 63) / 64;
    const float inv_sqrt_d = 1.0f / sqrtf((float)hd);
    float *mc = malloc(nch * 4), *lc = malloc(nch * 4), *nc = malloc(nch * 4), *oc = malloc(nch * hd * 4);
    for (size_t h = 0; h < heads; ++h) {
        const float *qh = q + h * hd;
        const float *kh = kc + (h / kv_mul) * max_seq * hd;
        const float *vh = vc + (h / kv_mul) * max_seq * hd;
        for (size_t t = 0; t <= pos; ++t) att[t] = dot_lanes(qh, kh + t * hd, hd) * inv_sqrt_d;
        for (size_t t = pos / 8 * 8; t <= pos; ++t)
            att[t] = dot_tail(qh, kh + t * hd, hd) * inv_sqrt_d;
        for (size_t c = 0; c < nch; ++c) {
            const size_t t0 = 64 * c, rows = n - t0 < 64 ? n - t0 : 64;
            float m = -INFINITY, mn = INFINITY;
            for (size_t i = 0; i < rows; ++i) {
                m = fmaxf(m, att[t0 + i]);
                if (att[t0 + i] > -INFINITY) mn = fminf(mn, att[t0 + i]);
            }
            nc[c] = mn;
            float e[64];
            for (size_t i = 0; i < 64; ++i)
                e[i] = (i < rows && att[t0 + i] > -INFINITY && isfinite(m))
                           ? orc_exp256(att[t0 + i] - m) : 0.0f;
            float b[64];
            memcpy(b, e, sizeof b);
            for (size_t off = 32; off > 0; off >>= 1) {
                float nb[64];
                for (size_t i = 0; i < 64; ++i) nb[i] = b[i] + b[i ^ off];
                memcpy(b, nb, sizeof b);
            }
            mc[c] = m;
            lc[c] = b[0];
            for (size_t d = 0; d < hd; ++d) {
                float acc = 0.0f;
                for (size_t i = 0; i < rows; ++i) acc = fmaf(e[i], vh[(t0 + i) * hd + d], acc);
                oc[c * hd + d] = acc;
            }
        }
        float M = -INFINITY;
        for (size_t c = 0; c < nch; ++c) M = fmaxf(M, mc[c]);
        int vanish = 0;
        for (size_t c = 0; c < nch; ++c)
            if (isfinite(M) && nc[c] < INFINITY && orc_exp256(nc[c] - M) == -INFINITY) vanish = 1;
        for (size_t d = 0; d < hd; ++d) {
            if (vanish) {
                out[h * hd + d] = 0.0f;
                continue;
            }
            float L = 0.0f, O = 0.0f;
            for (size_t c = 0; c < nch; ++c) {
                const float w = (isfinite(M) && mc[c] > -INFINITY) ? orc_exp256(mc[c] - M) : 0.0f;
                L = fmaf(w, lc[c], L);
                O = fmaf(w, oc[c * hd + d], O);
            }
            out[h * hd + d] = (L > 0.0f && isfinite(L)) ? O * (1.0f / L) : 0.0f;
        }
    }
    free(mc), free(lc), free(nc), free(oc);
}

/* model/src/forward.cpp:458-720 forward_text for a text token at `pos`.
 * flags bit 0 (ORC_KV_FP16): the caches hold fp16 bits (uint16) and new K/V
 * rows are rounded to fp16 on store; clear: fp32 caches as in the reference
 * (lm:348-349). Bit 1 (ORC_ATTN_CHUNKED): orc_attention_chunked in place of
 * the reference's attention. Returns greedy_decode(logits); logits [vocab]
 * if non-null. */
int32_t orc_decode_step(const orc_model *m, void *k_cache, void *v_cache, int flags,
                        int32_t token, size_t pos, float *logits) {
    const int kv_fp16 = flags & ORC_KV_FP16;
    const size_t H = (size_t)m->hidden, I = (size_t)m->inter, NH = (size_t)m->heads;
    const size_t NKV = (size_t)m->kv_heads, D = (size_t)m->head_dim, S = (size_t)m->max_seq;
    const size_t gs = (size_t)m->gs, V = (size_t)m->vocab, L = (size_t)m->layers;
    const size_t QD = NH * D, KD = NKV * D;
    float *x = malloc(H * 4), *t = malloc(H * 4), *q = malloc(QD * 4), *k = malloc(KD * 4);
    float *v = malloc(KD * 4), *ao = malloc(QD * 4), *gt = malloc(I * 4), *up = malloc(I * 4);
    float *att = malloc((pos + 1) * 4), *kl = malloc(NKV * S * D * 4), *vl = malloc(NKV * S * D * 4);
    float *lg = logits ? logits : malloc(V * 4);

    orc_embed(m->emb_w, m->emb_s, H, gs, token, x); /* :478-485 */
    const float *cos_row = m->rope_cos + pos * (D / 2), *sin_row = m->rope_sin + pos * (D / 2);
    for (size_t l = 0; l < L; ++l) {
        /* :493 pre-attention RMSNorm (the reference's rms_ffn_w) */
        orc_rms_norm_i8(x, m->anorm_w + l * H, m->anorm_s + l * H / gs, H, gs, m->eps, t);
        /* :506-528 q, k, v */
        orc_linear_i8(t, m->wq + l * QD * H, m->sq + l * QD * H / gs, q, NULL, 1, QD, H, gs);
        orc_linear_i8(t, m->wk + l * KD * H, m->sk + l * KD * H / gs, k, NULL, 1, KD, H, gs);
        orc_linear_i8(t, m->wv + l * KD * H, m->sv + l * KD * H / gs, v, NULL, 1, KD, H, gs);
        /* :531-538 QK RMSNorm per head */
        orc_rms_norm_inplace_i8(q, m->qnorm_w + l * D, m->qnorm_s + l * D / gs, D, gs, m->eps, NH);
        orc_rms_norm_inplace_i8(k, m->knorm_w + l * D, m->knorm_s + l * D / gs, D, gs, m->eps, NKV);
        /* :545-562 RoPE on q and k, K/V rows written at pos */
        orc_rope(q, cos_row, sin_row, NH, D);
        orc_rope(k, cos_row, sin_row, NKV, D);
        const size_t lo = l * NKV * S * D;
        for (size_t hh = 0; hh < NKV; ++hh) {
            const size_t o = lo + (hh * S + pos) * D;
            for (size_t d = 0; d < D; ++d) {
                if (kv_fp16) {
                    ((uint16_t *)k_cache)[o + d] = orc_float_to_half(k[hh * D + d]);
                    ((uint16_t *)v_cache)[o + d] = orc_float_to_half(v[hh * D + d]);
                } else {
                    ((float *)k_cache)[o + d] = k[hh * D + d];
                    ((float *)v_cache)[o + d] = v[hh * D + d];
                }
            }
        }
        /* widen this layer's cache rows [0, pos] */
        for (size_t hh = 0; hh < NKV; ++hh)
            for (size_t tt = 0; tt <= pos; ++tt)
                for (size_t d = 0; d < D; ++d) {
                    const size_t src = lo + (hh * S + tt) * D + d, dst = (hh * S + tt) * D + d;
                    if (kv_fp16) {
                        kl[dst] = orc_half_to_float(((uint16_t *)k_cache)[src]);
                        vl[dst] = orc_half_to_float(((uint16_t *)v_cache)[src]);
                    } else {
                        kl[dst] = ((float *)k_cache)[src];
                        vl[dst] = ((float *)v_cache)[src];
                    }
                }
        /* :571-581 attention */
        if (flags & ORC_ATTN_CHUNKED)
            orc_attention_chunked(q, kl, vl, NH, NKV, D, S, pos, att, ao);
        else
            orc_attention(q, kl, vl, NH, NKV, D, S, pos, att, ao);
        /* :592-604 output projection + residual */
        orc_linear_i8(ao, m->wo + l * H * QD, m->so + l * H * QD / gs, t, NULL, 1, H, QD, gs);
        for (size_t i = 0; i < H; ++i) x[i] += t[i];
        /* :611-661 post-attention RMSNorm, gate/up, swiglu, down, residual */
        orc_rms_norm_i8(x, m->mnorm_w + l * H, m->mnorm_s + l * H / gs, H, gs, m->eps, t);
        orc_linear_i8(t, m->wg + l * I * H, m->sg + l * I * H / gs, gt, NULL, 1, I, H, gs);
        orc_linear_i8(t, m->wu + l * I * H, m->su + l * I * H / gs, up, NULL, 1, I, H, gs);
        orc_swiglu(gt, up, I);
        orc_linear_i8(gt, m->wd + l * H * I, m->sd + l * H * I / gs, t, NULL, 1, H, I, gs);
        for (size_t i = 0; i < H; ++i) x[i] += t[i];
    }
    /* :693-705 final RMSNorm (in place) and the tied int8 classifier */
    orc_rms_norm_inplace_i8(x, m->fnorm_w, m->fnorm_s, H, gs, m->eps, 1);
    orc_linear_i8(x, m->emb_w, m->emb_s, lg, NULL, 1, V, H, gs);
    const int32_t id = orc_argmax(lg, V);
    free(x), free(t), free(q), free(k), free(v), free(ao), free(gt), free(up), free(att);
    free(kl), free(vl);
    if (!logits) free(lg);
    return id;
}
