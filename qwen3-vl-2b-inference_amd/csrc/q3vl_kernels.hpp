// q3vl_kernels.hpp -- host-side launchers of the gfx950 kernels (internal to
// libq3vl_int8.so; the public surface is include/q3vl_int8.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q3vl {

// ---------------------------------------------------------------- quantizer
hipError_t launch_quantize_i16(const float *A, int16_t *q, float *a_s, int M, int K,
                               int gs, hipStream_t st);
// fp16 images of q (exact: |q| <= 1016) with row stride ldq, and a_s stored
// transposed as a_sT[g * lda_s + m] for the GEMM epilogue.
hipError_t launch_quantize_f16(const float *A, _Float16 *q, float *a_sT, int M, int K,
                               int gs, int ldq, int lda_s, hipStream_t st);
// The exporter's weight quantizer: int8 values and one fp32 scale per group
// of `group` consecutive values.
hipError_t launch_quantize_export(const float *x, size_t count, size_t group, int8_t *q,
                                  float *scales, hipStream_t st);

// ------------------------------------------------------------ GEMV (M <= 8)
// Up to three weight matrices stacked along N share one quantized activation.
struct GemvSeg {
    const int8_t *W;  // [N, K] int8, reference layout (mat_B_transpose=true)
    const float *S;   // [N, K/gs] fp32 group scales
    float *Y;         // [M, N] fp32 output (row stride N)
    int32_t *G;       // optional [M, N, K/gs] int32 group sums (debug), or null
    int N;
};

enum GemvMode : int {
    GEMV_PLAIN = 0,   // Y_s = A W_s^T for every segment
    GEMV_SWIGLU = 1,  // seg0 = gate, seg1 = up: seg0.Y = silu(gate) * up
    GEMV_ARGMAX = 2,  // seg0 only: per-row argmax partials (+ logits if Y)
};

struct GemvArgs {
    const float *A;   // [M, K] fp32 activations
    GemvSeg seg[3];
    int nseg;
    int M, K, gs;
    int mode;
    int accumulate;   // GEMV_PLAIN: Y += A W^T (the decode step's residual add)
    float *part_val;  // GEMV_ARGMAX: [grid, M] block partial maxima
    int32_t *part_idx;  // [grid, M] block partial indices (-1: none)
    // Optional RMSNorm of the activation row before quantization (M == 1):
    // A' = w * ((s_g * inv) * A), inv = 1/sqrt(sum(A^2)/K + eps) with the sum
    // in the 8-lane order (text_layer.cpp:110-147 / 234-270, int8 group
    // weight with the GEMV's group size). norm_w == nullptr: no norm.
    const int8_t *norm_w;
    const float *norm_s;
    float norm_eps;
};

// lanes=true: the reference's M=1 path (i8:122-224 / 327-455) -- per-lane
// fp32 FMA chains and the fixed 8-lane tree. lanes=false: the general path
// (i8:477-662) -- acc = fma(G*a_s, w_s, acc), M <= 8.
// Returns the grid size used (argmax partial count) through *grid_out.
hipError_t launch_gemv(const GemvArgs &a, bool lanes, int *grid_out, hipStream_t st);

// Final argmax over block partials: ids[m] = first index of the maximum;
// *pos_inc += 1 afterwards when pos_inc is non-null (decode step position).
hipError_t launch_argmax_final(const float *part_val, const int32_t *part_idx,
                               int nparts, int M, int32_t *ids, hipStream_t st,
                               int32_t *pos_inc = nullptr);
// Block partials of greedy argmax over rows of logits ([nparts, M] layout).
hipError_t launch_argmax_partials(const float *logits, int M, int V, float *part_val,
                                  int32_t *part_idx, int nparts, hipStream_t st);
// Stand-alone greedy argmax over rows of logits (partials + final).
hipError_t launch_argmax_rows(const float *logits, int M, int V, float *part_val,
                              int32_t *part_idx, int nparts, int32_t *ids,
                              hipStream_t st);
// Stand-alone swiglu: gate[i] = silu(gate[i]) * up[i].
hipError_t launch_swiglu(float *gate, const float *up, size_t n, hipStream_t st);
// p[0..n) = 0 (32-bit words), by a kernel.
hipError_t launch_zero_words(void *p, size_t n, hipStream_t st);

// ------------------------------------------------------------ decode step
struct AttnArgs {
    const float *q, *k, *v;                 // raw projections [heads*hd], [kv_heads*hd]
    const int8_t *qnorm_w, *knorm_w;        // this layer's [hd] int8 norm weights
    const float *qnorm_s, *knorm_s;
    const float *rope_cos, *rope_sin;       // [max_seq, hd/2]
    uint16_t *k_cache, *v_cache;            // fp16 [layers, kv_heads, max_seq, hd]
    const int32_t *pos;                     // device: position of the new token
    float *scores, *cmax;                   // scratch [heads, max_seq], [heads, max_chunks]
    float *part_o, *part_ml;                // chunked order: [heads, max_chunks, hd], [heads, max_chunks, 4]: m, l, min, 0
    int order;                              // 0: the reference's order, 1: chunked
    float *out;                             // [heads*hd]
    int layer, heads, kv_heads, head_dim, max_seq, max_chunks, gs;
    float eps, inv_sqrt_d;
};
// Embedding row of *token (a NaN row for a token outside [0, vocab)).
hipError_t launch_embed(const int8_t *w, const float *s, const int32_t *token, float *x, int H,
                        int gs, int vocab, hipStream_t st);
hipError_t launch_attention(const AttnArgs &a, hipStream_t st);
constexpr int kAttnChunk = 64;  // positions per attention score chunk
// Dynamic LDS the softmax/value kernel needs; at most kAttnMaxLds (160 KiB
// less room for its static LDS).
size_t attention_lds_bytes(int heads, int kv_heads, int max_seq);
constexpr size_t kAttnMaxLds = 160 * 1024 - 4096;

// ---------------------------------------------------------- GEMM (MFMA)
struct GemmArgs {
    const _Float16 *Aq;  // [M, lda] exact fp16 images of the int16 activations
    const float *a_s;    // transposed: a_s[g * lda_s + m]
    int lda;
    int lda_s;
    const int8_t *W0;    // [N, K] (gate when swiglu)
    const float *S0;
    const int8_t *W1;    // up weights when swiglu, else null
    const float *S1;
    float *C;            // [M, N] output (H when swiglu)
    int32_t *G;          // optional [M, N, K/gs] group sums (not with swiglu)
    int M, N, K, gs;
    bool swiglu;
};
hipError_t launch_gemm(const GemmArgs &a, hipStream_t st);

// Group size 64: activations quantized into MFMA fragment order
// (launch_quantize_frag), then the fragment-order GEMM.
struct GemmMfArgs {
    const _Float16 *Af;  // [Mt][K/64][4][64][8] fp16 fragments of q (Mt = ceil(M/32))
    const float *asf;    // [Mt][K/64][2][16] activation scales in accumulator order
    int Mt;
    const int8_t *W0;    // [N, K] (gate when swiglu)
    const float *S0;     // [N, K/64]
    const int8_t *W1;    // up weights when swiglu, else null
    const float *S1;
    float *C;            // [M, N] (H when swiglu)
    int M, N, K;
    // optional (not with swiglu): greedy-argmax partials of each block's
    // columns per row, [ceil(N / gemm_mf_argmax_cols(...))][M], for
    // launch_argmax_final
    float *part_val = nullptr;
    int32_t *part_idx = nullptr;
    // optional (swiglu, N % 64 == 0): H is not stored; instead it is
    // quantized as launch_quantize_frag would quantize it, into hq
    // [Mt][N/64][4][64][8] and hqs [Mt][N/64][2][16] (the operand of a GEMM
    // with K = N)
    _Float16 *hq = nullptr;
    float *hqs = nullptr;
};
// Columns per argmax partial of launch_gemm_mf for an M-row plain product.
int gemm_mf_argmax_cols(int M);
// qf must hold 32*ceil(M/32)*K halves, asf 32*ceil(M/32)*K/64 floats.
hipError_t launch_quantize_frag(const float *A, _Float16 *qf, float *asf, int M, int K,
                                hipStream_t st);
// Whether the fragment-order GEMM serves an M x N x K product (else
// launch_gemm's kernels, with launch_quantize_f16), on a device of `cus` CUs.
bool gemm_mf_serves(int M, int N, int K, bool swiglu, int cus);
hipError_t launch_gemm_mf(const GemmMfArgs &a, bool swiglu, int cus, hipStream_t st);
// 16 or fewer rows of fp32 activations A [M, K] against a wide weight (K %
// 512 == 0, K <= 2048): quantized inside the kernel, 16 x 16 MFMA tiles with
// the weights loaded straight into the operands. With argmax partial buffers
// it leaves gemm_mf_wide_parts(N, cus) partials per row, [parts][M]; C may
// then be null.
bool gemm_mf_wide_serves(int M, int N, int K);
int gemm_mf_wide_parts(int N, int cus);
hipError_t launch_gemm_mf_wide(const float *A, const int8_t *W, const float *S, float *C, int M, int N,
                               int K, float *part_val, int32_t *part_idx, int cus, hipStream_t st);

}  // namespace q3vl
