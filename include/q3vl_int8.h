/*
 * q3vl_int8.h -- C ABI of the MI355X (gfx950) int8 group-quantized matmul
 * library libq3vl_int8.so.
 *
 * It replaces the int8 branch of the reference engine's matmul entry point
 *   void linear(const void *A, const void *B, const void *B_scale,
 *               const void *bias, const void *bias_scale, void *C,
 *               size_t M, size_t N, size_t K, bool B_transpose,
 *               DType::Type ta, DType::Type tb, DType::Type tb_scale,
 *               DType::Type tc, bool group_quantized, size_t group_size)
 * (matmul/include/cpu_wrapper.hpp:10-16, matmul/src/cpu_wrapper.cpp:308-357)
 * and its consumers on the decode path: SwiGLU (layers/src/text_layer.cpp:
 * 420-434), the lm_head classifier_gemm (layers/src/text_layer.cpp:302-314)
 * and greedy_decode (tokenizer/src/utils.cpp:34-44).
 *
 * Conventions (identical to the reference's int8 path):
 *   A  fp32 [M, K] row-major activations;
 *   W  int8 [N, K] row-major weights (the reference's B with
 *      mat_B_transpose = true);
 *   S  fp32 [N, K/gs] row-major group scales, S[n*K/gs + g];
 *   C  fp32 [M, N], overwritten.
 * Activations are quantized per row and per K-group to int16 with an RMS
 * scale; int32 group sums are exact; the fp32 results reproduce the
 * reference's operation order bit for bit:
 *   M==1 && N>=1024 && K>=1024 : per-lane FMA chains + fixed 8-lane tree
 *                                (cpu_f32a_i8f32sb_f32c_avx2.cpp:122-224);
 *   otherwise                  : acc = fma(float(G)*a_s, w_s, acc) per group
 *                                (cpu_f32a_i8f32sb_f32c_avx2.cpp:477-662).
 *
 * All pointers passed to compute entry points are DEVICE pointers (HIP
 * allocations visible to the current device). Every call is asynchronous on
 * `stream` (a hipStream_t; NULL = the null stream) and returns a status code;
 * q3vl_last_error() gives the message of this thread's last failure.
 *
 * Shape support: K % group_size == 0. M <= 8 runs the HBM-bound GEMV kernels
 * (group_size in {16,32,64,128,256}, K <= 8192, K % 16 == 0); M > 8 runs the
 * matrix-core GEMM (group_size in {32,64,128}, K % 64 == 0). A and W must be
 * 16-byte aligned.
 *
 * Workspace: entry points that need scratch device memory take `workspace`
 * and `workspace_bytes` (>= q3vl_workspace_bytes()). Passing NULL makes the
 * library use its own per-device buffer, grown on demand with hipMalloc
 * (not allowed while the stream is being captured into a HIP graph; capture
 * callers pass their own workspace). A caller's workspace must be 256-byte
 * aligned; its contents need no initialization (every call writes what it
 * reads). Calls sharing one workspace must be ordered on one stream.
 */
#ifndef Q3VL_INT8_H
#define Q3VL_INT8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *q3vl_stream; /* hipStream_t */

enum q3vl_status {
    Q3VL_OK = 0,
    Q3VL_ERR_INVALID_ARGUMENT = 1, /* null / misaligned pointer, bad shape   */
    Q3VL_ERR_UNSUPPORTED = 2,      /* dtype combination or shape not served  */
    Q3VL_ERR_HIP = 3,              /* a HIP runtime call failed              */
    Q3VL_ERR_OUT_OF_MEMORY = 4,    /* workspace or registry allocation failed */
    Q3VL_ERR_STALE_WEIGHT = 5      /* registry entry no longer matches host  */
};

/* DType values of the reference (utils/include/tensor.hpp:38). */
enum q3vl_dtype {
    Q3VL_DTYPE_FP32 = 0,
    Q3VL_DTYPE_INT32 = 1,
    Q3VL_DTYPE_FP16 = 2,
    Q3VL_DTYPE_INT8 = 3,
    Q3VL_DTYPE_INT4 = 4
};

/* Message of this thread's last failing call ("" if none). */
const char *q3vl_last_error(void);
/* ABI version of this header (bumped on any signature or struct layout
 * change; 3: q3vl_text_model.attn_order). */
int q3vl_abi_version(void);
#define Q3VL_ABI_VERSION 3

/* Scratch bytes needed by q3vl_linear_i8* / q3vl_lm_head_argmax for a shape. */
size_t q3vl_workspace_bytes(size_t M, size_t N, size_t K, size_t group_size);

/* Dispatch check of linear() (matmul/src/cpu_wrapper.cpp:320-357): returns
 * Q3VL_OK when (ta, tb, tb_scale, tc, has_bias, group_quantized, B_transpose)
 * is the int8 group-quantized combination this library serves, else
 * Q3VL_ERR_UNSUPPORTED with a message naming the combination. */
int q3vl_check_dtypes(int ta, int tb, int tb_scale, int tc, int has_bias,
                      int group_quantized, int b_transpose);

/* 1 when (M, N, K) takes the reference's M=1 lane-ordered GEMV
 * (cpu_f32a_i8f32sb_f32c_avx2.cpp:464), 0 for the general path. */
int q3vl_uses_lane_path(size_t M, size_t N, size_t K);

/* Activation quantizer (cpu_f32a_i8f32sb_f32c_avx2.cpp:135-177):
 * A [M,K] fp32 -> q [M,K] int16, a_s [M,K/gs] fp32. */
int q3vl_quantize_rows(const float *A, int16_t *q, float *a_s, size_t M,
                       size_t K, size_t group_size, q3vl_stream stream);

/* The int8 branch of linear() (cpu_wrapper.cpp:339-348): C = A W^T. */
int q3vl_linear_i8(const float *A, const int8_t *W, const float *S, float *C,
                   size_t M, size_t N, size_t K, size_t group_size,
                   void *workspace, size_t workspace_bytes, q3vl_stream stream);

/* As q3vl_linear_i8, also writing the exact int32 group accumulators
 * G[(m*N + n)*(K/gs) + g] = sum_{k in g} q[m,k]*W[n,k] (a parity probe; the
 * GEMM variant that writes G is slower). */
int q3vl_linear_i8_groups(const float *A, const int8_t *W, const float *S,
                          float *C, int32_t *G, size_t M, size_t N, size_t K,
                          size_t group_size, void *workspace,
                          size_t workspace_bytes, q3vl_stream stream);

/* Up to three linears over the same activation in one pass (the decode
 * step's q/k/v projections, model/src/forward.cpp:506-528): C[i] = A W[i]^T,
 * each with the numerics linear() gives its own (M, N[i], K). */
int q3vl_linear_i8_multi(const float *A, size_t M, size_t K, size_t group_size,
                         int count, const int8_t *const *W,
                         const float *const *S, float *const *C,
                         const size_t *N, void *workspace,
                         size_t workspace_bytes, q3vl_stream stream);

/* gate and up projections plus swiglu (model/src/forward.cpp:623-642,
 * layers/src/text_layer.cpp:420-434) in one pass:
 * H[m,n] = silu(A Wg^T)[m,n] * (A Wu^T)[m,n], Wg/Wu [N,K]. */
int q3vl_linear_i8_swiglu(const float *A, const int8_t *Wg, const float *Sg,
                          const int8_t *Wu, const float *Su, float *H,
                          size_t M, size_t N, size_t K, size_t group_size,
                          void *workspace, size_t workspace_bytes,
                          q3vl_stream stream);

/* The MLP block of forward_text (model/src/forward.cpp:619-654): the gate
 * and up linear() calls, swiglu (layers/src/text_layer.cpp:420-434) and the
 * down linear() call: Y = (silu(A Wg^T) * (A Wu^T)) Wd^T with A [M,H],
 * Wg/Wu [I,H], Wd [H,I], Y [M,H]; the numerics of those four calls (the down
 * projection quantizes h as the reference's linear() quantizes state->gate).
 * With M > 8, group size 64 and H, I multiples of 512, the gate|up GEMM's
 * epilogue quantizes h straight into the down GEMM's operand (no h in
 * memory, one quantizer launch fewer); otherwise the two calls run through
 * an h buffer in the workspace (>= q3vl_mlp_workspace_bytes()). */
int q3vl_mlp_i8(const float *A, const int8_t *Wg, const float *Sg,
                const int8_t *Wu, const float *Su, const int8_t *Wd,
                const float *Sd, float *Y, size_t M, size_t H, size_t I,
                size_t group_size, void *workspace, size_t workspace_bytes,
                q3vl_stream stream);
size_t q3vl_mlp_workspace_bytes(size_t M, size_t H, size_t I, size_t group_size);

/* lm_head (classifier_gemm, layers/src/text_layer.cpp:302-314) fused with
 * greedy_decode (tokenizer/src/utils.cpp:34-44): ids[m] = first index of the
 * maximum of row m of A W^T (W [V,K]). logits may be NULL (not stored) for
 * M <= 8. */
int q3vl_lm_head_argmax(const float *A, const int8_t *W, const float *S,
                        float *logits, int32_t *ids, size_t M, size_t V,
                        size_t K, size_t group_size, void *workspace,
                        size_t workspace_bytes, q3vl_stream stream);

/* greedy_decode over each row of logits [M, V]. */
int q3vl_argmax_rows(const float *logits, int32_t *ids, size_t M, size_t V,
                     void *workspace, size_t workspace_bytes,
                     q3vl_stream stream);

/* swiglu (layers/src/text_layer.cpp:420-434): gate = silu(gate) * up. */
int q3vl_swiglu(float *gate, const float *up, size_t n, q3vl_stream stream);

/* ---- the decode step that calls the int8 path (model/src/forward.cpp:
 * 458-720): one text token through every layer and the tied lm_head, on an
 * int8 group-quantized model held in device memory. Per-layer tensors are
 * stacked [layers, ...] and contiguous. The KV caches are fp16
 * [layers, kv_heads, max_seq, head_dim]. `token` and `pos` live in device
 * memory: the call reads the token at position *pos, writes the greedy next
 * token into *token and increments *pos, so a captured HIP graph of one call
 * can be replayed step after step. A *pos outside [0, max_seq) leaves the
 * caches untouched and makes the attention outputs (so the logits) NaN, as
 * a token outside [0, vocab) does. head_dim must be 128; every linear must
 * take the M=1 lane-ordered GEMV (dimensions >= 1024, <= 8192). */
typedef struct q3vl_text_model {
    int vocab, hidden, intermediate, layers, heads, kv_heads, head_dim, max_seq, group_size;
    float rms_eps;
    const int8_t *embed_w;      const float *embed_s;      /* [vocab, hidden], tied lm_head */
    const int8_t *final_norm_w; const float *final_norm_s; /* [hidden] */
    const int8_t *attn_norm_w;  const float *attn_norm_s;  /* [layers, hidden] pre-attention */
    const int8_t *mlp_norm_w;   const float *mlp_norm_s;   /* [layers, hidden] pre-MLP */
    const int8_t *q_norm_w;     const float *q_norm_s;     /* [layers, head_dim] */
    const int8_t *k_norm_w;     const float *k_norm_s;     /* [layers, head_dim] */
    const int8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;        /* [layers, N, K] */
    const float *sq, *sk, *sv, *so, *sg, *su, *sd;         /* [layers, N, K/gs] */
    const float *rope_cos, *rope_sin;                      /* [max_seq, head_dim/2] */
    /* Order of the attention's softmax and value sum. Q3VL_ATTN_REFERENCE
     * (0, what a zero-initialized struct holds): the reference's
     * (text_layer.cpp:436-535, 655-710) -- one max, sum and value chain over
     * all positions. Q3VL_ATTN_CHUNKED (1): no counterpart in the reference;
     * per 64-position chunk a max, a sum and a value chain, folded chunk by
     * chunk. It differs from the reference order by the error of the
     * reference's exp256 polynomial (up to a few 1e-4 of the output scale;
     * each order is that far from an exact softmax), and the test oracle
     * restates it exactly. It zeroes a head exactly where the reference
     * does (some score's exp256(s - M) is -inf): each chunk keeps its
     * smallest finite score for that check. */
    int attn_order;
} q3vl_text_model;

#define Q3VL_ATTN_REFERENCE 0
#define Q3VL_ATTN_CHUNKED 1

/* Scratch bytes q3vl_decode_step needs for a model. */
size_t q3vl_decode_workspace_bytes(const q3vl_text_model *m);

/* One decode step; logits [vocab] are stored when non-NULL. No allocation
 * when `workspace` is given. */
int q3vl_decode_step(const q3vl_text_model *m, uint16_t *k_cache, uint16_t *v_cache,
                     int32_t *token, int32_t *pos, float *logits, void *workspace,
                     size_t workspace_bytes, q3vl_stream stream);

/* q3vl_decode_step without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Its scratch is a static device array of
 * q3vl_decode_static_scratch_bytes() (1 MiB) per device, held until the
 * process ends; the first call on a device looks up that device's copy. A
 * model whose decode scratch (q3vl_decode_workspace_bytes) exceeds it is
 * refused with Q3VL_ERR_UNSUPPORTED before any device work. Every call on a
 * device shares the one array, so calls that overlap on one device (other
 * streams, other threads) race; the scratch holds no state between calls.
 * Same kernels and results as q3vl_decode_step. */
int q3vl_decode_step_static(const q3vl_text_model *m, uint16_t *k_cache, uint16_t *v_cache,
                            int32_t *token, int32_t *pos, float *logits, q3vl_stream stream);
size_t q3vl_decode_static_scratch_bytes(void);

/* ---- checkpoint files: the reference's single-file .bin
 * (model/src/load_model.cpp:50-246, written by
 * export_bin/export_qwen_bin.py:212-420). A 100-byte header
 * (q3vl_checkpoint_header, little-endian int32 / float32), then tensor
 * groups in a fixed order. An int8 group stores all of its fp32 scales, then
 * all of its int8 values; an fp16 / fp32 group stores its values. The text
 * groups, in file order (q3vl_checkpoint_tensor): embed_tokens [vocab,
 * hidden]; input_layernorm [layers, hidden] (applied before attention: the
 * reference's rms_ffn_w, forward.cpp:494); mlp down [layers, hidden, inter];
 * gate, up [layers, inter, hidden]; post_attention_layernorm [layers,
 * hidden] (before the MLP: rms_attn_w, forward.cpp:612); k_norm [layers,
 * head_dim]; k [layers, kv_heads*head_dim, hidden]; o [layers, hidden,
 * hidden]; q_norm; q [layers, heads*head_dim, hidden]; v; the final norm
 * [hidden]. The vision groups follow. Norm tensors are group-quantized
 * always; the other int8 tensors when group_quantized != 0, else with one
 * scale per row. */
typedef struct q3vl_checkpoint_header {
    int vocab, hidden, intermediate, layers, heads, kv_heads, max_position, rope_theta;
    float rms_eps;
    int vision_hidden, vision_depth, vision_patch, vision_spatial_merge, vision_temporal_patch,
        vision_heads, vision_intermediate, out_hidden;
    int image_token_id, vision_start_token_id, vision_end_token_id, video_token_id;
    int text_bits, group_size, vision_bits, group_quantized;
} q3vl_checkpoint_header; /* the file's first 100 bytes */

enum q3vl_checkpoint_tensor {
    Q3VL_CK_EMBED = 0, Q3VL_CK_ATTN_NORM, Q3VL_CK_DOWN, Q3VL_CK_GATE, Q3VL_CK_UP,
    Q3VL_CK_MLP_NORM, Q3VL_CK_K_NORM, Q3VL_CK_K, Q3VL_CK_O, Q3VL_CK_Q_NORM, Q3VL_CK_Q,
    Q3VL_CK_V, Q3VL_CK_FINAL_NORM, Q3VL_CK_TEXT_TENSORS
};

/* One tensor group's place in the file. */
typedef struct q3vl_checkpoint_span {
    size_t scales_offset; /* byte offset of the fp32 scales (int8 groups) */
    size_t scales_count;  /* number of scales (0 for fp16 / fp32 groups) */
    size_t data_offset;   /* byte offset of the values */
    size_t data_count;    /* number of values */
    int bits;             /* 8, 16 or 32 */
    int group;            /* values per scale (int8 groups) */
} q3vl_checkpoint_span;

/* The header of a checkpoint file (the field reads of load_model.cpp:62-91).
 * Host only. Q3VL_ERR_INVALID_ARGUMENT for a missing or short file. */
int q3vl_checkpoint_read_header(const char *path, q3vl_checkpoint_header *hdr);

/* The text groups' places, spans[Q3VL_CK_TEXT_TENSORS], as map_tensor walks
 * the file (load_model.cpp:146-195). Host only. */
int q3vl_checkpoint_text_layout(const q3vl_checkpoint_header *hdr, q3vl_checkpoint_span *spans);

/* RoPE tables for text positions 0..rows-1 (the T section of
 * qwen_rope_precompute, load_model.cpp:416-490; a text position has its
 * three sections equal): cos[p][i] = cosf(p * inv_freq[i]),
 * inv_freq[i] = 1.0f / powf(theta, (2.0f * i) / head_dim), fp32 with the
 * host's libm. Host only; cos_out and sin_out hold rows * head_dim/2. */
int q3vl_rope_tables(int rope_theta, int head_dim, int rows, float *cos_out, float *sin_out);

/* A checkpoint's text model in device memory on the current device: one
 * allocation, every tensor 256-byte aligned, and RoPE tables for max_seq
 * positions (the device-resident counterpart of init_model_weights and the
 * run state's tables, load_model.cpp:50-195 and :413-490). Needs int8 text
 * weights, group-quantized with a group size the decode step serves, and
 * head_dim 128; Q3VL_ERR_UNSUPPORTED names what does not fit. The copies are
 * complete when the call returns. */
typedef struct q3vl_checkpoint q3vl_checkpoint;
int q3vl_checkpoint_load(const char *path, int max_seq, q3vl_stream stream,
                         q3vl_checkpoint **out);
/* The loaded model (valid until q3vl_checkpoint_free). */
const q3vl_text_model *q3vl_checkpoint_text_model(const q3vl_checkpoint *ck);
int q3vl_checkpoint_header_of(const q3vl_checkpoint *ck, q3vl_checkpoint_header *hdr);
void q3vl_checkpoint_free(q3vl_checkpoint *ck);

/* The exporter's weight quantizer on the device (quantize_groupwise,
 * export_bin/export_qwen_bin.py:260-275): per group of `group` consecutive
 * values, m = max|x| + 1e-8, s = m / 127 (fp32), q = round half to even of
 * x / s, clipped to [-127, 127]; scales[i] = s of group i. quantize_rowwise
 * (:242-258) is the case group = row length. count must be a multiple of
 * group; x must be finite. Device pointers, asynchronous on `stream`. */
int q3vl_quantize_groupwise(const float *x, size_t count, size_t group, int8_t *q,
                            float *scales, q3vl_stream stream);

/* ---- weight registry for host-pointer callers (the drop-in linear()).
 * The reference hands linear() mmapped host pointers to weights and scales
 * (model/src/load_model.cpp:146-181); the registry uploads a weight once and
 * maps its host address to device copies (256-byte aligned).
 *
 * An entry is identified by host_W together with host_S, N, K, group_size
 * and a fingerprint of the host bytes (64-bit hash over the first and last
 * 256 bytes of W, 16 strided 64-byte samples of it, and the first and last
 * 64 bytes of S). q3vl_weight_register returns the existing copies when all
 * of these match; when host_W is registered with anything else (the engine
 * unmapped one model and mapped another at the same address, or passes
 * another shape) it frees the old copies and uploads the new weight. The
 * fingerprint is a sampled check: a caller that replaces weights in place
 * releases them (q3vl_weight_release) before the next call. */
int q3vl_weight_register(const int8_t *host_W, const float *host_S, size_t N,
                         size_t K, size_t group_size, const int8_t **dev_W,
                         const float **dev_S);
/* Device copies of a registered host weight. Q3VL_OK only if host_W is
 * registered with the same host_S, N, K, group_size and fingerprint;
 * Q3VL_ERR_INVALID_ARGUMENT if host_W is not registered;
 * Q3VL_ERR_STALE_WEIGHT if it is registered with any of them different (the
 * caller re-registers; nothing is returned). */
int q3vl_weight_lookup(const void *host_W, const float *host_S, size_t N, size_t K,
                       size_t group_size, const int8_t **dev_W, const float **dev_S);
int q3vl_weight_release(const void *host_W);
int q3vl_weight_release_all(void);

#ifdef __cplusplus
}
#endif

#endif /* Q3VL_INT8_H */
