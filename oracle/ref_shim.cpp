// ref_shim.cpp -- C entry points over the reference's own sources, compiled
// from /root/reference by oracle/Makefile into oracle/_ref/ (never committed).
//
// TEST INFRASTRUCTURE ONLY. It lets tests and the golden-vector writer call the
// reference's real linear() (matmul/src/cpu_wrapper.cpp:308), its text-layer
// ops (layers/src/text_layer.cpp) and its decode step forward_text()
// (model/src/forward.cpp:458), its checkpoint loader init_model_weights()
// (model/src/load_model.cpp:50) and RoPE tables qwen_rope_precompute()
// (model/src/load_model.cpp:413), and lets bench.py time the reference CPU path.
// Nothing here is linked into the HIP library.
#include <fcntl.h>
#include <unistd.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "layers/include/text_layer.hpp"
#include "matmul/module.hpp"
#include "model/include/forward.hpp"
#include "model/include/load_model.hpp"

namespace {

// The reference's Tensor constructors print to stdout; keep stdout clean for
// callers that print machine-readable output.
struct Silence {
    int saved = -1;
    Silence() {
        fflush(stdout);
        saved = dup(1);
        int devnull = open("/dev/null", O_WRONLY);
        if (devnull >= 0) {
            dup2(devnull, 1);
            close(devnull);
        }
    }
    ~Silence() {
        fflush(stdout);
        if (saved >= 0) {
            dup2(saved, 1);
            close(saved);
        }
    }
};

// Tensor's destructor unmaps buffers it does not own (utils/src/tensor.cpp:
// 83-101), so wrappers over caller memory drop their pointers first.
void release(Tensor *t) {
    if (!t) return;
    t->buf = nullptr;
    t->scale_buf = nullptr;
    delete t;
}

Tensor *f32(std::vector<size_t> shape, void *buf) { return new Tensor(shape, buf, DType::FP32); }

Tensor *i8(std::vector<size_t> shape, const void *w, const void *s, size_t gs) {
    return new Tensor(shape, const_cast<void *>(w), const_cast<void *>(s), gs, true, DType::INT8,
                      DType::FP32);
}

}  // namespace

extern "C" {

// The int8 group-quantized branch of linear(): FP32 A, INT8 B [N,K]
// (mat_B_transpose=true), FP32 group scales, FP32 C, no bias.
void ref_linear_i8(const float *A, const int8_t *W, const float *S, float *C, size_t M, size_t N,
                   size_t K, size_t gs) {
    linear(A, W, S, nullptr, nullptr, C, M, N, K, true, DType::FP32, DType::INT8, DType::FP32,
           DType::FP32, true, gs);
}

void ref_swiglu(float *gate, const float *up, size_t n) {
    Silence quiet;
    Tensor *g = f32({n}, gate), *u = f32({n}, const_cast<float *>(up));
    swiglu(g, u, n);
    release(g);
    release(u);
}

// rms_norm (text_layer.cpp:52), int8 group-quantized weight, one row.
void ref_rms_norm_i8(const float *x, const int8_t *w, const float *ws, size_t n, size_t gs,
                     float eps, float *out) {
    Silence quiet;
    Tensor *tx = f32({1, n}, const_cast<float *>(x)), *to = f32({1, n}, out);
    Tensor *tw = i8({n}, w, ws, gs);
    rms_norm(tx, tw, to, eps, 1, 0);
    release(tx), release(to), release(tw);
}

// rms_norm_inplace (text_layer.cpp:177), int8 group weight, `batches` rows.
void ref_rms_norm_inplace_i8(float *x, const int8_t *w, const float *ws, size_t n, size_t gs,
                             float eps, size_t batches) {
    Silence quiet;
    Tensor *tx = f32({batches, n}, x);
    Tensor *tw = i8({n}, w, ws, gs);
    rms_norm_inplace(tx, tw, eps, batches, 0);
    release(tx), release(tw);
}

// apply_rotary (text_layer.cpp:712): cos/sin tables [S, hd/2], row `pos`.
void ref_rope(float *x, const float *cos_t, const float *sin_t, size_t S, int heads, int hd,
              int pos) {
    Silence quiet;
    Tensor *tx = f32({(size_t)heads * hd}, x);
    Tensor *tc = f32({S, (size_t)hd / 2}, const_cast<float *>(cos_t));
    Tensor *ts = f32({S, (size_t)hd / 2}, const_cast<float *>(sin_t));
    apply_rotary(tx, tc, ts, heads, hd, pos);
    release(tx), release(tc), release(ts);
}

void ref_softmax(float *x, size_t n) { softmax(x, n); }

// attn_scores_all_heads + attn_weighted_sum_all_heads (text_layer.cpp:575,
// 655) for one layer: caches fp32 [kv_heads][S][hd], q [heads][hd].
void ref_attention(const float *q, const float *kc, const float *vc, int heads, int kv_heads,
                   int hd, size_t S, int pos, float *out) {
    Silence quiet;
    Tensor *tq = f32({1, (size_t)heads, (size_t)hd}, const_cast<float *>(q));
    std::vector<float> att((size_t)heads * S);
    Tensor *ta = f32({1, (size_t)heads, S}, att.data());
    Tensor *to = f32({1, (size_t)heads * hd}, out);
    attn_scores_all_heads(kc, tq, ta, heads, heads / kv_heads, hd, kv_heads * hd, S * hd, pos);
    attn_weighted_sum_all_heads(vc, ta, to, heads, heads / kv_heads, hd, kv_heads * hd, S * hd,
                                pos);
    release(tq), release(ta), release(to);
}

// Synthetic int8 text model for forward_text (model/src/forward.cpp:458).
// Field meaning as orc_model (oracle/oracle.h); the caller owns every buffer.
struct ref_model_desc {
    int vocab, hidden, inter, layers, heads, kv_heads, head_dim, max_seq, gs;
    float eps;
    const int8_t *emb_w;   const float *emb_s;
    const int8_t *fnorm_w; const float *fnorm_s;
    const int8_t *anorm_w; const float *anorm_s;
    const int8_t *mnorm_w; const float *mnorm_s;
    const int8_t *qnorm_w; const float *qnorm_s;
    const int8_t *knorm_w; const float *knorm_s;
    const int8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    const float *sq, *sk, *sv, *so, *sg, *su, *sd;
    const float *rope_cos, *rope_sin;
};

struct RefDecoder {
    QwenConfig cfg{};
    QwenWeight w{};
    QwenRunState st{};
    std::vector<float> x, t, q, k, v, att, qkv, gate, up, cosb, sinb, logits;
    std::vector<Tensor *> owned;
};

// Builds the reference's model/run-state structs over the caller's weights
// and fp32 KV caches [L][kv_heads][max_seq][head_dim].
void *ref_decoder_create(const ref_model_desc *d, float *k_cache, float *v_cache) {
    Silence quiet;
    auto *r = new RefDecoder();
    const size_t V = d->vocab, H = d->hidden, I = d->inter, L = d->layers, NH = d->heads,
                 NKV = d->kv_heads, D = d->head_dim, S = d->max_seq, gs = d->gs;
    QwenConfig &c = r->cfg;
    c.seq_len = (int)S;
    c.vocab_size = (int)V;
    c.hidden_size = (int)H;
    c.intermediate_size = (int)I;
    c.num_hidden_layers = (int)L;
    c.num_attention_heads = (int)NH;
    c.num_key_value_heads = (int)NKV;
    c.rms_norm_eps = d->eps;
    c.image_token_id = -100;
    c.video_token_id = -100;
    c.vision_deep_stack_depth = 3;
    c.group_quantized = 1;
    c.group_size = (int)gs;
    c.text_bits = 8;
    auto keep = [&](Tensor *t) {
        r->owned.push_back(t);
        return t;
    };
    QwenWeight &w = r->w;
    w.token_embedding_table = keep(i8({V, H}, d->emb_w, d->emb_s, gs));
    w.rms_out_w = keep(i8({H}, d->fnorm_w, d->fnorm_s, gs));
    // forward_text normalizes with rms_ffn_w before attention (:493) and with
    // rms_attn_w before the MLP (:611)
    w.rms_ffn_w = keep(i8({L, H}, d->anorm_w, d->anorm_s, gs));
    w.rms_attn_w = keep(i8({L, H}, d->mnorm_w, d->mnorm_s, gs));
    w.w_attn_q_norm = keep(i8({L, D}, d->qnorm_w, d->qnorm_s, gs));
    w.w_attn_k_norm = keep(i8({L, D}, d->knorm_w, d->knorm_s, gs));
    w.w_attn_q = keep(i8({L, NH * D, H}, d->wq, d->sq, gs));
    w.w_attn_k = keep(i8({L, NKV * D, H}, d->wk, d->sk, gs));
    w.w_attn_v = keep(i8({L, NKV * D, H}, d->wv, d->sv, gs));
    w.w_attn_o = keep(i8({L, H, NH * D}, d->wo, d->so, gs));
    w.w_mlp_gate = keep(i8({L, I, H}, d->wg, d->sg, gs));
    w.w_mlp_up = keep(i8({L, I, H}, d->wu, d->su, gs));
    w.w_mlp_down = keep(i8({L, H, I}, d->wd, d->sd, gs));
    r->x.assign(H, 0.f);
    r->t.assign(H, 0.f);
    r->q.assign(NH * D, 0.f);
    r->k.assign(NH * D, 0.f);
    r->v.assign(NH * D, 0.f);
    r->att.assign(NH * S, 0.f);
    r->qkv.assign(H, 0.f);
    r->gate.assign(I, 0.f);
    r->up.assign(I, 0.f);
    r->logits.assign(V, 0.f);
    r->cosb.assign(3 * S * (D / 2), 0.f);
    r->sinb.assign(3 * S * (D / 2), 0.f);
    for (int p = 0; p < 3; ++p) {  // text positions read plane 0 only
        memcpy(&r->cosb[p * S * (D / 2)], d->rope_cos, S * (D / 2) * 4);
        memcpy(&r->sinb[p * S * (D / 2)], d->rope_sin, S * (D / 2) * 4);
    }
    QwenRunState &s = r->st;
    s.x = keep(f32({1, H}, r->x.data()));
    s.t = keep(f32({1, H}, r->t.data()));
    s.q = keep(f32({1, NH, D}, r->q.data()));
    s.k = keep(f32({1, NH, D}, r->k.data()));
    s.v = keep(f32({1, NH, D}, r->v.data()));
    s.att = keep(f32({1, NH, S}, r->att.data()));
    s.qkv_out = keep(f32({1, H}, r->qkv.data()));
    s.gate = keep(f32({1, I}, r->gate.data()));
    s.up = keep(f32({1, I}, r->up.data()));
    s.cos_tensor = keep(f32({3, S, D / 2}, r->cosb.data()));
    s.sin_tensor = keep(f32({3, S, D / 2}, r->sinb.data()));
    s.logits = keep(f32({1, V}, r->logits.data()));
    s.key_cache = keep(f32({1, L, NKV, S, D}, k_cache));
    s.value_cache = keep(f32({1, L, NKV, S, D}, v_cache));
    return r;
}

// forward_text for a text token at pos; logits [vocab] copied out. Returns 0,
// or -1 without calling forward_text when pos is outside the caches
// (pos >= max_seq) or the token outside the vocabulary: forward_text checks
// neither and would write the K/V cache rows at pos and att[h * S + t] past
// the buffers (model/src/forward.cpp:550-584).
int ref_decoder_step(void *h, int token, size_t pos, float *logits) {
    auto *r = static_cast<RefDecoder *>(h);
    if (pos >= (size_t)r->cfg.seq_len || token < 0 || token >= r->cfg.vocab_size) return -1;
    Silence quiet;
    const float *out = forward_text(&r->cfg, &r->st, &r->w, token, pos);
    memcpy(logits, out, r->logits.size() * 4);
    return 0;
}

void ref_decoder_destroy(void *h) {
    auto *r = static_cast<RefDecoder *>(h);
    for (Tensor *t : r->owned) release(t);
    delete r;
}

// ---- checkpoint loader (model/src/load_model.cpp:50-246)
struct ref_ck_tensor {
    const void *data;    // mapped values
    const void *scales;  // mapped fp32 scales (int8 tensors), else null
    size_t count;        // values
    size_t group;        // values per scale (int8 tensors)
    int dtype;           // DType::Type
};

struct RefCheckpoint {
    QwenConfig cfg{};
    QwenWeight w{};
};

// Maps a checkpoint with init_model_weights. cfg25 receives the 25 header
// fields in file order (rms_norm_eps as its float bits); out receives the 13
// text tensors in file order, then the 27 vision tensors in file order.
// Returns null when the loader mapped nothing.
void *ref_checkpoint_open(const char *path, int *cfg25, ref_ck_tensor *out) {
    Silence quiet;
    auto *r = new RefCheckpoint();
    init_model_weights(path, &r->cfg, &r->w);
    if (!r->w.rms_out_w) {
        delete r;
        return nullptr;
    }
    const QwenConfig &c = r->cfg;
    int eps_bits;
    memcpy(&eps_bits, &c.rms_norm_eps, 4);
    const int f[25] = {c.vocab_size, c.hidden_size, c.intermediate_size, c.num_hidden_layers,
                       c.num_attention_heads, c.num_key_value_heads, c.max_position_embeddings,
                       c.rope_theta, eps_bits, c.vision_hidden_size, c.vision_depth,
                       c.vision_patch_size, c.vision_spatial_merge_size,
                       c.vision_temporal_patch_size, c.vision_num_heads,
                       c.vision_intermediate_size, c.out_hidden_size, c.image_token_id,
                       c.vision_start_token_id, c.vision_end_token_id, c.video_token_id,
                       c.text_bits, c.group_size, c.vision_bits, c.group_quantized};
    memcpy(cfg25, f, sizeof f);
    const QwenWeight &w = r->w;
    const Tensor *ts[] = {
        w.token_embedding_table, w.rms_ffn_w, w.w_mlp_down, w.w_mlp_gate, w.w_mlp_up,
        w.rms_attn_w, w.w_attn_k_norm, w.w_attn_k, w.w_attn_o, w.w_attn_q_norm, w.w_attn_q,
        w.w_attn_v, w.rms_out_w,
        w.vl_patch_emb_b, w.vl_patch_emb_w, w.vl_pos_emb_w, w.vl_attn_proj_b, w.vl_attn_proj_w,
        w.vl_attn_qkv_b, w.vl_attn_qkv_w, w.vl_mlp1_b, w.vl_mlp1_w, w.vl_mlp2_b, w.vl_mlp2_w,
        w.vl_norm1_b, w.vl_norm1_w, w.vl_norm2_b, w.vl_norm2_w,
        w.vl_d_mlp1_b, w.vl_d_mlp1_w, w.vl_d_mlp2_b, w.vl_d_mlp2_w, w.vl_d_norm_b, w.vl_d_norm_w,
        w.vl_merge_mlp1_b, w.vl_merge_mlp1_w, w.vl_merge_mlp2_b, w.vl_merge_mlp2_w,
        w.vl_merge_norm_b, w.vl_merge_norm_w};
    for (size_t i = 0; i < sizeof ts / sizeof ts[0]; ++i) {
        const Tensor *t = ts[i];
        out[i].data = t->buf;
        out[i].scales = t->scale_buf;
        out[i].count = t->num_elem();
        out[i].group = t->group_size;
        out[i].dtype = (int)t->dtype;
    }
    return r;
}

void ref_checkpoint_close(void *h) {
    auto *r = static_cast<RefCheckpoint *>(h);
    free_model_weights(&r->w);
    free_model_config(&r->cfg);
    delete r;
}

// qwen_rope_precompute over caller buffers cos3/sin3 [3][seq_len][head_dim/2].
void ref_rope_precompute(int rope_theta, int hidden, int heads, int seq_len, float *cos3,
                         float *sin3) {
    Silence quiet;
    QwenConfig c{};
    int sections[3] = {24, 20, 20};  // load_model.cpp:96-98
    c.seq_len = seq_len;
    c.hidden_size = hidden;
    c.num_attention_heads = heads;
    c.rope_theta = rope_theta;
    c.mrope_section = sections;
    c.num_dimensions = 3;
    const size_t half = (size_t)(hidden / heads) / 2;
    Tensor *tc = f32({3, (size_t)seq_len, half}, cos3);
    Tensor *tsn = f32({3, (size_t)seq_len, half}, sin3);
    qwen_rope_precompute(tc, tsn, &c);
    release(tc);
    release(tsn);
}

}  // extern "C"
