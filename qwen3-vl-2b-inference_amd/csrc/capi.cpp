// capi.cpp -- extern "C" entry points of libq3vl_int8.so (include/q3vl_int8.h).
//
// Validates arguments, turns the reference's fprintf+exit(1) failure modes
// into status codes, manages scratch memory and the host-weight registry, and
// dispatches to the gfx950 kernels exactly as the reference's shape dispatch
// (matmul/src/cpu_f32a_i8f32sb_f32c_avx2.cpp:464-475) selects its numerics.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <atomic>
#include <fcntl.h>
#include <mutex>
#include <string>
#include <thread>
#include <unistd.h>
#include <unordered_map>
#include <vector>

#include "q3vl_int8.h"
#include "q3vl_kernels.hpp"

using namespace q3vl;

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(Q3VL_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define Q3VL_HIP(call, what)                          \
    do {                                              \
        hipError_t e_ = (call);                       \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

constexpr size_t kMaxGemvParts = 8192;  // >= grid of any GEMV launch
constexpr int kGemmArgmaxParts = 64;    // argmax partials per row after a GEMM

bool gs_ok_gemv(size_t gs) { return gs == 16 || gs == 32 || gs == 64 || gs == 128 || gs == 256; }
bool gs_ok_gemm(size_t gs) { return gs == 32 || gs == 64 || gs == 128; }

// ---- workspace layout
struct WsLayout {
    size_t parts_val = 0, parts_idx = 0;  // argmax partials
    size_t aq = 0, as = 0;                // GEMM: fp16 activations, transposed scales
    size_t logits = 0;                    // lm_head M > 8 without caller logits
    size_t total = 0;
    int lda_s = 0;
};

WsLayout layout(size_t M, size_t N, size_t K, size_t gs) {
    WsLayout L;
    size_t off = 0;
    const size_t mm = M ? M : 1;
    L.parts_val = off;
    off += align256(kMaxGemvParts * mm * sizeof(float));
    L.parts_idx = off;
    off += align256(kMaxGemvParts * mm * sizeof(int32_t));
    if (M > 8) {
        // rows padded to whole 32-row m-tiles (the fragment-order layout of
        // the group-64 GEMM; the transposed scales of the others use the same
        // stride)
        const size_t Kg = gs ? K / gs : 0;
        const size_t Mpad = (M + 31) & ~(size_t)31;
        L.lda_s = (int)Mpad;
        L.aq = off;
        off += align256(Mpad * K * 2);
        L.as = off;
        off += align256(Kg * Mpad * 4);
        L.logits = off;
        off += align256(M * N * 4);
    }
    L.total = off;
    return L;
}

// ---- library-owned default workspace (per device, grow-only)
struct DefaultWs {
    std::mutex mu;
    std::vector<void *> buf;
    std::vector<size_t> size;
};
DefaultWs g_ws;

int resolve_ws(void *user, size_t user_bytes, size_t need, char **out) {
    if (user) {
        if (user_bytes < need)
            return fail(Q3VL_ERR_INVALID_ARGUMENT,
                        "workspace too small: %zu bytes given, %zu needed", user_bytes, need);
        if (((uintptr_t)user & 255u) != 0)
            return fail(Q3VL_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
        *out = static_cast<char *>(user);
        return Q3VL_OK;
    }
    int dev = 0;
    Q3VL_HIP(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_ws.mu);
    if ((size_t)dev >= g_ws.buf.size()) {
        g_ws.buf.resize(dev + 1, nullptr);
        g_ws.size.resize(dev + 1, 0);
    }
    if (g_ws.size[dev] < need) {
        if (g_ws.buf[dev]) {
            // Work queued on any stream may still read the old buffer.
            Q3VL_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
            Q3VL_HIP(hipFree(g_ws.buf[dev]), "hipFree(workspace)");
            g_ws.buf[dev] = nullptr;
            g_ws.size[dev] = 0;
        }
        size_t sz = need < (1u << 20) ? (1u << 20) : need;
        void *p = nullptr;
        if (hipMalloc(&p, sz) != hipSuccess)
            return fail(Q3VL_ERR_OUT_OF_MEMORY, "workspace hipMalloc(%zu) failed", sz);
        g_ws.buf[dev] = p;
        g_ws.size[dev] = sz;
    }
    *out = static_cast<char *>(g_ws.buf[dev]);
    return Q3VL_OK;
}

// Compute units of the current device (cached per device).
int device_cus(int *cus) {
    static std::atomic<int> cache[64];
    int dev = 0;
    Q3VL_HIP(hipGetDevice(&dev), "hipGetDevice");
    if (dev >= 0 && dev < 64) {
        const int c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0) {
            *cus = c;
            return Q3VL_OK;
        }
    }
    int c = 0;
    Q3VL_HIP(hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev), "CU count");
    if (c < 1) c = 1;
    if (dev >= 0 && dev < 64) cache[dev].store(c, std::memory_order_relaxed);
    *cus = c;
    return Q3VL_OK;
}

int check_common(const void *A, const void *W, const void *S, size_t M, size_t N,
                 size_t K, size_t gs) {
    if (gs == 0 || K % gs != 0)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "K=%zu must be a multiple of group_size=%zu", K, gs);
    if (M && N && K && (!A || !W || !S))
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "null A/W/S pointer");
    if ((A && !aligned16(A)) || (W && !aligned16(W)))
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "A and W must be 16-byte aligned");
    if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff || N * K > 0x7fffffffULL ||
        M * K > 0x7fffffffULL)
        return fail(Q3VL_ERR_UNSUPPORTED, "shape too large (M=%zu N=%zu K=%zu)", M, N, K);
    return Q3VL_OK;
}

bool gemv_path_ok(size_t M, size_t K, size_t gs) {
    return M <= 8 && K % 16 == 0 && K / 16 <= 512 && gs_ok_gemv(gs);
}

// Shared-activation runner: segments ride one GEMV launch (M <= 8) or one
// quantization followed by one GEMM per segment (M > 8).
int run_linear(const float *A, int nseg, const int8_t *const *W, const float *const *S,
               float *const *C, int32_t *const *G, const size_t *Ns, size_t M, size_t K,
               size_t gs, int mode, void *ws, size_t wsb, hipStream_t st, int32_t *ids) {
    size_t Nmax = 0;
    for (int i = 0; i < nseg; ++i) {
        int rc = check_common(A, W[i], S[i], M, Ns[i], K, gs);
        if (rc) return rc;
        if (Ns[i] > Nmax) Nmax = Ns[i];
    }
    if (M == 0 || Nmax == 0) return Q3VL_OK;
    if (K == 0) {  // the reference's general path leaves C = 0 (and argmax 0)
        for (int i = 0; i < nseg; ++i)
            if (C[i]) Q3VL_HIP(launch_zero_words(C[i], M * Ns[i], st), "zero fill (C)");
        if (ids) Q3VL_HIP(launch_zero_words(ids, M, st), "zero fill (ids)");
        return Q3VL_OK;
    }
    const WsLayout L = layout(M, Nmax, K, gs);
    char *wbase = nullptr;
    int rc = resolve_ws(ws, wsb, L.total, &wbase);
    if (rc) return rc;

    // 5..8 rows against a very wide weight (the lm_head over a batch of
    // rows): the MFMA kernels below (16-row tiles, see wide16) stream the
    // weights faster than the general GEMV's integer dot products.
    bool wide_mf = M >= 5 && M <= 8 && gs == 64 && mode != GEMV_SWIGLU;
    for (int i = 0; wide_mf && i < nseg; ++i)
        wide_mf = !(G && G[i]) && (size_t)Ns[i] * K >= ((size_t)1 << 26) &&
                  (size_t)Ns[i] * K <= 0x7fffffffULL;
    if (wide_mf) {
        int cus = 0;
        rc = device_cus(&cus);
        if (rc) return rc;
        for (int i = 0; wide_mf && i < nseg; ++i)
            wide_mf = gemm_mf_serves((int)M, (int)Ns[i], (int)K, false, cus);
    }
    if (gemv_path_ok(M, K, gs) && !wide_mf) {
        // Lane numerics apply per segment shape; segments sharing one launch
        // must agree on the path.
        const bool lanes = q3vl_uses_lane_path(M, Ns[0], K);
        for (int i = 1; i < nseg; ++i)
            if (q3vl_uses_lane_path(M, Ns[i], K) != (int)lanes) {
                for (int j = 0; j < nseg; ++j) {
                    rc = run_linear(A, 1, &W[j], &S[j], &C[j], &G[j], &Ns[j], M, K, gs,
                                    GEMV_PLAIN, ws, wsb, st, nullptr);
                    if (rc) return rc;
                }
                return Q3VL_OK;
            }
        if (lanes && K < 1024) return fail(Q3VL_ERR_INVALID_ARGUMENT, "internal: lane path K");
        GemvArgs a{};
        a.A = A;
        a.nseg = nseg;
        for (int i = 0; i < nseg; ++i) a.seg[i] = {W[i], S[i], C[i], G ? G[i] : nullptr, (int)Ns[i]};
        a.M = (int)M;
        a.K = (int)K;
        a.gs = (int)gs;
        a.mode = mode;
        a.part_val = reinterpret_cast<float *>(wbase + L.parts_val);
        a.part_idx = reinterpret_cast<int32_t *>(wbase + L.parts_idx);
        int grid = 0;
        Q3VL_HIP(launch_gemv(a, lanes, &grid, st), "gemv launch");
        if (mode == GEMV_ARGMAX)
            Q3VL_HIP(launch_argmax_final(a.part_val, a.part_idx, grid, (int)M, ids, st),
                     "argmax final launch");
        return Q3VL_OK;
    }

    if (M <= 8 && q3vl_uses_lane_path(M, Nmax, K))
        return fail(Q3VL_ERR_UNSUPPORTED,
                    "M=1 lane-ordered GEMV needs K <= 8192 (K=%zu, group_size=%zu)", K, gs);
    if (!gs_ok_gemm(gs) || K % 64 != 0)
        return fail(Q3VL_ERR_UNSUPPORTED,
                    "GEMM path needs group_size in {32,64,128} and K %% 64 == 0 "
                    "(M=%zu K=%zu group_size=%zu)", M, K, gs);
    // M > 8 (or an M <= 8 shape the GEMV kernels do not take or that runs
    // faster on the GEMM): quantize once.
    const WsLayout LG = layout(M > 8 ? M : 9, Nmax, K, gs);
    if (LG.total > L.total) {
        rc = resolve_ws(ws, wsb, LG.total, &wbase);
        if (rc) return rc;
    }
    _Float16 *aq = reinterpret_cast<_Float16 *>(wbase + LG.aq);
    float *asT = reinterpret_cast<float *>(wbase + LG.as);
    // Group size 64 without group sums: the fragment-order GEMM where it
    // serves every segment's shape (it addresses its buffers with 32-bit byte
    // offsets), with the activations quantized into MFMA fragment order; one
    // GEMM per segment, gate and up together under SwiGLU.
    bool use_mf = gs == 64 && ((M + 31) & ~(size_t)31) * K * 2 <= 0x7fffffffULL &&
                  (size_t)Ns[0] * K <= 0x7fffffffULL;
    int cus = 0;
    if (use_mf) {
        rc = device_cus(&cus);
        if (rc) return rc;
    }
    for (int i = 0; use_mf && i < nseg; ++i)
        use_mf = !(G && G[i]) && (size_t)Ns[i] * K <= 0x7fffffffULL &&
                 gemm_mf_serves((int)M, (int)Ns[i], (int)K, mode == GEMV_SWIGLU, cus);
    if (use_mf) {
        const int Mt = (int)((M + 31) / 32);
        // 5..16 rows against a very wide weight (the lm_head over a batch of
        // rows): 16-row MFMA tiles with the weights loaded straight into the
        // operands, the activations quantized inside the kernel
        bool wide16 = Mt == 1 && M >= 5 && mode != GEMV_SWIGLU;
        for (int i = 0; wide16 && i < nseg; ++i)
            wide16 = (size_t)Ns[i] * K >= ((size_t)1 << 26) &&
                     gemm_mf_wide_serves((int)M, (int)Ns[i], (int)K);
        if (wide16) {
            for (int i = 0; i < nseg; ++i) {
                float *pv = nullptr;
                int32_t *pi = nullptr;
                int nparts = 0;
                if (mode == GEMV_ARGMAX) {
                    pv = reinterpret_cast<float *>(wbase + LG.parts_val);
                    pi = reinterpret_cast<int32_t *>(wbase + LG.parts_idx);
                    nparts = gemm_mf_wide_parts((int)Ns[i], cus);
                    if ((size_t)nparts > kMaxGemvParts)
                        return fail(Q3VL_ERR_UNSUPPORTED, "argmax: %d partials exceed %zu", nparts,
                                    kMaxGemvParts);
                }
                Q3VL_HIP(launch_gemm_mf_wide(A, W[i], S[i], C[i], (int)M, (int)Ns[i], (int)K, pv, pi, cus, st),
                         "wide gemm launch");
                if (mode == GEMV_ARGMAX)
                    Q3VL_HIP(launch_argmax_final(pv, pi, nparts, (int)M, ids, st), "argmax launch");
            }
            return Q3VL_OK;
        }
        Q3VL_HIP(launch_quantize_frag(A, aq, asT, (int)M, (int)K, st), "quantize launch");
        if (mode == GEMV_SWIGLU) {
            GemmMfArgs g{aq, asT, Mt, W[0], S[0], W[1], S[1], C[0], (int)M, (int)Ns[0], (int)K};
            Q3VL_HIP(launch_gemm_mf(g, true, cus, st), "gemm launch");
            return Q3VL_OK;
        }
        for (int i = 0; i < nseg; ++i) {
            GemmMfArgs g{aq, asT, Mt, W[i], S[i], nullptr, nullptr, C[i], (int)M, (int)Ns[i], (int)K};
            int nparts = 0;
            if (mode == GEMV_ARGMAX) {
                // the GEMM leaves each block's per-row argmax partial; the
                // logits are stored only when the caller asked for them
                g.part_val = reinterpret_cast<float *>(wbase + LG.parts_val);
                g.part_idx = reinterpret_cast<int32_t *>(wbase + LG.parts_idx);
                const int cols = gemm_mf_argmax_cols((int)M);
                nparts = (int)((Ns[i] + cols - 1) / cols);
                if ((size_t)nparts > kMaxGemvParts)
                    return fail(Q3VL_ERR_UNSUPPORTED, "argmax: %d partials exceed %zu", nparts,
                                kMaxGemvParts);
            }
            Q3VL_HIP(launch_gemm_mf(g, false, cus, st), "gemm launch");
            if (mode == GEMV_ARGMAX)
                Q3VL_HIP(launch_argmax_final(g.part_val, g.part_idx, nparts, (int)M, ids, st),
                         "argmax launch");
        }
        return Q3VL_OK;
    }
    Q3VL_HIP(launch_quantize_f16(A, aq, asT, (int)M, (int)K, (int)gs, (int)K, LG.lda_s, st),
             "quantize launch");
    if (mode == GEMV_SWIGLU) {
        GemmArgs g{aq, asT, (int)K, LG.lda_s, W[0], S[0], W[1], S[1], C[0], nullptr,
                   (int)M, (int)Ns[0], (int)K, (int)gs, true};
        Q3VL_HIP(launch_gemm(g, st), "gemm launch");
        return Q3VL_OK;
    }
    for (int i = 0; i < nseg; ++i) {
        float *Ci = C[i];
        if (mode == GEMV_ARGMAX && !Ci) Ci = reinterpret_cast<float *>(wbase + LG.logits);
        GemmArgs g{aq, asT, (int)K, LG.lda_s, W[i], S[i], nullptr, nullptr, Ci,
                   G ? G[i] : nullptr, (int)M, (int)Ns[i], (int)K, (int)gs, false};
        Q3VL_HIP(launch_gemm(g, st), "gemm launch");
        if (mode == GEMV_ARGMAX)
            Q3VL_HIP(launch_argmax_rows(Ci, (int)M, (int)Ns[i],
                                        reinterpret_cast<float *>(wbase + LG.parts_val),
                                        reinterpret_cast<int32_t *>(wbase + LG.parts_idx),
                                        kGemmArgmaxParts, ids, st),
                     "argmax launch");
    }
    return Q3VL_OK;
}

// ---- host-weight registry
struct RegEntry {
    void *dW = nullptr;
    void *dS = nullptr;
    const float *hS = nullptr;
    size_t N = 0, K = 0, gs = 0;
    uint64_t fp = 0;
};
std::mutex g_reg_mu;
std::unordered_map<const void *, RegEntry> g_reg;

// FNV-1a over byte ranges.
uint64_t fnv1a(uint64_t h, const unsigned char *p, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 0x100000001b3ull;
    }
    return h;
}

// Sampled fingerprint of a host weight: the first and last 256 bytes of W,
// 16 strided 64-byte samples of it, the first and last 64 bytes of S.
uint64_t weight_fingerprint(const int8_t *W, const float *S, size_t N, size_t K, size_t gs) {
    const auto *w = reinterpret_cast<const unsigned char *>(W);
    const auto *s = reinterpret_cast<const unsigned char *>(S);
    const size_t wb = N * K, sb = gs ? N * (K / gs) * 4 : 0;
    uint64_t h = 0xcbf29ce484222325ull;
    auto take = [&](const unsigned char *base, size_t total, size_t off, size_t n) {
        if (off >= total) return;
        if (n > total - off) n = total - off;
        h = fnv1a(h, base + off, n);
    };
    take(w, wb, 0, 256);
    take(w, wb, wb > 256 ? wb - 256 : 0, 256);
    for (size_t i = 1; i <= 16; ++i) take(w, wb, wb / 17 * i, 64);
    take(s, sb, 0, 64);
    take(s, sb, sb > 64 ? sb - 64 : 0, 64);
    return h;
}

bool reg_matches(const RegEntry &e, const float *host_S, size_t N, size_t K, size_t gs, uint64_t fp) {
    return e.hS == host_S && e.N == N && e.K == K && e.gs == gs && e.fp == fp;
}

void reg_free(RegEntry &e) {
    (void)hipFree(e.dW);
    (void)hipFree(e.dS);
    e.dW = e.dS = nullptr;
}

// ------------------------------------------------------------ decode step
struct DecodeLayout {
    size_t lin;  // linear() scratch (argmax partials)
    size_t x, q, k, v, ao, h, scores, cmax, part_o, part_ml;
    size_t total;
    int max_chunks;
};

DecodeLayout decode_layout(const q3vl_text_model *m) {
    DecodeLayout L{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += align256(bytes);
        return o;
    };
    const size_t H = m->hidden, I = m->intermediate, NH = m->heads, NKV = m->kv_heads,
                 D = m->head_dim, S = m->max_seq;
    L.max_chunks = (int)((S + kAttnChunk - 1) / kAttnChunk);
    L.lin = take(layout(1, m->vocab, H, m->group_size).total);
    L.x = take(H * 4);
    L.q = take(NH * D * 4);
    L.k = take(NKV * D * 4);
    L.v = take(NKV * D * 4);
    L.ao = take(NH * D * 4);
    L.h = take(I * 4);
    L.scores = take(NH * S * 4);
    L.cmax = take(NH * (size_t)L.max_chunks * 4);
    // the chunked attention order's per-chunk partials
    const bool chunked = m->attn_order == Q3VL_ATTN_CHUNKED;
    L.part_o = chunked ? take(NH * (size_t)L.max_chunks * D * 4) : 0;
    L.part_ml = chunked ? take(NH * (size_t)L.max_chunks * 4 * 4) : 0;  // (m, l, min, 0) per chunk
    L.total = off;
    return L;
}

// The shapes the decode step serves (no pointers read).
int check_model_dims(const q3vl_text_model *m) {
    const long H = m->hidden, I = m->intermediate, D = m->head_dim, gs = m->group_size;
    if (D != 128 || m->heads <= 0 || m->kv_heads <= 0 || m->heads % m->kv_heads ||
        m->heads / m->kv_heads > 3)
        return fail(Q3VL_ERR_UNSUPPORTED, "decode step needs head_dim 128 and heads/kv_heads <= 3");
    const long dims[] = {H, I, (long)m->heads * D, (long)m->kv_heads * D};
    for (long d : dims)
        if (d < 1024 || d > 8192 || d % 16 || !gs || d % gs)
            return fail(Q3VL_ERR_UNSUPPORTED,
                        "decode step needs every linear dimension in [1024, 8192], "
                        "a multiple of 16 and of group_size (got %ld)", d);
    if (!gs_ok_gemv((size_t)gs) || D % gs)
        return fail(Q3VL_ERR_UNSUPPORTED, "group_size %ld not served", gs);
    if (m->vocab < 1024 || m->layers < 1 || m->max_seq < 8 || m->max_seq % 8)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "bad vocab / layers / max_seq (a multiple of 8)");
    if (m->attn_order != Q3VL_ATTN_REFERENCE && m->attn_order != Q3VL_ATTN_CHUNKED)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "attn_order %d is neither Q3VL_ATTN_REFERENCE nor "
                    "Q3VL_ATTN_CHUNKED", m->attn_order);
    if (attention_lds_bytes(m->heads, m->kv_heads, m->max_seq) > kAttnMaxLds)
        return fail(Q3VL_ERR_UNSUPPORTED,
                    "max_seq %d too long for the attention kernel's LDS (heads/kv_heads %d)",
                    m->max_seq, m->heads / m->kv_heads);
    return Q3VL_OK;
}

int check_model(const q3vl_text_model *m) {
    if (!m) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null model");
    if (int rc = check_model_dims(m)) return rc;
    const void *ptrs[] = {m->embed_w, m->embed_s, m->final_norm_w, m->final_norm_s,
                          m->attn_norm_w, m->attn_norm_s, m->mlp_norm_w, m->mlp_norm_s,
                          m->q_norm_w, m->q_norm_s, m->k_norm_w, m->k_norm_s, m->wq, m->wk,
                          m->wv, m->wo, m->wg, m->wu, m->wd, m->sq, m->sk, m->sv, m->so, m->sg,
                          m->su, m->sd, m->rope_cos, m->rope_sin};
    for (const void *p : ptrs)
        if (!p) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null model tensor");
    const void *w16[] = {m->embed_w, m->wq, m->wk, m->wv, m->wo, m->wg, m->wu, m->wd};
    for (const void *p : w16)
        if (!aligned16(p)) return fail(Q3VL_ERR_INVALID_ARGUMENT, "weights must be 16-byte aligned");
    const void *w8[] = {m->final_norm_w, m->attn_norm_w, m->mlp_norm_w};
    for (const void *p : w8)
        if (((uintptr_t)p & 7u) != 0)
            return fail(Q3VL_ERR_INVALID_ARGUMENT, "norm weights must be 8-byte aligned");
    return Q3VL_OK;
}

int decode_step_on(const q3vl_text_model *m, uint16_t *k_cache, uint16_t *v_cache,
                   int32_t *token, int32_t *pos, float *logits, char *w, hipStream_t st);

// ---- static scratch of q3vl_decode_step_static (no allocation per call).
// The array's host-side name is not a device address: each device's copy is
// found once with hipGetSymbolAddress (with that device current) and that
// pointer is what the kernels receive.
constexpr size_t kStaticScratchBytes = (size_t)1 << 20;  // 1 MiB per device
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

int static_scratch(char **out) {
    int dev = 0;
    Q3VL_HIP(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(Q3VL_ERR_UNSUPPORTED, "device %d", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        Q3VL_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (!p || ((uintptr_t)p & 255u))
            return fail(Q3VL_ERR_HIP, "static scratch at %p is not 256-byte aligned", p);
        g_scratch_ptr[dev] = p;
    }
    *out = static_cast<char *>(g_scratch_ptr[dev]);
    return Q3VL_OK;
}

GemvArgs gemv1(const float *A, int K, int gs) {
    GemvArgs a{};
    a.A = A;
    a.M = 1;
    a.K = K;
    a.gs = gs;
    a.mode = GEMV_PLAIN;
    return a;
}

}  // namespace

extern "C" {

const char *q3vl_last_error(void) { return g_err.c_str(); }

int q3vl_abi_version(void) { return Q3VL_ABI_VERSION; }

size_t q3vl_workspace_bytes(size_t M, size_t N, size_t K, size_t group_size) {
    // The GEMM-path layout (M >= 9) is a superset of the GEMV-path one, and
    // an M <= 8 shape may fall back to the GEMM kernels.
    return layout(M > 9 ? M : 9, N, K, group_size ? group_size : 1).total;
}

int q3vl_check_dtypes(int ta, int tb, int tb_scale, int tc, int has_bias, int group_quantized,
                      int b_transpose) {
    if (ta == Q3VL_DTYPE_FP32 && tc == Q3VL_DTYPE_FP32 && tb == Q3VL_DTYPE_INT8 &&
        tb_scale == Q3VL_DTYPE_FP32 && !has_bias) {
        if (!group_quantized)
            return fail(Q3VL_ERR_UNSUPPORTED,
                        "DType matmul not supported: row-quantized int8 (group_quantized=0)");
        if (!b_transpose)
            return fail(Q3VL_ERR_UNSUPPORTED,
                        "DType matmul not supported: int8 weights need mat_B_transpose=1");
        return Q3VL_OK;
    }
    return fail(Q3VL_ERR_UNSUPPORTED,
                "DType matmul not supported: type_a=%d, type_b=%d, type_b_scale=%d, type_c=%d, "
                "bias=%d, group_quantized=%d",
                ta, tb, tb_scale, tc, has_bias, group_quantized);
}

int q3vl_uses_lane_path(size_t M, size_t N, size_t K) {
    return M == 1 && N >= 1024 && K >= 1024;
}

int q3vl_quantize_rows(const float *A, int16_t *q, float *a_s, size_t M, size_t K,
                       size_t group_size, q3vl_stream stream) {
    if (!gs_ok_gemv(group_size) || K % group_size != 0)
        return fail(Q3VL_ERR_UNSUPPORTED, "group_size=%zu / K=%zu not supported", group_size, K);
    if (M == 0 || K == 0) return Q3VL_OK;
    if (!A || !q || !a_s) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null pointer");
    if (M > 65535) return fail(Q3VL_ERR_UNSUPPORTED, "M=%zu > 65535", M);
    Q3VL_HIP(launch_quantize_i16(A, q, a_s, (int)M, (int)K, (int)group_size,
                                 (hipStream_t)stream),
             "quantize launch");
    return Q3VL_OK;
}

int q3vl_linear_i8(const float *A, const int8_t *W, const float *S, float *C, size_t M,
                   size_t N, size_t K, size_t group_size, void *workspace,
                   size_t workspace_bytes, q3vl_stream stream) {
    if (!C && M && N) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null C");
    int32_t *G = nullptr;
    return run_linear(A, 1, &W, &S, &C, &G, &N, M, K, group_size, GEMV_PLAIN, workspace,
                      workspace_bytes, (hipStream_t)stream, nullptr);
}

int q3vl_linear_i8_groups(const float *A, const int8_t *W, const float *S, float *C,
                          int32_t *G, size_t M, size_t N, size_t K, size_t group_size,
                          void *workspace, size_t workspace_bytes, q3vl_stream stream) {
    if ((!C || !G) && M && N) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null C or G");
    return run_linear(A, 1, &W, &S, &C, &G, &N, M, K, group_size, GEMV_PLAIN, workspace,
                      workspace_bytes, (hipStream_t)stream, nullptr);
}

int q3vl_linear_i8_multi(const float *A, size_t M, size_t K, size_t group_size, int count,
                         const int8_t *const *W, const float *const *S, float *const *C,
                         const size_t *N, void *workspace, size_t workspace_bytes,
                         q3vl_stream stream) {
    if (count < 1 || count > 3 || !W || !S || !C || !N)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "count must be 1..3 with non-null arrays");
    for (int i = 0; i < count; ++i)
        if (!C[i] && M && N[i]) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null C[%d]", i);
    int32_t *G[3] = {nullptr, nullptr, nullptr};
    return run_linear(A, count, W, S, C, G, N, M, K, group_size, GEMV_PLAIN, workspace,
                      workspace_bytes, (hipStream_t)stream, nullptr);
}

int q3vl_linear_i8_swiglu(const float *A, const int8_t *Wg, const float *Sg, const int8_t *Wu,
                          const float *Su, float *H, size_t M, size_t N, size_t K,
                          size_t group_size, void *workspace, size_t workspace_bytes,
                          q3vl_stream stream) {
    if (!H && M && N) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null H");
    const int8_t *W[2] = {Wg, Wu};
    const float *S[2] = {Sg, Su};
    float *C[2] = {H, nullptr};
    int32_t *G[2] = {nullptr, nullptr};
    const size_t Ns[2] = {N, N};
    return run_linear(A, 2, W, S, C, G, Ns, M, K, group_size, GEMV_SWIGLU, workspace,
                      workspace_bytes, (hipStream_t)stream, nullptr);
}

// The MLP block: h = swiglu(A Wg^T, A Wu^T) [M, I], then Y = h Wd^T [M, H].
// Fused where the fragment-order GEMMs serve both products: A quantized
// once, the gate|up GEMM's epilogue quantizes h into the down GEMM's operand
// (no h in memory, no quantizer launch for it). Elsewhere: the two calls
// through an h buffer at the start of the workspace.
struct MlpLayout {
    bool fused = false;
    size_t aq = 0, as = 0, hq = 0, hs = 0;  // fused
    size_t h = 0, inner = 0;                // two calls: h, then the calls' own workspace
    size_t total = 0;
};

static MlpLayout mlp_layout(size_t M, size_t H, size_t I, size_t gs, bool fused) {
    MlpLayout L;
    L.fused = fused;
    size_t off = 0;
    if (fused) {
        const size_t Mpad = (M + 31) & ~(size_t)31;
        L.aq = off;
        off += align256(Mpad * H * 2);
        L.as = off;
        off += align256(Mpad * (H / 64) * 4);
        L.hq = off;
        off += align256(Mpad * I * 2);
        L.hs = off;
        off += align256(Mpad * (I / 64) * 4);
    } else {
        L.h = off;
        off += align256(M * I * 4);
        L.inner = off;
        const size_t a = q3vl_workspace_bytes(M, I, H, gs), b = q3vl_workspace_bytes(M, H, I, gs);
        off += a > b ? a : b;
    }
    L.total = off;
    return L;
}

static bool mlp_fuses(size_t M, size_t H, size_t I, size_t gs, int cus) {
    const size_t Mpad = (M + 31) & ~(size_t)31;
    return M > 8 && gs == 64 && H % 512 == 0 && I % 512 == 0 && Mpad * (H > I ? H : I) * 2 <= 0x7fffffffULL &&
           H * I <= 0x7fffffffULL && gemm_mf_serves((int)M, (int)I, (int)H, true, cus) &&
           gemm_mf_serves((int)M, (int)H, (int)I, false, cus);
}

size_t q3vl_mlp_workspace_bytes(size_t M, size_t H, size_t I, size_t group_size) {
    const size_t a = mlp_layout(M, H, I, group_size ? group_size : 1, false).total;
    const size_t b = (group_size == 64 && H % 512 == 0 && I % 512 == 0 && M > 8)
                         ? mlp_layout(M, H, I, 64, true).total : 0;
    return a > b ? a : b;
}

int q3vl_mlp_i8(const float *A, const int8_t *Wg, const float *Sg, const int8_t *Wu, const float *Su,
                const int8_t *Wd, const float *Sd, float *Y, size_t M, size_t H, size_t I,
                size_t group_size, void *workspace, size_t workspace_bytes, q3vl_stream stream) {
    const hipStream_t st = (hipStream_t)stream;
    if (!Y && M && H) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null Y");
    int rc = check_common(A, Wg, Sg, M, I, H, group_size);
    if (!rc) rc = check_common(A, Wu, Su, M, I, H, group_size);
    if (!rc) rc = check_common(A, Wd, Sd, M, H, I, group_size);
    if (rc) return rc;
    if (M == 0 || H == 0) return Q3VL_OK;
    int cus = 0;
    rc = device_cus(&cus);
    if (rc) return rc;
    const bool fused = I > 0 && mlp_fuses(M, H, I, group_size, cus);
    const MlpLayout L = mlp_layout(M, H, I, group_size, fused);
    char *wbase = nullptr;
    rc = resolve_ws(workspace, workspace_bytes, L.total, &wbase);
    if (rc) return rc;
    if (fused) {
        _Float16 *aq = reinterpret_cast<_Float16 *>(wbase + L.aq);
        float *as = reinterpret_cast<float *>(wbase + L.as);
        _Float16 *hq = reinterpret_cast<_Float16 *>(wbase + L.hq);
        float *hs = reinterpret_cast<float *>(wbase + L.hs);
        const int Mt = (int)((M + 31) / 32);
        Q3VL_HIP(launch_quantize_frag(A, aq, as, (int)M, (int)H, st), "quantize launch");
        GemmMfArgs gu{aq, as, Mt, Wg, Sg, Wu, Su, nullptr, (int)M, (int)I, (int)H};
        gu.hq = hq;
        gu.hqs = hs;
        Q3VL_HIP(launch_gemm_mf(gu, true, cus, st), "gate|up gemm launch");
        GemmMfArgs dn{hq, hs, Mt, Wd, Sd, nullptr, nullptr, Y, (int)M, (int)H, (int)I};
        Q3VL_HIP(launch_gemm_mf(dn, false, cus, st), "down gemm launch");
        return Q3VL_OK;
    }
    // the two calls, h in the workspace
    float *h = reinterpret_cast<float *>(wbase + L.h);
    char *inner = wbase + L.inner;
    const size_t inner_bytes = L.total - L.inner;
    rc = q3vl_linear_i8_swiglu(A, Wg, Sg, Wu, Su, h, M, I, H, group_size, inner, inner_bytes, stream);
    if (rc) return rc;
    return q3vl_linear_i8(h, Wd, Sd, Y, M, H, I, group_size, inner, inner_bytes, stream);
}

int q3vl_lm_head_argmax(const float *A, const int8_t *W, const float *S, float *logits,
                        int32_t *ids, size_t M, size_t V, size_t K, size_t group_size,
                        void *workspace, size_t workspace_bytes, q3vl_stream stream) {
    if (!ids && M) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null ids");
    if (M == 0) return Q3VL_OK;
    if (V == 0 || V > 0x7fffffff)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "vocabulary size V=%zu", V);
    int32_t *G = nullptr;
    return run_linear(A, 1, &W, &S, &logits, &G, &V, M, K, group_size, GEMV_ARGMAX, workspace,
                      workspace_bytes, (hipStream_t)stream, ids);
}

int q3vl_argmax_rows(const float *logits, int32_t *ids, size_t M, size_t V, void *workspace,
                     size_t workspace_bytes, q3vl_stream stream) {
    if (M == 0) return Q3VL_OK;
    if (!logits || !ids) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null pointer");
    if (V == 0 || V > 0x7fffffff || M > 65535)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "bad shape M=%zu V=%zu", M, V);
    const int nparts = 64;
    const size_t need = 2 * align256((size_t)nparts * M * 4);
    char *w = nullptr;
    int rc = resolve_ws(workspace, workspace_bytes, need, &w);
    if (rc) return rc;
    float *pv = reinterpret_cast<float *>(w);
    int32_t *pi = reinterpret_cast<int32_t *>(w + align256((size_t)nparts * M * 4));
    Q3VL_HIP(launch_argmax_rows(logits, (int)M, (int)V, pv, pi, nparts, ids,
                                (hipStream_t)stream),
             "argmax launch");
    return Q3VL_OK;
}

int q3vl_swiglu(float *gate, const float *up, size_t n, q3vl_stream stream) {
    if (n == 0) return Q3VL_OK;
    if (!gate || !up) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null pointer");
    Q3VL_HIP(launch_swiglu(gate, up, n, (hipStream_t)stream), "swiglu launch");
    return Q3VL_OK;
}

size_t q3vl_decode_workspace_bytes(const q3vl_text_model *m) {
    if (!m || m->head_dim <= 0 || m->group_size <= 0) return 0;
    return decode_layout(m).total;
}

int q3vl_decode_step(const q3vl_text_model *m, uint16_t *k_cache, uint16_t *v_cache,
                     int32_t *token, int32_t *pos, float *logits, void *workspace,
                     size_t workspace_bytes, q3vl_stream stream) {
    int rc = check_model(m);
    if (rc) return rc;
    if (!k_cache || !v_cache || !token || !pos)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "null cache / token / pos");
    const DecodeLayout L = decode_layout(m);
    char *w = nullptr;
    rc = resolve_ws(workspace, workspace_bytes, L.total, &w);
    if (rc) return rc;
    return decode_step_on(m, k_cache, v_cache, token, pos, logits, w, (hipStream_t)stream);
}

size_t q3vl_decode_static_scratch_bytes(void) { return kStaticScratchBytes; }

int q3vl_decode_step_static(const q3vl_text_model *m, uint16_t *k_cache, uint16_t *v_cache,
                            int32_t *token, int32_t *pos, float *logits, q3vl_stream stream) {
    int rc = check_model(m);
    if (rc) return rc;
    if (!k_cache || !v_cache || !token || !pos)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "null cache / token / pos");
    const size_t need = decode_layout(m).total;
    if (need > kStaticScratchBytes)
        return fail(Q3VL_ERR_UNSUPPORTED,
                    "decode step needs %zu bytes of scratch, more than the %zu of the static "
                    "scratch (use q3vl_decode_step with a caller workspace)",
                    need, kStaticScratchBytes);
    char *w = nullptr;
    rc = static_scratch(&w);
    if (rc) return rc;
    return decode_step_on(m, k_cache, v_cache, token, pos, logits, w, (hipStream_t)stream);
}

}  // extern "C"

namespace {

// The decode step's launches over a resolved workspace w (decode_layout(m)).
int decode_step_on(const q3vl_text_model *m, uint16_t *k_cache, uint16_t *v_cache,
                   int32_t *token, int32_t *pos, float *logits, char *w, hipStream_t st) {
    const DecodeLayout L = decode_layout(m);
    const int H = m->hidden, I = m->intermediate, NH = m->heads, NKV = m->kv_heads;
    const int D = m->head_dim, gs = m->group_size, V = m->vocab;
    const int QD = NH * D, KD = NKV * D;
    auto F = [&](size_t off) { return reinterpret_cast<float *>(w + off); };
    float *x = F(L.x), *q = F(L.q), *k = F(L.k), *v = F(L.v), *ao = F(L.ao);
    float *hb = F(L.h);
    const WsLayout LL = layout(1, V, H, gs);
    float *pv = reinterpret_cast<float *>(w + L.lin + LL.parts_val);
    int32_t *pi = reinterpret_cast<int32_t *>(w + L.lin + LL.parts_idx);

    Q3VL_HIP(launch_embed(m->embed_w, m->embed_s, token, x, H, gs, V, st), "embed");  // :478-485
    AttnArgs aa{};
    aa.q = q;
    aa.k = k;
    aa.v = v;
    aa.rope_cos = m->rope_cos;
    aa.rope_sin = m->rope_sin;
    aa.k_cache = k_cache;
    aa.v_cache = v_cache;
    aa.pos = pos;
    aa.scores = F(L.scores);
    aa.cmax = F(L.cmax);
    aa.order = m->attn_order;
    if (m->attn_order == Q3VL_ATTN_CHUNKED) {
        aa.part_o = F(L.part_o);
        aa.part_ml = F(L.part_ml);
    }
    aa.out = ao;
    aa.heads = NH;
    aa.kv_heads = NKV;
    aa.head_dim = D;
    aa.max_seq = m->max_seq;
    aa.max_chunks = L.max_chunks;
    aa.gs = gs;
    aa.eps = m->rms_eps;
    aa.inv_sqrt_d = 1.0f / sqrtf((float)D);  // text_layer.cpp:582
    int grid = 0;
    for (int l = 0; l < m->layers; ++l) {
        const size_t lH = (size_t)l * H, lD = (size_t)l * D;
        // :493 pre-attention RMSNorm fused into the q, k, v GEMV (:506-528)
        GemvArgs g = gemv1(x, H, gs);
        g.norm_w = m->attn_norm_w + lH;
        g.norm_s = m->attn_norm_s + lH / gs;
        g.norm_eps = m->rms_eps;
        g.nseg = 3;
        g.seg[0] = {m->wq + (size_t)l * QD * H, m->sq + (size_t)l * QD * H / gs, q, nullptr, QD};
        g.seg[1] = {m->wk + (size_t)l * KD * H, m->sk + (size_t)l * KD * H / gs, k, nullptr, KD};
        g.seg[2] = {m->wv + (size_t)l * KD * H, m->sv + (size_t)l * KD * H / gs, v, nullptr, KD};
        Q3VL_HIP(launch_gemv(g, true, &grid, st), "qkv gemv");
        // :531-581 QK norm, RoPE, KV store, attention
        aa.layer = l;
        aa.qnorm_w = m->q_norm_w + lD;
        aa.qnorm_s = m->q_norm_s + lD / gs;
        aa.knorm_w = m->k_norm_w + lD;
        aa.knorm_s = m->k_norm_s + lD / gs;
        Q3VL_HIP(launch_attention(aa, st), "attention");
        // :592-604 output projection, residual add into x
        g = gemv1(ao, QD, gs);
        g.nseg = 1;
        g.accumulate = 1;
        g.seg[0] = {m->wo + (size_t)l * H * QD, m->so + (size_t)l * H * QD / gs, x, nullptr, H};
        Q3VL_HIP(launch_gemv(g, true, &grid, st), "o gemv");
        // :611-661 pre-MLP RMSNorm fused into gate/up + swiglu, then down and
        // the residual add
        g = gemv1(x, H, gs);
        g.norm_w = m->mlp_norm_w + lH;
        g.norm_s = m->mlp_norm_s + lH / gs;
        g.norm_eps = m->rms_eps;
        g.nseg = 2;
        g.mode = GEMV_SWIGLU;
        g.seg[0] = {m->wg + (size_t)l * I * H, m->sg + (size_t)l * I * H / gs, hb, nullptr, I};
        g.seg[1] = {m->wu + (size_t)l * I * H, m->su + (size_t)l * I * H / gs, nullptr, nullptr, I};
        Q3VL_HIP(launch_gemv(g, true, &grid, st), "gate/up gemv");
        g = gemv1(hb, I, gs);
        g.nseg = 1;
        g.accumulate = 1;
        g.seg[0] = {m->wd + (size_t)l * H * I, m->sd + (size_t)l * H * I / gs, x, nullptr, H};
        Q3VL_HIP(launch_gemv(g, true, &grid, st), "down gemv");
    }
    // :693-705 final RMSNorm fused into the tied classifier, greedy_decode
    GemvArgs g = gemv1(x, H, gs);
    g.norm_w = m->final_norm_w;
    g.norm_s = m->final_norm_s;
    g.norm_eps = m->rms_eps;
    g.nseg = 1;
    g.mode = GEMV_ARGMAX;
    g.seg[0] = {m->embed_w, m->embed_s, logits, nullptr, V};
    g.part_val = pv;
    g.part_idx = pi;
    Q3VL_HIP(launch_gemv(g, true, &grid, st), "lm_head gemv");
    Q3VL_HIP(launch_argmax_final(pv, pi, grid, 1, token, st, pos), "argmax final");
    return Q3VL_OK;
}

}  // namespace

extern "C" {

int q3vl_weight_register(const int8_t *host_W, const float *host_S, size_t N, size_t K,
                         size_t group_size, const int8_t **dev_W, const float **dev_S) {
    if (!host_W || !host_S || !group_size || K % group_size)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "bad weight registration arguments");
    const uint64_t fp = weight_fingerprint(host_W, host_S, N, K, group_size);
    std::lock_guard<std::mutex> lk(g_reg_mu);
    auto it = g_reg.find(host_W);
    if (it != g_reg.end() && !reg_matches(it->second, host_S, N, K, group_size, fp)) {
        // A stale entry (another weight now lives at host_W): work queued on
        // any stream may still read the old copies.
        Q3VL_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
        reg_free(it->second);
        g_reg.erase(it);
        it = g_reg.end();
    }
    if (it == g_reg.end()) {
        RegEntry e;
        e.hS = host_S;
        e.N = N;
        e.K = K;
        e.gs = group_size;
        e.fp = fp;
        const size_t wb = N * K, sb = N * (K / group_size) * 4;
        if (hipMalloc(&e.dW, wb ? wb : 1) != hipSuccess ||
            hipMalloc(&e.dS, sb ? sb : 1) != hipSuccess) {
            if (e.dW) (void)hipFree(e.dW);
            return fail(Q3VL_ERR_OUT_OF_MEMORY, "weight upload: hipMalloc failed");
        }
        hipError_t err = hipMemcpy(e.dW, host_W, wb, hipMemcpyHostToDevice);
        if (err == hipSuccess) err = hipMemcpy(e.dS, host_S, sb, hipMemcpyHostToDevice);
        if (err != hipSuccess) {
            reg_free(e);
            return hip_fail(err, "weight upload");
        }
        it = g_reg.emplace(host_W, e).first;
    }
    if (dev_W) *dev_W = static_cast<const int8_t *>(it->second.dW);
    if (dev_S) *dev_S = static_cast<const float *>(it->second.dS);
    return Q3VL_OK;
}

int q3vl_weight_lookup(const void *host_W, const float *host_S, size_t N, size_t K,
                       size_t group_size, const int8_t **dev_W, const float **dev_S) {
    if (!host_W || !host_S || !group_size || K % group_size)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "bad weight lookup arguments");
    const uint64_t fp =
        weight_fingerprint(static_cast<const int8_t *>(host_W), host_S, N, K, group_size);
    std::lock_guard<std::mutex> lk(g_reg_mu);
    auto it = g_reg.find(host_W);
    if (it == g_reg.end())
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "host weight %p is not registered", host_W);
    const RegEntry &e = it->second;
    if (!reg_matches(e, host_S, N, K, group_size, fp))
        return fail(Q3VL_ERR_STALE_WEIGHT,
                    "host weight %p is registered as [%zu x %zu] group %zu with scales %p; called "
                    "with [%zu x %zu] group %zu, scales %p%s",
                    host_W, e.N, e.K, e.gs, (const void *)e.hS, N, K, group_size,
                    (const void *)host_S, e.fp != fp ? " and other contents" : "");
    if (dev_W) *dev_W = static_cast<const int8_t *>(e.dW);
    if (dev_S) *dev_S = static_cast<const float *>(e.dS);
    return Q3VL_OK;
}

int q3vl_weight_release(const void *host_W) {
    std::lock_guard<std::mutex> lk(g_reg_mu);
    auto it = g_reg.find(host_W);
    if (it == g_reg.end())
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "host weight %p is not registered", host_W);
    Q3VL_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    reg_free(it->second);
    g_reg.erase(it);
    return Q3VL_OK;
}

int q3vl_weight_release_all(void) {
    std::lock_guard<std::mutex> lk(g_reg_mu);
    if (!g_reg.empty()) Q3VL_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    for (auto &kv : g_reg) reg_free(kv.second);
    g_reg.clear();
    return Q3VL_OK;
}

}  // extern "C"

// ------------------------------------------------------------ checkpoint files
struct q3vl_checkpoint {
    q3vl_checkpoint_header hdr;
    q3vl_text_model model;
    void *dev;  // one allocation holding every tensor and the RoPE tables
    int device;
};

namespace {

constexpr size_t kCkHeaderBytes = 100;
static_assert(sizeof(q3vl_checkpoint_header) == kCkHeaderBytes,
              "the header struct is the file's first 100 bytes");

// map_tensor's walk over the text groups (load_model.cpp:146-195): per group,
// the scales (int8) then the values; norm tensors always group-quantized.
// One byte range of a checkpoint file and where it goes in device memory.
struct FilePiece {
    size_t file_off, bytes, dev_off;
};

// Copies file byte ranges to device memory on the current device. kReaders
// threads each take 16 MB jobs in turn, read them with pread into one of
// their own two pinned buffers and copy them on their own stream, so the
// file reads (memcpy-bound from the page cache) run in parallel and overlap
// the host-to-device copies. Synchronous: every copy has landed on return.
int copy_file_to_device(int fd, const char *path, const std::vector<FilePiece> &pieces,
                        unsigned char *d) {
    constexpr int kReaders = 4;
    constexpr size_t kJob = (size_t)16 << 20;
    std::vector<FilePiece> jobs;
    for (const FilePiece &p : pieces)
        for (size_t o = 0; o < p.bytes; o += kJob)
            jobs.push_back({p.file_off + o, p.bytes - o < kJob ? p.bytes - o : kJob, p.dev_off + o});
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return fail(Q3VL_ERR_HIP, "hipGetDevice failed");
    std::atomic<size_t> next{0};
    std::atomic<bool> stop{false};
    std::mutex mu;
    int err_code = Q3VL_OK;
    std::string err_msg;
    auto set_err = [&](int code, std::string msg) {
        std::lock_guard<std::mutex> lk(mu);
        if (err_code == Q3VL_OK) {
            err_code = code;
            err_msg = std::move(msg);
        }
        stop = true;
    };
    auto worker = [&]() {
        if (hipSetDevice(device) != hipSuccess) return set_err(Q3VL_ERR_HIP, "hipSetDevice failed");
        hipStream_t st = nullptr;
        void *stage[2] = {nullptr, nullptr};
        hipEvent_t done[2] = {nullptr, nullptr};
        bool used[2] = {false, false};
        bool ok = hipStreamCreateWithFlags(&st, hipStreamNonBlocking) == hipSuccess;
        for (int j = 0; j < 2 && ok; ++j)
            ok = hipHostMalloc(&stage[j], kJob, hipHostMallocDefault) == hipSuccess &&
                 hipEventCreateWithFlags(&done[j], hipEventDisableTiming) == hipSuccess;
        if (!ok) set_err(Q3VL_ERR_OUT_OF_MEMORY, "pinned staging buffers / reader stream");
        for (int k = 0; ok && !stop; k ^= 1) {
            const size_t j = next++;
            if (j >= jobs.size()) break;
            const FilePiece &jb = jobs[j];
            if (used[k] && hipEventSynchronize(done[k]) != hipSuccess) {
                set_err(Q3VL_ERR_HIP, "hipEventSynchronize failed");
                break;
            }
            size_t got = 0;
            while (got < jb.bytes) {
                const ssize_t n = pread(fd, static_cast<char *>(stage[k]) + got, jb.bytes - got,
                                        (off_t)(jb.file_off + got));
                if (n <= 0) break;
                got += (size_t)n;
            }
            if (got != jb.bytes) {
                char buf[256];
                snprintf(buf, sizeof buf, "%s: read failed at %zu", path, jb.file_off + got);
                set_err(Q3VL_ERR_INVALID_ARGUMENT, buf);
                break;
            }
            hipError_t e = hipMemcpyAsync(d + jb.dev_off, stage[k], jb.bytes, hipMemcpyHostToDevice, st);
            if (e == hipSuccess) e = hipEventRecord(done[k], st);
            if (e != hipSuccess) {
                set_err(Q3VL_ERR_HIP, std::string("checkpoint copy: ") + hipGetErrorString(e));
                break;
            }
            used[k] = true;
        }
        if (st && hipStreamSynchronize(st) != hipSuccess) set_err(Q3VL_ERR_HIP, "reader stream sync failed");
        for (int j = 0; j < 2; ++j) {
            if (done[j]) (void)hipEventDestroy(done[j]);
            if (stage[j]) (void)hipHostFree(stage[j]);
        }
        if (st) (void)hipStreamDestroy(st);
    };
    const int nthreads = (int)(jobs.size() < (size_t)kReaders ? jobs.size() : (size_t)kReaders);
    std::vector<std::thread> pool;
    for (int t = 0; t < nthreads; ++t) pool.emplace_back(worker);
    for (std::thread &t : pool) t.join();
    if (err_code != Q3VL_OK) return fail(err_code, "%s", err_msg.c_str());
    return Q3VL_OK;
}

int ck_layout(const q3vl_checkpoint_header *h, q3vl_checkpoint_span *sp) {
    if (!h || !sp) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null header / spans");
    if (h->vocab <= 0 || h->hidden <= 0 || h->intermediate <= 0 || h->layers <= 0 ||
        h->heads <= 0 || h->kv_heads <= 0 || h->hidden % h->heads)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "bad checkpoint dimensions");
    if (h->text_bits != 8 && h->text_bits != 16 && h->text_bits != 32)
        return fail(Q3VL_ERR_UNSUPPORTED, "text_bits %d not read (8, 16 or 32)", h->text_bits);
    if (h->text_bits == 8 && h->group_size <= 0)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "group_size %d", h->group_size);
    const size_t L = h->layers, H = h->hidden, I = h->intermediate, V = h->vocab;
    const size_t hd = H / h->heads, QD = (size_t)h->heads * hd, KV = (size_t)h->kv_heads * hd;
    size_t off = kCkHeaderBytes;
    int rc = Q3VL_OK;
    auto put = [&](int idx, size_t count, size_t rowlen, bool norm) {
        q3vl_checkpoint_span t{};
        t.bits = h->text_bits;
        t.data_count = count;
        if (h->text_bits == 8) {
            const size_t grp = (h->group_quantized || norm) ? (size_t)h->group_size : rowlen;
            if (count % grp) {
                rc = fail(Q3VL_ERR_INVALID_ARGUMENT, "tensor %d: %zu values, not whole groups of %zu",
                          idx, count, grp);
                return;
            }
            t.group = (int)grp;
            t.scales_offset = off;
            t.scales_count = count / grp;
            off += t.scales_count * 4;
            t.data_offset = off;
            off += count;
        } else {
            t.data_offset = off;
            off += count * (size_t)(h->text_bits / 8);
        }
        sp[idx] = t;
    };
    put(Q3VL_CK_EMBED, V * H, H, false);
    put(Q3VL_CK_ATTN_NORM, L * H, H, true);
    put(Q3VL_CK_DOWN, L * H * I, I, false);
    put(Q3VL_CK_GATE, L * I * H, H, false);
    put(Q3VL_CK_UP, L * I * H, H, false);
    put(Q3VL_CK_MLP_NORM, L * H, H, true);
    put(Q3VL_CK_K_NORM, L * hd, hd, true);
    put(Q3VL_CK_K, L * KV * H, H, false);
    put(Q3VL_CK_O, L * H * H, H, false);  // {L, H, H} as load_model.cpp:186
    put(Q3VL_CK_Q_NORM, L * hd, hd, true);
    put(Q3VL_CK_Q, L * QD * H, H, false);
    put(Q3VL_CK_V, L * KV * H, H, false);
    put(Q3VL_CK_FINAL_NORM, H, H, true);
    return rc;
}

}  // namespace

extern "C" {

int q3vl_checkpoint_read_header(const char *path, q3vl_checkpoint_header *hdr) {
    if (!path || !hdr) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null path / header");
    FILE *f = fopen(path, "rb");
    if (!f) return fail(Q3VL_ERR_INVALID_ARGUMENT, "cannot open %s", path);
    unsigned char buf[kCkHeaderBytes];
    const size_t got = fread(buf, 1, sizeof buf, f);
    fclose(f);
    if (got != sizeof buf) return fail(Q3VL_ERR_INVALID_ARGUMENT, "%s: shorter than the header", path);
    memcpy(hdr, buf, sizeof buf);
    return Q3VL_OK;
}

int q3vl_checkpoint_text_layout(const q3vl_checkpoint_header *hdr, q3vl_checkpoint_span *spans) {
    return ck_layout(hdr, spans);
}

int q3vl_rope_tables(int rope_theta, int head_dim, int rows, float *cos_out, float *sin_out) {
    if (!cos_out || !sin_out || head_dim <= 0 || head_dim % 2 || rows < 0)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "bad RoPE table arguments");
    const int half = head_dim / 2;
    std::vector<float> inv_freq(half);
    for (int i = 0; i < half; ++i)
        inv_freq[i] = 1.0f / powf((float)rope_theta, (2.0f * i) / (float)head_dim);
    for (int pos = 0; pos < rows; ++pos)
        for (int i = 0; i < half; ++i) {
            const float freq = pos * inv_freq[i];
            cos_out[(size_t)pos * half + i] = cosf(freq);
            sin_out[(size_t)pos * half + i] = sinf(freq);
        }
    return Q3VL_OK;
}

int q3vl_checkpoint_load(const char *path, int max_seq, q3vl_stream stream,
                         q3vl_checkpoint **out) {
    if (!out) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null output");
    *out = nullptr;
    q3vl_checkpoint_header h;
    int rc = q3vl_checkpoint_read_header(path, &h);
    if (rc) return rc;
    q3vl_checkpoint_span sp[Q3VL_CK_TEXT_TENSORS];
    if ((rc = ck_layout(&h, sp))) return rc;
    if (h.text_bits != 8)
        return fail(Q3VL_ERR_UNSUPPORTED, "text_bits %d: the decode step runs int8 weights", h.text_bits);
    if (!h.group_quantized)
        return fail(Q3VL_ERR_UNSUPPORTED,
                    "per-row scales (group_quantized = 0) are not served by the decode step");
    if (max_seq <= 0) return fail(Q3VL_ERR_INVALID_ARGUMENT, "max_seq %d", max_seq);
    const size_t end = sp[Q3VL_CK_FINAL_NORM].data_offset + sp[Q3VL_CK_FINAL_NORM].data_count;
    {
        q3vl_text_model dm{};
        dm.vocab = h.vocab;
        dm.hidden = h.hidden;
        dm.intermediate = h.intermediate;
        dm.layers = h.layers;
        dm.heads = h.heads;
        dm.kv_heads = h.kv_heads;
        dm.head_dim = h.hidden / h.heads;
        dm.max_seq = max_seq;
        dm.group_size = h.group_size;
        if ((rc = check_model_dims(&dm))) return rc;  // before any allocation
    }

    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(Q3VL_ERR_INVALID_ARGUMENT, "cannot open %s", path);
    const off_t fsize = lseek(fd, 0, SEEK_END);
    if (fsize < 0 || (size_t)fsize < end) {
        close(fd);
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "%s: %lld bytes, the text tensors end at %zu", path,
                    (long long)fsize, end);
    }

    // device layout: every piece 256-byte aligned
    const int hd = h.hidden / h.heads, half = hd / 2;
    size_t off = 0;
    std::vector<FilePiece> pieces;
    size_t sc_at[Q3VL_CK_TEXT_TENSORS], da_at[Q3VL_CK_TEXT_TENSORS];
    for (int i = 0; i < Q3VL_CK_TEXT_TENSORS; ++i) {
        sc_at[i] = off;
        pieces.push_back({sp[i].scales_offset, sp[i].scales_count * 4, off});
        off += align256(sp[i].scales_count * 4);
        da_at[i] = off;
        pieces.push_back({sp[i].data_offset, sp[i].data_count, off});
        off += align256(sp[i].data_count);
    }
    const size_t rope_bytes = (size_t)max_seq * half * 4;
    const size_t cos_at = off;
    off += align256(rope_bytes);
    const size_t sin_at = off;
    off += align256(rope_bytes);

    q3vl_checkpoint *ck = new q3vl_checkpoint{};
    ck->hdr = h;
    if (hipGetDevice(&ck->device) != hipSuccess || hipMalloc(&ck->dev, off) != hipSuccess) {
        close(fd);
        delete ck;
        return fail(Q3VL_ERR_OUT_OF_MEMORY, "checkpoint hipMalloc(%zu) failed", off);
    }
    unsigned char *d = static_cast<unsigned char *>(ck->dev);
    rc = copy_file_to_device(fd, path, pieces, d);
    close(fd);
    if (!rc) {
        hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        std::vector<float> cs((size_t)max_seq * half), sn((size_t)max_seq * half);
        rc = q3vl_rope_tables(h.rope_theta, hd, max_seq, cs.data(), sn.data());
        if (!rc) {
            hipError_t e = hipMemcpyAsync(d + cos_at, cs.data(), rope_bytes, hipMemcpyHostToDevice, st);
            if (e == hipSuccess) e = hipMemcpyAsync(d + sin_at, sn.data(), rope_bytes, hipMemcpyHostToDevice, st);
            if (e == hipSuccess) e = hipStreamSynchronize(st);
            if (e != hipSuccess) rc = hip_fail(e, "RoPE table copy");
        }
    }
    if (rc) {
        (void)hipFree(ck->dev);
        delete ck;
        return rc;
    }

    q3vl_text_model &m = ck->model;
    m.vocab = h.vocab;
    m.hidden = h.hidden;
    m.intermediate = h.intermediate;
    m.layers = h.layers;
    m.heads = h.heads;
    m.kv_heads = h.kv_heads;
    m.head_dim = hd;
    m.max_seq = max_seq;
    m.group_size = h.group_size;
    m.rms_eps = h.rms_eps;
    auto W = [&](int i) { return reinterpret_cast<const int8_t *>(d + da_at[i]); };
    auto S = [&](int i) { return reinterpret_cast<const float *>(d + sc_at[i]); };
    m.embed_w = W(Q3VL_CK_EMBED);           m.embed_s = S(Q3VL_CK_EMBED);
    m.final_norm_w = W(Q3VL_CK_FINAL_NORM); m.final_norm_s = S(Q3VL_CK_FINAL_NORM);
    m.attn_norm_w = W(Q3VL_CK_ATTN_NORM);   m.attn_norm_s = S(Q3VL_CK_ATTN_NORM);
    m.mlp_norm_w = W(Q3VL_CK_MLP_NORM);     m.mlp_norm_s = S(Q3VL_CK_MLP_NORM);
    m.q_norm_w = W(Q3VL_CK_Q_NORM);         m.q_norm_s = S(Q3VL_CK_Q_NORM);
    m.k_norm_w = W(Q3VL_CK_K_NORM);         m.k_norm_s = S(Q3VL_CK_K_NORM);
    m.wq = W(Q3VL_CK_Q); m.sq = S(Q3VL_CK_Q);
    m.wk = W(Q3VL_CK_K); m.sk = S(Q3VL_CK_K);
    m.wv = W(Q3VL_CK_V); m.sv = S(Q3VL_CK_V);
    m.wo = W(Q3VL_CK_O); m.so = S(Q3VL_CK_O);
    m.wg = W(Q3VL_CK_GATE); m.sg = S(Q3VL_CK_GATE);
    m.wu = W(Q3VL_CK_UP);   m.su = S(Q3VL_CK_UP);
    m.wd = W(Q3VL_CK_DOWN); m.sd = S(Q3VL_CK_DOWN);
    m.rope_cos = reinterpret_cast<const float *>(d + cos_at);
    m.rope_sin = reinterpret_cast<const float *>(d + sin_at);
    if ((rc = check_model(&m))) {
        (void)hipFree(ck->dev);
        delete ck;
        return rc;
    }
    *out = ck;
    return Q3VL_OK;
}

const q3vl_text_model *q3vl_checkpoint_text_model(const q3vl_checkpoint *ck) {
    return ck ? &ck->model : nullptr;
}

int q3vl_checkpoint_header_of(const q3vl_checkpoint *ck, q3vl_checkpoint_header *hdr) {
    if (!ck || !hdr) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null checkpoint / header");
    *hdr = ck->hdr;
    return Q3VL_OK;
}

void q3vl_checkpoint_free(q3vl_checkpoint *ck) {
    if (!ck) return;
    int cur = 0;
    const bool switched = hipGetDevice(&cur) == hipSuccess && cur != ck->device &&
                          hipSetDevice(ck->device) == hipSuccess;
    (void)hipDeviceSynchronize();
    (void)hipFree(ck->dev);
    if (switched) (void)hipSetDevice(cur);
    delete ck;
}

int q3vl_quantize_groupwise(const float *x, size_t count, size_t group, int8_t *q, float *scales,
                            q3vl_stream stream) {
    if (!x || !q || !scales) return fail(Q3VL_ERR_INVALID_ARGUMENT, "null pointer");
    if (!group || count % group)
        return fail(Q3VL_ERR_INVALID_ARGUMENT, "count %zu is not a multiple of group %zu", count, group);
    if (group > (size_t)INT32_MAX) return fail(Q3VL_ERR_UNSUPPORTED, "group %zu too large", group);
    Q3VL_HIP(launch_quantize_export(x, count, group, q, scales, reinterpret_cast<hipStream_t>(stream)),
             "quantize_export");
    return Q3VL_OK;
}

}  // extern "C"
