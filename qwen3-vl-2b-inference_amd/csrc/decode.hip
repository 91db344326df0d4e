// decode.hip -- support kernels of the text decode step that calls the int8
// path (model/src/forward.cpp:458-720), gfx950.
//
// Every floating-point step follows the reference's order, including the
// orders its compiler picks for `omp simd` reductions on 8-wide AVX2: the
// RMS sums of squares and the scores of the last partial block of 8
// positions use 8 FMA lane chains folded left to right, the softmax sums 8
// float lanes then adds them in double, and the value-weighted sum is one
// FMA chain over positions per output element. The decode step is therefore
// bit-exact with the CPU oracle in its fp16-cache mode.
#include <float.h>

#include <type_traits>

#include "q3vl_device.hpp"
#include "q3vl_kernels.hpp"

namespace q3vl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ helpers
// layers/include/simd_utils.hpp:7-47 exp256_ps, one lane (2^n is -inf for
// n = -128, as in the reference).
__device__ __forceinline__ float exp256(float x) {
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
    return y * __uint_as_float((uint32_t)(n + 127) << 23);
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// fp32 -> fp16 bits, round to nearest even (NaN -> sign | 0x7E00), as one
// v_cvt_f16_f32 on the fp32 value. A plain (_Float16) conversion lets the
// compiler fuse it with the fmaf that produced the value (v_fma_mixlo_f16
// rounds the exact result once, straight to fp16), which differs from the
// reference's fp32 result rounded to fp16 whenever that result lies exactly
// halfway between two fp16 values; the asm keeps the conversion on its own.
// It equals the integer rounding (sign, rebiased exponent, 13 dropped
// mantissa bits rounded half to even, subnormals below 2^-14, overflow from
// 65520 on) for all 2^32 inputs, checked exhaustively on the device.
__device__ __forceinline__ uint16_t f2h(float f) {
    uint32_t h;
    asm("v_cvt_f16_f32 %0, %1" : "=v"(h) : "v"(f));
    return (uint16_t)h;
}

// s_waitcnt lgkmcnt(0) alone. A batch of 16 LDS reads issued behind another
// 16 exceeds what the 4-bit lgkm counter can tell apart, so the compiler's
// own wait before the first batch's use would also wait for most of the
// second; waiting for the first batch before issuing the second avoids that.
__device__ __forceinline__ void lgkm_wait0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Sixteen chain steps acc = fma(p_c of lane k of this row of 16 lanes,
// v[k - k0].c, acc) for k = k0 .. k0+3 (k0 a multiple of 4), c = 0..3:
// v_fmac_f32 with the DPP row_newbcast:k operand, one instruction per step
// (the row broadcast replaces an LDS read of p per step). One asm block
// holds the sixteen steps, so no wait states are placed between them; the
// caller keeps 2 instructions between a VALU write of p and its first use.
#define Q3VL_F4(K, V0, V1, V2, V3)                                  \
    "v_fmac_f32_dpp %0, %1, " V0 " row_newbcast:" #K " row_mask:0xf bank_mask:0xf\n\t" \
    "v_fmac_f32_dpp %0, %2, " V1 " row_newbcast:" #K " row_mask:0xf bank_mask:0xf\n\t" \
    "v_fmac_f32_dpp %0, %3, " V2 " row_newbcast:" #K " row_mask:0xf bank_mask:0xf\n\t" \
    "v_fmac_f32_dpp %0, %4, " V3 " row_newbcast:" #K " row_mask:0xf bank_mask:0xf\n\t"
#define Q3VL_FMAC16_BC(K0, K1, K2, K3)                                                        \
    case K0:                                                                                 \
        asm volatile(Q3VL_F4(K0, "%5", "%6", "%7", "%8") Q3VL_F4(K1, "%9", "%10", "%11", "%12") \
                         Q3VL_F4(K2, "%13", "%14", "%15", "%16")                              \
                             Q3VL_F4(K3, "%17", "%18", "%19", "%20")                          \
                     : "+v"(acc)                                                              \
                     : "v"(p0), "v"(p1), "v"(p2), "v"(p3), "v"(v[0].x), "v"(v[0].y),         \
                       "v"(v[0].z), "v"(v[0].w), "v"(v[1].x), "v"(v[1].y), "v"(v[1].z),       \
                       "v"(v[1].w), "v"(v[2].x), "v"(v[2].y), "v"(v[2].z), "v"(v[2].w),       \
                       "v"(v[3].x), "v"(v[3].y), "v"(v[3].z), "v"(v[3].w));                   \
        break;
__device__ __forceinline__ void fmac16_row_bcast(float &acc, float p0, float p1, float p2, float p3,
                                                 const float4 *v, int k) {
    switch (k) {
        Q3VL_FMAC16_BC(0, 1, 2, 3) Q3VL_FMAC16_BC(4, 5, 6, 7)
        Q3VL_FMAC16_BC(8, 9, 10, 11) Q3VL_FMAC16_BC(12, 13, 14, 15)
    }
}
#undef Q3VL_FMAC16_BC
#undef Q3VL_F4

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Maximum over the 64 lanes (fmaxf, so NaN lanes drop out), wave-uniform:
// quad swaps, then the mirror inside 8 and 16 lanes (each lane ends with the
// maximum of its row of 16), then the four rows' lane 0.
__device__ __forceinline__ float wave_max(float v) {
#define Q3VL_DPPM(x, ctrl) \
    __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), ctrl, 0xF, 0xF, false))
    v = fmaxf(v, Q3VL_DPPM(v, 0xB1));   // quad_perm [1,0,3,2]
    v = fmaxf(v, Q3VL_DPPM(v, 0x4E));   // quad_perm [2,3,0,1]
    v = fmaxf(v, Q3VL_DPPM(v, 0x141));  // row_half_mirror
    v = fmaxf(v, Q3VL_DPPM(v, 0x140));  // row_mirror
#undef Q3VL_DPPM
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// Minimum over the 64 lanes, wave-uniform (the same moves as wave_max).
__device__ __forceinline__ float wave_min(float v) {
#define Q3VL_DPPM(x, ctrl) \
    __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), ctrl, 0xF, 0xF, false))
    v = fminf(v, Q3VL_DPPM(v, 0xB1));
    v = fminf(v, Q3VL_DPPM(v, 0x4E));
    v = fminf(v, Q3VL_DPPM(v, 0x141));
    v = fminf(v, Q3VL_DPPM(v, 0x140));
#undef Q3VL_DPPM
    return fminf(fminf(readlane_f(v, 0), readlane_f(v, 16)), fminf(readlane_f(v, 32), readlane_f(v, 48)));
}

// Left-to-right fold of the 8 lane accumulators held by lanes 0..7:
// ((c0 + c1) + c2) + ... + c7; wave-uniform result.
__device__ __forceinline__ float fold8_lanes(float c) {
    float s = readlane_f(c, 0);
#pragma unroll
    for (int l = 1; l < 8; ++l) s = s + readlane_f(c, l);
    return s;
}

// Sum of squares of a 128-vector held by one wave as (lo = x[lane],
// hi = x[lane + 64]) in the reference's order (text_layer.cpp:247-250 as
// compiled): chain c = lane & 7 takes x[c], x[c+8], ..., x[c+120] with one
// FMA each -- lo of lanes c, c+8, ..., c+56, then hi of the same lanes --
// and the 8 chains are folded left to right.
__device__ __forceinline__ float wave_sumsq128(float lo, float hi) {
    const int c = __lane_id() & 7;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float v = __shfl(lo, c + 8 * k);
        acc = fmaf(v, v, acc);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float v = __shfl(hi, c + 8 * k);
        acc = fmaf(v, v, acc);
    }
    return fold8_lanes(acc);
}

// layers/src/text_layer.cpp:240-270 (int8 group weight, in place) on one
// head of 128 held by a wave, then RoPE (text_layer.cpp:712-760) with the
// pair (x[i], x[i+64]) in one lane. The lane's inputs are loaded beforehand
// (NormRopeIn) so that their loads can be issued ahead of larger ones.
struct NormRopeIn {
    float lo, hi;  // x[lane], x[lane + 64]
    int wl, wh;    // int8 norm weights of the two elements (converted at use)
    float sl, sh;  // their group scales
    float c, s;    // rope cos / sin at (pos, lane)
};

__device__ __forceinline__ void norm_rope128(const NormRopeIn &in, float eps, float &lo, float &hi) {
    // opaque copies: keeps the int8 -> float conversions (and their waits)
    // here rather than next to the loads
    int wl = in.wl, wh = in.wh;
    asm volatile("" : "+v"(wl), "+v"(wh));
    const float ss = wave_sumsq128(in.lo, in.hi);
    const float inv = rcp_rn(sqrt_rn(ss * (1.0f / 128.0f) + eps));  // 1.0f / sqrtf(...)
    const float a = (float)wl * ((in.sl * inv) * in.lo);
    const float b = (float)wh * ((in.sh * inv) * in.hi);
    lo = fmaf(a, in.c, -(b * in.s));
    hi = fmaf(a, in.s, b * in.c);
}

// ----------------------------------------------------------------- embedding
// layers/src/text_layer.cpp:3-49, int8 group-quantized table. A token outside
// [0, vocab) gives a NaN row instead of a read outside the table.
__global__ __launch_bounds__(256) void embed_kernel(const int8_t *w, const float *s,
                                                    const int32_t *token, float *x, int H,
                                                    int gs, int vocab) {
    const int tok = *token;
    const bool ok = tok >= 0 && tok < vocab;
    const size_t base = (size_t)(ok ? tok : 0) * H;
    for (int i = threadIdx.x + blockIdx.x * blockDim.x; i < H; i += blockDim.x * gridDim.x)
        x[i] = ok ? (float)w[base + i] * s[(base + i) / gs] : __builtin_nanf("");
}

// --------------------------------------------------------------- attention
// Two kernels per layer. Their blocks are numbered kv head first (blockIdx.x
// = kv head), so with 8 kv heads every block of one kv head sits on the same
// XCD (workgroups go round-robin over the 8 XCDs) and the scores one kernel
// writes are read back from that XCD's L2.
//
// A: per (kv head, chunk of ATT_CH positions), one wave per query head of the
// group. The waves normalize + rotate their query heads (q RMSNorm + RoPE,
// forward.cpp:531-545); the chunk holding `pos` also normalizes + rotates the
// new key and stores it and the new value as fp16 at pos (forward.cpp:
// 548-562). Scores follow text_layer.cpp:598-620 exactly: 8 FMA lane chains
// over the head dimension, the fixed tree (the left-to-right fold for the
// positions of the last partial block of 8), times 1/sqrt(hd).
//
// PAR (the chunked order, Q3VL_ATTN_CHUNKED; no counterpart in the
// reference, whose softmax and value sum run over all positions in one
// order): the block also forms its chunk's share of the softmax and of the
// value sum, per query head h and chunk c (positions t of the chunk, t < n):
//   m_c = max of the chunk's scores,
//   e_t = exp256(s_t - m_c)  (0 for s_t = -inf or m_c not finite),
//   l_c = the e_t of the 64 lanes (0 past the context) summed by the xor
//         butterfly, offsets 32, 16, 8, 4, 2, 1 (each lane adds the partner
//         lane's value to its own),
//   o_c[d] = fma chain over the chunk's t ascending of e_t * v_t[d];
// attn_combine_kernel folds the chunks. A value chain is then at most 64
// steps instead of pos + 1.
constexpr int ATT_CH = 64;
constexpr int ATT_HD = 128;
constexpr int ATT_KSTR = ATT_HD + 8;  // halves per LDS key row (272 B: bank-spread)
constexpr int ATT_THREADS = 256;
constexpr int ATT_KITEMS = ATT_CH * (ATT_HD / 8) / ATT_THREADS;  // 16-byte key pieces per thread

// The attention kernels take what their entry loads need as leading plain
// arguments (the position pointer first), which the dispatcher preloads into
// scalar registers: the position's load then waits for no argument fetch.
// The rest is read from the AttnArgs copy after them.
template <bool PAR>
__global__ __launch_bounds__(ATT_THREADS) void attn_scores_kernel(
    const int32_t *pos_p, uint16_t *k_cache_p, const float *q_p, const float *k_p,
    const int8_t *qnorm_w_p, int layer_p, int heads_p, int kv_heads_p, int max_seq_p, AttnArgs args) {
    AttnArgs a = args;
    a.pos = pos_p;
    a.k_cache = k_cache_p;
    a.q = q_p;
    a.k = k_p;
    a.qnorm_w = qnorm_w_p;
    a.layer = layer_p;
    a.heads = heads_p;
    a.kv_heads = kv_heads_p;
    a.max_seq = max_seq_p;
    __shared__ __align__(16) float qsh[3][ATT_HD];
    __shared__ uint16_t ksh[ATT_CH * ATT_KSTR];
    __shared__ __align__(16) uint16_t vnew[PAR ? ATT_HD : 1];
    __shared__ __align__(16) uint32_t vsh[PAR ? ATT_CH / 2 * ATT_HD : 1];  // [t/2][d]: (v_2r[d], v_2r+1[d])
    __shared__ __align__(16) float esh[PAR ? 3 : 1][ATT_CH];
    const int kvh = blockIdx.x, ch = blockIdx.y;
    const int kvm = a.heads / a.kv_heads;
    const int S = a.max_seq;
    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    const int t0 = ch * ATT_CH;
    const size_t lay = ((size_t)a.layer * a.kv_heads + kvh) * S * ATT_HD;
    uint16_t *kc = a.k_cache + lay;
    uint16_t *vc = a.v_cache + lay;
    const bool q_wave = wid < kvm, k_wave = wid == kvm;

    // Loads that need no `pos` go out first, so that their latency overlaps
    // that of `pos` itself: the norm inputs of the query heads (and of the
    // new key and value), then the key tile (and the value tile) with rows
    // clamped into the cache -- rows at or past the context are replaced
    // when staged. vmcnt retires in order, so the norms wait only for their
    // own loads.
    // (the position's scalar load goes first: vector loads can wait at
    // issue for queue room, and it must not wait behind them)
    const int pos = *a.pos;
    __builtin_amdgcn_sched_barrier(0);
    NormRopeIn nri{};
    float vlo = 0.0f, vhi = 0.0f;
    if (q_wave || k_wave) {
        const float *x = q_wave ? a.q + (kvh * kvm + wid) * ATT_HD : a.k + kvh * ATT_HD;
        const int8_t *w = q_wave ? a.qnorm_w : a.knorm_w;
        const float *ws = q_wave ? a.qnorm_s : a.knorm_s;
        nri.lo = x[lane];
        nri.hi = x[lane + 64];
        nri.wl = w[lane];
        nri.wh = w[lane + 64];
        nri.sl = ws[lane / a.gs];
        nri.sh = ws[(lane + 64) / a.gs];
        if (k_wave) {
            vlo = a.v[kvh * ATT_HD + lane];
            vhi = a.v[kvh * ATT_HD + 64 + lane];
        }
    }
    u32x4 kr[ATT_KITEMS];
#pragma unroll
    for (int it = 0; it < ATT_KITEMS; ++it) {
        const int idx = it * ATT_THREADS + tid, r = idx >> 4, c8 = idx & 15;
        kr[it] = *reinterpret_cast<const u32x4 *>(kc + (size_t)min(t0 + r, S - 1) * ATT_HD + c8 * 8);
    }
    // PAR: the value tile, by row pairs -- piece it of thread tid is pair
    // rp = (it*256 + tid) / 16, dims 8 * (tid % 16) .. + 7 of both rows
    constexpr int VIT = PAR ? ATT_CH / 2 * (ATT_HD / 8) / ATT_THREADS : 1;
    u32x4 vr[VIT][2];
    if constexpr (PAR) {
#pragma unroll
        for (int it = 0; it < VIT; ++it) {
            const int idx = it * ATT_THREADS + tid, rp = idx >> 4, c8 = idx & 15;
#pragma unroll
            for (int o = 0; o < 2; ++o)
                vr[it][o] = *reinterpret_cast<const u32x4 *>(vc + (size_t)min(t0 + 2 * rp + o, S - 1) * ATT_HD + c8 * 8);
        }
    }

    if (pos < 0 || pos >= S) return;  // no cache row for it: nothing is touched
    const int n = pos + 1;
    if (t0 >= n) return;  // uniform: chunk past the context
    const bool own_pos = pos >= t0 && pos < t0 + ATT_CH;
    const bool nr_q = q_wave, nr_k = k_wave && own_pos;
    if (nr_q || nr_k) {  // the rope row of pos
        nri.c = a.rope_cos[(size_t)pos * (ATT_HD / 2) + lane];
        nri.s = a.rope_sin[(size_t)pos * (ATT_HD / 2) + lane];
    }
    __builtin_amdgcn_sched_barrier(0);

    if (nr_q) {
        float lo, hi;
        norm_rope128(nri, a.eps, lo, hi);
        qsh[wid][lane] = lo;
        qsh[wid][lane + 64] = hi;
    } else if (nr_k) {
        float lo, hi;
        norm_rope128(nri, a.eps, lo, hi);
        const uint16_t l16 = f2h(lo), h16 = f2h(hi);
        kc[(size_t)pos * ATT_HD + lane] = l16;
        kc[(size_t)pos * ATT_HD + 64 + lane] = h16;
        // row pos of the key tile, written here (the staging below skips it)
        ksh[(pos - t0) * ATT_KSTR + lane] = l16;
        ksh[(pos - t0) * ATT_KSTR + 64 + lane] = h16;
        const uint16_t vl16 = f2h(vlo), vh16 = f2h(vhi);
        vc[(size_t)pos * ATT_HD + lane] = vl16;
        vc[(size_t)pos * ATT_HD + 64 + lane] = vh16;
        if constexpr (PAR) {
            vnew[lane] = vl16;
            vnew[lane + 64] = vh16;
        }
    }
#pragma unroll
    for (int it = 0; it < ATT_KITEMS; ++it) {
        const int idx = it * ATT_THREADS + tid, r = idx >> 4, c8 = idx & 15;
        const int t = t0 + r;
        u32x4 v = kr[it];
        if (t >= n) v = (u32x4){0u, 0u, 0u, 0u};
        if (t != pos) *reinterpret_cast<u32x4 *>(ksh + r * ATT_KSTR + c8 * 8) = v;
    }
    if constexpr (PAR) {
        lds_barrier();  // vnew
        // pairs (v_2rp[d], v_2rp+1[d]); rows past the context as zeros, row
        // pos from vnew
#pragma unroll
        for (int it = 0; it < VIT; ++it) {
            const int idx = it * ATT_THREADS + tid, rp = idx >> 4, c8 = idx & 15;
            u32x4 rw[2];
#pragma unroll
            for (int o = 0; o < 2; ++o) {
                const int t = t0 + 2 * rp + o;
                rw[o] = vr[it][o];
                if (t >= n) rw[o] = (u32x4){0u, 0u, 0u, 0u};
                else if (t == pos) rw[o] = *reinterpret_cast<const u32x4 *>(vnew + c8 * 8);
            }
            const uint32_t l4[4] = {rw[0].x, rw[0].y, rw[0].z, rw[0].w};
            const uint32_t h4[4] = {rw[1].x, rw[1].y, rw[1].z, rw[1].w};
            uint32_t w[8];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                w[2 * k] = __builtin_amdgcn_perm(h4[k], l4[k], 0x05040100u);      // dim 2k
                w[2 * k + 1] = __builtin_amdgcn_perm(h4[k], l4[k], 0x07060302u);  // dim 2k+1
            }
            uint32_t *dst = vsh + rp * ATT_HD + c8 * 8;
            *reinterpret_cast<u32x4 *>(dst) = (u32x4){w[0], w[1], w[2], w[3]};
            *reinterpret_cast<u32x4 *>(dst + 4) = (u32x4){w[4], w[5], w[6], w[7]};
        }
    }
    lds_barrier();  // ksh, qsh, vsh
    if (wid < kvm) {
    const int h = kvh * kvm + wid;
    const int t = t0 + lane;
    const int rows = min(ATT_CH, n - t0);
    float score = -INFINITY;
    if (lane < rows) {
        // 8 lane chains over the 128 dims (chain l takes dims i + l), in
        // batches of 32 dims: a batch's key words and query values (12 LDS
        // reads, within what the lgkm counter tells apart) are issued before
        // the previous batch's 32 FMAs, two register sets used in turn
        float cc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        const uint16_t *kr2 = ksh + lane * ATT_KSTR;
        const float4 *q4 = reinterpret_cast<const float4 *>(qsh[wid]);
        u32x4 KA[4], KB[4];
        float4 QA[8], QB[8];
        auto ld = [&](u32x4 *K, float4 *Q, int i0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) K[u] = *reinterpret_cast<const u32x4 *>(kr2 + i0 + 8 * u);
#pragma unroll
            for (int u = 0; u < 8; ++u) Q[u] = q4[i0 / 4 + u];
        };
        // the chains pass through an empty asm before and after each batch:
        // otherwise instruction selection, which keeps plain arithmetic in
        // no order against the waits, gathers the FMAs of the later batches
        // behind the last reads and every batch's read latency is waited out
        auto pin = [&]() {
            asm volatile("" : "+v"(cc[0]), "+v"(cc[1]), "+v"(cc[2]), "+v"(cc[3]),
                              "+v"(cc[4]), "+v"(cc[5]), "+v"(cc[6]), "+v"(cc[7]));
        };
        auto run = [&](const u32x4 *K, const float4 *Q) {
            pin();
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t kw[4] = {K[u].x, K[u].y, K[u].z, K[u].w};
                const float qv[8] = {Q[2 * u].x, Q[2 * u].y, Q[2 * u].z, Q[2 * u].w,
                                     Q[2 * u + 1].x, Q[2 * u + 1].y, Q[2 * u + 1].z, Q[2 * u + 1].w};
#pragma unroll
                for (int l = 0; l < 8; ++l) {
                    const uint16_t hb = (uint16_t)(kw[l >> 1] >> (16 * (l & 1)));
                    cc[l] = fmaf(qv[l], h2f(hb), cc[l]);
                }
            }
            pin();
        };
        ld(KA, QA, 0);
#pragma unroll
        for (int b = 0; b < 4; b += 2) {
            lgkm_wait0();
            __builtin_amdgcn_sched_barrier(0);
            ld(KB, QB, 32 * (b + 1));
            run(KA, QA);
            __builtin_amdgcn_sched_barrier(0);
            lgkm_wait0();
            __builtin_amdgcn_sched_barrier(0);
            if (b + 2 < 4) ld(KA, QA, 32 * (b + 2));
            run(KB, QB);
            __builtin_amdgcn_sched_barrier(0);
        }
        float dot;
        if (t >= (pos & ~7)) {  // text_layer.cpp:626-633: lanes folded left to right
            dot = cc[0];
#pragma unroll
            for (int l = 1; l < 8; ++l) dot = dot + cc[l];
        } else {                // text_layer.cpp:598-620: the fixed tree
            dot = tree8(cc[0], cc[1], cc[2], cc[3], cc[4], cc[5], cc[6], cc[7]);
        }
        score = dot * a.inv_sqrt_d;
        a.scores[(size_t)h * a.max_seq + t] = score;
    }
    const float m = wave_max(score);
    if (lane == 0) a.cmax[h * a.max_chunks + ch] = m;
    if constexpr (PAR) {
        const float e = (lane < rows && score > -INFINITY && __builtin_isfinite(m)) ? exp256(score - m) : 0.0f;
        esh[wid][lane] = e;
        float l = e;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) l = l + __shfl_xor(l, off);
        // the chunk's smallest score above -inf (+inf if none): the fold
        // zeroes the head when exp256(min_c - M) is -inf, as the reference's
        // softmax does when any of its terms is
        const float mn = wave_min(lane < rows && score > -INFINITY ? score : INFINITY);
        if (lane == 0)
            *reinterpret_cast<float4 *>(a.part_ml + ((size_t)h * a.max_chunks + ch) * 4) = make_float4(m, l, mn, 0.0f);
    }
    }
    if constexpr (PAR) {
        lds_barrier();  // esh
        // the chunk's value chains: thread tid runs query head tid / 128 of
        // the group at dim tid % 128; with three query heads per kv head,
        // threads below 128 also run head 2 at the same dim
        const int dA = tid & (ATT_HD - 1), hA = tid >> 7;
        const bool runA = hA < kvm, runB = kvm == 3 && tid < ATT_HD;
        const int rows4 = (min(ATT_CH, n - t0) + 3) & ~3;  // e and V are zero past the context
        float accA = 0.0f, accB = 0.0f;
        if (runA) {
            const float *eA = esh[min(hA, kvm - 1)], *eB = esh[min(2, kvm - 1)];
            for (int t = 0; t < rows4; t += 4) {
                const float4 pa = *reinterpret_cast<const float4 *>(eA + t);
                const uint32_t v01 = vsh[(t / 2) * ATT_HD + dA], v23 = vsh[(t / 2 + 1) * ATT_HD + dA];
                const float v0 = h2f((uint16_t)(v01 & 0xFFFFu)), v1 = h2f((uint16_t)(v01 >> 16));
                const float v2 = h2f((uint16_t)(v23 & 0xFFFFu)), v3 = h2f((uint16_t)(v23 >> 16));
                accA = fmaf(pa.x, v0, accA);
                accA = fmaf(pa.y, v1, accA);
                accA = fmaf(pa.z, v2, accA);
                accA = fmaf(pa.w, v3, accA);
                if (runB) {
                    const float4 pb = *reinterpret_cast<const float4 *>(eB + t);
                    accB = fmaf(pb.x, v0, accB);
                    accB = fmaf(pb.y, v1, accB);
                    accB = fmaf(pb.z, v2, accB);
                    accB = fmaf(pb.w, v3, accB);
                }
            }
            a.part_o[((size_t)(kvh * kvm + hA) * a.max_chunks + ch) * ATT_HD + dA] = accA;
            if (runB) a.part_o[((size_t)(kvh * kvm + 2) * a.max_chunks + ch) * ATT_HD + dA] = accB;
        }
    }
}

// The chunked order's fold (PAR above), per query head h and dim d, chunks
// c ascending:
//   M = max_c m_c, w_c = exp256(m_c - M) (0 for m_c = -inf or M not finite),
//   L = fma chain of w_c * l_c, O[d] = fma chain of w_c * o_c[d],
//   out[d] = O[d] * (1.0f / L), or 0 where L is not finite and positive,
//   and 0 for the whole head when M is finite and exp256(min_c - M) is -inf
//   for some chunk (min_c its smallest score above -inf): then the
//   reference's exp256(s_t - M) is -inf for that score (exp256 is -inf on a
//   whole half-line and fl(s - M) is monotone in s), its sum is not finite
//   and it zeroes the head (text_layer.cpp:512-515).
// One block of 128 threads per query head. Every load is issued before the
// values it feeds are needed: the (m_c, l_c, min_c) of all chunks go to LDS
// in one pass (one chunk per thread), the o_c[d] in batches of 16.
constexpr int ATT_MAX_CHUNKS = 256;  // max_seq <= 16384
__global__ __launch_bounds__(ATT_HD) void attn_combine_kernel(
    const int32_t *pos_p, const float *part_ml_p, const float *part_o_p, int max_chunks_p, int max_seq_p,
    AttnArgs args) {
    AttnArgs a = args;  // leading arguments preloaded, as in the kernels above
    a.pos = pos_p;
    a.part_ml = const_cast<float *>(part_ml_p);
    a.part_o = const_cast<float *>(part_o_p);
    a.max_chunks = max_chunks_p;
    a.max_seq = max_seq_p;
    __shared__ float wsh[ATT_MAX_CHUNKS], lsh[ATT_MAX_CHUNKS], msh[ATT_MAX_CHUNKS], nsh[ATT_MAX_CHUNKS];
    __shared__ float mred[2];
    const int h = blockIdx.x, d = threadIdx.x, lane = d & 63;
    const float *ml = a.part_ml + (size_t)h * a.max_chunks * 4;
    const float *po = a.part_o + (size_t)h * a.max_chunks * ATT_HD + d;
    // the first chunks' partials go out before `pos` is known (indices
    // clamped into the buffers; chunks past the context are not used)
    const float4 ml0 = *reinterpret_cast<const float4 *>(ml + 4 * min(d, a.max_chunks - 1));
    float ob[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) ob[i] = po[(size_t)min(i, a.max_chunks - 1) * ATT_HD];
    const int pos = *a.pos;
    if (pos < 0 || pos >= a.max_seq) {  // no cache row for it: NaN outputs
        a.out[h * ATT_HD + d] = __builtin_nanf("");
        return;
    }
    const int nch = (pos + ATT_CH) / ATT_CH;
    float m = -INFINITY;
    if (d < nch) {
        msh[d] = ml0.x;
        lsh[d] = ml0.y;
        nsh[d] = ml0.z;
        m = ml0.x;
    }
    for (int c = d + ATT_HD; c < nch; c += ATT_HD) {
        const float4 v = *reinterpret_cast<const float4 *>(ml + 4 * c);
        msh[c] = v.x;
        lsh[c] = v.y;
        nsh[c] = v.z;
        m = fmaxf(m, v.x);
    }
    // M: the max of the m_c (a max is the same in any order: DPP moves
    // instead of wave shuffles, which are LDS round trips)
    m = wave_max(m);
    if (lane == 0) mred[d >> 6] = m;
    __syncthreads();
    const float M = fmaxf(mred[0], mred[1]);
    const bool fin = __builtin_isfinite(M);
    int vanish = 0;  // some score's exp256(s - M) is -inf
    for (int c = d; c < nch; c += ATT_HD) {
        const float mc = msh[c], mn = nsh[c];
        wsh[c] = (fin && mc > -INFINITY) ? exp256(mc - M) : 0.0f;
        if (fin && mn < INFINITY && exp256(mn - M) == -INFINITY) vanish = 1;
    }
    if (__syncthreads_or(vanish)) {
        a.out[h * ATT_HD + d] = 0.0f;
        return;
    }
    float L = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += 16) {
        float nb[16];
        const bool more = c0 + 16 < nch;  // uniform
        if (more) {
#pragma unroll
            for (int i = 0; i < 16; ++i) nb[i] = po[(size_t)min(c0 + 16 + i, nch - 1) * ATT_HD];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if (c0 + i < nch) {  // uniform
                const float w = wsh[c0 + i];
                L = fmaf(w, lsh[c0 + i], L);
                O = fmaf(w, ob[i], O);
            }
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < 16; ++i) ob[i] = nb[i];
        }
    }
    const bool ok = L > 0.0f && __builtin_isfinite(L);
    a.out[h * ATT_HD + d] = ok ? O * (1.0f / L) : 0.0f;
}

// B: softmax (text_layer.cpp:436-535) and the value-weighted sum
// (text_layer.cpp:655-710) in the reference's order. Block (kv head kvh,
// slice db) serves the kvm query heads of kvh and the PV_D output dims
// [db*PV_D, db*PV_D + PV_D). Per head:
//   M = max of the scores (exact: the scores kernel's chunk maxima),
//   e_t = exp256(s_t - M) (0 for s_t = -inf),
//   sum = double(l_0) + ... + double(l_7) + e_nb + ... + e_pos (in double),
//     l_j = sequential fp32 sum of e_t over t = j (mod 8), t < nb = n/8*8,
//   p_t = e_t * (float)(1/sum)   (all zero if M or sum is not finite/positive),
//   out[d] = fma chain over t = 0..pos of p_t * v_t[d].
// The chain is inherently sequential (one dependent FMA per position), so
// everything else is arranged around it. Loads are issued at entry (the
// position first, then chunk maxima, the scores of the kvm heads and, in
// the staging waves, the first V chunk, in order of use), so the softmax runs
// while V is still arriving. The block's 8 waves (two per SIMD) share the
// e pass; waves 2, 3, 6 and 7 stage V: widened to fp32 into LDS, transposed
// ([d][t]) with 16-byte row writes of 4 positions, chunk 0 while waves 0 ..
// kvm-1 form the denominators, later chunks while the chain runs, so the
// chain wave issues no global loads. The chains read 64
// positions ahead with the reads spread between the FMAs. e also lives
// lane-major (row j holds e_j, e_{j+8}, ...), which the denominator's
// segmented sums read.
constexpr int PV_D = 16;
constexpr int PV_TC = 1024;
constexpr int PV_THREADS = 512;  // 8 waves, two per SIMD
constexpr int PV_RS = PV_TC + 4;                    // floats per LDS row of vt
// every chunk is staged by waves 2, 3, 6 and 7 (PV_QN quads a thread)
constexpr int PV_NST = PV_THREADS / 2;  // staging threads
constexpr int PV_QN = PV_TC * (PV_D / 8) / PV_NST / 4;
static_assert(4 * (PV_NST / 2) * PV_QN == PV_TC, "the staging quads cover the chunk");
// float4 score groups per head held in registers from entry (2048
// positions; later ones are loaded when n is known)
constexpr int PV_SREG = 2;

// V staging: thread (vsg, vb) of a staging group holds the 8-dim half vsg
// of the NQ quads of positions 4*(vb + QSTR*q) + i (item 4q + i) of a
// chunk, so each of its dims becomes one 16-byte LDS row write. Rows are
// clamped into the cache when loaded.
template <int NQ, int QSTR>
__device__ __forceinline__ void pv_load(u32x4 *vr, const uint16_t *vc, int t0, int S, int vsg, int vb) {
#pragma unroll
    for (int it = 0; it < 4 * NQ; ++it) {
        const int t = t0 + 4 * (vb + QSTR * (it >> 2)) + (it & 3);
        vr[it] = *reinterpret_cast<const u32x4 *>(vc + (size_t)min(t, S - 1) * ATT_HD + vsg * 8);
    }
}
// Widens the staged V to fp32 rows vt[d][t]. Rows past pos are stored as
// zeros (their steps then add exact +0, even where the row at pos holds an
// infinity); quads at or past lim (the chunk-relative end of what the chains
// read, a multiple of 64) are not stored at all. (The chunk without rows
// past pos takes a loop of its own, free of selects.)
template <int NQ, int QSTR>
__device__ __forceinline__ void pv_store(float *vt, const u32x4 *vr, int vsg, int vb, int t0, int lim, int pos) {
    auto quad = [&](int q, bool masked) {
        const int p0 = 4 * (vb + QSTR * q);
        if (p0 >= lim) return;
        float4 f[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 v = vr[4 * q + i];
            const bool past = masked && t0 + p0 + i > pos;
            const uint32_t w[4] = {past ? 0u : v.x, past ? 0u : v.y, past ? 0u : v.z, past ? 0u : v.w};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float x = h2f((uint16_t)(w[k >> 1] >> (16 * (k & 1))));
                if (i == 0) f[k].x = x;
                if (i == 1) f[k].y = x;
                if (i == 2) f[k].z = x;
                if (i == 3) f[k].w = x;
            }
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) *reinterpret_cast<float4 *>(vt + (vsg * 8 + k) * PV_RS + p0) = f[k];
    };
    if (t0 + PV_TC <= pos + 1) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) quad(q, false);
    } else {
#pragma unroll
        for (int q = 0; q < NQ; ++q) quad(q, true);
    }
}

// Lane-major e rows hold max_seq/8 terms rounded up to a multiple of 32 (the
// summing batch), plus 4 floats of padding against bank conflicts.
__host__ __device__ __forceinline__ int pv_et_stride(int max_seq) {
    return (max_seq / 8 + 31) / 32 * 32 + 4;
}

template <int KVM>
__global__ __launch_bounds__(PV_THREADS) void attn_softmax_pv_kernel(
    const int32_t *pos_p, const float *scores_p, const float *cmax_p, const uint16_t *v_cache_p,
    int layer_p, int heads_p, int kv_heads_p, int max_seq_p, int max_chunks_p, AttnArgs args) {
    AttnArgs a = args;
    a.pos = pos_p;
    a.scores = const_cast<float *>(scores_p);
    a.cmax = const_cast<float *>(cmax_p);
    a.v_cache = const_cast<uint16_t *>(v_cache_p);
    a.layer = layer_p;
    a.heads = heads_p;
    a.kv_heads = kv_heads_p;
    a.max_seq = max_seq_p;
    a.max_chunks = max_chunks_p;
    extern __shared__ __align__(16) float smem[];
    constexpr int kvm = KVM;  // query heads per kv head (a.heads / a.kv_heads)
    const int S = a.max_seq, ets = pv_et_stride(S);
    // e and et first: the chains' p reads then use small constant offsets
    float *e = smem;                        // [kvm][S]: e_t, then p_t
    float *et = e + kvm * S;                // [kvm][8][ets]
    float *vt = et + kvm * 8 * ets;         // [PV_D][PV_RS] fp32 (16-byte aligned: S % 8 == 0, ets % 4 == 0)
    __shared__ float hmax[4], hinv[4];
    const int kvh = blockIdx.x, db = blockIdx.y;
    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    const uint16_t *vc = a.v_cache + ((size_t)a.layer * a.kv_heads + kvh) * S * ATT_HD + db * PV_D;

    // ---- entry loads. The position's scalar load goes first (the vector
    // loads below can wait at issue for queue room, and it must not wait
    // behind them); the others follow in order of use, all issued before
    // `pos` is known (their latency overlaps its own). Indices are clamped
    // into the buffers; values past the context are masked once pos is
    // known.
    const int pos = *a.pos;
    __builtin_amdgcn_sched_barrier(0);
    // chunk maxima: wave hh < kvm, lane c (one pass covers 4096 positions)
    const int wh = min(wid, kvm - 1);
    const float cm = a.cmax[(kvh * kvm + wh) * a.max_chunks + min(lane, a.max_chunks - 1)];
    // scores: for head hh, thread tid holds positions 4*(ti + PV_THREADS*k)
    // + 0..3 with ti = tid on even heads and PV_THREADS-1-tid on odd ones,
    // so the float4s past a multiple of PV_THREADS fall to wave 0 on one
    // head and to the last wave on the next, and no wave computes every
    // head's tail
    float4 sreg[kvm][PV_SREG];
#pragma unroll
    for (int hh = 0; hh < kvm; ++hh) {
        const float4 *sc = reinterpret_cast<const float4 *>(a.scores + (size_t)(kvh * kvm + hh) * S);
        const int ti = (hh & 1) ? PV_THREADS - 1 - tid : tid;
#pragma unroll
        for (int k = 0; k < PV_SREG; ++k) sreg[hh][k] = sc[min(ti + PV_THREADS * k, S / 4 - 1)];
    }
    // V: waves 2, 3, 6 and 7 stage every chunk (staging thread s = 64
    // (wid & 1 | wid / 4 * 2) + lane: vsg = s & 1, vb = s >> 1, quads vb +
    // PV_NST/2 q), chunk 0 loaded here and widened into LDS while waves 0 ..
    // kvm-1 form the denominators, each later chunk loaded while the chain
    // runs on the one before, so the chain wave issues no global loads. The
    // other waves load no V. (Waves go to the CU's four SIMDs in turn, wave w
    // to SIMD w % 4: the stagers then share SIMDs 2 and 3, and the sums and
    // the chain, on SIMDs 0 and 1, share theirs with waves 4 and 5, idle by
    // then.)
    u32x4 vrn[4 * PV_QN];
    const int wu = __builtin_amdgcn_readfirstlane(wid);  // wave-uniform
    const bool stager = (wu & 2) != 0;
    const int vsg = tid & 1, vb = ((((wu & 1) | (wu >> 2) << 1)) * 64 + lane) >> 1;
    const int n = pos + 1;
    const int nb = n & ~7;
    const int nch = (n + ATT_CH - 1) / ATT_CH;
    auto chunk_lim = [&](int t0) { return (min(PV_TC, n - t0) + 63) & ~63; };

    // The position check, M and the e pass, written out once for the
    // stagers (with their V loads) and once for the other waves: the
    // compiler's wait counts at a join cover the loads of either path, so
    // one copy after a conditional V load would make the stagers' first
    // score use wait for the V transfer too. The stagers issue V after the
    // barrier that follows M, when every wave's entry loads have gone out:
    // issued at entry, V's many cache lines held the later waves' chunk
    // maxima and scores back in the CU's memory pipeline, and the barrier
    // with them. Returns false when pos has no cache row.
    float Mw = 0.0f;  // M of head wid, in waves wid < kvm
    auto front = [&](auto stg) -> bool {
        if (pos < 0 || pos >= S) {  // no cache row for it: NaN outputs
            if (wid == 0 && (lane >> 4) < kvm)
                a.out[(kvh * kvm + (lane >> 4)) * ATT_HD + db * PV_D + (lane & 15)] = __builtin_nanf("");
            return false;
        }
        // ---- M per head from the chunk maxima (beyond one pass: loop)
        if (wid < kvm) {
            const float *cmh = a.cmax + (kvh * kvm + wid) * a.max_chunks;
            float m = lane < nch ? cm : -INFINITY;  // loaded for head wh == wid
            for (int c = lane + 64; c < nch; c += 64) m = fmaxf(m, cmh[c]);
            m = wave_max(m);  // (any order: DPP moves, no LDS round trips)
            if (lane == 0) hmax[wid] = m;
            Mw = m;
        }
        lds_barrier();
        if constexpr (decltype(stg)::value) {
            __builtin_amdgcn_sched_barrier(0);
            pv_load<PV_QN, PV_NST / 2>(vrn, vc, 0, S, vsg, vb);
            __builtin_amdgcn_sched_barrier(0);
        }
        // ---- e_t (text_layer.cpp:486-493, 501-509), stored both ways,
        // computed and selected without per-position branches
#pragma unroll
        for (int hh = 0; hh < kvm; ++hh) {
            const float M = hmax[hh];
            const bool fin = __builtin_isfinite(M);
            float *eh = e + hh * S, *eth = et + hh * 8 * ets;
            auto ev_of = [&](float v) {
                const float x = exp256(v - M);
                return (fin && v > -INFINITY) ? x : 0.0f;
            };
            auto put4 = [&](int t, float4 v) {  // positions t..t+3, t % 4 == 0
                float4 ev;
                ev.x = ev_of(v.x);
                ev.y = ev_of(v.y);
                ev.z = ev_of(v.z);
                ev.w = ev_of(v.w);
                if (t < n) *reinterpret_cast<float4 *>(eh + t) = ev;  // t + 3 < S
                if (t < nb) {  // nb % 8 == 0: all four below nb
                    const int c = t >> 3, j = t & 7;
                    eth[(j + 0) * ets + c] = ev.x;
                    eth[(j + 1) * ets + c] = ev.y;
                    eth[(j + 2) * ets + c] = ev.z;
                    eth[(j + 3) * ets + c] = ev.w;
                }
            };
            // zeros after the lane sums' last term, up to a whole batch of
            // 32 per lane: adding +0 to a sum of non-negative terms is exact
            const int zend = (nb + 255) & ~255;
            for (int t = nb + tid; t < zend; t += PV_THREADS) eth[(t & 7) * ets + (t >> 3)] = 0.0f;
            // a wave skips a k with no position below n (uniform: its lowest
            // float4 index is 64*wid + PV_THREADS*k, mirrored on odd heads)
            const int ti = (hh & 1) ? PV_THREADS - 1 - tid : tid;
            const int wlo = (hh & 1) ? PV_THREADS - 64 * (wu + 1) : 64 * wu;
#pragma unroll
            for (int k = 0; k < PV_SREG; ++k)
                if (4 * (wlo + PV_THREADS * k) < n) put4(4 * (ti + PV_THREADS * k), sreg[hh][k]);
            const float4 *sc = reinterpret_cast<const float4 *>(a.scores + (size_t)(kvh * kvm + hh) * S);
            for (int i = tid + PV_THREADS * PV_SREG; 4 * i < n; i += PV_THREADS) put4(4 * i, sc[i]);
        }
        return true;
    };
    if (stager) {
        if (!front(std::true_type{})) return;
    } else {
        if (!front(std::false_type{})) return;
    }
    lds_barrier();
    // ---- sums and the fp32 inverse, one wave per head; the staging waves
    // widen V chunk 0 into LDS meanwhile. Lane sum l (the sequential fp32 sum over
    // t = l mod 8) is cut into segments of 32 terms; in a pass over 256 terms
    // lane 8l+s holds segment s of sum l in registers. Every lane adds its
    // segment's terms in each round, and a DPP row shift hands each lane's
    // value to the next segment's lane between rounds (row_ror:9 from the
    // last lane of one pass to the first of the next), so lane 8l+s carries
    // sum l through segment s in round s: the same adds in the same order as
    // one lane summing the whole row, with no LDS read between them.
    if (wid < kvm) {
        const int cnt = ((nb >> 3) + 31) & ~31;  // terms per lane sum, zero-padded
        const float *rowl = et + wid * 8 * ets + (lane >> 3) * ets + 32 * (lane & 7);
        const float *eh = e + wid * S;
        // the tail e_nb .. e_pos (at most 7), one per lane
        const float tl = lane < n - nb ? eh[nb + lane] : 0.0f;
        float acc = 0.0f;
        int last = 7;  // segment lane that ends with the sums
        for (int p0 = 0; p0 < cnt; p0 += 256) {
            const int nr = min(8, (cnt - p0) >> 5);  // segments in this pass
            // (segments past cnt read LDS words whose sums are never kept)
            float4 X[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) X[u] = reinterpret_cast<const float4 *>(rowl + p0)[u];
            if (p0 > 0)
                acc = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                          0, __builtin_bit_cast(int, acc), 0x129, 0xF, 0xF, false));
            for (int r = 0; r < nr; ++r) {
                if (r > 0)  // row_shr:1 (lane i takes lane i-1 inside each row of 16)
                    acc = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                              0, __builtin_bit_cast(int, acc), 0x111, 0xF, 0xF, false));
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    acc = acc + X[u].x;
                    acc = acc + X[u].y;
                    acc = acc + X[u].z;
                    acc = acc + X[u].w;
                }
            }
            last = nr - 1;
        }
        // the 8 lane sums, then the tail terms, in double and in order; the
        // terms are gathered first so that only the adds form the chain, and
        // all 7 tail lanes are added (0 past pos: adding +0 to the sum, never
        // -0, leaves it unchanged)
        float part[15];
#pragma unroll
        for (int l = 0; l < 8; ++l) part[l] = readlane_f(acc, 8 * l + last);  // lane sum l
#pragma unroll
        for (int l = 0; l < 7; ++l) part[8 + l] = readlane_f(tl, l);
        double sum = 0.0;
#pragma unroll
        for (int i = 0; i < 15; ++i) sum += (double)part[i];
        const bool ok = __builtin_isfinite(Mw) && sum > 0.0 && __builtin_isfinite(sum);
        const float inv = ok ? (float)(1.0 / sum) : 0.0f;
        if (lane == 0) hinv[wid] = inv;
    }
    if (stager) pv_store<PV_QN, PV_NST / 2>(vt, vrn, vsg, vb, 0, chunk_lim(0), pos);  // V chunk 0

    // ---- value-weighted sums. Wave 0 runs the chains: row r of 16 lanes is
    // query head r, lane d of the row output dim db*PV_D + d. Per batch of 64
    // positions tb..tb+63, lane k of a row holds p_{tb+4k+c} = e * inv
    // (c < 4, formed in registers; 0 past the context, which leaves the
    // chain unchanged: acc is never -0, and fma(0, v, acc) = acc for finite
    // v) and every step broadcasts one of them across the row. Only the
    // chunk's last batch can reach past the context, so only it masks p by
    // position.
    const int rl = lane & 15, hrow = min(lane >> 4, kvm - 1);
    const bool chain = wid == 0 && (lane >> 4) < kvm;
    float acc = 0.0f;
    for (int t0 = 0; t0 < n; t0 += PV_TC) {
        if (t0 > 0) {
            lds_barrier();  // previous chains done with vt
            if (stager) pv_store<PV_QN, PV_NST / 2>(vt, vrn, vsg, vb, t0, chunk_lim(t0), pos);
        }
        lds_barrier();      // vt (and inv) ready
        if (stager && t0 + PV_TC < n) pv_load<PV_QN, PV_NST / 2>(vrn, vc, t0 + PV_TC, S, vsg, vb);
        if (chain) {
            const float invh = hinv[hrow];
            const float *eph = e + hrow * S + t0;
            const float *vrow = vt + rl * PV_RS;
            const int len = min(PV_TC, n - t0);
            float4 Ae, Be, Av[16], Bv[16];
            // the LDS reads of a batch: its e (part 0) and V[k .. k+3]
            auto ldpart = [&](float4 &E, float4 *V, int tb, int k) {
                if (k == 0) E = *reinterpret_cast<const float4 *>(eph + tb + 4 * rl);
#pragma unroll
                for (int u = k; u < k + 4; ++u) V[u] = *reinterpret_cast<const float4 *>(vrow + tb + 4 * u);
            };
            // a head whose sum is not finite and positive has invh = 0 (a
            // finite positive sum is at most n, so its inverse is not 0):
            // the reference zeroes its p (text_layer.cpp:512-515), and e * 0
            // would be NaN for an e of -inf
            const bool live = invh > 0.0f;
            // pre(k) issues part k of the next batch's reads before block k
            // of 16 steps: spread over the steps, the reads enter the LDS
            // queue while the chain runs instead of holding its first step
            // back until all of them are issued
            auto run64 = [&](const float4 &E, const float4 *V, int tb, auto last_c, auto pre) {
                float p0, p1, p2, p3;
                if constexpr (decltype(last_c)::value) {
                    const int t = tb + 4 * rl;
                    p0 = live && t + 0 < len ? E.x * invh : 0.0f;
                    p1 = live && t + 1 < len ? E.y * invh : 0.0f;
                    p2 = live && t + 2 < len ? E.z * invh : 0.0f;
                    p3 = live && t + 3 < len ? E.w * invh : 0.0f;
                } else {  // every position of the batch is below len
                    p0 = live ? E.x * invh : 0.0f;
                    p1 = live ? E.y * invh : 0.0f;
                    p2 = live ? E.z * invh : 0.0f;
                    p3 = live ? E.w * invh : 0.0f;
                }
                asm volatile("s_nop 1" ::"v"(p0), "v"(p1), "v"(p2), "v"(p3));  // DPP read-after-write
#pragma unroll
                for (int k = 0; k < 16; k += 4) {
                    // the last batch stops at the first block of 16 steps
                    // wholly past the context (their p are 0: no change)
                    if (decltype(last_c)::value && tb + 4 * k >= len) break;  // uniform
                    pre(k);
                    __builtin_amdgcn_sched_barrier(0);
                    fmac16_row_bcast(acc, p0, p1, p2, p3, V + k, k);
                    __builtin_amdgcn_sched_barrier(0);
                }
            };
            const std::integral_constant<bool, false> full{};
            const std::integral_constant<bool, true> last{};
            auto none = [](int) {};
            // batches of 64 in two register sets used in turn: the next
            // batch's LDS reads go out during the current batch's steps
            // (every read of the set in use has completed before its first
            // step); batches 0 .. nbat-2 are whole, nbat-1 the last
            const int nbat = (len + 63) >> 6, nfull = nbat - 1;
#pragma unroll
            for (int k = 0; k < 16; k += 4) ldpart(Ae, Av, 0, k);
            int bi = 0;
            for (; bi + 2 <= nfull; bi += 2) {
                lgkm_wait0();
                __builtin_amdgcn_sched_barrier(0);
                run64(Ae, Av, 64 * bi, full, [&](int k) { ldpart(Be, Bv, 64 * (bi + 1), k); });
                lgkm_wait0();
                __builtin_amdgcn_sched_barrier(0);
                // bi + 2 <= nfull < nbat
                run64(Be, Bv, 64 * (bi + 1), full, [&](int k) { ldpart(Ae, Av, 64 * (bi + 2), k); });
            }
            if (bi < nfull) {  // A holds whole batch bi, the last is bi + 1
                lgkm_wait0();
                __builtin_amdgcn_sched_barrier(0);
                run64(Ae, Av, 64 * bi, full, [&](int k) { ldpart(Be, Bv, 64 * (bi + 1), k); });
                lgkm_wait0();
                __builtin_amdgcn_sched_barrier(0);
                run64(Be, Bv, 64 * (bi + 1), last, none);
            } else {  // A holds the last batch
                lgkm_wait0();
                __builtin_amdgcn_sched_barrier(0);
                run64(Ae, Av, 64 * bi, last, none);
            }
        }
    }
    if (chain) a.out[(kvh * kvm + hrow) * ATT_HD + db * PV_D + rl] = acc;
}

// ------------------------------------------------------------------ launch
hipError_t launch_embed(const int8_t *w, const float *s, const int32_t *token, float *x, int H,
                        int gs, int vocab, hipStream_t st) {
    embed_kernel<<<(H + 255) / 256, 256, 0, st>>>(w, s, token, x, H, gs, vocab);
    return hipGetLastError();
}

size_t attention_lds_bytes(int heads, int kv_heads, int max_seq) {
    const size_t kvm = (size_t)(heads / kv_heads);
    return (size_t)PV_D * PV_RS * 4 + kvm * max_seq * 4 + kvm * 8 * (size_t)pv_et_stride(max_seq) * 4;
}

template <int KVM>
static hipError_t launch_softmax_pv(const AttnArgs &a, size_t lds, hipStream_t st) {
    // raise the dynamic LDS limit once per process and instantiation
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&attn_softmax_pv_kernel<KVM>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)kAttnMaxLds);
    if (attr != hipSuccess) return attr;
    attn_softmax_pv_kernel<KVM><<<dim3(a.kv_heads, ATT_HD / PV_D), PV_THREADS, lds, st>>>(
        a.pos, a.scores, a.cmax, a.v_cache, a.layer, a.heads, a.kv_heads, a.max_seq, a.max_chunks, a);
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t st) {
    const int kvm = a.heads / a.kv_heads;
    if (a.head_dim != ATT_HD || a.heads % a.kv_heads != 0 || kvm < 1 || kvm > 3 ||
        a.max_seq % 8 != 0 || a.max_chunks * ATT_CH < a.max_seq)
        return hipErrorInvalidValue;
    const size_t lds = attention_lds_bytes(a.heads, a.kv_heads, a.max_seq);
    if (lds > kAttnMaxLds) return hipErrorInvalidValue;
    if (a.order == 1) {  // chunked order
        if (!a.part_o || !a.part_ml || a.max_chunks > ATT_MAX_CHUNKS) return hipErrorInvalidValue;
        attn_scores_kernel<true><<<dim3(a.kv_heads, a.max_chunks), ATT_THREADS, 0, st>>>(
            a.pos, a.k_cache, a.q, a.k, a.qnorm_w, a.layer, a.heads, a.kv_heads, a.max_seq, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        attn_combine_kernel<<<a.heads, ATT_HD, 0, st>>>(a.pos, a.part_ml, a.part_o, a.max_chunks,
                                                         a.max_seq, a);
        return hipGetLastError();
    }
    attn_scores_kernel<false><<<dim3(a.kv_heads, a.max_chunks), ATT_THREADS, 0, st>>>(
        a.pos, a.k_cache, a.q, a.k, a.qnorm_w, a.layer, a.heads, a.kv_heads, a.max_seq, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    switch (kvm) {
    case 1: return launch_softmax_pv<1>(a, lds, st);
    case 2: return launch_softmax_pv<2>(a, lds, st);
    default: return launch_softmax_pv<3>(a, lds, st);
    }
}

}  // namespace q3vl
