// gemm_mf.hip -- int8-weight GEMM for M > 8 at group size 64 (gfx950), with
// activations in MFMA fragment order.
//
// Reference: the general path of linear_int8_fp32s_int32acc_transpose,
// matmul/src/cpu_f32a_i8f32sb_f32c_avx2.cpp:477-662: for each output and
// each K-group g in ascending order, G = sum_{k in g} q[m,k] * w[n,k] exactly
// (int32), then acc = fma(float(G) * a_s[m,g], w_s[n,g], acc) (:613-617,
// 652; GCC contracts the multiply-add, which the golden vectors pin).
//
// Exactness. q (int16, |q| <= 1016) and w (int8) are exact in fp16, and every
// partial sum of one group is an integer below 2^24, so
// v_mfma_f32_32x32x16_f16 over the group's 64 k with a zero initial
// accumulator yields G exactly. The fp32 epilogue consumes it group by group.
//
// Data movement, from what this hardware measured (per CU: LDS reads about
// 110 B/clk, L1 about 62 B/clk, one 32x32x16 MFMA about 34 cycles; the
// epilogue's two fp32 operations per output and group cost as much VALU time
// as the MFMAs). Per-phase cycle counts showed the waves stalled at issuing
// their global loads: the vector memory path, not the MFMAs or the VALU,
// was the limit, so every operand is loaded once per block and staged into
// LDS, and the weight scales, which a per-group load fetched one cache line
// per weight row at a time, come in tiles of several groups:
// * A: the quantizer writes q in fragment order -- per 32-row m-tile t and
//   group g a 4 KB chunk [slice s][lane l][8 halves] holding
//   q[32t + l%32][64g + 32(l/32) + 8s + j]. Either (AL) wave w loads slice w
//   of each of the block's m-tiles (one coalesced 1 KB read each) and stores
//   it to LDS unchanged, every wave then reading its fragments with one
//   ds_read_b128 per slice and m-tile; or each wave loads the four slices
//   of its own m-tiles straight into its registers (the L1 path carries A,
//   LDS only B and the scales: faster wherever two or more m-tiles share a
//   block). The a_s come in the matching order: [t][g][l/32][16]
//   holds a_s of rows 32t + 8(e/4) + 4(l/32) + e%4, the rows a lane's 16
//   accumulators hold.
// * B: the block loads its weight rows (64 bytes per row and group) once,
//   widens them to fp16 (one SDWA conversion a byte) and stores them in LDS in the
//   same fragment order, two buffers deep, so every wave reads its B
//   fragments with one ds_read_b128 per slice and n-tile. The 16-byte slots
//   are swizzled (slot ^ 4*(s/2) ^ 8*(l/32)) so that the writers' and the
//   readers' 16-lane passes each hit 16 distinct bank groups.
// * w_s: every SG groups (8) the block loads the next SG scales of each of
//   its weight rows, 2 threads per row, contiguous 4 SG bytes per row, into
//   a second LDS tile slot.
// * The k order inside a group: slice s of lane half h covers k = 32h + 8s +
//   j; A and B use the same map, so each MFMA pairs matching k and the four
//   slices cover the group's 64 k once.
// * Block: 4 waves in WM x (4/WM), wave tile (32 TM) x (32 TN); two to four
//   blocks share a CU, so one block's epilogue overlaps another's MFMAs and
//   its loads another's waits. One barrier per group (an LDS-only fence).
//   WM = 1 serves M <= 32 (one m-tile): all four waves take output columns.
//   SWIGLU: the block's B rows are 32 TN gate rows and the same up rows; wave
//   wn holds gate n-tile wn and up n-tile 2 + wn, so silu(gate) * up needs no
//   exchange.
#include "q3vl_device.hpp"
#include "q3vl_kernels.hpp"

namespace q3vl {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------- fragment-order quantizer
// The reference quantizer (cpu_f32a_i8f32sb_f32c_avx2.cpp:135-177) writing q
// as fp16 in the fragment order above and a_s in its fragment order; rows
// M .. 32*Mt-1 are written as zeros. 16 lanes per (row, group): lane u loads
// the float4 of elements 4u .. 4u+3 (one coalesced 256-byte row piece per 16
// lanes). The group's sum of squares runs in the reference order in
// registers: chain 4(u & 3) + k takes elements 16t + 4(u & 3) + k, t = 0..3,
// whose step t lives in lane 4t + (u & 3), so each of four rounds extends the
// chain value of lane u - 4 (row_shr:4; 0 into lanes 0..3) and lanes 12..15
// end with the 16 chains; V[i] = P0[i] + P1[i] (lanes 12, 13 take lanes 14,
// 15: row_shl:2), lane 12 takes lane 13's half (row_shl:1), runs the fixed
// tree, and the row takes lane 12's sum (row_newbcast:12). Each lane then
// quantizes its 4 values and stores them as 8 bytes of fp16: elements 4u ..
// 4u+3 are halves 4(u & 1) .. of slice (u & 7) / 2 in lane half u / 8. A
// block takes 8 rows x 2 groups: a 128-byte line of the fragment order holds
// 16 bytes of each of 8 consecutive rows, so every line is written whole by
// one block (rows of a line spread over blocks on several XCDs would leave
// partial lines in several L2s).
__global__ __launch_bounds__(256) void quantize_frag_kernel(const float *__restrict__ A,
                                                            _Float16 *__restrict__ qf,
                                                            float *__restrict__ asf, int M, int K) {
    const int Kg = K / 64;
    const int u = threadIdx.x & 15;
    const int pair = threadIdx.x >> 4;  // row (pair & 3) + 4 (pair >> 3), group pair >> 2 & 1
    const int g = blockIdx.x * 2 + ((pair >> 2) & 1);
    const int m = blockIdx.y * 8 + (pair & 3) + 4 * (pair >> 3);
    if (g >= Kg) return;  // whole 16-lane rows leave together
    const bool real = m < M;
    float4 xv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (real) xv = reinterpret_cast<const float4 *>(A + (size_t)m * K + (size_t)g * 64)[u];
#define Q3VL_DPPF(v, ctrl) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false))
    float c0 = fmaf(xv.x, xv.x, 0.0f), c1 = fmaf(xv.y, xv.y, 0.0f);
    float c2 = fmaf(xv.z, xv.z, 0.0f), c3 = fmaf(xv.w, xv.w, 0.0f);
#pragma unroll
    for (int t = 1; t < 4; ++t) {
        c0 = fmaf(xv.x, xv.x, Q3VL_DPPF(c0, 0x114));
        c1 = fmaf(xv.y, xv.y, Q3VL_DPPF(c1, 0x114));
        c2 = fmaf(xv.z, xv.z, Q3VL_DPPF(c2, 0x114));
        c3 = fmaf(xv.w, xv.w, Q3VL_DPPF(c3, 0x114));
    }
    const float v0 = c0 + Q3VL_DPPF(c0, 0x102), v1 = c1 + Q3VL_DPPF(c1, 0x102);
    const float v2 = c2 + Q3VL_DPPF(c2, 0x102), v3 = c3 + Q3VL_DPPF(c3, 0x102);
    const float w0 = Q3VL_DPPF(v0, 0x101), w1 = Q3VL_DPPF(v1, 0x101);
    const float w2 = Q3VL_DPPF(v2, 0x101), w3 = Q3VL_DPPF(v3, 0x101);
    const float sumsq = Q3VL_DPPF(tree8(v0, v1, v2, v3, w0, w1, w2, w3), 0x15C);
#undef Q3VL_DPPF
    const float s = group_scale(sumsq, 1.0f / 64.0f);
    const float inv = rcp_rn(s);
    uint32_t q0 = quant_pair_finite(xv.x * inv, xv.y * inv);
    uint32_t q1 = quant_pair_finite(xv.z * inv, xv.w * inv);
    if (__builtin_expect(!__builtin_isfinite(s), 0)) {  // a non-finite group (rare)
        q0 = quant_pair(xv.x * inv, xv.y * inv);
        q1 = quant_pair(xv.z * inv, xv.w * inv);
    }
    // int16 pairs -> fp16 pairs (exact: |q| <= 32768 fits; rows past M: 0)
    const uint32_t h0 = real ? __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(
                                   (float)(int16_t)(q0 & 0xFFFF), (float)(int16_t)(q0 >> 16)))
                             : 0u;
    const uint32_t h1 = real ? __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(
                                   (float)(int16_t)(q1 & 0xFFFF), (float)(int16_t)(q1 >> 16)))
                             : 0u;
    const int mt = m >> 5, r = m & 31;
    const int sl = (u & 7) >> 1, hh = u >> 3;
    const size_t piece = (((size_t)mt * Kg + g) * 4 + sl) * 64 + r + 32 * hh;  // 16-byte piece
    *reinterpret_cast<uint2 *>(reinterpret_cast<char *>(qf) + piece * 16 + 8 * (u & 1)) = make_uint2(h0, h1);
    if (u == 0) {
        const int ah = (r >> 2) & 1, e = 4 * (r >> 3) + (r & 3);
        asf[(((size_t)mt * Kg + g) * 2 + ah) * 16 + e] = real ? s : 0.0f;
    }
}

hipError_t launch_quantize_frag(const float *A, _Float16 *qf, float *asf, int M, int K,
                                hipStream_t st) {
    if (K % 64 != 0 || M < 1) return hipErrorInvalidValue;
    const int Mt = (M + 31) / 32;
    dim3 grid((K / 64 + 1) / 2, Mt * 4);
    quantize_frag_kernel<<<grid, 256, 0, st>>>(A, qf, asf, M, K);
    return hipGetLastError();
}

// ---------------------------------------------------------------- the GEMM
// 4 int8 bytes -> 4 fp16 values in two dwords (bytes 0, 1 -> lo, 2, 3 -> hi),
// one conversion per byte: v_cvt_f16_i16 reading the byte sign-extended
// (SDWA source select) and writing one half of the destination (the other
// half kept), exact for every int8.
__device__ __forceinline__ void widen4_mf(uint32_t x, uint32_t &lo, uint32_t &hi) {
    asm("v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%2) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3"
        : "=&v"(lo), "=&v"(hi)
        : "v"(x));
}

// Swizzled 16-byte slot of (slice s, lane l) inside an n-tile's 4 KB.
__device__ __forceinline__ int bslot(int s, int l) {
    return s * 64 + (l ^ ((s & 2) << 1) ^ ((l & 32) >> 2));
}

// BPC: blocks per CU the register budget is sized for. D: groups whose
// global loads are in flight (a ring of D register sets; D divides kWsTile).
// AL: the block's A fragments are loaded once per block (each wave a share)
// and staged into LDS beside B, instead of each wave loading its own from
// L1/L2. The weight scales come as tiles of kWsTile groups: per weight row
// 4 * kWsTile contiguous bytes in one or two 16-byte loads, where a per-group
// load would touch a cache line of every row each group. A ring value is
// consumed by the staging (or, for A without AL, by the MFMAs) before its
// slot is reloaded; a value copied out of the ring into other registers
// would make each reload wait for that copy's load, which the in-order
// return turns into a wait for the whole ring. SG: groups per w_s tile (a
// power of two, at most kWsTile; K must be a multiple of 64 kWsTile).
constexpr int kWsTile = 8;
// HQ (SwiGLU only): the epilogue quantizes h into the down GEMM's operand
// (GemmMfArgs::hq) instead of storing it.
template <int TM, int TN, bool SWIGLU, int D, int BPC, int WM = 2, bool AL = true, int SG = kWsTile,
          bool HQ = false>
// What the entry loads need comes first, as plain arguments that the
// dispatcher preloads into scalar registers (the up scales and the rest are
// read from the GemmMfArgs copy).
__global__ __launch_bounds__(256, BPC) void gemm_mf_kernel(
    const _Float16 *Af_p, const float *asf_p, const int8_t *W0_p, const float *S0_p, int Mt_p,
    int N_p, int K_p, int M_p, const int8_t *W1_p, GemmMfArgs args) {
    GemmMfArgs a = args;
    a.Af = Af_p;
    a.asf = asf_p;
    a.W0 = W0_p;
    a.S0 = S0_p;
    a.Mt = Mt_p;
    a.N = N_p;
    a.K = K_p;
    a.M = M_p;
    a.W1 = W1_p;
    constexpr int WN = 4 / WM;              // waves along N
    constexpr int MTB = WM * TM;            // m-tiles of the block
    constexpr int BN = 32 * WN * TN;        // weight rows of the block
    constexpr int NT = BN / 32;             // n-tiles in the B buffer
    constexpr int BCH = BN * 4 / 256;       // 16-byte weight chunks per thread and group
    constexpr int BBUF = NT * 4 * 64 * 16;  // bytes of one B buffer
    constexpr int ABUF = AL ? MTB * 4 * 1024 : 0;  // bytes of one A buffer
    constexpr int WB = SG * 4 / 2;          // bytes of a row's tile that one thread loads (2 per row)
    constexpr int WCH = (2 * BN + 255) / 256;  // w_s tile chunks per thread
    static_assert(SG >= 2 && SG <= kWsTile && (SG & (SG - 1)) == 0 && kWsTile % SG == 0, "w_s tile");
    static_assert(!SWIGLU || (TN == 2 && WM == 2), "SwiGLU pairs one gate and one up n-tile per wave");
    static_assert(WM == 1 || WM == 2, "2 x 2 or 1 x 4 waves");
    static_assert(D >= 2 && SG % D == 0, "group g+1 is staged from loads issued a group earlier");
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char *Asm = smem + 2 * BBUF;                        // [2][MTB][4 slices][64 lanes][16 B]
    float *asl = reinterpret_cast<float *>(Asm + 2 * ABUF);      // [2][MTB m-tiles][32]
    float *wsl = asl + 2 * 32 * MTB;                              // [2 tiles][SG][BN]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int wm = wid % WM, wn = wid / WM;
    const int M = a.M, N = a.N, K = a.K, Kg = K / 64, Mt = a.Mt;
    const int ncols = SWIGLU ? BN / 2 : BN;  // output columns of the block
    // XCD-aware tile order. Workgroups go to the 8 XCDs round-robin (block b
    // to XCD b % 8), and each XCD has its own L2. Tile t = xcd * per + b / 8
    // gives XCD x the contiguous tiles [x per, (x+1) per), taken M-tile
    // fastest: a few columns of weight rows (which then stay in that XCD's
    // L2) against all activation rows, read by the XCD's blocks in step.
    const int tiles_m = (Mt + MTB - 1) / MTB;
    const int tiles = tiles_m * ((N + ncols - 1) / ncols);
    const int per = (tiles + 7) / 8;
    const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (t >= tiles) return;  // whole block: before any barrier
    const int n0 = (t / tiles_m) * ncols;
    const int mt0 = (t % tiles_m) * MTB;  // first m-tile of the block

    // Global loads go through buffer resources (SGPR base and size, 32-bit
    // per-lane offsets, the per-group advance in the scalar offset); a read
    // past a buffer's size returns zeros.
    constexpr int kRsrcWord3 = 0x00020000;
    const __amdgpu_buffer_rsrc_t rA =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.Af, 0, Mt * Kg * 4096, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rAS =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.asf, 0, Mt * Kg * 128, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rW0 =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.W0, 0, N * K, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rW1 =
        __builtin_amdgcn_make_buffer_rsrc((void *)(SWIGLU ? a.W1 : a.W0), 0, N * K, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rS0 =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.S0, 0, N * Kg * 4, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rS1 =
        __builtin_amdgcn_make_buffer_rsrc((void *)(SWIGLU ? a.S1 : a.S0), 0, N * Kg * 4, kRsrcWord3);

    // ---- A: with AL, wave w loads slice w of each of the block's MTB
    // m-tiles (1 KB each, m-tiles clamped into the buffer), in the LDS layout
    // of the fragments [m-tile][slice][lane][16 B]; without AL, each wave
    // loads the four slices of its own TM m-tiles
    constexpr int AU = AL ? MTB : TM;  // A ring entries per thread (AL: 1 slice; else 4)
    int aoff[AU];
#pragma unroll
    for (int i = 0; i < AU; ++i) {
        const int mt = min(mt0 + (AL ? i : wm * TM + i), Mt - 1);
        aoff[i] = ((mt * Kg * 4 + (AL ? wid : 0)) * 64 + lane) * 16;
    }
    // ---- B staging: chunk q = tid + 256 i -> row q / 4, 16-byte piece q % 4
    // (under SWIGLU the chunks with i >= BCH / 2 are the up rows)
    int boff[BCH];
    int bdst0[BCH], bdst1[BCH];
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
        const int q = tid + 256 * i;
        const int row = q >> 2, c = q & 3;
        const int nrow = min(n0 + (SWIGLU && row >= BN / 2 ? row - BN / 2 : row), N - 1);
        boff[i] = nrow * K + 16 * c;
        const int nt = row >> 5, l = (row & 31) + 32 * (c >> 1), s0 = 2 * (c & 1);
        bdst0[i] = (nt * 256 + bslot(s0, l)) * 16;
        bdst1[i] = (nt * 256 + bslot(s0 + 1, l)) * 16;
    }
    // ---- a_s staging: 8 MTB threads copy one float4 each (MTB m-tiles of
    // 32 scales per group); every thread loads and stores, the others a
    // duplicate of thread tid % (8 MTB) -- the same value to the same place,
    // so no path leaves a scale load outstanding into the loop
    int as_off, as_dst;
    {
        const int q = tid % (8 * MTB);
        const int i = q >> 3, part = q & 7;  // m-tile i of the block, 16 B piece
        const int mt = min(mt0 + i, Mt - 1);
        as_off = (mt * Kg * 32 + 4 * part) * 4;
        as_dst = i * 32 + 4 * part;
    }
    // ---- w_s tiles: chunk q = tid + 256 c -> B row (q / 2) % BN, groups
    // (SG / 2) (q % 2) .. of the tile (chunks past the rows duplicate a row:
    // the same values to the same place). Under SWIGLU rows >= BN / 2 are the
    // up rows, taken by whole waves, so the resource stays scalar.
    static_assert(!SWIGLU || BN == 128 || BN == 256, "SwiGLU w_s chunks split at a wave");
    int wso[WCH], wsr[WCH], wsh[WCH];
    bool wsu[WCH];
#pragma unroll
    for (int c = 0; c < WCH; ++c) {
        const int q = tid + 256 * c, row = (q >> 1) % BN;
        wsu[c] = SWIGLU && __builtin_amdgcn_readfirstlane(row) >= BN / 2;  // whole waves
        wsr[c] = row;
        wsh[c] = q & 1;
        const int nrow = min(n0 + (wsu[c] ? row - BN / 2 : row), N - 1);
        wso[c] = (nrow * Kg + (SG / 2) * (q & 1)) * 4;
    }
    // ---- this lane's output columns (n-tile bt[j] of the B buffer)
    int bt[TN];
    int ncol[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        if (SWIGLU) {
            bt[j] = j == 0 ? wn : 2 + wn;
            ncol[j] = n0 + 32 * wn + (lane & 31);
        } else {
            bt[j] = TN * wn + j;
            ncol[j] = n0 + 32 * (TN * wn + j) + (lane & 31);
        }
    }
    const int h = lane >> 5;

    // ---- the ring of in-flight loads: group g's operands in slot g % D
    u32x4 araw[D][AU][AL ? 1 : 4];
    u32x4 braw[D][BCH];
    float4 asraw[D];
    typedef float wsv_t __attribute__((ext_vector_type(SG / 2)));
    wsv_t wst[WCH];  // the next w_s tile
    auto load_group = [&](int sl, int g) {
#pragma unroll
        for (int i = 0; i < AU; ++i)
#pragma unroll
            for (int s = 0; s < (AL ? 1 : 4); ++s)
                araw[sl][i][s] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(rA, aoff[i], g * 4096 + s * 1024, 0));
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
            const bool up = SWIGLU && i >= BCH / 2;
            braw[sl][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        up ? rW1 : rW0, boff[i], 64 * g, 0));
        }
        asraw[sl] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rAS, as_off, 128 * g, 0));
    };
    // w_s tile of groups g .. g + SG - 1
    auto load_ws = [&](int g) {
#pragma unroll
        for (int c = 0; c < WCH; ++c) {
            if constexpr (WB == 16)
                wst[c] = __builtin_bit_cast(wsv_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                       wsu[c] ? rS1 : rS0, wso[c], 4 * g, 0));
            else if constexpr (WB == 8)
                wst[c] = __builtin_bit_cast(wsv_t, __builtin_amdgcn_raw_buffer_load_b64(
                                                       wsu[c] ? rS1 : rS0, wso[c], 4 * g, 0));
            else
                wst[c] = __builtin_bit_cast(wsv_t, __builtin_amdgcn_raw_buffer_load_b32(
                                                       wsu[c] ? rS1 : rS0, wso[c], 4 * g, 0));
        }
    };
    auto store_ws = [&](int g) {  // into tile slot (g / SG) % 2
        float *slot = wsl + ((g / SG) & 1) * SG * BN;
#pragma unroll
        for (int c = 0; c < WCH; ++c)
#pragma unroll
            for (int k = 0; k < SG / 2; ++k) slot[((SG / 2) * wsh[c] + k) * BN + wsr[c]] = wst[c][k];
    };
    // group g (ring slot sl) goes to the A (with AL) and B buffers g % 2, its
    // a_s to slot g % 2 (every ring value is consumed here, before its slot
    // is reloaded, so a reload never waits for the load it replaces)
    auto stage = [&](int sl, int g) {
        if constexpr (AL) {
            unsigned char *As = Asm + (g & 1) * ABUF;
#pragma unroll
            for (int i = 0; i < MTB; ++i)
                *reinterpret_cast<u32x4 *>(As + ((i * 4 + wid) * 64 + lane) * 16) = araw[sl][i][0];
        }
        unsigned char *Bs = smem + (g & 1) * BBUF;
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
            const u32x4 v = braw[sl][i];
            uint32_t w[8];
            widen4_mf(v.x, w[0], w[1]);
            widen4_mf(v.y, w[2], w[3]);
            widen4_mf(v.z, w[4], w[5]);
            widen4_mf(v.w, w[6], w[7]);
            *reinterpret_cast<u32x4 *>(Bs + bdst0[i]) = (u32x4){w[0], w[1], w[2], w[3]};
            *reinterpret_cast<u32x4 *>(Bs + bdst1[i]) = (u32x4){w[4], w[5], w[6], w[7]};
        }
        *reinterpret_cast<float4 *>(asl + (g & 1) * 32 * MTB + as_dst) = asraw[sl];
    };

    // one accumulator set: the MFMA -> epilogue chain of one wave is hidden
    // by the other blocks on the CU
    float16_t acc[TM][TN], out[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) out[i][j] = (float16_t)(0.0f);

    // ---- prologue: w_s tile 0 and groups 0 .. D-1 in flight (clamped: a
    // repeated load of the last group keeps the ring full), w_s tile 0 and
    // group 0 staged
    load_ws(0);
#pragma unroll
    for (int j = 0; j < D; ++j) load_group(j, min(j, Kg - 1));
    store_ws(0);
    stage(0, 0);
    // Enter the loop with no load outstanding (vmcnt(0); group 0's data had
    // to arrive anyway, the others were issued right behind it): the
    // compiler's wait counts at the loop head then follow the loop's own
    // order of loads alone, not a merge with the prologue's.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();

    // The MFMAs of group g (B from LDS buffer g % 2; A from LDS buffer g % 2
    // with AL, else from ring slot sl): the fragments of slice s + 1 are read
    // while slice s multiplies
    auto mfmas = [&](int g, int sl) {
        const unsigned char *As = Asm + (g & 1) * ABUF + (wm * TM * 4 * 64 + lane) * 16;
        const unsigned char *Bs = smem + (g & 1) * BBUF;
        half8_t afr[2][TM], bfr[2][TN];
        auto rd = [&](int s) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
                afr[s & 1][i] = AL ? *reinterpret_cast<const half8_t *>(As + (i * 4 + s) * 1024)
                                   : __builtin_bit_cast(half8_t, araw[sl][AL ? 0 : i][AL ? 0 : s]);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bfr[s & 1][j] = *reinterpret_cast<const half8_t *>(Bs + (bt[j] * 256 + bslot(s, lane)) * 16);
        };
        rd(0);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s + 1 < 4) rd(s + 1);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                        afr[s & 1][i], bfr[s & 1][j], s == 0 ? (float16_t)(0.0f) : acc[i][j], 0, 0, 0);
        }
    };
    // epilogue of group g, reference order: out = fma(G * a_s, w_s, out)
    auto epilogue = [&](int g) {
        const float *as_g = asl + (g & 1) * 32 * MTB + wm * TM * 32 + h * 16;
        const float *ws_t = wsl + ((g / SG) & 1) * SG * BN + (g % SG) * BN;
        float ws_g[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) ws_g[j] = ws_t[bt[j] * 32 + (lane & 31)];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            float asv[16];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 v = *reinterpret_cast<const float4 *>(as_g + i * 32 + 4 * q4);
                asv[4 * q4] = v.x;
                asv[4 * q4 + 1] = v.y;
                asv[4 * q4 + 2] = v.z;
                asv[4 * q4 + 3] = v.w;
            }
            // The single-m-tile variant (M <= 32) skips the accumulator
            // quads whose rows (8 (e / 4) + e % 4, and 4 more) are all past M:
            // their outputs are never stored.
            int nq = 4;
            if constexpr (MTB == 1) nq = min(4, (M - 32 * mt0 + 7) >> 3);  // uniform
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (q >= nq) break;
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int e = 4 * q; e < 4 * q + 4; ++e)
                        out[i][j][e] = fmaf(acc[i][j][e] * asv[e], ws_g[j], out[i][j][e]);
            }
        }
    };
    // group g = g0 + j (ring slot sl = j % D): MFMAs, reload slot sl with
    // group g+D (and at j = 0 the w_s tile after the current one), the
    // epilogue, stage group g+1 (slot (g+1) % D, loaded D-1 groups ago; at
    // j = SG-1 also the w_s tile loaded SG-1 groups ago), barrier. The
    // scheduling barriers keep that order: staging group g+1 any earlier
    // (say beside the MFMAs) would wait for its loads sooner, instead of the
    // MFMAs of the other blocks on the CU hiding this wave's MFMA -> epilogue
    // dependency.
    auto group = [&](int g0, int j) {
        const int g = g0 + j, sl = j % D;
        mfmas(g, sl);
        // slot sl was consumed (staged one group ago; without AL its A just
        // went into the MFMAs), so it takes group g+D now. Unconditional (the
        // last group is reloaded near the end), so the compiler's count of
        // loads in flight is the same on every path.
        load_group(sl, min(g + D, Kg - 1));
        if (j == 0) load_ws(min(g0 + SG, Kg - SG));  // j is a compile-time constant
        __builtin_amdgcn_sched_barrier(0);
        epilogue(g);
        __builtin_amdgcn_sched_barrier(0);
        // also after the last group (the buffers and slots it fills are not
        // read again; ring and tile hold clamped reloads), so every path
        // waits for the same loads. Buffers (g+1) % 2 were last read before
        // the previous barrier, as were a_s slot (g+1) % 2 (by the epilogues
        // of group g-1); w_s tile slot ((g+1) / SG) % 2 is not the one the
        // epilogues of group g read.
        stage((sl + 1) % D, g + 1);
        if (j == SG - 1) store_ws(g + 1);
        // LDS-only barrier: a __syncthreads() here would also wait for every
        // global load in flight and empty the load ring at each group
        lds_barrier();
        // nothing crosses from one group to the next: global loads hoisted
        // over the barrier would pile up in registers across the unrolled
        // groups
        __builtin_amdgcn_sched_barrier(0);
    };
    // unrolled by SG (Kg is a multiple of SG and SG of D): ring slots and
    // tile steps are static, and the loop body has no exit inside (a path
    // that left part of it would reach the loop head with other loads
    // outstanding, and the compiler's wait counts at the head cover every
    // path)
    for (int g0 = 0; g0 < Kg; g0 += SG) {
#pragma unroll
        for (int j = 0; j < SG; ++j) group(g0, j);
    }

    // ---- greedy-argmax partials of the block's columns (plain products):
    // per row the larger value, equal values the lower column, values that
    // are not above -FLT_MAX (NaN, -inf, -FLT_MAX) never win -- the strict >
    // scan from -FLT_MAX, as argmax_part_kernel combines it. Each lane
    // reduces its TN columns, the 32 lanes of its half (one row per
    // accumulator) by xor shuffles, the WN waves that share the rows through
    // LDS (free: the last group's barrier has passed).
    if constexpr (!SWIGLU) {
        if (a.part_val) {  // uniform
            float *rv = reinterpret_cast<float *>(smem);          // [4 waves][TM][16][2]
            int32_t *ri = reinterpret_cast<int32_t *>(rv + 4 * TM * 32);
#pragma unroll
            for (int i = 0; i < TM; ++i) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    // rows 8 (e / 4) + (e % 4) and 4 more: past M for both
                    // halves -> nothing to reduce (uniform)
                    if (32 * (mt0 + wm * TM + i) + 8 * (e >> 2) + (e & 3) >= M) continue;
                    float bv = -FLT_MAX;
                    int32_t bi = -1;
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        const float v = out[i][j][e];
                        if (ncol[j] < N && v > -FLT_MAX) am_combine(bv, bi, v, ncol[j]);
                    }
#pragma unroll
                    for (int off = 16; off > 0; off >>= 1) {
                        const float ov = __shfl_xor(bv, off);
                        const int32_t oi = __shfl_xor(bi, off);
                        am_combine(bv, bi, ov, oi);
                    }
                    if ((lane & 31) == 0) {
                        rv[((wid * TM + i) * 16 + e) * 2 + h] = bv;
                        ri[((wid * TM + i) * 16 + e) * 2 + h] = bi;
                    }
                }
            }
            lds_barrier();
            if (tid < MTB * 32) {
                const int li = tid >> 5, r = tid & 31;  // block m-tile li, row r of it
                const int wmr = li / TM, i = li % TM;
                const int e = 4 * (r >> 3) + (r & 3), hr = (r >> 2) & 1;
                float bv = -FLT_MAX;
                int32_t bi = -1;
#pragma unroll
                for (int w = 0; w < WN; ++w) {
                    const int src = ((wmr + WM * w) * TM + i) * 16 + e;
                    am_combine(bv, bi, rv[src * 2 + hr], ri[src * 2 + hr]);
                }
                const int mrow = 32 * (mt0 + li) + r;
                if (mrow < M) {
                    a.part_val[(size_t)(n0 / ncols) * M + mrow] = bv;
                    a.part_idx[(size_t)(n0 / ncols) * M + mrow] = bi;
                }
            }
        }
    }

    // ---- SwiGLU with hq: the block's h tile (MTB m-tiles x 64 columns, one
    // whole group of the down projection's K) quantized straight into the
    // down GEMM's fragment-order operand, with quantize_frag_kernel's layout
    // and numerics (i8:135-177: the 16 chains over elements 16t + c, V[i] =
    // P[i] + P[i+8], the fixed tree, s = rms * fp32(1/127), RNE(h / s)), in
    // place of storing h: a quad of lanes per (row, group), lane u holding
    // elements 16t + 4u .. 4u + 3 (chains 4u .. 4u + 3). Rows past M get q = 0
    // and a_s = 0, as the quantizer's padding rows do.
    if constexpr (SWIGLU && HQ) {
        {
            constexpr int HLD = 68;  // floats per h row in LDS (64 + 4)
            float *ht = reinterpret_cast<float *>(smem);  // (the last group's barrier has passed)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int rr = 32 * (wm * TM + i) + 4 * h + 8 * (e >> 2) + (e & 3);
                    ht[rr * HLD + 32 * wn + (lane & 31)] = silu_mul(out[i][0][e], out[i][1][e]);
                }
            lds_barrier();
            const int Kgo = N / 64, go = n0 / 64;
            // (the thread index is rebuilt from mbcnt here rather than kept
            // live across the K loop, where one more VGPR spills per group)
            const int lid = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
#pragma unroll
            for (int p = 0; p < MTB * 128 / 256; ++p) {
                const int idx = 64 * wid + lid + 256 * p, rr = idx >> 2, u = idx & 3;
                const int mt = mt0 + (rr >> 5), r = rr & 31;
                const bool real = 32 * mt + r < M;  // the same for the quad
                float4 cv[4];
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    cv[t] = real ? *reinterpret_cast<const float4 *>(ht + rr * HLD + 16 * t + 4 * u)
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    p0 = fmaf(cv[t].x, cv[t].x, p0);
                    p1 = fmaf(cv[t].y, cv[t].y, p1);
                    p2 = fmaf(cv[t].z, cv[t].z, p2);
                    p3 = fmaf(cv[t].w, cv[t].w, p3);
                }
#define Q3VL_QUAD(v, ctrl) \
    __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false))
                // lanes 0, 1 take lanes 2, 3 (quad_perm [2,3,2,3]); lane 0 takes
                // lane 1's V[4..7] ([1,1,1,1]); lane 0's sum to the quad ([0,0,0,0])
                const float v0 = p0 + Q3VL_QUAD(p0, 0xEE), v1 = p1 + Q3VL_QUAD(p1, 0xEE);
                const float v2 = p2 + Q3VL_QUAD(p2, 0xEE), v3 = p3 + Q3VL_QUAD(p3, 0xEE);
                const float w0 = Q3VL_QUAD(v0, 0x55), w1 = Q3VL_QUAD(v1, 0x55);
                const float w2 = Q3VL_QUAD(v2, 0x55), w3 = Q3VL_QUAD(v3, 0x55);
                const float sumsq = Q3VL_QUAD(tree8(v0, v1, v2, v3, w0, w1, w2, w3), 0x00);
#undef Q3VL_QUAD
                const float sc = group_scale(sumsq, 1.0f / 64.0f);
                const float inv = rcp_rn(sc);
                if (mt < Mt) {  // (a block's last m-tile may lie past the product)
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        uint32_t q0 = quant_pair_finite(cv[t].x * inv, cv[t].y * inv);
                        uint32_t q1 = quant_pair_finite(cv[t].z * inv, cv[t].w * inv);
                        if (__builtin_expect(!__builtin_isfinite(sc), 0)) {
                            q0 = quant_pair(cv[t].x * inv, cv[t].y * inv);
                            q1 = quant_pair(cv[t].z * inv, cv[t].w * inv);
                        }
                        const uint32_t h0 = real ? __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(
                                                       (float)(int16_t)(q0 & 0xFFFF), (float)(int16_t)(q0 >> 16)))
                                                 : 0u;
                        const uint32_t h1 = real ? __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(
                                                       (float)(int16_t)(q1 & 0xFFFF), (float)(int16_t)(q1 >> 16)))
                                                 : 0u;
                        // element 16t + 4u of the group: quarter 4t + u of
                        // quantize_frag_kernel (slice 2 (t & 1) + u / 2, half t / 2)
                        const int sl = 2 * (t & 1) + (u >> 1), hh = t >> 1;
                        const size_t piece = (((size_t)mt * Kgo + go) * 4 + sl) * 64 + r + 32 * hh;
                        *reinterpret_cast<uint2 *>(reinterpret_cast<char *>(a.hq) + piece * 16 + 8 * (u & 1)) =
                            make_uint2(h0, h1);
                    }
                    if (u == 0) {
                        const int ah = (r >> 2) & 1, e = 4 * (r >> 3) + (r & 3);
                        a.hqs[(((size_t)mt * Kgo + go) * 2 + ah) * 16 + e] = real ? sc : 0.0f;
                    }
                }
            }
            return;
        }
    }

    // ---- store (an argmax caller that wants no logits passes C = null)
    if (!a.C) return;  // uniform
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int rbase = 32 * (mt0 + wm * TM + i) + 4 * h;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int mrow = rbase + 8 * (e >> 2) + (e & 3);
            if (mrow >= M) continue;
            if constexpr (SWIGLU) {
                if (ncol[0] < N) a.C[(size_t)mrow * N + ncol[0]] = silu_mul(out[i][0][e], out[i][1][e]);
            } else {
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    if (ncol[j] < N) a.C[(size_t)mrow * N + ncol[j]] = out[i][j][e];
            }
        }
    }
}

template <int TM, int TN, bool SWIGLU, int D, int BPC, int WM = 2, bool AL = true, int SG = kWsTile,
          bool HQ = false>
static hipError_t launch_mf(const GemmMfArgs &a, hipStream_t st) {
    constexpr int BN = 32 * (4 / WM) * TN, MTB = WM * TM;
    const int ncols = SWIGLU ? BN / 2 : BN;
    // argmax partials: one per block column range, counted by the caller
    if (a.part_val && ncols != gemm_mf_argmax_cols(a.M)) return hipErrorInvalidValue;
    const int tiles = ((a.N + ncols - 1) / ncols) * ((a.Mt + MTB - 1) / MTB);
    const int grid = 8 * ((tiles + 7) / 8);  // see the tile order in the kernel
    const size_t lds = 2 * (BN / 32) * 4 * 64 * 16 + (AL ? 2 * MTB * 4096 : 0) + 2 * 32 * MTB * 4 + 2 * SG * BN * 4;
    gemm_mf_kernel<TM, TN, SWIGLU, D, BPC, WM, AL, SG, HQ><<<grid, 256, lds, st>>>(
        a.Af, a.asf, a.W0, a.S0, a.Mt, a.N, a.K, a.M, a.W1, a);
    return hipGetLastError();
}

// Where this kernel serves (the caller quantizes in fragment order for it)
// and with which tiles, from timings of the prefill, vision and lm_head
// shapes on MI355X: every group-64 product whose K is a whole number of w_s
// tiles (K % 512 == 0). SwiGLU: 64 x (64 gate + 64 up) tiles at 3 blocks per
// CU, each wave loading its own A slices, while the grid fits one round of
// the device, else 128-row tiles at 2 blocks per CU. Plain: one
// m-tile (M <= 32, e.g. the lm_head over a few rows) takes 32 x 128 tiles of
// 1 x 4 waves, its A staged once per block; more m-tiles take 64 x 64 tiles
// at 4 blocks per CU, each wave loading its A slices itself (3-8% faster
// there: the L1 path takes A, LDS only B and the scales).
static long mf_blocks(const GemmMfArgs &a, int tm, int ncols) {
    return (long)((a.N + ncols - 1) / ncols) * ((a.Mt + 2 * tm - 1) / (2 * tm));
}

bool gemm_mf_serves(int M, int N, int K, bool swiglu, int cus) {
    (void)swiglu;
    (void)cus;
    return K % (64 * kWsTile) == 0 && K > 0 && M >= 1 && N >= 1;  // whole w_s tiles
}

// The output columns per block of the plain tiles launch_gemm_mf picks
// below (32 x 128 for one m-tile, 64 x 64 otherwise): one argmax partial each.
int gemm_mf_argmax_cols(int M) { return (M + 31) / 32 == 1 ? 128 : 64; }

hipError_t launch_gemm_mf(const GemmMfArgs &a, bool swiglu, int cus, hipStream_t st) {
    if (a.K % (64 * kWsTile) != 0 || a.K <= 0 || a.M < 1 || a.N < 1) return hipErrorInvalidValue;
    if (swiglu && a.part_val) return hipErrorInvalidValue;
    // h quantized in the epilogue: SwiGLU only, whole 64-column groups
    if (a.hq && (!swiglu || !a.hqs || a.N % 64 != 0)) return hipErrorInvalidValue;
    if (swiglu && a.hq) {
        if (mf_blocks(a, 1, 64) <= 3L * cus) return launch_mf<1, 2, true, 2, 3, 2, false, 8, true>(a, st);
        return launch_mf<2, 2, true, 2, 2, 2, true, 8, true>(a, st);
    }
    if (swiglu) {
        if (mf_blocks(a, 1, 64) <= 3L * cus) return launch_mf<1, 2, true, 2, 3, 2, false, 8>(a, st);
        return launch_mf<2, 2, true, 2, 2, 2, true, 8>(a, st);
    }
    if (a.Mt == 1) return launch_mf<1, 1, false, 2, 3, 1, true, 8>(a, st);
    return launch_mf<1, 1, false, 2, 4, 2, false, 8>(a, st);
}

// ------------------------------------------------ wide products, few rows
// 16 or fewer activation rows against a very wide weight (the lm_head over a
// batch of rows): the product is 16 rows x N, so the 32-row tiles above would
// pad it, and they stage every weight row through LDS. Here one wave computes
// 16 weight rows x the 16 activation rows with v_mfma_f32_16x16x32_f16, the
// weights going straight from the load into the MFMA operand:
// * B (weights): lane l takes weight row n = l % 16 of the tile and, of each
//   group's 64 bytes, bytes 16c .. 16c + 15 (c = l / 16) -- one 16-byte load a
//   lane and group; widened to fp16 (widen4_mf), its first 8 k feed the
//   group's first MFMA, the other 8 the second.
// * A: MFMA u of lane l takes row l % 16, k = 16c + 8u + j (j = 0..7) -- the k
//   the weight bytes hold. Each block quantizes the activations itself into
//   LDS in that lane order, 16-byte pieces [group][u][lane], and the a_s as
//   [group][row] (rows M..15 zero), so no quantizer launch precedes it: a
//   team of 4 lanes per (row, group) runs the reference quantizer
//   (i8:135-177) in its own order -- the 16 FMA chains over x[16t + i]^2,
//   P0[i] + P1[i], the fixed tree, s = sqrt(sumsq/64 + 1e-6) / 127 as
//   quantize_frag_kernel's group_scale, q = rne(x * (1/s)) saturated to
//   int16, as fp16 (exact: |q| <= 1016 wherever s is finite).
// * G of a group is the MFMA pair's exact integer sum (as in gemm_mf_kernel);
//   lane l holds rows 4c + i, column n, and folds out = fma(G * a_s, w_s, out)
//   group by group in ascending order (i8:613-617, 652).
// * Each wave takes a contiguous run of 16-row tiles (the runs differ by at
//   most one tile); its loads run D quads (4 groups each) ahead, across its
//   tiles. Per tile it keeps the greedy-argmax candidate of each row
//   (am_combine over its columns; values not above -FLT_MAX never win), and
//   at the end leaves one partial per row (an empty one without tiles).
template <int D, int NW, int MINB>
__global__ __launch_bounds__(64 * NW, MINB) void gemm_mf_wide_kernel(const float *A,
                                                                 const int8_t *W, const float *S, int N,
                                                                 int K, int M, int nwaves, int ntiles,
                                                                 float *C, float *part_val,
                                                                 int32_t *part_idx) {
    constexpr int NT = 64 * NW;  // threads
    extern __shared__ __align__(16) unsigned char smem[];
    const int Kg = K / 64, qpt = Kg / 4;  // groups; quads per tile
    u32x4 *Al = reinterpret_cast<u32x4 *>(smem);                  // [Kg][2][64]
    float *asl = reinterpret_cast<float *>(smem + Kg * 2 * 64 * 16);  // [Kg][16]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gw = (int)blockIdx.x * NW + wid;  // this wave's partial
    // tiles [t0, t1): the waves' shares differ by at most one tile
    const int t0 = (int)((long)gw * ntiles / nwaves), t1 = (int)((long)(gw + 1) * ntiles / nwaves);

    constexpr int kRsrcWord3 = 0x00020000;
    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc((void *)W, 0, N * K, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rS = __builtin_amdgcn_make_buffer_rsrc((void *)S, 0, N * Kg * 4, kRsrcWord3);
    const int c = lane >> 4, nl = lane & 15;
    // weight row of tile t (clamped into the weight; columns past N are not
    // kept) and its byte offset of quad q
    u32x4 wr[D][4];
    float4 wsr[D];
    const int nq = max(t1 - t0, 0) * qpt;  // quads over the wave's tiles
    auto load = [&](int sl, int Q) __attribute__((always_inline)) {
        const int t = t0 + Q / qpt, g0 = 4 * (Q % qpt);
        const int row = min(16 * t + nl, N - 1);
#pragma unroll
        for (int u = 0; u < 4; ++u)
            wr[sl][u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      rW, row * K + 16 * c, 64 * (g0 + u), 0));
        wsr[sl] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rS, row * Kg * 4, 4 * g0, 0));
    };
    // ---- quantize A into LDS (every thread of the block, before its
    // barrier). A team of 4 lanes per (row, group), rows 0..RW-1, groups
    // fastest (a wave's loads read 16 consecutive 256-byte groups, 64 bytes
    // a team each); rows past M are zeros, and with RW = 8 rows 8..15 are
    // zero-filled. Lane j of a team holds x[16v + 4j + c] (v, c = 0..3):
    // the whole chains i = 4j + c of the sum of squares, t = v ascending.
    // v_i = P_i + P_{i+8} pairs lanes j and j + 2, the tree's v_i + v_{i+4}
    // lanes 0 and 1, then (s0 + s1) + (s2 + s3) in lane 0. The teams go in
    // batches of QB passes whose loads are all issued before any of them is
    // used (rows clamped into A, no branch around a load); the first batch
    // goes out ahead of the weight stream, so waiting for it leaves the
    // weights in flight.
    const int RW = M <= 8 ? 8 : 16;
    const int nteam = RW * Kg;  // a multiple of NT / 4 (Kg is a multiple of 8)
    const int tj = tid & 3;
    constexpr int QB = 4;
    float4 xb[QB][4];
    auto load_batch = [&](int tb) __attribute__((always_inline)) {
#pragma unroll
        for (int it = 0; it < QB; ++it) {
            const int tm = min((tid >> 2) + tb + (NT / 4) * it, nteam - 1);
            const float *xr = A + (size_t)min(tm / Kg, M - 1) * K + 64 * (tm % Kg) + 4 * tj;
#pragma unroll
            for (int v = 0; v < 4; ++v) xb[it][v] = *reinterpret_cast<const float4 *>(xr + 16 * v);
        }
    };
    load_batch(0);
    // the weight stream starts before the activations are quantized; the
    // slots are issued in ring order, as the loop reissues them (the wait
    // counts at the loop head cover both paths: any other order here would
    // make every quad's first use wait for nearly every load in flight)
    if (nq > 0) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            load(j, min(j, nq - 1));
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if (RW == 8) {
        for (int q = tid; q < Kg * 16; q += NT) {  // (group, u, c) pieces of rows 8..15
            const int g = q >> 4, u = (q >> 3) & 1, cc = (q >> 1) & 3, r = 8 + 4 * (q & 1);
            u32x4 *d = Al + (g * 2 + u) * 64 + 16 * cc + r;
#pragma unroll
            for (int z = 0; z < 4; ++z) d[z] = (u32x4){0u, 0u, 0u, 0u};
        }
        for (int q = tid; q < Kg * 8; q += NT) asl[(q >> 3) * 16 + 8 + (q & 7)] = 0.0f;
    }
    // batch tb's teams (their loads in xb)
    auto quant_batch = [&](int tb) __attribute__((always_inline)) {
#pragma unroll
        for (int it = 0; it < QB; ++it) {
            const int tm = (tid >> 2) + tb + (NT / 4) * it;
            if (tm >= nteam) break;  // wave-uniform (16 teams a wave)
            const int g = tm % Kg, m = tm / Kg;
            const bool real = m < M;
            float4 xv[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float4 f = xb[it][v];
                xv[v] = real ? f : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
            float P[4];
            P[0] = fmaf(xv[0].x, xv[0].x, 0.0f);
            P[1] = fmaf(xv[0].y, xv[0].y, 0.0f);
            P[2] = fmaf(xv[0].z, xv[0].z, 0.0f);
            P[3] = fmaf(xv[0].w, xv[0].w, 0.0f);
#pragma unroll
            for (int v = 1; v < 4; ++v) {
                P[0] = fmaf(xv[v].x, xv[v].x, P[0]);
                P[1] = fmaf(xv[v].y, xv[v].y, P[1]);
                P[2] = fmaf(xv[v].z, xv[v].z, P[2]);
                P[3] = fmaf(xv[v].w, xv[v].w, P[3]);
            }
            float V[4], T[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) V[c] = P[c] + __shfl_xor(P[c], 2, 4);  // lanes 0, 1: v_{4j+c}
#pragma unroll
            for (int c = 0; c < 4; ++c) T[c] = V[c] + __shfl_xor(V[c], 1, 4);  // lane 0: s_c
            const float sumsq = __shfl((T[0] + T[1]) + (T[2] + T[3]), 0, 4);
            const float sc = group_scale(sumsq, 1.0f / 64.0f);
            const float inv = rcp_rn(sc);
            // q = rne(x * inv): for a finite scale |q| <= 1016, and adding and
            // removing 1.5 * 2^23 rounds to the integer, ties to even, exactly
            // in fp16 (quant_pair_finite's integer); otherwise the saturating
            // conversion of the reference, as int16 converted to fp16
            uint32_t h[8];  // h[2v + e]: elements 16v + 4tj + 2e, +1
            if (__builtin_expect(__builtin_isfinite(sc), 1)) {
                constexpr float kMagic = 12582912.0f;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float r0 = (xv[v].x * inv + kMagic) - kMagic, r1 = (xv[v].y * inv + kMagic) - kMagic;
                    const float r2 = (xv[v].z * inv + kMagic) - kMagic, r3 = (xv[v].w * inv + kMagic) - kMagic;
                    h[2 * v] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1));
                    h[2 * v + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r2, r3));
                }
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const uint32_t q0 = quant_pair(xv[v].x * inv, xv[v].y * inv);
                    const uint32_t q1 = quant_pair(xv[v].z * inv, xv[v].w * inv);
                    h[2 * v] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(
                                                      (float)(int16_t)(q0 & 0xFFFF), (float)(int16_t)(q0 >> 16)));
                    h[2 * v + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(
                                                          (float)(int16_t)(q1 & 0xFFFF), (float)(int16_t)(q1 >> 16)));
                }
            }
            // elements 16v + 4tj + c are halves 4(tj % 2) + c of piece 2v + tj / 2,
            // i.e. (u, lane c') = (tj / 2, 16v + m)
            unsigned char *Ab = reinterpret_cast<unsigned char *>(Al);
#pragma unroll
            for (int v = 0; v < 4; ++v)
                *reinterpret_cast<uint2 *>(Ab + ((g * 2 + (tj >> 1)) * 64 + 16 * v + m) * 16 + 8 * (tj & 1)) =
                    real ? make_uint2(h[2 * v], h[2 * v + 1]) : make_uint2(0u, 0u);
            if (tj == 0) asl[g * 16 + m] = real ? sc : 0.0f;
        }
    };
    // the first batch straight-line: its loads went out before the weight
    // ring's, and this code's wait for them leaves the ring in flight
    quant_batch(0);
    for (int tb = QB * (NT / 4); tb < nteam; tb += QB * (NT / 4)) {
        load_batch(tb);
        quant_batch(tb);
    }
    __syncthreads();
    if (nq == 0) {  // no tile for this wave: an empty partial (no barrier follows)
        if (part_val && (lane & 15) == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (4 * (lane >> 4) + i < M) {
                    part_val[(size_t)gw * M + 4 * (lane >> 4) + i] = -FLT_MAX;
                    part_idx[(size_t)gw * M + 4 * (lane >> 4) + i] = -1;
                }
        }
        return;
    }

    float4 out = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float bv[4] = {-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX};
    int32_t bi[4] = {-1, -1, -1, -1};
    auto step = [&](int sl, int Q) __attribute__((always_inline)) {
        const int g0 = 4 * (Q % qpt);
        half8_t bf[4][2];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const u32x4 v = wr[sl][u];
            uint32_t w[8];
            widen4_mf(v.x, w[0], w[1]);
            widen4_mf(v.y, w[2], w[3]);
            widen4_mf(v.z, w[4], w[5]);
            widen4_mf(v.w, w[6], w[7]);
            bf[u][0] = __builtin_bit_cast(half8_t, (u32x4){w[0], w[1], w[2], w[3]});
            bf[u][1] = __builtin_bit_cast(half8_t, (u32x4){w[4], w[5], w[6], w[7]});
        }
        // the scales copied out by real moves: kept as the slot's registers,
        // they would be live across the reload, which then takes other
        // registers and the loop's back edge copies them after a wait for
        // every load in flight
        float ws[4];
        asm volatile("v_mov_b32 %0, %1" : "=v"(ws[0]) : "v"(wsr[sl].x));
        asm volatile("v_mov_b32 %0, %1" : "=v"(ws[1]) : "v"(wsr[sl].y));
        asm volatile("v_mov_b32 %0, %1" : "=v"(ws[2]) : "v"(wsr[sl].z));
        asm volatile("v_mov_b32 %0, %1" : "=v"(ws[3]) : "v"(wsr[sl].w));
        // the slot's reload goes out here, after its values are consumed and
        // before this quad's MFMAs (pinned: left to itself, the scheduler
        // hoists reloads into fresh registers ahead of earlier uses, and the
        // ring's loads then retire in an order that makes each use wait for
        // nearly every load in flight)
        __builtin_amdgcn_sched_barrier(0);
        load(sl, min(Q + D, nq - 1));  // (past the last quad: the last again)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int g = g0 + u;
            const half8_t a0 = __builtin_bit_cast(half8_t, Al[(g * 2 + 0) * 64 + lane]);
            const half8_t a1 = __builtin_bit_cast(half8_t, Al[(g * 2 + 1) * 64 + lane]);
            const float4 as4 = *reinterpret_cast<const float4 *>(asl + g * 16 + 4 * c);
            float4_t acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bf[u][0], (float4_t){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bf[u][1], acc, 0, 0, 0);
            out.x = fmaf(acc[0] * as4.x, ws[u], out.x);
            out.y = fmaf(acc[1] * as4.y, ws[u], out.y);
            out.z = fmaf(acc[2] * as4.z, ws[u], out.z);
            out.w = fmaf(acc[3] * as4.w, ws[u], out.w);
        }
        if (Q % qpt == qpt - 1) {  // uniform: the tile's last quad
            const int col = 16 * (t0 + Q / qpt) + nl;
            const float o4[4] = {out.x, out.y, out.z, out.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 4 * c + i;
                if (row < M && col < N) {
                    if (C) C[(size_t)row * N + col] = o4[i];
                    if (o4[i] > -FLT_MAX) am_combine(bv[i], bi[i], o4[i], col);
                }
            }
            out = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    // nq is a multiple of D (D divides the quads of a tile): whole ring turns
    for (int Q0 = 0; Q0 < nq; Q0 += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) step(j, Q0 + j);
    }
    // ---- the wave's partial per row: the 16 lanes of row group c
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv[i], off);
            const int32_t oi = __shfl_xor(bi[i], off);
            am_combine(bv[i], bi[i], ov, oi);
        }
        const int row = 4 * c + i;
        if (part_val && nl == 0 && row < M) {
            part_val[(size_t)gw * M + row] = bv[i];
            part_idx[(size_t)gw * M + row] = bi[i];
        }
    }
}

constexpr int kWideD = 2;   // quads in flight per wave of gemm_mf_wide_kernel
constexpr int kWideNW = 4;  // waves per block
constexpr int kWideBPC = 1; // blocks per CU

bool gemm_mf_wide_serves(int M, int N, int K) {
    // K: whole quads of groups, the ring's D quads dividing a tile's, and the
    // block's A fragments (32 K bytes) within half of a CU's LDS
    return M >= 1 && M <= 16 && N >= 16 && K > 0 && K % (256 * kWideD) == 0 && K <= 2048;
}

// Waves: kWideBPC blocks of kWideNW waves per CU, fewer where the weight has
// fewer 16-row tiles; one argmax partial each. (Fewer, longer waves measured
// faster than two blocks per CU: the blocks' prologue quantizers repeat the
// same work.)
int gemm_mf_wide_parts(int N, int cus) {
    const int ntiles = (N + 15) / 16;
    const int blocks = min(kWideBPC * max(cus, 1), (ntiles + kWideNW - 1) / kWideNW);
    return blocks * kWideNW;
}

hipError_t launch_gemm_mf_wide(const float *A, const int8_t *W, const float *S, float *C, int M, int N,
                               int K, float *part_val, int32_t *part_idx, int cus, hipStream_t st) {
    if (!gemm_mf_wide_serves(M, N, K) || (size_t)N * K > 0x7fffffffULL || (!part_val) != (!part_idx) ||
        (!C && !part_val))
        return hipErrorInvalidValue;
    const int ntiles = (N + 15) / 16, nwaves = gemm_mf_wide_parts(N, cus);
    const size_t lds = (size_t)(K / 64) * (2 * 64 * 16 + 16 * 4);
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&gemm_mf_wide_kernel<kWideD, kWideNW, 2>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)((2048 / 64) * (2 * 64 * 16 + 16 * 4)));
    if (attr != hipSuccess) return attr;
    gemm_mf_wide_kernel<kWideD, kWideNW, 2><<<nwaves / kWideNW, 64 * kWideNW, lds, st>>>(
        A, W, S, N, K, M, nwaves, ntiles, C, part_val, part_idx);
    return hipGetLastError();
}

}  // namespace q3vl
