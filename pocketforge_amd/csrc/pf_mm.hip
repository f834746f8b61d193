// Int8-activation x block-quantized matrix products for gfx950, on the
// 32-row group layout of pf_layout.h.
//
//  * k_gemv  M <= 8 activation rows (decode passes).  One workgroup owns a
//            32-row group and all of K: its waves split the 256-column chunks
//            and meet in LDS, so every output is final inside the workgroup
//            and no partial sum leaves it.  The workgroup quantizes its own
//            copy of the activation rows first (prologue: RMSNorm + quantize,
//            or quantize, or a copy of rows quantized elsewhere) while its
//            weight loads are in flight, and applies the consumer's step to
//            the outputs (epilogue: store, residual add, RoPE + Q/K/V split,
//            SwiGLU of interleaved gate/up rows).
//  * k_gemm  M > 8 rows (prompt passes, many-sequence verify): the same
//            exact arithmetic over 32-row activation tiles quantized by the
//            row kernels, with the same epilogues; a workgroup shares each
//            activation tile among its waves through LDS.
//
// Arithmetic: v_mfma_i32_32x32x32_i8 gives the exact int32 dot p of one
// 32-element block of an activation row and a weight row; the output is
// y = (float)(a_s * sum_b d_b * p_b) with the sum exact in fp64 (every term is
// a multiple of the smallest block-scale ulp of the row and the row's scales
// span at most 15 binades, checked at upload), so any association order
// gives the same bits; k_gemm keeps the same sum as an exact int64 multiple
// of the row's smallest scale binade.  The activation quantization and RMSNorm follow
// src/matmul_neon.cpp:16-29 and :231-239 in the canonical orders of
// pf_gemv.hip.
#include "pf_device.h"

namespace pf {

typedef int pf_v4i __attribute__((ext_vector_type(4)));
typedef int pf_v16i __attribute__((ext_vector_type(16)));

enum Pro : int { PRO_NORM = 0, PRO_QUANT = 1, PRO_INT8 = 2, PRO_QPART = 3, PRO_MERGE = 4 };
enum Epi : int { EPI_STORE = 0, EPI_RESID = 1, EPI_QKV = 2, EPI_SWIGLU = 3 };
// Hand-offs through LL words (pf_device.h) inside one launch:
//   LL_IN : the NORM / QUANT prologue's input rows are LL words, lli.ll[m xs + col]
//   LL_OLD: the RESID epilogue's old values are LL words, e.llold[m y_stride + n]
//   LL_OUT: the RESID / SWIGLU epilogue writes LL words to e.ll instead of e.y
//   LL_COPY: with LL_OUT, RESID also stores the rows to e.y2 (for a later launch)
//   LL_GATE: the weight loads wait for the word lli.gate[lli.gate_off], so that
//            they start after an earlier stage's own loads
//   LL_NEXT: with LL_OUT, the words carry the next layer's flag (the residual
//            rows a layer hands to the next one in a launch of several layers)
enum LLMode : int { LL_IN = 1, LL_OLD = 2, LL_OUT = 4, LL_COPY = 8, LL_GATE = 16, LL_NEXT = 32 };

// Consumer step applied to the outputs.  Row n is a device row (pf_layout.h).
struct MmEpi {
    float* y;                  // STORE: y[m][logical n]; RESID: y[m][n] += ; SWIGLU: y[m][j]
    uint32_t y_stride;
    uint32_t ilv;              // STORE: the matrix holds two halves interleaved by 16 rows
    const uint32_t* skipm;     // RESID: rows m with skipm[m] != 0 take no residual (layer skip)
    float *q, *k, *v;          // QKV: [rows][D] each
    const float *rc, *rs;      // QKV: RoPE cos/sin [position][head_dim / 2]
    const PassDesc* pd;        // QKV: positions of the pass rows
    uint32_t D, hd;
    float* pmax;               // SWIGLU (GEMV): per-workgroup row maxima of |output| [M][N / 32], or null
    float* y2;                 // RESID: a copy of the updated rows (a pass's hidden output, or with LL_OUT the rows for a later launch), or null
    // QKV of a one-launch QKV + attention pass: instead of q/k/v, the rows
    // go to ll[m][3 D] as 8-byte words (value bits, flag) written with one
    // device-scope store each, flag = ep[0] * fmul + fadd (the pass epoch
    // and the layer), so a reader that sees the flag sees the value
    unsigned long long* ll;
    const uint32_t* ep;
    uint32_t fmul, fadd;
    const unsigned long long* llold;   // RESID with LL_OLD
};

// Logical row of device row n of a matrix whose halves [0, N/2) and
// [N/2, N) are interleaved by 16 rows.
__device__ __forceinline__ uint32_t ilv_logical(uint32_t n, uint32_t N) {
    const uint32_t g = n >> 5, r = n & 31u;
    return r < 16u ? 16u * g + r : N / 2u + 16u * g + (r - 16u);
}

// Operands of the epilogue that come from memory, loaded before the
// product so that their latency overlaps it: RESID the old value (a) and
// the skip flag (b != 0: no residual); QKV the RoPE cos (a) and sin (b).
struct EpiPre { float a, b; uint32_t f; };

template <int EPI, int LLM = 0>
__device__ __forceinline__ EpiPre epi_prefetch(const MmEpi& e, uint32_t m, uint32_t n, uint32_t flag = 0u,
                                               uint32_t* err = nullptr, uint32_t lay = 0u) {
    EpiPre p{0.0f, 0.0f, (LLM & LL_NEXT) ? flag + 1u : flag};
    if constexpr (EPI == EPI_RESID && (LLM & LL_OLD)) {
        const uint32_t off[1] = {m * e.y_stride + n};
        float v[1];
        ll_wait<1>(e.llold, off, v, flag, err);
        p.a = v[0];
    } else if constexpr (EPI == EPI_RESID) {
        p.a = e.y[(size_t)m * e.y_stride + n];
        p.b = (e.skipm && e.skipm[m]) ? 1.0f : 0.0f;
    } else if constexpr (EPI == EPI_QKV) {
        const uint32_t sec = n / e.D, i = n - sec * e.D;
        if (sec < 2u) {
            const uint32_t half = e.hd >> 1, t = (i % e.hd) >> 1;
            const uint32_t pos = row_pos(e.pd, m);
            p.a = e.rc[(size_t)pos * half + t];
            p.b = e.rs[(size_t)pos * half + t];
        }
        if (e.ll) p.f = ll_epoch(e.ep) * e.fmul + e.fadd + lay;
    }
    return p;
}

// y is this lane's output for (row m, device row n); y1 and y16 are the
// outputs of rows n ^ 1 and n ^ 16 of the same m (lane partners).  Returns
// the value a SWIGLU lane stores (0 for the others).
template <int EPI, int LLM = 0>
__device__ __forceinline__ float epi_apply(const MmEpi& e, const EpiPre& p, uint32_t N, uint32_t m, uint32_t n,
                                           float y, float y1, float y16) {
    if constexpr (EPI == EPI_STORE) {
        e.y[(size_t)m * e.y_stride + (e.ilv ? ilv_logical(n, N) : n)] = y;
    } else if constexpr (EPI == EPI_RESID && (LLM & LL_OUT)) {
        ll_store(e.ll + (size_t)m * e.y_stride + n, p.a + y, p.f);
        if constexpr ((LLM & LL_COPY) != 0) e.y2[(size_t)m * e.y_stride + n] = p.a + y;
    } else if constexpr (EPI == EPI_RESID) {
        if (p.b == 0.0f) e.y[(size_t)m * e.y_stride + n] = p.a + y;
        if (e.y2) e.y2[(size_t)m * e.y_stride + n] = p.b == 0.0f ? p.a + y : p.a;
    } else if constexpr (EPI == EPI_QKV) {
        // src/engine.cpp:693-715 (Q, K, V rows of the fused matrix) and the
        // RoPE of :732-749 for Q and K: pair (2t, 2t+1) of a head
        const uint32_t sec = n / e.D, i = n - sec * e.D;
        float out = y;
        if (sec < 2u) out = (n & 1u) ? __builtin_fmaf(y1, p.b, y * p.a) : __builtin_fmaf(y, p.a, -(y1 * p.b));
        if (e.ll) {
            __hip_atomic_store(e.ll + (size_t)m * 3u * e.D + n, ((unsigned long long)p.f << 32) | f2u(out),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            float* dst = sec == 0u ? e.q : (sec == 1u ? e.k : e.v);
            dst[(size_t)m * e.D + i] = out;
        }
    } else {
        // SwiGLU of src/engine.cpp:832-838 on gate row j (group rows 0-15)
        // and up row j (rows 16-31): g * (1 / (1 + exp(-g))) * u
        if ((n & 31u) < 16u) {
            const uint32_t j = 16u * (n >> 5) + (n & 31u);
            const float sig = 1.0f / (1.0f + expf_c(-y));
            const float f = y * sig * y16;
            if constexpr ((LLM & LL_OUT) != 0) ll_store(e.ll + (size_t)m * e.y_stride + j, f, p.f);
            else e.y[(size_t)m * e.y_stride + j] = f;
            return f;
        }
    }
    return 0.0f;
}

// ------------------------------------------------------------ operands

// B operand (16 signed codes, element order) of block t of a 256-column
// chunk for this lane (row lane % 32, elements 16 (lane / 32) ..): cw holds
// the lane's 16-byte words of the chunk's sets.
template <int FMT>
__device__ __forceinline__ pf_v4i b_operand(const uint4* cw, uint32_t t) {
    constexpr uint32_t ADD = (0x80u - (uint32_t)code_offset(FMT)) * 0x01010101u;
    pf_v4i v;
    if constexpr (FMT == FMT_Q8) {
        const uint4 c = cw[t];
        v.x = (int)c.x; v.y = (int)c.y; v.z = (int)c.z; v.w = (int)c.w;
    } else if constexpr (FMT == FMT_Q4) {
        const uint4 c = cw[t >> 1];
        const uint32_t x0 = (t & 1u) ? c.z : c.x, x1 = (t & 1u) ? c.w : c.y, mk = 0x0F0F0F0Fu;
        v.x = (int)(((x0 & mk) + ADD) ^ 0x80808080u);
        v.y = (int)(((x1 & mk) + ADD) ^ 0x80808080u);
        v.z = (int)((((x0 >> 4) & mk) + ADD) ^ 0x80808080u);
        v.w = (int)((((x1 >> 4) & mk) + ADD) ^ 0x80808080u);
    } else {
        const uint4 c = cw[t >> 2];
        const uint32_t s = t & 3u;
        const uint32_t x = s == 0u ? c.x : (s == 1u ? c.y : (s == 2u ? c.z : c.w)), mk = 0x03030303u;
        v.x = (int)(((x & mk) + ADD) ^ 0x80808080u);
        v.y = (int)((((x >> 2) & mk) + ADD) ^ 0x80808080u);
        v.z = (int)((((x >> 4) & mk) + ADD) ^ 0x80808080u);
        v.w = (int)((((x >> 6) & mk) + ADD) ^ 0x80808080u);
    }
    return v;
}

// The same block's codes as stored (0 .. 15 for Q4, 0 .. 3 for the 2-bit
// formats), without the offset: v_dot4 over them gives the block's dot plus
// offset x the activation codes' sum, which the one-row product removes by
// starting its v_dot4 chain at -offset x that sum (integers: exact).
template <int FMT>
__device__ __forceinline__ pf_v4i b_operand_raw(const uint4* cw, uint32_t t) {
    static_assert(FMT != FMT_Q8, "Q8 codes are signed bytes");
    pf_v4i v;
    if constexpr (FMT == FMT_Q4) {
        const uint4 c = cw[t >> 1];
        const uint32_t x0 = (t & 1u) ? c.z : c.x, x1 = (t & 1u) ? c.w : c.y, mk = 0x0F0F0F0Fu;
        v.x = (int)(x0 & mk);
        v.y = (int)(x1 & mk);
        v.z = (int)((x0 >> 4) & mk);
        v.w = (int)((x1 >> 4) & mk);
    } else {
        const uint4 c = cw[t >> 2];
        const uint32_t s = t & 3u;
        const uint32_t x = s == 0u ? c.x : (s == 1u ? c.y : (s == 2u ? c.z : c.w)), mk = 0x03030303u;
        v.x = (int)(x & mk);
        v.y = (int)((x >> 2) & mk);
        v.z = (int)((x >> 4) & mk);
        v.w = (int)((x >> 6) & mk);
    }
    return v;
}

template <int FMT>
constexpr int sets_of() { return FMT == FMT_Q8 ? 8 : (FMT == FMT_Q4 ? 4 : 2); }

// =============================================================== GEMV

constexpr int GEMV_WAVES = 8;
constexpr uint32_t GEMV_MAX_M = 8;

struct GemvArgs {
    const uint8_t* W;
    uint32_t N, K, M;
    const float* x;            // NORM / QUANT / QPART input rows [M][xs]
    uint32_t xs;
    const float* nw;           // NORM weight [K]
    const int8_t* a8;          // INT8 input: codes [M][xs] and row scales [M]
    const float* a8s;
    const float* pin;          // QPART: row maxima partials of the input [M][np]
    uint32_t np;
    const uint32_t* gate;      // gated instances: 0 -> nothing to compute
    const float* S;            // MERGE: per (head, chunk) maximum and sum [H][s_stride] of row 0
    uint32_t s_stride;
    const float* Up;           // MERGE: chunk-weighted V [H][cstride][hd] of row 0
    uint32_t cstride;
    uint32_t ncap;             // MERGE: chunks the loads cover without reading the pass (heads * ncap <= 2048), or 0
    KvGeom g;                  // MERGE: chunk count of row 0's list
    MmEpi e;
    Prefetch nx;               // the next product's weights: nx.blocks more workgroups load them
    LLIn lli;                  // LL_IN / LL_OLD / LL_OUT: input words, epoch, flag terms, timeout flag
};

// Dynamic LDS of k_gemv (bytes), laid out as: fp64 partials [waves][64][4],
// int8 rows [M][K + 16], tile sums [M][K / 64], maxima [M][4 waves], row
// statistics [3][8], and for one row the offset terms of the raw-code
// products [2][K / 32] (int32).
__host__ __device__ constexpr uint32_t gemv_kp(uint32_t K) { return K + 16u; }
__host__ __device__ constexpr uint32_t gemv_smem(uint32_t M, uint32_t K) {
    return (uint32_t)GEMV_WAVES * 64u * 4u * 8u + M * gemv_kp(K) + M * (K / 64u) * 4u +
           M * 4u * (uint32_t)GEMV_WAVES * 4u + 3u * 8u * 4u + (M == 1u ? K / 16u * 4u : 0u);
}
// MERGE adds the chunk maxima and sums [2][2048] (heads * chunks <= 2048),
// the head maxima and 1 / T [2][128] and a block reduction [16].
constexpr uint32_t GEMV_MERGE_SMEM = (2u * 2048u + 2u * 128u + 16u) * 4u;

// Codes of four values with the row's 127 / amax.
__device__ __forceinline__ uint32_t pack_codes(float4 v, float q) {
    const uint32_t b0 = (uint8_t)quant_code(v.x, q), b1 = (uint8_t)quant_code(v.y, q);
    const uint32_t b2 = (uint8_t)quant_code(v.z, q), b3 = (uint8_t)quant_code(v.w, q);
    return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

__device__ __forceinline__ float max4abs(float4 v) {
    return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// Grid N / 32 (one 32-row group per workgroup) + nx.blocks prefetch
// workgroups, 64 * GEMV_WAVES threads, gemv_smem(M, K) bytes of dynamic LDS.
// K % 256 == 0, K <= 1024 CPW (CPW chunks of 256 columns per wave, held in
// registers), M <= MR <= 8.
//
// The workgroup first loads everything its prologue needs, then its weight
// words (wave w takes chunks [nch w / W, nch (w + 1) / W)), then the
// epilogue's operands, so that the prologue's arithmetic waits only for the
// first loads while the weights are in flight.  Every load is issued
// unconditionally from a clamped address (rows past M reload row M - 1 and
// are not used), so no load sits behind a branch:
//   NORM : K = D <= 2048.  Wave w, row q of 16 lanes takes tile T = w + 8q;
//          lane i holds elements i, i + 16, i + 32, i + 48 of the tile in
//          every row m, so the tile's halving tree (offsets 32 and 16 first)
//          starts inside the lane and ends with DPP steps.  Tile sums in
//          column order give 1 / rms; amax = max|x * w| * inv (rounding is
//          monotone); codes of (x * w) * inv.
//   QUANT: the row held (CPW float4 per thread and row), amax, codes.
//   QPART: the same, amax from the producer's per-workgroup maxima.
//   INT8 : rows quantized by another kernel, copied.
//   MERGE: (M == 1, K = heads * head_dim <= 2048) the attention's chunk
//          results of the row merged per head exactly as merge_quant_row
//          does (max over the chunk maxima, f_c = exp(m_c - max), T and U
//          fmaf chains over c in order, U * (1 / (T + 1e-10))), then the
//          row quantized (quantize_activation_row).
//
// gemv_body is the workgroup's work as workgroup bx of gx; k_gemv runs it
// as its own grid, k_qkv_attn and k_o_ffn as workgroups of a wider one.  The
// weights, input rows and norm weights come as parameters (a kernel may
// pass them as preloaded arguments), the rest from a.
// With LL_IN the prologue's input words are waited for after the weight
// loads have been issued, so the weights stream in during the wait.  `lay`
// adds to every flag (the layer of a launch of several layers).
template <int FMT, int PRO, int EPI, bool GATED, int CPW, int MR, int LLM = 0>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, uint32_t bx, uint32_t gx, uint8_t* smem,
                                          const uint8_t* __restrict__ Wm, const float* __restrict__ xin,
                                          const float* __restrict__ nwv, uint32_t lay = 0u) {
    static_assert(!(LLM & LL_IN) || PRO == PRO_NORM || PRO == PRO_QUANT, "LL input rows: NORM or QUANT prologue");
    static_assert(!(LLM & LL_OLD) || (LLM & LL_IN), "LL old values come with LL input rows");
    constexpr uint32_t TB = g32_tile_bytes(FMT), CODES = g32_code_bytes(FMT);
    constexpr int SETS = sets_of<FMT>();
    constexpr uint32_t NT = 64u * GEMV_WAVES;
    if (bx >= (a.N >> 5)) {   // workgroups past the groups prefetch the next product's weights
        prefetch_groups(a.nx, bx, bx - (a.N >> 5), gx - (a.N >> 5));
        return;
    }
    if constexpr (GATED)
        if (*a.gate == 0u) return;   // no row of the pass needs this product
    double* red = reinterpret_cast<double*>(smem);
    int8_t* act = reinterpret_cast<int8_t*>(smem + GEMV_WAVES * 64 * 4 * 8);
    const uint32_t K = a.K, M = a.M, kp = gemv_kp(K), nt = K / 64u, xs = a.xs, mlast = M - 1u;
    float* tss = reinterpret_cast<float*>(act + M * kp);
    float* wmx = tss + M * nt;                 // [M][4 GEMV_WAVES]
    float* st = wmx + M * 4u * GEMV_WAVES;
    float* st_q = st + 8;                      // 127 / amax
    float* st_as = st + 16;                    // amax / 127
    const uint32_t t = threadIdx.x, lane = t & 63u, r = lane & 31u, h = lane >> 5;
    const uint32_t wid = __builtin_amdgcn_readfirstlane(t >> 6);
    const float* __restrict__ xg = xin;
    const uint32_t llflag = LLM ? ll_epoch(a.lli.ep) * a.lli.fmul + a.lli.fadd + lay : 0u;

    // ---- prologue loads
    const uint32_t li = lane & 15u, q = lane >> 4, T = wid + GEMV_WAVES * q;   // NORM tile of this lane
    float xv[MR][4], wv[4];
    float4 hv[MR][CPW];
    float pv[MR];
    uint4 iv[2];
    const uint32_t per4 = K / 4u, per16 = K / 16u;
    if constexpr (PRO == PRO_NORM) {
        const uint32_t col = 64u * min(T, nt - 1u) + li;
#pragma unroll
        for (int k = 0; k < 4; k++) wv[k] = nwv[col + 16u * k];
        if constexpr (!(LLM & LL_IN)) {
#pragma unroll
            for (uint32_t m = 0; m < MR; m++)
#pragma unroll
                for (int k = 0; k < 4; k++) xv[m][k] = xg[(size_t)min(m, mlast) * xs + col + 16u * k];
        }
    } else if constexpr (PRO == PRO_INT8) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t i = t + NT * k, m = min(i / per16, mlast), c = i % per16;
            iv[k] = *reinterpret_cast<const uint4*>(a.a8 + (size_t)m * xs + 16u * c);
        }
    }
    // MERGE: the row's (head, chunk) maxima and sums (entry i = h ncl + c,
    // heads * ncl <= 2048), and the first MG chunks of its columns
    // 4t .. 4t + 3 (head 4t >> hs, elements 4t & (hd - 1) ..; head_dim is a
    // power of two).  With ncap set the loads cover ncl = ncap chunks, the
    // capacity, whatever the pass's count nc, so they issue without waiting
    // for the pass descriptor; entries past nc are never used.  Otherwise
    // ncl = nc.  Chunk loads past ncl repeat its last chunk, so every group
    // issues the same loads and the waits stay exact.
    constexpr int MK = 2048 / NT;
    constexpr uint32_t MG = 12;
    uint32_t nc = 1, ncl = 1, hs = 0;
    uint32_t sh[MK], sc[MK];                  // head and chunk of S entry t + NT k
    float sm[MK], sv[MK];
    float4 uc[MG];
    const float* upc = nullptr;               // this thread's columns in chunk 0
    if constexpr (PRO == PRO_MERGE) {
        static_assert(MR == 1, "the merge prologue serves one row");
        if (a.ncap) ncl = a.ncap;
        else ncl = (kv_view(a.g, row_pos(pass_head(a.e.pd), 0)).count() + 1u + 255u) / 256u;
        const uint32_t hn = a.g.n_heads * ncl;
        hs = (uint32_t)__builtin_ctz(a.e.hd);
        const float rnc = 1.0f / (float)ncl;
#pragma unroll
        for (int k = 0; k < MK; k++) {
            const uint32_t i = min(t + NT * k, hn - 1u);
            uint32_t hh = (uint32_t)((float)i * rnc);     // i / ncl, corrected below
            hh -= hh * ncl > i ? 1u : 0u;
            hh += (hh + 1u) * ncl <= i ? 1u : 0u;
            sh[k] = hh;
            sc[k] = t + NT * k < hn ? i - hh * ncl : 0xFFFFFFFFu;
            sm[k] = a.S[(size_t)hh * a.s_stride + 2u * (i - hh * ncl)];
            sv[k] = a.S[(size_t)hh * a.s_stride + 2u * (i - hh * ncl) + 1u];
        }
        const uint32_t i4 = min(4u * t, K - 4u);
        upc = a.Up + (size_t)(i4 >> hs) * a.cstride * a.e.hd + (i4 & (a.e.hd - 1u));
#pragma unroll
        for (uint32_t u = 0; u < MG; u++)
            uc[u] = *reinterpret_cast<const float4*>(upc + (size_t)min(u, ncl - 1u) * a.e.hd);
    } else if constexpr (PRO != PRO_INT8 && PRO != PRO_NORM && !(LLM & LL_IN)) {
#pragma unroll
        for (uint32_t m = 0; m < MR; m++)
#pragma unroll
            for (int k = 0; k < CPW; k++) {
                const uint32_t c = min(t + NT * k, per4 - 1u);
                hv[m][k] = *reinterpret_cast<const float4*>(xg + (size_t)min(m, mlast) * xs + 4u * c);
            }
        if constexpr (PRO == PRO_QPART) {
            const uint32_t ti = min(t, a.np - 1u);
#pragma unroll
            for (uint32_t m = 0; m < MR; m++) pv[m] = a.pin[(size_t)min(m, mlast) * a.np + ti];
        }
    }

    // ---- weight loads (after the gate word, with LL_GATE: wave 0 polls it
    // and the others wait at a barrier, so that a workgroup keeps one poll
    // in flight rather than eight)
    if constexpr ((LLM & LL_GATE) != 0) {
        const uint32_t go[1] = {a.lli.gate_off};
        float gv[1];
        if (wid == 0) ll_wait<1>(a.lli.gate, go, gv, llflag - a.lli.gate_back, a.lli.err);
        __syncthreads();
    }
    const uint32_t nch = K >> 8, c0 = nch * wid / GEMV_WAVES, c1 = nch * (wid + 1) / GEMV_WAVES;
    const uint8_t* tiles = Wm + (size_t)bx * nch * TB;
    uint4 cw[CPW][SETS], sw[CPW];
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        const uint8_t* tile = tiles + (size_t)min(c0 + j, nch - 1u) * TB;
#pragma unroll
        for (int s = 0; s < SETS; s++) cw[j][s] = *reinterpret_cast<const uint4*>(tile + s * 1024 + lane * 16);
        sw[j] = *reinterpret_cast<const uint4*>(tile + CODES + r * 16);
    }
    // ---- epilogue operands from memory (thread t outputs row om of device
    // row on), issued before the LL input wait so that their latency overlaps
    // it; an LL old value is loaded beside the input words (below)
    const uint32_t om = t >> 5, on = 32u * bx + (t & 31u);
    EpiPre pre{};
    if constexpr (!(LLM & LL_OLD)) pre = epi_prefetch<EPI, LLM>(a.e, min(om, mlast), on, llflag, a.lli.err, lay);
    // ---- LL input rows, after the weight loads: the sentinel word first
    // (wave 0 polls it, one request per round, while the others wait at a
    // barrier), then the
    // thread's own words row by row (rows past M repeat row M - 1); the old
    // value's word (LL_OLD, written by an earlier stage than the input's) is
    // loaded with them and waited for only if its flag is not yet there
    unsigned long long wold = 0;
    if constexpr ((LLM & LL_IN) != 0) {
        const uint32_t so[1] = {a.lli.sent};
        float sv[1];
        if (wid == 0) ll_wait<1>(a.lli.ll, so, sv, llflag, a.lli.err);
        __syncthreads();
    }
    if constexpr ((LLM & LL_OLD) != 0) wold = ll_load(a.e.llold + (size_t)min(om, mlast) * a.e.y_stride + on);
    if constexpr ((LLM & LL_IN) && PRO == PRO_NORM) {
        const uint32_t col = 64u * min(T, nt - 1u) + li;
#pragma unroll
        for (uint32_t m = 0; m < MR; m++) {
            uint32_t off[4];
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) off[k] = (MR == 1 ? 0u : min(m, mlast) * xs) + col + 16u * k;
            ll_wait<4>(a.lli.ll, off, v, llflag, a.lli.err);
#pragma unroll
            for (int k = 0; k < 4; k++) xv[m][k] = v[k];
        }
    } else if constexpr ((LLM & LL_IN) && PRO == PRO_QUANT) {
#pragma unroll
        for (uint32_t m = 0; m < MR; m++) {
            uint32_t off[4 * CPW];
            float v[4 * CPW];
#pragma unroll
            for (int k = 0; k < CPW; k++) {
                const uint32_t c = min(t + NT * k, per4 - 1u);
#pragma unroll
                for (int j = 0; j < 4; j++) off[4 * k + j] = (MR == 1 ? 0u : min(m, mlast) * xs) + 4u * c + j;
            }
            ll_wait<4 * CPW>(a.lli.ll, off, v, llflag, a.lli.err);
#pragma unroll
            for (int k = 0; k < CPW; k++) hv[m][k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
        }
    }
    if constexpr ((LLM & LL_OLD) != 0) {
        if ((uint32_t)(wold >> 32) == llflag) {
            pre.a = __uint_as_float((uint32_t)wold);
            pre.f = (LLM & LL_NEXT) ? llflag + 1u : llflag;
        } else {
            pre = epi_prefetch<EPI, LLM>(a.e, min(om, mlast), on, llflag, a.lli.err, lay);
        }
    }

    // ---- prologue arithmetic
    if constexpr (PRO == PRO_MERGE) {
        float* fsm = st + 24;                    // [2048] chunk maxima, then f_c
        float* tsm = fsm + 2048;                 // [2048] chunk sums
        float* hiv = tsm + 2048 + 128;           // [128] 1 / (T + 1e-10) per head
        float* mred = hiv + 128;                 // [16]
        const uint32_t H = a.g.n_heads, hd = a.e.hd;
        if (a.ncap) nc = (kv_view(a.g, row_pos(pass_head(a.e.pd), 0)).count() + 1u + 255u) / 256u;
        else nc = ncl;
#pragma unroll
        for (int k = 0; k < MK; k++) {
            if (sc[k] < nc) {
                fsm[sh[k] * ncl + sc[k]] = sm[k];
                tsm[sh[k] * ncl + sc[k]] = sv[k];
            }
        }
        __syncthreads();
        // per head (thread h): the maximum over the chunk maxima, then
        // f_c = exp(m_c - max) in place and the T chain over c in order
        if (t < H) {
            float* f = fsm + t * ncl;
            const float* ts = tsm + t * ncl;
            float mx = f[0];
            for (uint32_t c = 1; c < nc; c++) mx = fmaxf(mx, f[c]);
            float T = 0.0f;
            for (uint32_t c = 0; c < nc; c++) {
                const float fc = expf_c(f[c] - mx);
                f[c] = fc;
                T = __builtin_fmaf(ts[c], fc, T);
            }
            hiv[t] = 1.0f / (T + 1e-10f);
        }
        __syncthreads();
        // U chains over c in order: the first MG chunks are held, later
        // groups (more than MG chunks) are loaded group by group
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float* f0 = fsm + (min(4u * t, K - 4u) >> hs) * ncl;
        for (uint32_t c0 = 0; c0 < nc; c0 += MG) {
            if (c0) {
#pragma unroll
                for (uint32_t u = 0; u < MG; u++)
                    uc[u] = *reinterpret_cast<const float4*>(upc + (size_t)min(c0 + u, nc - 1u) * hd);
            }
            const uint32_t nb = min(MG, nc - c0);
#pragma unroll
            for (uint32_t u = 0; u < MG; u++) {
                if (u < nb) {
                    const float f = f0[c0 + u];
                    v.x = __builtin_fmaf(uc[u].x, f, v.x);
                    v.y = __builtin_fmaf(uc[u].y, f, v.y);
                    v.z = __builtin_fmaf(uc[u].z, f, v.z);
                    v.w = __builtin_fmaf(uc[u].w, f, v.w);
                }
            }
        }
        // the row's amax: wave maxima meet in LDS behind one barrier
        const bool own = 4u * t < K;
        const float hv4 = hiv[min(4u * t, K - 4u) >> hs];
        v.x *= hv4;
        v.y *= hv4;
        v.z *= hv4;
        v.w *= hv4;
        float amax = own ? max4abs(v) : 0.0f;
        amax = wave_max(amax);
        if (lane == 0) mred[wid] = amax;
        __syncthreads();
        amax = mred[0];
#pragma unroll
        for (uint32_t w = 1; w < GEMV_WAVES; w++) amax = fmaxf(amax, mred[w]);
        const float qq = amax == 0.0f ? 1.0f : 127.0f / amax;
        if (own) *reinterpret_cast<uint32_t*>(act + 4u * t) = pack_codes(v, qq);
        if (t == 0) st_as[0] = amax == 0.0f ? 1.0f : amax / 127.0f;
    } else if constexpr (PRO == PRO_INT8) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t i = t + NT * k, m = i / per16, c = i % per16;
            if (m < M) *reinterpret_cast<uint4*>(act + m * kp + 16u * c) = iv[k];
        }
        if (t < M) st_as[t] = a.a8s[t];
    } else if constexpr (PRO == PRO_NORM) {
#pragma unroll
        for (uint32_t m = 0; m < MR; m++) {
            if (m >= M) break;
            float s = (xv[m][0] * xv[m][0] + xv[m][2] * xv[m][2]) + (xv[m][1] * xv[m][1] + xv[m][3] * xv[m][3]);
            s = row16_tree_sum(s);
            const float mx = row16_max(fmaxf(fmaxf(fabsf(xv[m][0] * wv[0]), fabsf(xv[m][1] * wv[1])),
                                             fmaxf(fabsf(xv[m][2] * wv[2]), fabsf(xv[m][3] * wv[3]))));
            if (li == 0) {
                if (T < nt) tss[m * nt + T] = s;
                wmx[m * 4u * GEMV_WAVES + 4u * wid + q] = T < nt ? mx : 0.0f;
            }
        }
        __syncthreads();
        if (t < M) {
            // tile sums in column order from +0 (all loaded first); rms of
            // src/matmul_neon.cpp:231-239
            float tv[32], wm[4 * GEMV_WAVES];
#pragma unroll
            for (uint32_t i = 0; i < 32; i += 4) {
                const float4 v4 = *reinterpret_cast<const float4*>(tss + t * nt + min(i, nt - 4u));
                tv[i] = v4.x; tv[i + 1] = v4.y; tv[i + 2] = v4.z; tv[i + 3] = v4.w;
            }
#pragma unroll
            for (uint32_t i = 0; i < 4 * GEMV_WAVES; i += 4) {
                const float4 v4 = *reinterpret_cast<const float4*>(wmx + t * 4u * GEMV_WAVES + i);
                wm[i] = v4.x; wm[i + 1] = v4.y; wm[i + 2] = v4.z; wm[i + 3] = v4.w;
            }
            float ss = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < 32; i++)
                if (i < nt) ss = ss + tv[i];
            const float inv = 1.0f / __builtin_sqrtf(ss / (float)K + 1e-6f);
            float mw = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < 4 * GEMV_WAVES; i++) mw = fmaxf(mw, wm[i]);
            const float amax = mw * inv;
            st[t] = inv;
            st_q[t] = amax == 0.0f ? 1.0f : 127.0f / amax;
            st_as[t] = amax == 0.0f ? 1.0f : amax / 127.0f;
        }
        __syncthreads();
        if (T < nt) {
#pragma unroll
            for (uint32_t m = 0; m < MR; m++) {
                if (m >= M) break;
                const float inv = st[m], qq = st_q[m];
#pragma unroll
                for (int k = 0; k < 4; k++)
                    act[m * kp + 64u * T + li + 16u * k] = quant_code((xv[m][k] * wv[k]) * inv, qq);
            }
        }
    } else {
#pragma unroll
        for (uint32_t m = 0; m < MR; m++) {
            if (m >= M) break;
            float mx;
            if constexpr (PRO == PRO_QPART) {
                mx = t < a.np ? pv[m] : 0.0f;
            } else {
                mx = 0.0f;
#pragma unroll
                for (int k = 0; k < CPW; k++) mx = fmaxf(mx, max4abs(hv[m][k]));
            }
            mx = row16_max(mx);
            if (li == 0) wmx[m * 4u * GEMV_WAVES + 4u * wid + q] = mx;
        }
        __syncthreads();
        if (t < M) {
            float wm[4 * GEMV_WAVES];
#pragma unroll
            for (uint32_t i = 0; i < 4 * GEMV_WAVES; i += 4) {
                const float4 v4 = *reinterpret_cast<const float4*>(wmx + t * 4u * GEMV_WAVES + i);
                wm[i] = v4.x; wm[i + 1] = v4.y; wm[i + 2] = v4.z; wm[i + 3] = v4.w;
            }
            float amax = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < 4 * GEMV_WAVES; i++) amax = fmaxf(amax, wm[i]);
            st_q[t] = amax == 0.0f ? 1.0f : 127.0f / amax;
            st_as[t] = amax == 0.0f ? 1.0f : amax / 127.0f;
        }
        __syncthreads();
#pragma unroll
        for (uint32_t m = 0; m < MR; m++) {
            if (m >= M) break;
            const float qq = st_q[m];
#pragma unroll
            for (int k = 0; k < CPW; k++) {
                const uint32_t c = t + NT * k;
                if (c < per4) *reinterpret_cast<uint32_t*>(act + m * kp + 4u * c) = pack_codes(hv[m][k], qq);
            }
        }
    }
    __syncthreads();
    // one row of a sub-byte format: -offset x the sum of each half block's
    // 16 activation codes, [half][block], the start of the product's chains
    int* nsum = reinterpret_cast<int*>(st + 24);
    if constexpr (MR == 1 && FMT != FMT_Q8) {
        for (uint32_t i = t; i < K / 16u; i += NT) {
            const pf_v4i v = *reinterpret_cast<const pf_v4i*>(act + 16u * i);
            int s = __builtin_amdgcn_sdot4(v.x, 0x01010101, 0, false);
            s = __builtin_amdgcn_sdot4(v.y, 0x01010101, s, false);
            s = __builtin_amdgcn_sdot4(v.z, 0x01010101, s, false);
            s = __builtin_amdgcn_sdot4(v.w, 0x01010101, s, false);
            nsum[(i & 1u) * (K / 32u) + (i >> 1)] = -code_offset(FMT) * s;
        }
        __syncthreads();
    }

    // ---- product
    if constexpr (MR == 1) {
        // One row: lane (r, h) takes the 16 codes 16h .. 16h + 15 of each
        // block of weight row r with the row's matching activation bytes
        // (the same LDS words for every lane of a half, a broadcast), four
        // v_dot4 give the exact int32 partial p, and d_b * p accumulates in
        // fp64; the halves and waves meet in LDS.  Every partial sum is a
        // sum of some of the exact terms d_b * p_b, so the result is the
        // same sum as the MFMA path's.  Sub-byte codes enter the v_dot4 as
        // stored, the chain starting at the half block's offset term.
        double S1 = 0.0;
        const int8_t* a0 = act + 16u * h;
#pragma unroll
        for (int j = 0; j < CPW; j++) {
            if (c0 + j >= c1) break;
            const uint32_t c = c0 + j;
            const uint16_t* sc = reinterpret_cast<const uint16_t*>(&sw[j]);
            pf_v4i A[8];
            int n0[8];
#pragma unroll
            for (uint32_t u = 0; u < 8; u++) A[u] = *reinterpret_cast<const pf_v4i*>(a0 + 32u * (8u * c + u));
            if constexpr (FMT != FMT_Q8) {
                const int4 p0 = *reinterpret_cast<const int4*>(nsum + h * (K / 32u) + 8u * c);
                const int4 p1 = *reinterpret_cast<const int4*>(nsum + h * (K / 32u) + 8u * c + 4u);
                n0[0] = p0.x; n0[1] = p0.y; n0[2] = p0.z; n0[3] = p0.w;
                n0[4] = p1.x; n0[5] = p1.y; n0[6] = p1.z; n0[7] = p1.w;
            }
#pragma unroll
            for (uint32_t u = 0; u < 8; u++) {
                pf_v4i B;
                int pp;
                if constexpr (FMT == FMT_Q8) {
                    B = b_operand<FMT>(cw[j], u);
                    pp = 0;
                } else {
                    B = b_operand_raw<FMT>(cw[j], u);
                    pp = n0[u];
                }
                pp = __builtin_amdgcn_sdot4(A[u].x, B.x, pp, false);
                pp = __builtin_amdgcn_sdot4(A[u].y, B.y, pp, false);
                pp = __builtin_amdgcn_sdot4(A[u].z, B.z, pp, false);
                pp = __builtin_amdgcn_sdot4(A[u].w, B.w, pp, false);
                S1 = __builtin_fma((double)h2f(sc[u]), (double)pp, S1);
            }
        }
        red[wid * 64 + lane] = S1;
        __syncthreads();
        float y = 0.0f;
        if (t < 32u) {
            double v = red[t] + red[t + 32u];
#pragma unroll
            for (uint32_t w = 1; w < GEMV_WAVES; w++) v += red[w * 64 + t] + red[w * 64 + t + 32u];
            y = (float)(v * (double)st_as[0]);
        }
        const float y1 = __shfl_xor(y, 1, 64), y16 = __shfl_xor(y, 16, 64);
        float f = 0.0f;
        if (om < M) f = epi_apply<EPI, LLM>(a.e, pre, a.N, om, on, y, y1, y16);
        if constexpr (EPI == EPI_SWIGLU) {
            float mx = fabsf(f);
#pragma unroll
            for (int off = 16; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            if (a.e.pmax && om < M && (t & 31u) == 0) a.e.pmax[(size_t)om * (a.N / 32u) + bx] = mx;
        }
        return;
    }
    double S[4] = {0.0, 0.0, 0.0, 0.0};
    const pf_v16i zero = {};
    const pf_v4i za = {0, 0, 0, 0};
    const int8_t* arow = act + min(r, mlast) * kp + 16u * h;
#pragma unroll
    for (int j = 0; j < CPW; j++) {
        if (c0 + j >= c1) break;
        const uint32_t c = c0 + j;
        const uint16_t* sc = reinterpret_cast<const uint16_t*>(&sw[j]);
        pf_v4i A[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; u++) {
            const pf_v4i v = *reinterpret_cast<const pf_v4i*>(arow + 32u * (8u * c + u));
            A[u] = r < M ? v : za;
        }
        // two blocks' MFMAs in flight before their results are scaled
#pragma unroll
        for (uint32_t u = 0; u < 8; u += 2) {
            const pf_v16i D0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[u], b_operand<FMT>(cw[j], u), zero, 0, 0, 0);
            const pf_v16i D1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[u + 1], b_operand<FMT>(cw[j], u + 1), zero, 0, 0, 0);
            const double d0 = (double)h2f(sc[u]), d1 = (double)h2f(sc[u + 1]);
#pragma unroll
            for (int i = 0; i < 4; i++) S[i] = __builtin_fma(d0, (double)D0[i], S[i]);
#pragma unroll
            for (int i = 0; i < 4; i++) S[i] = __builtin_fma(d1, (double)D1[i], S[i]);
        }
    }
    // lane (r, h) holds rows m = 4h + i of device row r; the waves meet in LDS
#pragma unroll
    for (int i = 0; i < 4; i++) red[(wid * 64 + lane) * 4 + i] = S[i];
    __syncthreads();
    float y = 0.0f;
    if (om < M) {
        const uint32_t L = (t & 31u) + 32u * (om >> 2), i = om & 3u;
        double v = red[L * 4 + i];
#pragma unroll
        for (uint32_t w = 1; w < GEMV_WAVES; w++) v += red[(w * 64 + L) * 4 + i];
        y = (float)(v * (double)st_as[om]);
    }
    const float y1 = __shfl_xor(y, 1, 64), y16 = __shfl_xor(y, 16, 64);
    float f = 0.0f;
    if (om < M) f = epi_apply<EPI, LLM>(a.e, pre, a.N, om, on, y, y1, y16);
    if constexpr (EPI == EPI_SWIGLU) {
        // row maximum of |f| over the group's 16 outputs (lanes of one m
        // are a half wave), for the consumer's quantization
        float mx = fabsf(f);
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        if (a.e.pmax && om < M && (t & 31u) == 0) a.e.pmax[(size_t)om * (a.N / 32u) + bx] = mx;
    }
}

template <int FMT, int PRO, int EPI, bool GATED, int CPW, int MR>
__global__ __launch_bounds__(64 * GEMV_WAVES) void k_gemv(GemvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    gemv_body<FMT, PRO, EPI, GATED, CPW, MR>(a, blockIdx.x, gridDim.x, smem, a.W, a.x, a.nw);
}

// =============================================================== GEMM

struct GemmArgs {
    const uint8_t* W;
    uint32_t N, K, M;
    const int8_t* act;         // [ceil(M / 32) * 32][act_stride] readable rows
    uint32_t act_stride;
    const float* as;           // [M]
    const uint32_t* gate;
    const uint8_t* xmin;       // [device rows]: smallest binade of the row's nonzero block scales
    MmEpi e;
};

// Integer form of a block scale for exact int64 sums: the fp16 scale d
// (low 16 bits of h) is M * 2^(X - 25) with M = significand (hidden bit
// included, 0 for zero) and X = max(biased exponent, 1); relative to the
// row's smallest binade xmin (nonzero scales only, so X >= xmin whenever
// M != 0) d = c * 2^(xmin - 25) with c = M << (X - xmin) < 2^26 (the
// upload keeps nonzero scales of a row within 15 binades).
__device__ __forceinline__ int32_t scale_multiplier(uint32_t h, uint32_t xmin) {
    const uint32_t e = (h >> 10) & 31u, mt = h & 1023u;
    const uint32_t mag = (e ? (mt | 1024u) : mt) << (((e ? e : 1u) - xmin) & 31u);
    return (h & 0x8000u) ? -(int32_t)mag : (int32_t)mag;
}

// One 256-column chunk of one wave's 32 x 32 output tile: eight blocks'
// exact int32 dots (MFMA) times the blocks' integer scale multipliers into
// int64 sums (|c p| < 2^41, so the sums of up to 8192 columns stay exact).
// The MFMAs of DI blocks are issued before their products are added, so
// the matrix core works while the adds of earlier blocks run.
template <int FMT, int DI>
__device__ __forceinline__ void gemm_chunk(int64_t (&S)[16], const uint8_t* arow, const uint4 (&cw)[sets_of<FMT>()],
                                           const uint4& sw, uint32_t xmin) {
    const pf_v16i zero = {};
    pf_v4i A[8];
#pragma unroll
    for (uint32_t u = 0; u < 8; u++) A[u] = *reinterpret_cast<const pf_v4i*>(arow + 32u * u);
    const uint32_t sx[4] = {sw.x, sw.y, sw.z, sw.w};
#pragma unroll
    for (uint32_t u0 = 0; u0 < 8; u0 += DI) {
        pf_v16i D[DI];
#pragma unroll
        for (uint32_t j = 0; j < (uint32_t)DI; j++)
            D[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[u0 + j], b_operand<FMT>(cw, u0 + j), zero, 0, 0, 0);
#pragma unroll
        for (uint32_t j = 0; j < (uint32_t)DI; j++) {
            const uint32_t u = u0 + j;
            const int32_t c = scale_multiplier(sx[u >> 1] >> (16u * (u & 1u)), xmin);
#pragma unroll
            for (int i = 0; i < 16; i++) S[i] += (int64_t)c * (int64_t)D[j][i];
        }
    }
}

// Grid (ceil(N / 32 / NW), ceil(M / 32 / MW)), 512 threads: 8 waves, wave
// w takes M tile mw = w % MW (32 activation rows),
// weight group nw = (w / MW) % NW of the workgroup's NW groups, and K slice
// kw = w / (MW NW) (chunks c with c % KW == kw).  Step s covers chunks
// KW s .. KW s + KW - 1: the workgroup copies their activation tiles
// (32 MW rows x 256 B each) once into LDS (double buffer, rows padded to
// 272 B) and every wave reads its rows from there, so a tile is fetched
// once per workgroup instead of once per wave; one barrier per step.  Loads
// run one step ahead (clamped, issued unconditionally), the weights into
// two register sets used on alternate steps, so that no copy waits for
// them.
// K slices meet in LDS (exact int64 sums).  Two waves per SIMD (up to 256
// VGPRs per lane): a 128-register budget spills.  Each lane keeps the 16
// outputs of its MFMA tile as int64 multiples of its row's 2^(xmin - 25);
// the epilogue converts them to fp64 exactly (|sum| < 2^53) and applies
// y = (float)(sum * 2^(xmin - 25) * a_s), the value of the fp64 block sum.
template <int MW, int KW>
constexpr uint32_t gemm_smem() { return 2u * KW * 32u * MW * 272u; }

template <int FMT, int EPI, bool GATED, int MW, int NW, int KW, int DI>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm(GemmArgs a) {
    static_assert(MW * NW * KW == 8, "eight waves");
    constexpr uint32_t TB = g32_tile_bytes(FMT), CODES = g32_code_bytes(FMT);
    constexpr int SETS = sets_of<FMT>();
    constexpr uint32_t ROWS = 32u * MW, AROW = 272u, STEP = KW * ROWS * AROW;
    constexpr uint32_t APT = KW * MW;                  // 16-byte activation pieces per thread and step
    static_assert((KW > 1 ? (KW - 1) * MW * NW * 64 * 16 * 8 : 0) <= 2 * STEP, "slice partials fit the buffers");
    __shared__ __align__(16) uint8_t smem[2 * STEP];
    if constexpr (GATED)
        if (*a.gate == 0u) return;
    const uint32_t t = threadIdx.x, lane = t & 63u, r = lane & 31u, h = lane >> 5;
    const uint32_t wid = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t mw = wid % MW, nw = (wid / MW) % NW, kw = wid / (MW * NW);
    const uint32_t m0 = blockIdx.y * ROWS, ng = a.N >> 5, g = blockIdx.x * NW + nw, gc = min(g, ng - 1u);
    const uint32_t nch = a.K >> 8, nsteps = (nch + KW - 1) / KW, mlast = a.M - 1u;
    const uint8_t* tiles = a.W + (size_t)gc * nch * TB;
    // piece u of thread t: row (t >> 4) + 32 (u % MW) of the tile, 16 bytes
    // at 16 (t & 15) of chunk KW s + u / MW
    const int8_t* abase[MW];
#pragma unroll
    for (uint32_t u = 0; u < (uint32_t)MW; u++)
        abase[u] = a.act + (size_t)min(m0 + (t >> 4) + 32u * u, mlast) * a.act_stride + 16u * (t & 15u);
    const uint32_t sbase = (t >> 4) * AROW + 16u * (t & 15u);
    pf_v4i av[APT];
#pragma unroll
    for (uint32_t u = 0; u < APT; u++)
        av[u] = *reinterpret_cast<const pf_v4i*>(abase[u % MW] + 256u * min(u / MW, nch - 1u));
    uint4 cw0[SETS], cw1[SETS], sw0, sw1;
    {
        const uint8_t* tile = tiles + (size_t)min(kw, nch - 1u) * TB;
#pragma unroll
        for (int q = 0; q < SETS; q++) cw0[q] = *reinterpret_cast<const uint4*>(tile + q * 1024 + lane * 16);
        sw0 = *reinterpret_cast<const uint4*>(tile + CODES + r * 16);
    }
    int64_t S[16];
#pragma unroll
    for (int i = 0; i < 16; i++) S[i] = 0;
    const uint32_t xmin = a.xmin[32u * gc + r];
    const uint32_t aoff = (kw * ROWS + 32u * mw + r) * AROW + 16u * h;
    for (uint32_t st = 0; st < nsteps; st += 2) {
#pragma unroll
        for (uint32_t ph = 0; ph < 2; ph++) {
            const uint32_t s = st + ph;
            if (ph == 1 && s >= nsteps) break;
            uint8_t* buf = smem + ph * STEP;
#pragma unroll
            for (uint32_t u = 0; u < APT; u++)
                *reinterpret_cast<pf_v4i*>(buf + (u / MW) * ROWS * AROW + 32u * (u % MW) * AROW + sbase) = av[u];
            __syncthreads();
            const uint32_t nx = s + 1u < nsteps ? s + 1u : s;
            const uint8_t* tile = tiles + (size_t)min(KW * nx + kw, nch - 1u) * TB;
            // two register sets: step s uses set s & 1, the loads fill the other
#pragma unroll
            for (int q = 0; q < SETS; q++) {
                const uint4 w = *reinterpret_cast<const uint4*>(tile + q * 1024 + lane * 16);
                if (ph == 0) cw1[q] = w; else cw0[q] = w;
            }
            const uint4 w = *reinterpret_cast<const uint4*>(tile + CODES + r * 16);
            if (ph == 0) sw1 = w; else sw0 = w;
#pragma unroll
            for (uint32_t u = 0; u < APT; u++)
                av[u] = *reinterpret_cast<const pf_v4i*>(abase[u % MW] + 256u * min(KW * nx + u / MW, nch - 1u));
            if (KW * s + kw < nch) {
                if (ph == 0) gemm_chunk<FMT, DI>(S, buf + aoff, cw0, sw0, xmin);
                else gemm_chunk<FMT, DI>(S, buf + aoff, cw1, sw1, xmin);
            }
        }
    }
    if constexpr (KW > 1) {
        int64_t* red = reinterpret_cast<int64_t*>(smem);   // [KW - 1][MW NW][16][64]: lanes on consecutive banks
        __syncthreads();
        if (kw > 0) {
#pragma unroll
            for (int i = 0; i < 16; i++) red[(((kw - 1u) * MW * NW + mw + MW * nw) * 16u + i) * 64u + lane] = S[i];
        }
        __syncthreads();
        if (kw == 0) {
#pragma unroll
            for (uint32_t k = 1; k < (uint32_t)KW; k++)
#pragma unroll
                for (int i = 0; i < 16; i++) S[i] += red[(((k - 1u) * MW * NW + mw + MW * nw) * 16u + i) * 64u + lane];
        }
    }
    if (kw != 0u || g >= ng) return;   // whole waves
    // output i of lane (r, h): activation row 8 (i / 4) + 4 h + i % 4 of the
    // wave's M tile, device row r of group g
    const uint32_t n = 32u * g + r;
    const double unit = __builtin_ldexp(1.0, (int)xmin - 25);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const uint32_t m = m0 + 32u * mw + 8u * (i / 4) + 4u * h + (i % 4);
        const float y = m < a.M ? (float)(((double)S[i] * unit) * (double)a.as[m]) : 0.0f;
        const float y1 = __shfl_xor(y, 1, 64), y16 = __shfl_xor(y, 16, 64);
        if (m < a.M) {
            const EpiPre pre = epi_prefetch<EPI>(a.e, m, n);
            epi_apply<EPI>(a.e, pre, a.N, m, n, y, y1, y16);
        }
    }
}

// ===================================================== row kernels (M > 8)

// The engine's RMSNorm of one row (1024 threads, element i = t + 1024 k) in
// the canonical tile order of the GEMV prologue: per 64-column tile a
// halving tree of x * x, tile sums added in column order from +0, then
// normed = (x * w) * inv.  K % 64 == 0, K <= 4096.
template <int PER>
__device__ __forceinline__ void norm_row_1024(float (&xv)[PER], const float (&wv)[PER], uint32_t K, float* row,
                                              float* tree, float* red) {
    const uint32_t t = threadIdx.x, wid = t >> 6, lane = t & 63u;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const uint32_t i = t + 1024u * k;
        if (i < K) row[i] = xv[k];
    }
    __syncthreads();
    for (uint32_t tl = wid; tl < K / 64u; tl += 16u) {
        const float v = row[64u * tl + lane];
        const float s = wave_tree_sum(v * v);
        if (lane == 0) tree[tl] = s;
    }
    __syncthreads();
    if (t == 0) {
        float ss = 0.0f;
        for (uint32_t tl = 0; tl < K / 64u; tl++) ss = ss + tree[tl];
        red[0] = ss;
    }
    __syncthreads();
    const float ss = red[0];
    __syncthreads();
    const float inv = 1.0f / __builtin_sqrtf(ss / (float)K + 1e-6f);
#pragma unroll
    for (int k = 0; k < PER; k++) xv[k] = (xv[k] * wv[k]) * inv;
}

// Grid M, 1024 threads: normed rows (fp32) of x into out; with nclear,
// block 0 zeroes that word (the layer-skip row counter of the layer).
template <int PER>
__global__ __launch_bounds__(1024) void k_norm_rows(const float* __restrict__ x, uint32_t K,
                                                    const float* __restrict__ w, float* __restrict__ out,
                                                    uint32_t* __restrict__ nclear) {
    __shared__ float row[4096];
    __shared__ float tree[64];
    __shared__ float red[16];
    const uint32_t m = blockIdx.x, t = threadIdx.x;
    if (nclear && m == 0 && t == 0) *nclear = 0u;
    float xv[PER], wv[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const uint32_t i = t + 1024u * k;
        xv[k] = i < K ? x[(size_t)m * K + i] : 0.0f;
        wv[k] = i < K ? w[i] : 0.0f;
    }
    norm_row_1024<PER>(xv, wv, K, row, tree, red);
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const uint32_t i = t + 1024u * k;
        if (i < K) out[(size_t)m * K + i] = xv[k];
    }
}

// Grid M, 1024 threads: normed rows quantized (quantize_activation_row)
// into q [M][q_stride] with row scales as[M].
template <int PER>
__global__ __launch_bounds__(1024) void k_norm_quant(const float* __restrict__ x, uint32_t K,
                                                     const float* __restrict__ w, int8_t* __restrict__ q,
                                                     uint32_t q_stride, float* __restrict__ as) {
    __shared__ float row[4096];
    __shared__ float tree[64];
    __shared__ float red[16];
    const uint32_t m = blockIdx.x, t = threadIdx.x;
    float xv[PER], wv[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const uint32_t i = t + 1024u * k;
        xv[k] = i < K ? x[(size_t)m * K + i] : 0.0f;
        wv[k] = i < K ? w[i] : 0.0f;
    }
    norm_row_1024<PER>(xv, wv, K, row, tree, red);
    __syncthreads();
    quantize_row_block<PER, 1024>(xv, K, q + (size_t)m * q_stride, as + m, nullptr, red);
}

}  // namespace pf
