// One decode pass (M <= 8 rows, every layer) as a single persistent kernel.
//
// One 256-thread workgroup per CU; the grid never exceeds what the device
// holds at once, so every workgroup is resident while others wait for it.
// Each layer has five phases, which every workgroup walks in order, taking
// its share of each:
//
//   QKV   a contiguous range of (64-row tile, 256-column split) items of the
//         fused QKV GEMV.  Each workgroup computes the RMSNorm statistics
//         and int8 codes of the whole residual rows itself (every workgroup
//         gets the same values), so no workgroup waits for another to
//         normalise.  Split sums meet in exact fp64 atomics; each item then
//         counts towards its head.
//   ATT   (head, 256-entry chunk) items over every row of the pass.  The
//         chunk's K/V rows from earlier passes are loaded before the head's
//         QKV sums are complete.  q/k/v, RoPE and the pass's own int8 K/V
//         rows are then formed from the sums (every item of a head forms
//         the same values; chunk 0 stores the rows), followed by the
//         scores, chunk max, exp, chunk sum and the V-weighted partials of
//         k_attn_chunk.  The last chunk of a head to finish merges the
//         head's chunks (k_attn_merge_quant's arithmetic) and publishes the
//         head's slice of the attention output and its row maxima.
//   O     (tile, split) items of the O projection; the last split of a tile
//         adds the tile to the residual rows.
//   GU    (gate|up tile pair, split) items; RMSNorm and codes of the whole
//         rows again in every workgroup; the last split of a pair applies
//         SwiGLU (src/engine.cpp:832-838) and publishes the pair's row
//         maxima.
//   DOWN  (tile, split) items; the last split of a tile adds the tile to
//         the residual rows and counts towards the next layer.
//
// Synchronisation.  Data that crosses workgroups is written and read with
// agent-scope (coherent) stores and loads, always issued in batches so that
// their latencies overlap.  A producer drains its memory operations
// (s_waitcnt 0) and the workgroup barrier before it counts, so a consumer
// that sees the count reads complete data.  Counters that workgroups poll
// only ever grow: a pass waits for (arrivals per pass) x epoch, the epoch
// being a device word that the last workgroup of a pass increments, so no
// counter is reset between passes.  Counters that only a last arrival
// reads are reset by that arrival.  Every wait is bounded in time; a
// timed-out wait sets the error word and every workgroup leaves.
//
// Every value is computed with the arithmetic and association order of the
// multi-kernel pass (k_resid_norm_quant, k_gemv_i8, k_qkv_post,
// k_attn_chunk, k_attn_merge_quant, k_swiglu_quant), so the two paths agree
// bit for bit.
#include "pf_device.h"

namespace pf {

// ------------------------------------------------------------ arguments

struct DecodeOffsets {
    uint32_t xin, xmid, acc_qkv, acc_o, acc_gu, acc_d, rs, amax_o, amax_f, o, f, S, Up, stats_a, stats_f;
};

enum : uint32_t { MAT_QKV = 0, MAT_O = 1, MAT_GU = 2, MAT_DOWN = 3 };

struct DecodeLayer {
    const uint8_t* w[4];     // tiled matrices: QKV, O, gate|up, down
    int32_t fmt[4];
    const float* an;         // attention-norm and FFN-norm weights [D]
    const float* fn;
};

struct DecodeArgs {
    const PassDesc* pd;
    KvGeom g;
    KvPlanes kv;
    const DecodeLayer* layers;   // [L]
    const float* rope_c;
    const float* rope_s;
    uint32_t L, D, F, H, hd;
    float* x;                    // [8][D] residual rows: input of layer 0, output of the last layer
    uint8_t* lbuf;               // per-layer buffers, lstride bytes per layer
    size_t lstride;
    DecodeOffsets off;           // byte offsets of the buffers within a layer
    uint32_t s_stride, cstride;  // floats per (row, head) of S; chunks per (row, head) of Up
    uint32_t* ctr;               // [L][ctr_layer] counter words
    uint32_t ctr_layer;
    uint32_t* glob;              // [0] workgroups done, [16] epoch (>= 1)
    uint32_t* err;               // nonzero after a timed-out wait
    uint64_t spin_limit;         // wall-clock ticks a wait may take
    uint64_t* trace;             // null, or [L][grid][DEC_TRACE] phase timestamps
};

// Buffers of one layer.  Each is written once per pass (by coherent
// stores or device-scope atomics) and read only after everything in it is
// complete, so its lines cannot be stale in any cache and consumers read it
// with plain loads.  Every buffer starts on a 256-byte boundary, so no
// cache line holds values of two buffers (a line read early for one buffer
// would be stale for the other).
struct LayerBufs {
    float* xin;                  // [8][D] input rows of the layer
    float* xmid;                 // [8][D] rows after the attention residual
    float* xout;                 // [8][D] output rows (the next layer's xin)
    double* acc_qkv;             // [8][3D], [8][D], [8][2F], [8][D]: zero before the pass,
    double* acc_o;               // cleared again by their consumers
    double* acc_gu;
    double* acc_d;
    float* rs;                   // [8] QKV input row scales
    float* amax_o;               // [H][8] row maxima of each head's output
    float* amax_f;               // [F / 64][8] row maxima of each SwiGLU tile
    float* o;                    // [8][D] attention output
    float* f;                    // [8][F] SwiGLU output
    float* S;                    // [8][H][s_stride] chunk max / sum
    float* Up;                   // [8][H][cstride][hd] chunk partials
    float* stats_a;              // [D / 64][8][2] tile statistics of xin (tree of x * x, max |x * w|)
    float* stats_f;              // the same for xmid
    float* stats_next;           // stats_a of the next layer (null in the last layer)
};

// Phase timestamps of one workgroup in one layer (wall clock, 100 MHz).
constexpr uint32_t DEC_TRACE = 32;
enum : uint32_t {
    TR_Q_WAIT = 0, TR_Q_NORM, TR_Q_DONE, TR_A_WAIT, TR_A_QKV, TR_A_DONE, TR_MERGE, TR_O_WAIT, TR_O_DONE,
    TR_O_FIN, TR_G_WAIT, TR_G_DONE, TR_G_FIN, TR_D_WAIT, TR_D_DONE, TR_D_FIN,
    TR_A_KVQ, TR_A_SELF, TR_A_SCORE, TR_A_EXP, TR_A_WSUM, TR_G_NORM, TR_O_AMAX, TR_D_AMAX,
    TR_SA_BEG, TR_SA_END, TR_SF_BEG, TR_SF_END, TR_Q_STATS, TR_G_STATS, TR_M_T, TR_M_END
};

// Counter words of one layer, each in its own 64-byte slot (16 words).
// Polled (grow by a fixed count per pass): x_ready, head_cnt, heads_done,
// xmid, pairs.  Last-arrival only (reset by the last arrival): att_cnt,
// o_tile, gu_pair, d_tile.
struct Ctr {
    uint32_t* base;
    uint32_t H, TD, TF;
    __device__ uint32_t* slot(uint32_t i) const { return base + 16u * i; }
    __device__ uint32_t* x_ready() const { return slot(0); }
    __device__ uint32_t* head_cnt(uint32_t h) const { return slot(1 + h); }
    __device__ uint32_t* att_cnt(uint32_t h) const { return slot(1 + H + h); }
    __device__ uint32_t* heads_done() const { return slot(1 + 2 * H); }
    __device__ uint32_t* o_tile(uint32_t t) const { return slot(2 + 2 * H + t); }
    __device__ uint32_t* xmid() const { return slot(2 + 2 * H + TD); }
    __device__ uint32_t* gu_pair(uint32_t p) const { return slot(3 + 2 * H + TD + p); }
    __device__ uint32_t* pairs() const { return slot(3 + 2 * H + TD + TF); }
    __device__ uint32_t* d_tile(uint32_t t) const { return slot(4 + 2 * H + TD + TF + t); }
};
__host__ __device__ constexpr uint32_t decode_ctr_slots(uint32_t H, uint32_t TD, uint32_t TF) {
    return 4 + 2 * H + 2 * TD + TF;
}

// ------------------------------------------------------------ shared memory
//
// One buffer, carved per phase:
//   GEMV  codes [8][2048] (QKV / GU: whole rows; O / DOWN: four 256-column
//         slots), block sums [8][64], fp64 wave partials [4][8][64]
//   ATT   V rows [256][144], fp32 q/k/v of the pass rows [3][8][128],
//         probabilities [8][256], V scales [256], wave partials
//         [8][4][128], int8 K/V rows of the pass [2][8][128], K rows
//         [256][144]
//   MERGE chunk maxima and sums [8][256][2], exp factors [8][256]
constexpr uint32_t DEC_MAXD = 2048;
// Items per prefetch batch (weights of a batch are loaded before the wait).
constexpr uint32_t DEC_IB = 3;
constexpr uint32_t G_SA = 0;
constexpr uint32_t G_SB = 8 * DEC_MAXD;                        // 16384
constexpr uint32_t G_RED = G_SB + 8 * 64 * 4;                 // 18432
constexpr uint32_t G_END = G_RED + 4 * 8 * 64 * 8;            // 34816
constexpr uint32_t A_VT = 0;                                  // [256][144]
constexpr uint32_t A_QS = 256 * 144;                          // 36864: [8][128] f32
constexpr uint32_t A_KF = A_QS + 8 * 128 * 4;
constexpr uint32_t A_VF = A_KF + 8 * 128 * 4;
constexpr uint32_t A_PE = A_VF + 8 * 128 * 4;                 // [8][256] f32
constexpr uint32_t A_VSC = A_PE + 8 * 256 * 4;                // [256] f32
constexpr uint32_t A_WP = A_VSC + 256 * 4;                    // [8][4][128] f32
constexpr uint32_t A_KQ = A_WP + 8 * 4 * 128 * 4;             // [8][128] i8
constexpr uint32_t A_VQ = A_KQ + 8 * 128;
constexpr uint32_t A_KT = A_VQ + 8 * 128;                    // [256][144] K rows
constexpr uint32_t A_END = A_KT + 256 * 144;
constexpr uint32_t M_SS = 0;                                  // [8][256][2] f32
constexpr uint32_t M_FS = M_SS + 8 * 256 * 2 * 4;             // [8][256] f32
constexpr uint32_t M_END = M_FS + 8 * 256 * 4;
constexpr uint32_t DEC_MAX_CHUNKS = 256;
constexpr uint32_t DEC_SMEM_AB = G_END > A_END ? G_END : A_END;
constexpr uint32_t DEC_SMEM = DEC_SMEM_AB > M_END ? DEC_SMEM_AB : M_END;

struct DecShared {
    uint32_t flag;
    float inv[8], invq[8], as[8];
    float red[4][8], red2[4][8];
    float mx[8], T[8], pself[8], selfs[8], ksn[8], vsn[8], hinv[8];
    float am[8 * 128];           // row maxima gathered from other workgroups
};

#define PF_TR(l, k)                                                                                  \
    do {                                                                                             \
        if (a.trace && threadIdx.x == 0)                                                             \
            a.trace[((size_t)(l) * gridDim.x + blockIdx.x) * DEC_TRACE + (k)] = wall_clock64();      \
    } while (0)

// Waits until the counter reaches target (wrapping compare: counters grow
// forever).  Thread 0 polls; every thread returns the verdict.  False when
// the wait timed out or another workgroup's did.
__device__ __forceinline__ bool wait_ge(const uint32_t* c, uint32_t target, const DecodeArgs& a, DecShared& sh) {
    if (threadIdx.x == 0) {
        uint32_t ok = 1;
        if ((int32_t)(ldc(c) - target) < 0) {
            const uint64_t t0 = wall_clock64();
            uint32_t it = 0;
            while ((int32_t)(ldc(c) - target) < 0) {
                __builtin_amdgcn_s_sleep(1);
                if ((++it & 15u) == 0u) {
                    if (ldc(a.err) != 0u) { ok = 0; break; }
                    if (wall_clock64() - t0 > a.spin_limit) {
                        atomicOr(a.err, 1u);
                        ok = 0;
                        break;
                    }
                }
            }
        }
        sh.flag = ok;
    }
    __syncthreads();
    const bool ok = sh.flag != 0u;
    __syncthreads();
    return ok;
}

// Thread 0 adds n to *c; every thread learns whether this made the count
// reach `total` (the last arrival).  Call after drain().
__device__ __forceinline__ bool arrive_last(uint32_t* c, uint32_t n, uint32_t total, DecShared& sh) {
    if (threadIdx.x == 0) sh.flag = (arrive_n(c, n) + n == total) ? 1u : 0u;
    __syncthreads();
    const bool last = sh.flag != 0u;
    __syncthreads();
    return last;
}

// ------------------------------------------------------------ row statistics

// sb[m][b] = sum of the int8 codes of 32-block b of row m (sa[m][DEC_MAXD]),
// for blocks b0 <= b < b0 + nb of rows m < M; exact v_dot4 sums against
// ones.  No barrier.
template <int M>
__device__ __forceinline__ void block_sums(const int8_t* sa, int32_t* sb, uint32_t b0, uint32_t nb) {
    for (uint32_t e = threadIdx.x; e < (uint32_t)M * nb; e += 256u) {
        const uint32_t m = e / nb, b = b0 + (e - m * nb);
        const int4 a0 = *reinterpret_cast<const int4*>(sa + m * DEC_MAXD + b * 32u);
        const int4 a1 = *reinterpret_cast<const int4*>(sa + m * DEC_MAXD + b * 32u + 16u);
        const int ones = 0x01010101;
        int sum = __builtin_amdgcn_sdot4(a0.x, ones, 0, false);
        sum = __builtin_amdgcn_sdot4(a0.y, ones, sum, false);
        sum = __builtin_amdgcn_sdot4(a0.z, ones, sum, false);
        sum = __builtin_amdgcn_sdot4(a0.w, ones, sum, false);
        sum = __builtin_amdgcn_sdot4(a1.x, ones, sum, false);
        sum = __builtin_amdgcn_sdot4(a1.y, ones, sum, false);
        sum = __builtin_amdgcn_sdot4(a1.z, ones, sum, false);
        sum = __builtin_amdgcn_sdot4(a1.w, ones, sum, false);
        sb[m * 64 + b] = sum;
    }
}

// The engine's RMSNorm (src/matmul_neon.cpp:231-239) in tile-canonical
// order, as k_resid_norm_quant computes it: the sum of squares of a row is
// the sequential sum over its 64-column tiles of each tile's halving tree
// of x * x, normed = (x * w) * inv, and quantize_activation_row's row
// maximum is fl(max |fl(x * w)| * inv) (rounding is monotone).  The wave
// holding (tile, row) with lane = column publishes the tile's tree and
// max |x * w| to st[tile][row].
__device__ __forceinline__ void tile_stat(float xv, float wv, float* st, uint32_t tile, uint32_t m) {
    const float s = wave_tree_sum(xv * xv);
    const float a = wave_max(fabsf(xv * wv));
    if ((threadIdx.x & 63u) == 0) {
        stc(st + (tile * 8u + m) * 2u, s);
        stc(st + (tile * 8u + m) * 2u + 1u, a);
    }
}

// Row factors from the tile statistics st[TD][8][2] (complete): sh.inv,
// sh.invq = 127 / amax, sh.as = amax / 127 (1 when amax is 0).
template <int M>
__device__ __forceinline__ void combine_stats(const float* st, uint32_t TD, uint32_t D, DecShared& sh) {
    const uint32_t t = threadIdx.x;
    if (t < TD * 8u) {
        const float2 v = *reinterpret_cast<const float2*>(st + 2u * t);
        sh.am[2u * t] = v.x;
        sh.am[2u * t + 1u] = v.y;
    }
    __syncthreads();
    if (t < (uint32_t)M) {
        float ss = 0.0f, ax = 0.0f;
        for (uint32_t t0 = 0; t0 < TD; t0 += 16) {
            float sv[16], av[16];
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const uint32_t tl = min(t0 + k, TD - 1u);
                sv[k] = sh.am[(tl * 8u + t) * 2u];
                av[k] = sh.am[(tl * 8u + t) * 2u + 1u];
            }
#pragma unroll
            for (int k = 0; k < 16; k++)
                if (t0 + k < TD) {
                    ss = ss + sv[k];
                    ax = fmaxf(ax, av[k]);
                }
        }
        const float inv = 1.0f / __builtin_sqrtf(ss / (float)D + 1e-6f);
        const float amax = ax * inv;
        sh.inv[t] = inv;
        sh.invq[t] = (amax == 0.0f) ? 1.0f : 127.0f / amax;
        sh.as[t] = (amax == 0.0f) ? 1.0f : amax / 127.0f;
    }
    __syncthreads();
}

// Codes of the 256-column slices [col0_i, col0_i + 256) of the normed rows
// (x[m] * w) * inv[m] with the row factors in sh: thread t takes column t
// of every slice and row (every load first).  Codes to sa[m][DEC_MAXD],
// then the slices' 32-block sums to sb.  Ends with a barrier.
template <int M>
__device__ __forceinline__ void norm_slices(const float* x, const float* w, uint32_t D, const uint32_t (&col0)[DEC_IB],
                                            uint32_t ns, int8_t* sa, int32_t* sb, DecShared& sh) {
    const uint32_t t = threadIdx.x;
    float v[DEC_IB][M], wv[DEC_IB];
#pragma unroll
    for (uint32_t i = 0; i < DEC_IB; i++) {
        const uint32_t c = col0[min(i, ns - 1u)] + t;
#pragma unroll
        for (int m = 0; m < M; m++) v[i][m] = x[(size_t)m * D + c];
        wv[i] = w[c];
    }
#pragma unroll
    for (uint32_t i = 0; i < DEC_IB; i++) {
        if (i >= ns) break;
#pragma unroll
        for (int m = 0; m < M; m++)
            sa[m * DEC_MAXD + col0[i] + t] = quant_code((v[i][m] * wv[i]) * sh.inv[m], sh.invq[m]);
    }
    __syncthreads();
    for (uint32_t i = 0; i < ns; i++) block_sums<M>(sa, sb, col0[i] >> 5, 8);
    __syncthreads();
}

// Codes of one 256-column slice of rows src[m] (row stride `stride`) with
// the row factors invq: thread t takes column t of every row (loads issued
// first).  Codes to sa[m][DEC_MAXD] at `col0`.  No barrier.
template <int M>
__device__ __forceinline__ void quant_slice256(const float* src, uint32_t stride, const float* invq, int8_t* sa,
                                               int32_t* sb, uint32_t col0) {
    const uint32_t t = threadIdx.x;
    float v[M];
#pragma unroll
    for (int m = 0; m < M; m++) v[m] = src[(size_t)m * stride + t];
#pragma unroll
    for (int m = 0; m < M; m++) sa[m * DEC_MAXD + col0 + t] = quant_code(v[m], invq[m]);
}

// Row factors of an input quantized with a global row maximum: amax[m] is
// the max over n values src[j * 8 + m] (gathered with batched loads),
// invq = 127 / amax, as = amax / 127 (1 when amax is 0).
template <int M>
__device__ __forceinline__ void gather_amax(const float* src_, uint32_t n, DecShared& sh) {
    const float* src = (const float*)(const __attribute__((address_space(1))) float*)src_;
    const uint32_t t = threadIdx.x;
    for (uint32_t e0 = 0; e0 < n * 8u; e0 += 1024u) {
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = src[min(e0 + t + 256u * k, n * 8u - 1u)];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t e = e0 + t + 256u * k;
            if (e < n * 8u) sh.am[e - e0] = v[k];
        }
        __syncthreads();
        if (t < (uint32_t)M) {
            float a = e0 == 0 ? 0.0f : sh.as[t];
            const uint32_t jn = min(128u, n - e0 / 8u);
            for (uint32_t j = 0; j < jn; j++) a = fmaxf(a, sh.am[j * 8u + t]);
            sh.as[t] = a;   // running maximum
        }
    }
    __syncthreads();
    if (t < (uint32_t)M) {
        const float amax = sh.as[t];
        sh.invq[t] = (amax == 0.0f) ? 1.0f : 127.0f / amax;
        sh.as[t] = (amax == 0.0f) ? 1.0f : amax / 127.0f;
    }
    __syncthreads();
}

// ------------------------------------------------------------ GEMV items

// Raw weight words of one wave's two blocks of a (tile, split) item: code
// bytes (4 dwords per block for Q4, 2 for Q2 / Q1.5) and the two fp16 block
// scales of the lane's row.
struct WRaw {
    uint32_t c[2][4];
    uint32_t s;
};

template <int FMT>
__device__ __forceinline__ void load_raw2(const uint8_t* W, uint32_t K, uint32_t tile, uint32_t split, uint32_t wid,
                                          uint32_t lane, WRaw& w) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    typedef unsigned int v2u __attribute__((ext_vector_type(2)));
    typedef const __attribute__((address_space(1))) uint8_t gu8;
    typedef const __attribute__((address_space(1))) v4u gu128;
    typedef const __attribute__((address_space(1))) v2u gu64;
    typedef const __attribute__((address_space(1))) uint32_t gu32;
    constexpr uint32_t TB = tile_bytes(FMT);
    constexpr uint32_t CODES = TILE_ROWS * TILE_BLOCKS * code_bytes(FMT);
    gu8* tp = (gu8*)W + ((size_t)tile * (K >> 8) + split) * TB;
    const uint32_t t0 = 2u * wid;
    if constexpr (FMT == FMT_Q4) {
        gu8* cp = tp + t0 * 1024u + lane * 16u;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const v4u c = *(gu128*)(cp + k * 1024);
            w.c[k][0] = c.x; w.c[k][1] = c.y; w.c[k][2] = c.z; w.c[k][3] = c.w;
        }
    } else {
        // blocks t0, t0 + 1 are one block pair: 1 KiB, 16 bytes per row
        const v4u c = *(gu128*)(tp + (t0 >> 1) * 1024u + lane * 16u);
        w.c[0][0] = c.x; w.c[0][1] = c.y; w.c[1][0] = c.z; w.c[1][1] = c.w;
        w.c[0][2] = w.c[0][3] = w.c[1][2] = w.c[1][3] = 0u;
    }
    w.s = *(gu32*)(tp + CODES + lane * 16u + t0 * 2u);
}

__device__ __forceinline__ void load_w2(int32_t fmt, const uint8_t* W, uint32_t K, uint32_t tile, uint32_t split,
                                        uint32_t wid, uint32_t lane, WRaw& w) {
    if (fmt == FMT_Q4) load_raw2<FMT_Q4>(W, K, tile, split, wid, lane, w);
    else if (fmt == FMT_Q2) load_raw2<FMT_Q2>(W, K, tile, split, wid, lane, w);
    else load_raw2<FMT_Q15>(W, K, tile, split, wid, lane, w);
}

// The eight code dwords of block k (unpack_codes' element order).
__device__ __forceinline__ void unpack_raw(int32_t fmt, const WRaw& w, int k, uint32_t u[8]) {
    if (fmt == FMT_Q4) {
        const uint32_t m = 0x0F0F0F0Fu;
        u[0] = w.c[k][0] & m; u[1] = w.c[k][1] & m; u[2] = w.c[k][2] & m; u[3] = w.c[k][3] & m;
        u[4] = (w.c[k][0] >> 4) & m; u[5] = (w.c[k][1] >> 4) & m;
        u[6] = (w.c[k][2] >> 4) & m; u[7] = (w.c[k][3] >> 4) & m;
    } else {
        const uint32_t m = 0x03030303u;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            u[2 * p] = (w.c[k][0] >> (2 * p)) & m;
            u[2 * p + 1] = (w.c[k][1] >> (2 * p)) & m;
        }
    }
}

// S[m] += the exact block products d_b * p_b of the wave's two blocks of
// an item for the lane's row (k_gemv_i8's body): p_b = dot(u, a) - off *
// sum(a) with v_dot4, activation codes and block sums read from LDS at
// block b0 (wave-uniform addresses).
template <int M>
__device__ __forceinline__ void item_dots(const WRaw& w, int32_t fmt, const int8_t* sa, const int32_t* sb, uint32_t b0,
                                          double (&S)[M]) {
    const int off = code_offset(fmt);
#pragma unroll
    for (int k = 0; k < 2; k++) {
        uint32_t u[8];
        unpack_raw(fmt, w, k, u);
        const double dk = (double)h2f((uint16_t)(w.s >> (16 * k)));
        const uint32_t b = b0 + (uint32_t)k;
        int4 a0[M], a1[M];
        int p[M];
#pragma unroll
        for (int m = 0; m < M; m++) {
            a0[m] = *reinterpret_cast<const int4*>(sa + m * DEC_MAXD + b * 32u);
            a1[m] = *reinterpret_cast<const int4*>(sa + m * DEC_MAXD + b * 32u + 16u);
            p[m] = -off * sb[m * 64 + b];
        }
        // the rows' integer chains interleaved (independent, exact)
#pragma unroll
        for (int m = 0; m < M; m++) p[m] = __builtin_amdgcn_sdot4((int)u[0], a0[m].x, p[m], false);
#pragma unroll
        for (int m = 0; m < M; m++) p[m] = __builtin_amdgcn_sdot4((int)u[1], a0[m].y, p[m], false);
#pragma unroll
        for (int m = 0; m < M; m++) p[m] = __builtin_amdgcn_sdot4((int)u[2], a0[m].z, p[m], false);
#pragma unroll
        for (int m = 0; m < M; m++) p[m] = __builtin_amdgcn_sdot4((int)u[3], a0[m].w, p[m], false);
#pragma unroll
        for (int m = 0; m < M; m++) p[m] = __builtin_amdgcn_sdot4((int)u[4], a1[m].x, p[m], false);
#pragma unroll
        for (int m = 0; m < M; m++) p[m] = __builtin_amdgcn_sdot4((int)u[5], a1[m].y, p[m], false);
#pragma unroll
        for (int m = 0; m < M; m++) p[m] = __builtin_amdgcn_sdot4((int)u[6], a1[m].z, p[m], false);
#pragma unroll
        for (int m = 0; m < M; m++) p[m] = __builtin_amdgcn_sdot4((int)u[7], a1[m].w, p[m], false);
#pragma unroll
        for (int m = 0; m < M; m++) S[m] = __builtin_fma(dk, (double)p[m], S[m]);
    }
}

// acc[m][col0 + r] += the four waves' S[m] of row r (exact fp64, so the
// order of the additions and of the atomics never changes a bit); S is
// cleared.
template <int M>
__device__ __forceinline__ void flush_tile(double (&S)[M], double* red, double* acc, uint32_t acc_stride,
                                           uint32_t col0) {
    const uint32_t t = threadIdx.x, lane = t & 63u, wid = t >> 6;
#pragma unroll
    for (int m = 0; m < M; m++) {
        red[(wid * 8 + m) * 64 + lane] = S[m];
        S[m] = 0.0;
    }
    __syncthreads();
    for (uint32_t e = t; e < (uint32_t)M * 64u; e += 256u) {
        const uint32_t m = e >> 6, r = e & 63u;
        const double v = red[(0 * 8 + m) * 64 + r] + red[(1 * 8 + m) * 64 + r] + red[(2 * 8 + m) * 64 + r] +
                         red[(3 * 8 + m) * 64 + r];
        atomicAdd(acc + (size_t)m * acc_stride + col0 + r, v);
    }
    __syncthreads();
}



// Contiguous item range [lo, hi) of workgroup w out of G for N items.
__device__ __forceinline__ void item_range(uint32_t N, uint32_t w, uint32_t G, uint32_t& lo, uint32_t& hi) {
    lo = (uint32_t)(((uint64_t)w * N) / G);
    hi = (uint32_t)(((uint64_t)(w + 1) * N) / G);
}

// Tiles (of `per` items each) t0 .. t0 + DEC_IB - 1 overlapping [lo, hi):
// thread 0 adds each tile's item count to its counter ctr(tile), every
// atomic in flight together; bit j of the result is set when tile t0 + j
// got its last arrival (its counter then reset for the next pass).  Call
// after drain().
template <class C>
__device__ __forceinline__ uint32_t arrive_tiles(C ctr, uint32_t t0, uint32_t lo, uint32_t hi, uint32_t per,
                                                 DecShared& sh) {
    if (threadIdx.x == 0) {
        uint32_t old[DEC_IB], n[DEC_IB];
#pragma unroll
        for (uint32_t j = 0; j < DEC_IB; j++) {
            const uint32_t tl = t0 + j, a0 = max(lo, tl * per), a1 = min(hi, (tl + 1) * per);
            n[j] = a1 > a0 ? a1 - a0 : 0u;
            old[j] = n[j] ? arrive_n(ctr(tl), n[j]) : 0u;
        }
        uint32_t mask = 0;
#pragma unroll
        for (uint32_t j = 0; j < DEC_IB; j++)
            if (n[j] && old[j] + n[j] == per) {
                mask |= 1u << j;
                stc(ctr(t0 + j), 0u);
            }
        sh.flag = mask;
    }
    __syncthreads();
    const uint32_t mask = sh.flag;
    __syncthreads();
    return mask;
}

// Tile of element group jj among the set bits of mask (bit j = tile t0 + j).
__device__ __forceinline__ uint32_t nth_tile(uint32_t mask, uint32_t t0, uint32_t jj) {
    uint32_t j = 0;
#pragma unroll
    for (uint32_t b = 0; b < DEC_IB; b++) {
        if (mask & (1u << b)) {
            if (jj == 0) j = b;
            jj = jj == 0 ? 0xFFFFFFFFu : jj - 1u;
        }
    }
    return t0 + j;
}

// xd[m][64 tile + r] = xs[...] + (float)(acc * as[m]) for the tiles of
// mask, acc cleared (k_resid_norm_quant's residual), and with wn (the next
// RMSNorm's weights) the tiles' statistics of xd to st; every load first.
// A wave holds one (tile, row) with lane = column.
template <int M>
__device__ __forceinline__ void finalize_resid(uint32_t mask, uint32_t t0, const float* xs, float* xd, double* acc,
                                               uint32_t D, const DecShared& sh, const float* wn, float* st) {
    constexpr uint32_t PER = (DEC_IB * M * 64 + 255) / 256;
    const uint32_t n = __builtin_popcount(mask) * (uint32_t)M * 64u;
    float xv[PER], wq[PER];
    double av[PER];
    size_t off[PER];
    uint32_t mr[PER];
#pragma unroll
    for (uint32_t k = 0; k < PER; k++) {
        const uint32_t e = min(threadIdx.x + 256u * k, n - 1u), jj = e / ((uint32_t)M * 64u), r = e - jj * M * 64u;
        const uint32_t m = r >> 6, col = nth_tile(mask, t0, jj) * 64u + (r & 63u);
        off[k] = (size_t)m * D + col;
        mr[k] = m;
        xv[k] = xs[off[k]];
        av[k] = acc[off[k]];
        wq[k] = wn ? wn[col] : 0.0f;
    }
#pragma unroll
    for (uint32_t k = 0; k < PER; k++) {
        if (threadIdx.x + 256u * k >= n) continue;   // wave-uniform (n % 64 == 0)
        const float xn = xv[k] + (float)(av[k] * (double)sh.as[mr[k]]);
        stc(xd + off[k], xn);
        stc(acc + off[k], 0.0);
        if (wn) tile_stat(xn, wq[k], st, (uint32_t)(off[k] % D) >> 6, mr[k]);
    }
}

// ------------------------------------------------------------ attention

// Entry j of a view whose position is >= pos0 (a row of this pass), or
// UINT32_MAX: sink entries hold positions 0.., window entry w holds
// position sink_size + w, pooled rows hold no single position.
__device__ __forceinline__ uint32_t entry_pass_row(const KvGeom& g, const KvView& v, uint32_t j, uint32_t pos0) {
    uint32_t p;
    if (j < v.sink) {
        p = j;
    } else {
        const uint32_t r = j - v.sink;
        if (r < v.pool) return 0xFFFFFFFFu;
        p = g.sink_size + v.win_lo + (r - v.pool);
    }
    return p >= pos0 ? p - pos0 : 0xFFFFFFFFu;
}

// Loads the K row (LDS kt[t]) and V row (LDS vt[t]) of entry j of view v
// for thread t, unless the entry is beyond `count` or a row of this pass
// (returned as its pass row, filled in later from the pass's own rows).
template <int PARTS>
__device__ __forceinline__ uint32_t load_entry(const KvGeom& g, const KvPlanes& kv, size_t plane, const KvView& v,
                                               uint32_t j, uint32_t count, uint32_t pos0, int8_t (*kt)[144],
                                               float& ks, float& vs, int8_t (*vt)[144]) {
    constexpr uint32_t hd = 16 * PARTS;
    ks = 0.0f;
    vs = 0.0f;
    if (j >= count) return 0xFFFFFFFEu;
    const uint32_t pr = entry_pass_row(g, v, j, pos0);
    if (pr != 0xFFFFFFFFu) return pr;
    const size_t row = plane * g.rows + kv_row(g, v, j);
    const int4* kr = reinterpret_cast<const int4*>(kv.k + row * hd);
    const int4* vr = reinterpret_cast<const int4*>(kv.v + row * hd);
    int4 kw[PARTS], vw[PARTS];
#pragma unroll
    for (int p = 0; p < PARTS; p++) {
        kw[p] = kr[p];
        vw[p] = vr[p];
    }
    ks = kv.ks[row];
    vs = kv.vs[row];
#pragma unroll
    for (int p = 0; p < PARTS; p++) {
        *reinterpret_cast<int4*>(&kt[threadIdx.x][p * 16]) = kw[p];
        *reinterpret_cast<int4*>(&vt[threadIdx.x][p * 16]) = vw[p];
    }
    return 0xFFFFFFFFu;
}

// Two views with the same sink / pool / window start map every list index
// to the same plane row (they differ only in their counts).
__device__ __forceinline__ bool same_map(const KvView& a, const KvView& b) {
    return a.sink == b.sink && a.pool == b.pool && a.win_lo == b.win_lo;
}

// Attention item (head h, chunk c) over rows m < pm of the pass, which
// share the fused QKV sums of the head.  Returns false on a failed wait.
template <int M, int PARTS>
__device__ __forceinline__ bool attn_item(const DecodeArgs& a, const LayerBufs& B, const Ctr& cc, uint32_t l, uint32_t h,
                                          uint32_t c, uint32_t pos0, uint32_t pm, uint32_t head_target, uint8_t* smem,
                                          DecShared& sh) {
    constexpr uint32_t hd = 16 * PARTS, half = hd / 2;
    const KvGeom& g = a.g;
    const uint32_t t = threadIdx.x, lane = t & 63u, wid = t >> 6;
    const uint32_t H = a.H, D = a.D;
    int8_t (*vt)[144] = reinterpret_cast<int8_t (*)[144]>(smem + A_VT);
    int8_t (*kt)[144] = reinterpret_cast<int8_t (*)[144]>(smem + A_KT);
    float* qs = reinterpret_cast<float*>(smem + A_QS);    // [8][128]
    float* kf = reinterpret_cast<float*>(smem + A_KF);
    float* vf = reinterpret_cast<float*>(smem + A_VF);
    float* pe = reinterpret_cast<float*>(smem + A_PE);    // [8][256]
    float* vsc = reinterpret_cast<float*>(smem + A_VSC);  // [256]
    float* wp = reinterpret_cast<float*>(smem + A_WP);    // [8][4][128]
    int8_t* kq = reinterpret_cast<int8_t*>(smem + A_KQ);  // [8][128]
    int8_t* vq = reinterpret_cast<int8_t*>(smem + A_VQ);
    const size_t plane = (size_t)l * g.n_heads + h;
    const uint32_t j = c * 256u + t;

    // first group of rows sharing one list -> plane-row map; its entries
    // are loaded before the wait
    uint32_t m0 = 0, m1 = 1;
    KvView v0 = kv_view(g, pos0);
    while (m1 < pm && same_map(kv_view(g, pos0 + m1), v0)) m1++;
    float ks, vs;
    uint32_t pr = load_entry<PARTS>(g, a.kv, plane, v0, j, kv_view(g, pos0 + m1 - 1).count(), pos0, kt, ks, vs, vt);

    PF_TR(l, TR_A_WAIT);
    if (!wait_ge(cc.head_cnt(h), head_target, a, sh)) return false;

    // q/k/v of the head for every pass row from the exact sums: RoPE
    // (src/engine.cpp:732-749), fp32 rows to LDS (k_qkv_post's arithmetic)
    {
        constexpr uint32_t NE = (M * half + 255) / 256;   // pairs per thread
        double aq[NE][2], ak[NE][2], av[NE][2];
        float sc[NE], cs[NE], sn[NE];
        // every load first (pairs past the pass rows re-read the last one)
#pragma unroll
        for (uint32_t k = 0; k < NE; k++) {
            const uint32_t e = min(t + 256u * k, pm * half - 1u), m = e / half, p = e - m * half;
            const double* r = B.acc_qkv + (size_t)m * 3 * D + h * hd + 2 * p;
            aq[k][0] = r[0]; aq[k][1] = r[1];
            ak[k][0] = r[D]; ak[k][1] = r[D + 1];
            av[k][0] = r[2 * D]; av[k][1] = r[2 * D + 1];
            sc[k] = B.rs[m];
            const uint32_t pos = pos0 + m;
            cs[k] = a.rope_c[(size_t)pos * half + p];
            sn[k] = a.rope_s[(size_t)pos * half + p];
        }
#pragma unroll
        for (uint32_t k = 0; k < NE; k++) {
            const uint32_t e = t + 256u * k, m = e / half, p = e - m * half;
            if (e >= pm * half) continue;
            const double s = (double)sc[k];
            const float q0 = (float)(aq[k][0] * s), q1 = (float)(aq[k][1] * s);
            const float k0 = (float)(ak[k][0] * s), k1 = (float)(ak[k][1] * s);
            qs[m * 128 + 2 * p] = __builtin_fmaf(q0, cs[k], -(q1 * sn[k]));
            qs[m * 128 + 2 * p + 1] = __builtin_fmaf(q0, sn[k], q1 * cs[k]);
            kf[m * 128 + 2 * p] = __builtin_fmaf(k0, cs[k], -(k1 * sn[k]));
            kf[m * 128 + 2 * p + 1] = __builtin_fmaf(k0, sn[k], k1 * cs[k]);
            vf[m * 128 + 2 * p] = (float)(av[k][0] * s);
            vf[m * 128 + 2 * p + 1] = (float)(av[k][1] * s);
        }
    }
    __syncthreads();
    PF_TR(l, TR_A_QKV);
    // int8 K/V rows of the pass (KVCache::quantize_row, src/kv_cache.cpp:
    // 19-28); wave w takes rows w, w + 4; chunk 0 stores them
    for (uint32_t m = wid; m < pm; m += 4) {
        const bool act = lane < half;
        const float k0 = act ? kf[m * 128 + 2 * lane] : 0.0f, k1 = act ? kf[m * 128 + 2 * lane + 1] : 0.0f;
        const float v0f = act ? vf[m * 128 + 2 * lane] : 0.0f, v1f = act ? vf[m * 128 + 2 * lane + 1] : 0.0f;
        float ak = act ? fmaxf(fabsf(k0), fabsf(k1)) : 0.0f;
        float av = act ? fmaxf(fabsf(v0f), fabsf(v1f)) : 0.0f;
        ak = wave_max(ak);
        av = wave_max(av);
        const float ik = (ak == 0.0f) ? 1.0f : 127.0f / ak;
        const float iv = (av == 0.0f) ? 1.0f : 127.0f / av;
        const float ksc = (ak == 0.0f) ? 1.0f : ak / 127.0f, vscl = (av == 0.0f) ? 1.0f : av / 127.0f;
        if (act) {
            kq[m * 128 + 2 * lane] = quant_code(k0, ik);
            kq[m * 128 + 2 * lane + 1] = quant_code(k1, ik);
            vq[m * 128 + 2 * lane] = quant_code(v0f, iv);
            vq[m * 128 + 2 * lane + 1] = quant_code(v1f, iv);
        }
        if (lane == 0) {
            sh.ksn[m] = ksc;
            sh.vsn[m] = vscl;
        }
        const uint32_t row = kv_store_row(g, pos0 + m);
        if (c == 0 && row != 0xFFFFFFFFu) {
            const size_t base = (plane * g.rows + row) * hd;
            if (act) {
                const uint32_t kc = (uint32_t)(uint8_t)quant_code(k0, ik) | ((uint32_t)(uint8_t)quant_code(k1, ik) << 8);
                const uint32_t vc = (uint32_t)(uint8_t)quant_code(v0f, iv) | ((uint32_t)(uint8_t)quant_code(v1f, iv) << 8);
                *reinterpret_cast<uint16_t*>(a.kv.k + base + 2 * lane) = (uint16_t)kc;
                *reinterpret_cast<uint16_t*>(a.kv.v + base + 2 * lane) = (uint16_t)vc;
            }
            if (lane == 0) {
                a.kv.ks[plane * g.rows + row] = ksc;
                a.kv.vs[plane * g.rows + row] = vscl;
            }
        }
    }
    __syncthreads();
    PF_TR(l, TR_A_KVQ);

    const float scale = 1.0f / __builtin_sqrtf((float)hd);
    for (bool first = true; m0 < pm; first = false) {
        if (!first) {
            v0 = kv_view(g, pos0 + m0);
            m1 = m0 + 1;
            while (m1 < pm && same_map(kv_view(g, pos0 + m1), v0)) m1++;
            __syncthreads();   // vt, pe, wp of the previous group are consumed
            pr = load_entry<PARTS>(g, a.kv, plane, v0, j, kv_view(g, pos0 + m1 - 1).count(), pos0, kt, ks, vs, vt);
        }
        // this pass's rows among the entries come from the int8 rows above
        if (pr < pm) {
#pragma unroll
            for (int p = 0; p < PARTS; p++) {
                *reinterpret_cast<int4*>(&kt[t][p * 16]) = *reinterpret_cast<const int4*>(kq + pr * 128 + 16 * p);
                *reinterpret_cast<int4*>(&vt[t][p * 16]) = *reinterpret_cast<const int4*>(vq + pr * 128 + 16 * p);
            }
            ks = sh.ksn[pr];
            vs = sh.vsn[pr];
        }
        vsc[t] = vs;
        uint32_t C[M];
        bool live[M];
#pragma unroll
        for (int m = 0; m < M; m++) {
            live[m] = (uint32_t)m >= m0 && (uint32_t)m < m1;
            C[m] = live[m] ? kv_view(g, pos0 + m).count() : 0u;
            live[m] = live[m] && c * 256u < C[m] + 1u;
        }
        // self scores: the lane whose entry is row m's own position
        // (sequential sum of the fp32 query and key, k_attn_chunk's order)
        uint32_t my = 0xFFFFFFFFu;
#pragma unroll
        for (int m = 0; m < M; m++)
            if (live[m] && j == C[m]) my = (uint32_t)m;
        __syncthreads();
        if (my != 0xFFFFFFFFu) {
            float self = 0.0f;
            for (uint32_t i = 0; i < hd; i++) self = self + qs[my * 128 + i] * kf[my * 128 + i];
            sh.selfs[my] = self * scale;
        }
        PF_TR(l, TR_A_SELF);
        // scores of every live row against this thread's entry: fmaf chains
        // over the dimensions, one per row, sharing the dequantized key
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; m++) acc[m] = 0.0f;
#pragma unroll 1
        for (int p = 0; p < PARTS; p++) {
            // every read of the step first (one LDS round trip per step),
            // then the dequantized key and the fmaf chains
            const int4 kc = *reinterpret_cast<const int4*>(&kt[t][p * 16]);
            float4 qv[M][4];
#pragma unroll
            for (int m = 0; m < M; m++)
#pragma unroll
                for (int b4 = 0; b4 < 4; b4++) qv[m][b4] = *reinterpret_cast<const float4*>(qs + m * 128 + p * 16 + b4 * 4);
            __builtin_amdgcn_sched_barrier(0);
            const int wv[4] = {kc.x, kc.y, kc.z, kc.w};
            float kd[16];
#pragma unroll
            for (int b = 0; b < 16; b++) kd[b] = (float)(int8_t)((wv[b >> 2] >> (8 * (b & 3))) & 0xFF) * ks;
#pragma unroll
            for (int m = 0; m < M; m++) {
                // every row, live or not (no branches); rows that are not
                // live are ignored
#pragma unroll
                for (int b4 = 0; b4 < 4; b4++) {
                    acc[m] = __builtin_fmaf(qv[m][b4].x, kd[4 * b4], acc[m]);
                    acc[m] = __builtin_fmaf(qv[m][b4].y, kd[4 * b4 + 1], acc[m]);
                    acc[m] = __builtin_fmaf(qv[m][b4].z, kd[4 * b4 + 2], acc[m]);
                    acc[m] = __builtin_fmaf(qv[m][b4].w, kd[4 * b4 + 3], acc[m]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();   // self scores published
        PF_TR(l, TR_A_SCORE);
        float s[M];
#pragma unroll
        for (int m = 0; m < M; m++) {
            s[m] = -__builtin_inff();
            if (live[m]) {
                if (j < C[m]) s[m] = acc[m] * scale;
                else if (j == C[m]) s[m] = sh.selfs[m];
            }
            const float w = wave_max(s[m]);
            if (lane == 0) sh.red[wid][m] = w;
        }
        __syncthreads();
        float ex[M];
#pragma unroll
        for (int m = 0; m < M; m++) {
            const float mx = fmaxf(fmaxf(fmaxf(sh.red[0][m], sh.red[1][m]), sh.red[2][m]), sh.red[3][m]);
            ex[m] = (live[m] && j < C[m] + 1u) ? expf_c(s[m] - mx) : 0.0f;
            pe[m * 256 + t] = (live[m] && j < C[m]) ? ex[m] : 0.0f;
            if (live[m] && j == C[m]) sh.pself[m] = ex[m];
            if (t == 0) sh.mx[m] = mx;
            const float w = wave_tree_sum(ex[m]);
            if (lane == 0) sh.red2[wid][m] = w;
        }
        __syncthreads();
        PF_TR(l, TR_A_EXP);
        // V-weighted partials: sub-chunk sc = wave, dims i0, i0 + 1 = lane
        // pair; entries in order, the pass row's own fp32 value last
        uint32_t nv_max = 0;
#pragma unroll
        for (int m = 0; m < M; m++)
            if (live[m]) nv_max = max(nv_max, min(256u, C[m] > c * 256u ? C[m] - c * 256u : 0u));
        const uint32_t sc = wid, i0 = 2u * lane;
        if (i0 < hd) {
            float w0[M], w1[M];
#pragma unroll
            for (int m = 0; m < M; m++) w0[m] = w1[m] = 0.0f;
            const uint32_t e_end = min(64u * sc + 64u, (nv_max + 7u) & ~7u);
            for (uint32_t e = 64u * sc; e < e_end; e += 8) {
                // every read of the step first (one LDS round trip)
                uint32_t cc2[8];
#pragma unroll
                for (int u = 0; u < 8; u++) cc2[u] = *reinterpret_cast<const uint16_t*>(&vt[e + u][i0]);
                const float4 vs0 = *reinterpret_cast<const float4*>(vsc + e);
                const float4 vs1 = *reinterpret_cast<const float4*>(vsc + e + 4);
                float4 pp0[M], pp1[M];
#pragma unroll
                for (int m = 0; m < M; m++) {
                    pp0[m] = *reinterpret_cast<const float4*>(pe + m * 256 + e);
                    pp1[m] = *reinterpret_cast<const float4*>(pe + m * 256 + e + 4);
                }
                __builtin_amdgcn_sched_barrier(0);
                const float vsu[8] = {vs0.x, vs0.y, vs0.z, vs0.w, vs1.x, vs1.y, vs1.z, vs1.w};
                float vv0[8], vv1[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    vv0[u] = (float)(int8_t)(cc2[u] & 0xFFu) * vsu[u];
                    vv1[u] = (float)(int8_t)(cc2[u] >> 8) * vsu[u];
                }
#pragma unroll
                for (int m = 0; m < M; m++) {
                    // rows that are not live have zero weights here
                    const float pw[8] = {pp0[m].x, pp0[m].y, pp0[m].z, pp0[m].w, pp1[m].x, pp1[m].y, pp1[m].z, pp1[m].w};
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        w0[m] = __builtin_fmaf(pw[u], vv0[u], w0[m]);
                        w1[m] = __builtin_fmaf(pw[u], vv1[u], w1[m]);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int m = 0; m < M; m++) {
                if (!live[m]) continue;
                const uint32_t js = C[m] - c * 256u;
                if (js < 256u && (js >> 6) == sc) {
                    const float p = sh.pself[m];
                    w0[m] = __builtin_fmaf(p, vf[m * 128 + i0], w0[m]);
                    w1[m] = __builtin_fmaf(p, vf[m * 128 + i0 + 1], w1[m]);
                }
                wp[(m * 4 + sc) * 128 + i0] = w0[m];
                wp[(m * 4 + sc) * 128 + i0 + 1] = w1[m];
            }
        }
        __syncthreads();
        PF_TR(l, TR_A_WSUM);
        for (uint32_t e = t; e < (uint32_t)M * hd; e += 256u) {
            const uint32_t m = e / hd, d = e - m * hd;
            bool lv = false;
#pragma unroll
            for (int mm = 0; mm < M; mm++)
                if ((uint32_t)mm == m) lv = live[mm];
            if (!lv) continue;
            float u = 0.0f;
            u = u + wp[(m * 4 + 0) * 128 + d];
            u = u + wp[(m * 4 + 1) * 128 + d];
            u = u + wp[(m * 4 + 2) * 128 + d];
            u = u + wp[(m * 4 + 3) * 128 + d];
            const size_t mh = (size_t)m * H + h;
            stc(B.Up + (mh * a.cstride + c) * hd + d, u);
        }
        if (t < (uint32_t)M) {
            bool lv = false;
#pragma unroll
            for (int mm = 0; mm < M; mm++)
                if ((uint32_t)mm == t) lv = live[mm];
            if (lv) {
                const float T = (sh.red2[0][t] + sh.red2[2][t]) + (sh.red2[1][t] + sh.red2[3][t]);
                const size_t mh = (size_t)t * H + h;
                stc(B.S + mh * a.s_stride + 2 * c, sh.mx[t]);
                stc(B.S + mh * a.s_stride + 2 * c + 1, T);
            }
        }
        m0 = m1;
    }
    return true;
}

// The last chunk of head h: every row's chunks merged (max of the chunk
// maxima, f_c = exp(m_c - max), T and U fmaf chains over c in order, out =
// U * (1 / (T + 1e-10))); rows past the pass are written as 0.  Publishes
// the head's output slice and row maxima, clears the head's QKV sums.
// Every load that does not depend on another is issued first: the clears,
// the thread's chunk partials of its outputs (first 16 chunks) and the
// chunk statistics.
template <int M>
__device__ __forceinline__ void merge_head(const DecodeArgs& a, const LayerBufs& B, uint32_t l, uint32_t h,
                                           uint32_t pos0, uint32_t pm, uint8_t* smem, DecShared& sh) {
    const KvGeom& g = a.g;
    const uint32_t hd = a.hd, H = a.H, D = a.D, t = threadIdx.x, lane = t & 63u, wid = t >> 6;
    float* ts = reinterpret_cast<float*>(smem + M_SS);   // [8][256] chunk sums
    float* fs = reinterpret_cast<float*>(smem + M_FS);   // [8][256] exp factors
    constexpr uint32_t KO = (M * 128 + 255) / 256;      // outputs per thread (head_dim <= 128)
    uint32_t nc[M];
#pragma unroll
    for (int m = 0; m < M; m++) nc[m] = (uint32_t)m < pm ? (kv_view(g, pos0 + m).count() + 1 + 255) / 256 : 0u;
    auto nc_of = [&](uint32_t m) {
        uint32_t r = 0;
#pragma unroll
        for (int mm = 0; mm < M; mm++)
            if ((uint32_t)mm == m) r = nc[mm];
        return r;
    };
    // the head's QKV sums are consumed by every chunk of the head: clear
    for (uint32_t e = t; e < (uint32_t)M * 3u * hd; e += 256u) {
        const uint32_t m = e / (3u * hd), r = e - m * 3u * hd, part = r / hd, i = r - part * hd;
        stc(B.acc_qkv + (size_t)m * 3 * D + (size_t)part * D + h * hd + i, 0.0);
    }
    // this thread's outputs e = t + 256 k: partials of the first 16 chunks
    float uv[KO][16];
#pragma unroll
    for (uint32_t k = 0; k < KO; k++) {
        const uint32_t e = min(t + 256u * k, (uint32_t)M * hd - 1u), m = e / hd, i = e - m * hd;
        const uint32_t ncr = max(nc_of(m), 1u);
        const float* up = B.Up + ((size_t)m * H + h) * a.cstride * hd + i;
#pragma unroll
        for (uint32_t c = 0; c < 16; c++) uv[k][c] = up[(size_t)min(c, ncr - 1u) * hd];
    }
    // chunk statistics: wave w takes rows w, w + 4, lane = chunk
    for (uint32_t m = wid; m < (uint32_t)M; m += 4) {
        const uint32_t ncr = nc_of(m);
        if (ncr == 0) continue;
        const float* st = B.S + ((size_t)m * H + h) * a.s_stride;
        float mv[4], tv[4];
#pragma unroll
        for (int gi = 0; gi < 4; gi++) {
            const uint32_t c = min(lane + 64u * gi, ncr - 1u);
            mv[gi] = st[2 * c];
            tv[gi] = st[2 * c + 1];
        }
        float mx = -__builtin_inff();
#pragma unroll
        for (int gi = 0; gi < 4; gi++)
            if (lane + 64u * gi < ncr) mx = fmaxf(mx, mv[gi]);
        mx = wave_max(mx);
#pragma unroll
        for (int gi = 0; gi < 4; gi++) {
            const uint32_t c = lane + 64u * gi;
            if (c < ncr) {
                fs[m * 256 + c] = expf_c(mv[gi] - mx);
                ts[m * 256 + c] = tv[gi];
            }
        }
    }
    __syncthreads();
    // T chains in chunk order (thread m < M), 16 values per LDS round trip
    if (t < (uint32_t)M) {
        const uint32_t ncr = nc_of(t);
        float T = 0.0f;
        for (uint32_t c0 = 0; c0 < ncr; c0 += 16) {
            float tq[16], fq[16];
#pragma unroll
            for (int k = 0; k < 16; k++) {
                tq[k] = ts[t * 256 + min(c0 + k, 255u)];
                fq[k] = fs[t * 256 + min(c0 + k, 255u)];
            }
#pragma unroll
            for (int k = 0; k < 16; k++)
                if (c0 + k < ncr) T = __builtin_fmaf(tq[k], fq[k], T);
        }
        sh.hinv[t] = 1.0f / (T + 1e-10f);
    }
    __syncthreads();
    PF_TR(l, TR_M_T);
    // U chains in chunk order
    float wmax[M];
#pragma unroll
    for (int m = 0; m < M; m++) wmax[m] = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < KO; k++) {
        const uint32_t e = t + 256u * k;
        if (e >= (uint32_t)M * hd) continue;
        const uint32_t m = e / hd, i = e - m * hd, ncr = nc_of(m);
        float fq[16];
#pragma unroll
        for (int c = 0; c < 16; c++) fq[c] = fs[m * 256 + c];
        float U = 0.0f;
#pragma unroll
        for (uint32_t c = 0; c < 16; c++)
            if (c < ncr) U = __builtin_fmaf(uv[k][c], fq[c], U);
        const float* up = B.Up + ((size_t)m * H + h) * a.cstride * hd + i;
        for (uint32_t c0 = 16; c0 < ncr; c0 += 16) {
            float u2[16];
#pragma unroll
            for (int c = 0; c < 16; c++) {
                u2[c] = up[(size_t)min(c0 + c, ncr - 1u) * hd];
                fq[c] = fs[m * 256 + min(c0 + c, 255u)];
            }
#pragma unroll
            for (uint32_t c = 0; c < 16; c++)
                if (c0 + c < ncr) U = __builtin_fmaf(u2[c], fq[c], U);
        }
        const float val = ncr ? U * sh.hinv[m] : 0.0f;
        stc(B.o + (size_t)m * D + h * hd + i, val);
#pragma unroll
        for (int mm = 0; mm < M; mm++)
            if ((uint32_t)mm == m) wmax[mm] = fmaxf(wmax[mm], fabsf(val));
    }
#pragma unroll
    for (int m = 0; m < M; m++) {
        const float w = wave_max(wmax[m]);
        if (lane == 0) sh.red[wid][m] = w;
    }
    __syncthreads();
    if (t < (uint32_t)M)
        stc(B.amax_o + h * 8u + t, fmaxf(fmaxf(fmaxf(sh.red[0][t], sh.red[1][t]), sh.red[2][t]), sh.red[3][t]));
}

// ------------------------------------------------------------ the kernel

// An LDS pointer passed through an empty asm statement: addresses derived
// from it inside the layer loop are not hoisted out of the loop, where
// they would occupy registers across every phase.
template <class T>
__device__ __forceinline__ T* lds_opaque(T* p) {
    auto q = (__attribute__((address_space(3))) T*)p;
    asm volatile("" : "+s"(q));
    return (T*)q;
}
// The same for a global pointer (its loads stay global instructions).
template <class T>
__device__ __forceinline__ T* opaque(T* p) {
    auto q = (__attribute__((address_space(1))) T*)p;
    asm volatile("" : "+s"(q));
    return (T*)q;
}

template <int M, int PARTS>
__global__ __launch_bounds__(256) void k_decode(DecodeArgs a0) {
    __shared__ __align__(16) uint8_t smem_[DEC_SMEM];
    __shared__ DecShared sh_;
    const uint32_t G = gridDim.x, wg = blockIdx.x, t = threadIdx.x, lane = t & 63u;
    const uint32_t wid = __builtin_amdgcn_readfirstlane(t >> 6);
    const KvGeom& g = a0.g;
    const uint32_t D = a0.D, F = a0.F, H = a0.H, hd = a0.hd;
    const uint32_t pos0 = a0.pd->pos0, pm = min(a0.pd->m, (uint32_t)M);
    const uint32_t TD = D / 64, TF = F / 64, NS = D / 256, NSF = F / 256;
    const uint32_t E = a0.glob[16];   // this pass's epoch (the previous kernel set it)
    // attention chunks of the pass (the last row has the longest list)
    const uint32_t NC = (kv_view(g, pos0 + (pm ? pm : 1u) - 1u).count() + 1 + 255) / 256;
    const uint32_t head_items = 3u * (hd / 64u) * NS;

    for (uint32_t l = 0; l < a0.L; l++) {
        DecodeArgs a = a0;
        a.ctr = opaque(a0.ctr);
        LayerBufs B;
        {
            uint8_t* lb = opaque(a0.lbuf) + (size_t)l * a0.lstride;
            uint8_t* ln = lb + a0.lstride;
            B.xin = l == 0 ? opaque(a0.x) : reinterpret_cast<float*>(lb + a0.off.xin);
            B.xmid = reinterpret_cast<float*>(lb + a0.off.xmid);
            B.xout = l + 1 == a0.L ? opaque(a0.x) : reinterpret_cast<float*>(ln + a0.off.xin);
            B.acc_qkv = reinterpret_cast<double*>(lb + a0.off.acc_qkv);
            B.acc_o = reinterpret_cast<double*>(lb + a0.off.acc_o);
            B.acc_gu = reinterpret_cast<double*>(lb + a0.off.acc_gu);
            B.acc_d = reinterpret_cast<double*>(lb + a0.off.acc_d);
            B.rs = reinterpret_cast<float*>(lb + a0.off.rs);
            B.amax_o = reinterpret_cast<float*>(lb + a0.off.amax_o);
            B.amax_f = reinterpret_cast<float*>(lb + a0.off.amax_f);
            B.o = reinterpret_cast<float*>(lb + a0.off.o);
            B.f = reinterpret_cast<float*>(lb + a0.off.f);
            B.S = reinterpret_cast<float*>(lb + a0.off.S);
            B.Up = reinterpret_cast<float*>(lb + a0.off.Up);
            B.stats_a = reinterpret_cast<float*>(lb + a0.off.stats_a);
            B.stats_f = reinterpret_cast<float*>(lb + a0.off.stats_f);
            B.stats_next = l + 1 < a0.L ? reinterpret_cast<float*>(ln + a0.off.stats_a) : nullptr;
        }
        a.kv.k = opaque(a0.kv.k);
        a.kv.v = opaque(a0.kv.v);
        a.kv.ks = opaque(a0.kv.ks);
        a.kv.vs = opaque(a0.kv.vs);
        a.layers = opaque(a0.layers);
        a.rope_c = opaque(a0.rope_c);
        a.rope_s = opaque(a0.rope_s);
        uint8_t* smem = lds_opaque(smem_);
        DecShared& sh = *lds_opaque(&sh_);
        int8_t* sa = reinterpret_cast<int8_t*>(smem + G_SA);
        int32_t* sb = reinterpret_cast<int32_t*>(smem + G_SB);
        double* red = reinterpret_cast<double*>(smem + G_RED);
        const DecodeLayer& Ly = a.layers[l];
        const Ctr cc{a.ctr + (size_t)l * a.ctr_layer, H, TD, TF};

        // ---------------------------------------------------------- layer 0 norm
        if (l == 0) {
            // tile statistics of the embedded rows (later layers get them
            // from the down projection's last splits); wave w takes rows w,
            // w + 4
            for (uint32_t tl = wg; tl < TD; tl += G) {
                for (uint32_t m = wid; m < (uint32_t)M; m += 4)
                    tile_stat(B.xin[(size_t)m * D + 64u * tl + lane], Ly.an[64u * tl + lane], B.stats_a, tl, m);
                drain();
                PF_TR(l, TR_SA_END);
                if (t == 0) arrive_n(cc.x_ready(), 1u);
            }
        }
        // ---------------------------------------------------------- QKV
        {
            const uint8_t* W = Ly.w[MAT_QKV];
            const int32_t fmt = Ly.fmt[MAT_QKV];
            uint32_t lo, hi;
            item_range(3 * TD * NS, wg, G, lo, hi);
            if (lo < hi) {
                WRaw wr[DEC_IB];
#pragma unroll
                for (uint32_t i = 0; i < DEC_IB; i++)
                    load_w2(fmt, W, D, min(lo + i, hi - 1) / NS, min(lo + i, hi - 1) % NS, wid, lane, wr[i]);
                PF_TR(l, TR_Q_WAIT);
                if (!wait_ge(cc.x_ready(), TD * E, a, sh)) return;
                combine_stats<M>(B.stats_a, TD, D, sh);
                PF_TR(l, TR_Q_STATS);
                // codes of the slices of this workgroup's items
                for (uint32_t i0 = lo; i0 < hi; i0 += DEC_IB) {
                    uint32_t col0[DEC_IB], ns = 0;
                    for (uint32_t it = i0; it < min(hi, i0 + DEC_IB); it++)
                        if (it == i0 || it % NS != (it - 1) % NS) col0[ns++] = 256u * (it % NS);
                    norm_slices<M>(B.xin, Ly.an, D, col0, ns, sa, sb, sh);
                }
                PF_TR(l, TR_Q_NORM);
                if (t < (uint32_t)M) stc(B.rs + t, sh.as[t]);
                double S[M];
#pragma unroll
                for (int m = 0; m < M; m++) S[m] = 0.0;
                for (uint32_t it = lo; it < hi; it += DEC_IB) {
                    if (it > lo) {
#pragma unroll
                        for (uint32_t i = 0; i < DEC_IB; i++)
                            load_w2(fmt, W, D, min(it + i, hi - 1) / NS, min(it + i, hi - 1) % NS, wid, lane, wr[i]);
                    }
                    uint32_t cur = it / NS;
#pragma unroll
                    for (uint32_t i = 0; i < DEC_IB; i++) {
                        if (it + i >= hi) break;
                        const uint32_t tile = (it + i) / NS, s = (it + i) % NS;
                        if (tile != cur) {
                            flush_tile<M>(S, red, B.acc_qkv, 3 * D, 64 * cur);
                            cur = tile;
                        }
                        item_dots<M>(wr[i], fmt, sa, sb, 8 * s + 2 * wid, S);
                    }
                    flush_tile<M>(S, red, B.acc_qkv, 3 * D, 64 * cur);
                }
                drain();
                if (t == 0) {
                    // one arrival per run of items of the same head
                    uint32_t hcur = ((lo / NS) % TD) / (hd / 64), n = 0;
                    for (uint32_t it = lo; it < hi; it++) {
                        const uint32_t hh = ((it / NS) % TD) / (hd / 64);
                        if (hh != hcur) {
                            arrive_n(cc.head_cnt(hcur), n);
                            hcur = hh;
                            n = 0;
                        }
                        n++;
                    }
                    arrive_n(cc.head_cnt(hcur), n);
                }
                PF_TR(l, TR_Q_DONE);
            }
        }
        // ---------------------------------------------------------- attention
        for (uint32_t ai = wg; ai < H * NC; ai += G) {
            const uint32_t c = ai / H, h = ai - c * H;
            bool ok;
            if (PARTS == 4) ok = attn_item<M, 4>(a, B, cc, l, h, c, pos0, pm, head_items * E, smem, sh);
            else ok = attn_item<M, 8>(a, B, cc, l, h, c, pos0, pm, head_items * E, smem, sh);
            if (!ok) return;
            drain();
            PF_TR(l, TR_A_DONE);
            if (arrive_last(cc.att_cnt(h), 1u, NC, sh)) {
                merge_head<M>(a, B, l, h, pos0, pm, smem, sh);
                if (t == 0) stc(cc.att_cnt(h), 0u);
                drain();
                PF_TR(l, TR_MERGE);
                if (t == 0) arrive_n(cc.heads_done(), 1u);
            }
        }
        // ---------------------------------------------------------- O
        {
            const uint8_t* W = Ly.w[MAT_O];
            const int32_t fmt = Ly.fmt[MAT_O];
            uint32_t lo, hi;
            item_range(TD * NS, wg, G, lo, hi);
            if (lo < hi) {
                WRaw wr[DEC_IB];
#pragma unroll
                for (uint32_t i = 0; i < DEC_IB; i++)
                    load_w2(fmt, W, D, min(lo + i, hi - 1) / NS, min(lo + i, hi - 1) % NS, wid, lane, wr[i]);
                PF_TR(l, TR_O_WAIT);
                if (!wait_ge(cc.heads_done(), H * E, a, sh)) return;
                gather_amax<M>(B.amax_o, H, sh);
                PF_TR(l, TR_O_AMAX);
                double S[M];
#pragma unroll
                for (int m = 0; m < M; m++) S[m] = 0.0;
                for (uint32_t it = lo; it < hi; it += DEC_IB) {
                    if (it > lo) {
#pragma unroll
                        for (uint32_t i = 0; i < DEC_IB; i++)
                            load_w2(fmt, W, D, min(it + i, hi - 1) / NS, min(it + i, hi - 1) % NS, wid, lane, wr[i]);
                    }
                    // codes of the batch's column slices
#pragma unroll
                    for (uint32_t i = 0; i < DEC_IB; i++) {
                        if (it + i >= hi) break;
                        const uint32_t s = (it + i) % NS;
                        quant_slice256<M>(B.o + 256 * s, D, sh.invq, sa, sb, 256 * s);
                    }
                    __syncthreads();
                    block_sums<M>(sa, sb, 0, D >> 5);
                    __syncthreads();
                    uint32_t cur = it / NS;
#pragma unroll
                    for (uint32_t i = 0; i < DEC_IB; i++) {
                        if (it + i >= hi) break;
                        const uint32_t tile = (it + i) / NS, s = (it + i) % NS;
                        if (tile != cur) {
                            flush_tile<M>(S, red, B.acc_o, D, 64 * cur);
                            cur = tile;
                        }
                        item_dots<M>(wr[i], fmt, sa, sb, 8 * s + 2 * wid, S);
                    }
                    flush_tile<M>(S, red, B.acc_o, D, 64 * cur);
                }
                drain();
                PF_TR(l, TR_O_DONE);
                // per tile: the last split adds the tile to the residual rows
                for (uint32_t t0 = lo / NS; t0 <= (hi - 1) / NS; t0 += DEC_IB) {
                    const uint32_t mask = arrive_tiles([&](uint32_t x) { return cc.o_tile(x); }, t0, lo, hi, NS, sh);
                    if (mask) {
                        finalize_resid<M>(mask, t0, B.xin, B.xmid, B.acc_o, D, sh, Ly.fn, B.stats_f);
                        drain();
                        PF_TR(l, TR_O_FIN);
                        if (t == 0) arrive_n(cc.xmid(), __builtin_popcount(mask));
                    }
                }
            }
        }
        // ---------------------------------------------------------- gate|up
        {
            const uint8_t* W = Ly.w[MAT_GU];
            const int32_t fmt = Ly.fmt[MAT_GU];
            uint32_t lo, hi;
            item_range(TF * NS, wg, G, lo, hi);
            if (lo < hi) {
                WRaw wg_[DEC_IB], wu_[DEC_IB];
#pragma unroll
                for (uint32_t i = 0; i < DEC_IB; i++) {
                    const uint32_t p = min(lo + i, hi - 1) / NS, s = min(lo + i, hi - 1) % NS;
                    load_w2(fmt, W, D, p, s, wid, lane, wg_[i]);
                    load_w2(fmt, W, D, p + TF, s, wid, lane, wu_[i]);
                }
                PF_TR(l, TR_G_WAIT);
                if (!wait_ge(cc.xmid(), TD * E, a, sh)) return;
                combine_stats<M>(B.stats_f, TD, D, sh);
                PF_TR(l, TR_G_STATS);
                for (uint32_t i0 = lo; i0 < hi; i0 += DEC_IB) {
                    uint32_t col0[DEC_IB], ns = 0;
                    for (uint32_t it = i0; it < min(hi, i0 + DEC_IB); it++)
                        if (it == i0 || it % NS != (it - 1) % NS) col0[ns++] = 256u * (it % NS);
                    norm_slices<M>(B.xmid, Ly.fn, D, col0, ns, sa, sb, sh);
                }
                PF_TR(l, TR_G_NORM);
                double Sg[M], Su[M];
#pragma unroll
                for (int m = 0; m < M; m++) Sg[m] = Su[m] = 0.0;
                for (uint32_t it = lo; it < hi; it += DEC_IB) {
                    if (it > lo) {
#pragma unroll
                        for (uint32_t i = 0; i < DEC_IB; i++) {
                            const uint32_t p = min(it + i, hi - 1) / NS, s = min(it + i, hi - 1) % NS;
                            load_w2(fmt, W, D, p, s, wid, lane, wg_[i]);
                            load_w2(fmt, W, D, p + TF, s, wid, lane, wu_[i]);
                        }
                    }
                    uint32_t cur = it / NS;
#pragma unroll
                    for (uint32_t i = 0; i < DEC_IB; i++) {
                        if (it + i >= hi) break;
                        const uint32_t p = (it + i) / NS, s = (it + i) % NS;
                        if (p != cur) {
                            flush_tile<M>(Sg, red, B.acc_gu, 2 * F, 64 * cur);
                            flush_tile<M>(Su, red, B.acc_gu, 2 * F, F + 64 * cur);
                            cur = p;
                        }
                        item_dots<M>(wg_[i], fmt, sa, sb, 8 * s + 2 * wid, Sg);
                        item_dots<M>(wu_[i], fmt, sa, sb, 8 * s + 2 * wid, Su);
                    }
                    flush_tile<M>(Sg, red, B.acc_gu, 2 * F, 64 * cur);
                    flush_tile<M>(Su, red, B.acc_gu, 2 * F, F + 64 * cur);
                }
                drain();
                PF_TR(l, TR_G_DONE);
                for (uint32_t t0 = lo / NS; t0 <= (hi - 1) / NS; t0 += DEC_IB) {
                    const uint32_t mask = arrive_tiles([&](uint32_t x) { return cc.gu_pair(x); }, t0, lo, hi, NS, sh);
                    if (!mask) continue;
                    // SwiGLU of the columns [64p, 64p + 64) of every last-
                    // arrived pair p (k_swiglu_quant's arithmetic); wave w
                    // takes (pair, row) combinations w, w + 4, ...; loads first
                    constexpr uint32_t KC = (DEC_IB * M + 3) / 4;
                    const uint32_t ncb = __builtin_popcount(mask) * (uint32_t)M;
                    double ga[KC], ua[KC];
#pragma unroll
                    for (uint32_t k = 0; k < KC; k++) {
                        const uint32_t c = min(wid + 4u * k, ncb - 1u), m = c % M;
                        const uint32_t col = nth_tile(mask, t0, c / M) * 64u + lane;
                        ga[k] = B.acc_gu[(size_t)m * 2 * F + col];
                        ua[k] = B.acc_gu[(size_t)m * 2 * F + F + col];
                    }
#pragma unroll
                    for (uint32_t k = 0; k < KC; k++) {
                        const uint32_t c = wid + 4u * k;
                        if (c >= ncb) continue;   // wave-uniform
                        const uint32_t m = c % M, p = nth_tile(mask, t0, c / M), col = p * 64u + lane;
                        double* gp = B.acc_gu + (size_t)m * 2 * F + col;
                        stc(gp, 0.0);
                        stc(gp + F, 0.0);
                        const double as = (double)sh.as[m];
                        const float gt = (float)(ga[k] * as);
                        const float uu = (float)(ua[k] * as);
                        const float sig = 1.0f / (1.0f + expf_c(-gt));
                        const float fv = gt * sig * uu;
                        stc(B.f + (size_t)m * F + col, fv);
                        const float wm = wave_max(fabsf(fv));
                        if (lane == 0) stc(B.amax_f + p * 8u + m, wm);
                    }
                    drain();
                    PF_TR(l, TR_G_FIN);
                    if (t == 0) arrive_n(cc.pairs(), __builtin_popcount(mask));
                }
            }
        }
        // ---------------------------------------------------------- down
        {
            const uint8_t* W = Ly.w[MAT_DOWN];
            const int32_t fmt = Ly.fmt[MAT_DOWN];
            uint32_t lo, hi;
            item_range(TD * NSF, wg, G, lo, hi);
            if (lo < hi) {
                WRaw wr[DEC_IB];
#pragma unroll
                for (uint32_t i = 0; i < DEC_IB; i++)
                    load_w2(fmt, W, F, min(lo + i, hi - 1) / NSF, min(lo + i, hi - 1) % NSF, wid, lane, wr[i]);
                PF_TR(l, TR_D_WAIT);
                if (!wait_ge(cc.pairs(), TF * E, a, sh)) return;
                gather_amax<M>(B.amax_f, TF, sh);
                PF_TR(l, TR_D_AMAX);
                double S[M];
#pragma unroll
                for (int m = 0; m < M; m++) S[m] = 0.0;
                for (uint32_t it = lo; it < hi; it += DEC_IB) {
                    if (it > lo) {
#pragma unroll
                        for (uint32_t i = 0; i < DEC_IB; i++)
                            load_w2(fmt, W, F, min(it + i, hi - 1) / NSF, min(it + i, hi - 1) % NSF, wid, lane, wr[i]);
                    }
                    // codes of the batch's column slices into slots i
#pragma unroll
                    for (uint32_t i = 0; i < DEC_IB; i++) {
                        if (it + i >= hi) break;
                        const uint32_t s = (it + i) % NSF;
                        quant_slice256<M>(B.f + 256 * s, F, sh.invq, sa, sb, 256 * i);
                    }
                    __syncthreads();
                    block_sums<M>(sa, sb, 0, 8 * min(DEC_IB, hi - it));
                    __syncthreads();
                    uint32_t cur = it / NSF;
#pragma unroll
                    for (uint32_t i = 0; i < DEC_IB; i++) {
                        if (it + i >= hi) break;
                        const uint32_t tile = (it + i) / NSF;
                        if (tile != cur) {
                            flush_tile<M>(S, red, B.acc_d, D, 64 * cur);
                            cur = tile;
                        }
                        item_dots<M>(wr[i], fmt, sa, sb, 8 * i + 2 * wid, S);
                    }
                    flush_tile<M>(S, red, B.acc_d, D, 64 * cur);
                }
                drain();
                PF_TR(l, TR_D_DONE);
                for (uint32_t t0 = lo / NSF; t0 <= (hi - 1) / NSF; t0 += DEC_IB) {
                    const uint32_t mask = arrive_tiles([&](uint32_t x) { return cc.d_tile(x); }, t0, lo, hi, NSF, sh);
                    if (mask) {
                        finalize_resid<M>(mask, t0, B.xmid, B.xout, B.acc_d, D, sh,
                                          B.stats_next ? a.layers[l + 1].an : nullptr, B.stats_next);
                        drain();
                        PF_TR(l, TR_D_FIN);
                        if (t == 0 && l + 1 < a.L) arrive_n(a.ctr + (size_t)(l + 1) * a.ctr_layer, __builtin_popcount(mask));
                    }
                }
            }
        }
    }
    // the last workgroup to finish advances the epoch for the next pass
    drain();
    if (arrive_last(a0.glob, 1u, G, sh_) && t == 0) {
        stc(a0.glob, 0u);
        stc(a0.glob + 16, E + 1u);
    }
}

}  // namespace pf
