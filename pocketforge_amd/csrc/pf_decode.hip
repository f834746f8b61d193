// One decode pass (M <= 8 rows, every layer) as a single persistent kernel.
//
// The layer's work is split into items processed by a grid of co-resident
// 256-thread workgroups (the grid never exceeds what the device holds at
// once).  Workgroup w takes items w, w + G, ... of every phase in order:
//
//   QKV   (tile, K split) of the fused QKV GEMV.  The activation slice is
//         normalised and quantized from the residual stream x and the
//         row statistics (1/rms, amax of the normed row).  The last
//         arrival of a head applies RoPE, writes q/k/v and the head's int8
//         K/V rows (src/engine.cpp:726-755) and raises the head's flag.
//   ATT   (head, 256-entry chunk, row): the first attention stage of
//         k_attn_chunk.  The last arrival of a head merges its chunks for
//         every row (k_attn_merge_quant's arithmetic), writes the head's
//         slice of the attention output and folds its amax into the row
//         amax.
//   O     (tile, K split) of the O projection; the last split of a tile
//         adds the tile to x, the last tile computes the FFN-norm row
//         statistics.
//   GU    (tile, K split) of the fused gate|up GEMV; the last arrival of a
//         gate/up tile pair applies SwiGLU (src/engine.cpp:832-838) and
//         folds the result's amax into the row amax.
//   DOWN  (tile, K split) of the down projection; the last split of a tile
//         adds the tile to x, the last tile computes the next layer's
//         attention-norm statistics.
//
// Every phase waits only for earlier phases, so co-residency makes the
// pass deadlock free; every wait is also bounded in time (a timed-out wait
// sets the error word and all workgroups leave).  Data that crosses
// workgroups is written and read with agent-scope (coherent) stores and
// loads; the split-K partial sums meet in exact fp64 atomics.  A producer
// drains its memory operations (s_waitcnt 0) and the workgroup barrier
// before its single counter update, so a consumer that has seen the count
// reads complete data.  No L2 write-back or invalidate is needed.
//
// Every value is computed with the arithmetic and association order of the
// multi-kernel pass (k_resid_norm_quant, k_gemv_i8, k_qkv_post,
// k_attn_chunk, k_attn_merge_quant, k_swiglu_quant, k_resid_add), so the
// two paths agree bit for bit.
#include "pf_device.h"

namespace pf {

// ------------------------------------------------------------ coherence

// A pointer read from memory is generic; re-deriving it through the global
// address space lets its loads be global (not flat) instructions.
template <class T>
__device__ __forceinline__ T* gptr(T* p) {
    return (T*)(__attribute__((address_space(1))) T*)p;
}

template <class T>
__device__ __forceinline__ T ldc(const T* p) {
    return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void stc(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t arrive(uint32_t* c) {
    return __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Every wave's memory operations complete, then the workgroup barrier.
__device__ __forceinline__ void drain() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

// ------------------------------------------------------------ arguments

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
    uint32_t bpw[4];             // blocks per wave of each matrix kind
    float* x;                    // [8][D] residual stream
    float* stats;                // [L][2][8][2]: 1/rms and amax of the normed row
    double* acc_qkv;             // [8][3D], [8][D], [8][2F], [8][D]; zero between uses
    double* acc_o;
    double* acc_gu;
    double* acc_d;
    float *q, *k, *v;            // [8][D]
    float* S;                    // attention chunk max / sum, [8][H][s_stride]
    float* Up;                   // attention chunk partials, [8][H][cstride][hd]
    uint32_t s_stride, cstride;
    float* o;                    // [8][D] attention output
    float* f;                    // [8][F] SwiGLU output
    uint32_t* ctr;               // per-layer counters, zeroed before the pass
    uint32_t ctr_layer;          // counter words per layer
    uint32_t* err;               // nonzero after a timed-out wait
    uint64_t spin_limit;         // wall-clock ticks a wait may take
    uint64_t* trace;             // null, or [L][grid][DEC_TRACE] phase timestamps
};

// Phase timestamps of one workgroup in one layer (wall clock, 100 MHz):
// per phase the start and end of its wait, the end of its GEMV or
// attention work and the ends of its epilogues.
constexpr uint32_t DEC_TRACE = 48;

// Counter words of one layer, each in its own 64-byte slot (16 words).
struct Ctr {
    uint32_t* base;
    uint32_t H, TD, TF;    // heads, D / 64, F / 64
    __device__ uint32_t* slot(uint32_t i) const { return base + 16u * i; }
    __device__ uint32_t* x_ready() const { return slot(0); }
    __device__ uint32_t* head_cnt(uint32_t h) const { return slot(1 + h); }
    __device__ uint32_t* head_flag(uint32_t h) const { return slot(1 + H + h); }
    __device__ uint32_t* att_cnt(uint32_t h) const { return slot(1 + 2 * H + h); }
    __device__ uint32_t* heads_done() const { return slot(1 + 3 * H); }
    __device__ uint32_t* o_tile(uint32_t t) const { return slot(2 + 3 * H + t); }
    __device__ uint32_t* o_tiles() const { return slot(2 + 3 * H + TD); }
    __device__ uint32_t* xmid_ready() const { return slot(3 + 3 * H + TD); }
    __device__ uint32_t* gu_pair(uint32_t p) const { return slot(4 + 3 * H + TD + p); }
    __device__ uint32_t* pairs() const { return slot(4 + 3 * H + TD + TF); }
    __device__ uint32_t* d_tile(uint32_t t) const { return slot(5 + 3 * H + TD + TF + t); }
    __device__ uint32_t* d_tiles() const { return slot(5 + 3 * H + 2 * TD + TF); }
    __device__ uint32_t* amax_o() const { return slot(6 + 3 * H + 2 * TD + TF); }   // [8] float bits
    __device__ uint32_t* amax_f() const { return slot(7 + 3 * H + 2 * TD + TF); }
};
__host__ __device__ constexpr uint32_t decode_ctr_slots(uint32_t H, uint32_t TD, uint32_t TF) {
    return 8 + 3 * H + 2 * TD + TF;
}

// ------------------------------------------------------------ shared memory

constexpr uint32_t DEC_SA = 8 * 1024;                   // int8 codes [8][1024]
constexpr uint32_t DEC_SB = 8 * 32 * 4;                 // block sums [8][32]
constexpr uint32_t DEC_RED = 4 * 8 * 64 * 8;            // fp64 wave partials [4][8][64]
constexpr uint32_t DEC_GEMV = DEC_SA + DEC_SB + DEC_RED;
constexpr uint32_t DEC_MERGE = (2 * 2048 + 8) * 4;
constexpr uint32_t DEC_SMEM_A = DEC_GEMV > DEC_MERGE ? DEC_GEMV : DEC_MERGE;
constexpr uint32_t DEC_SMEM = DEC_SMEM_A > ATT_SMEM ? DEC_SMEM_A : ATT_SMEM;

struct DecShared {
    uint32_t flag;
    float red[16];
    float wsum[4][8], wmax[4][8];
    float inv[8], amax[8], invq[8], as[8];
};

#define PF_TR(l, k)                                                                                  \
    do {                                                                                             \
        if (a.trace && threadIdx.x == 0)                                                             \
            a.trace[((size_t)(l) * gridDim.x + blockIdx.x) * DEC_TRACE + (k)] = wall_clock64();      \
    } while (0)

// Waits until *c >= target (thread 0 polls; every thread returns the
// verdict).  False when the wait timed out or another workgroup's did.
__device__ __forceinline__ bool wait_ge(const uint32_t* c, uint32_t target, const DecodeArgs& a, DecShared& sh) {
    if (threadIdx.x == 0) {
        uint32_t ok = 1;
        if (ldc(c) < target) {
            const uint64_t t0 = wall_clock64();
            uint32_t it = 0;
            while (ldc(c) < target) {
                __builtin_amdgcn_s_sleep(1);
                if ((++it & 31u) == 0u) {
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

// Thread 0 adds one to *c; every thread learns whether it was the last of
// `total` arrivals.  Call after drain().
__device__ __forceinline__ bool arrive_last(uint32_t* c, uint32_t total, DecShared& sh) {
    if (threadIdx.x == 0) sh.flag = (arrive(c) == total - 1u) ? 1u : 0u;
    __syncthreads();
    const bool last = sh.flag != 0u;
    __syncthreads();
    return last;
}

// ------------------------------------------------------------ row statistics

// For rows m < M of x ([M][D]): 1/rms with the CANON(4) sum of squares of
// k_resid_norm_quant (canonical lane l < 256 takes elements l, l + 256, ...
// with an fmaf chain; trees over canonical waves; (W0 + W2) + (W1 + W3))
// and the amax of the normed row x * inv * w.  Written to st[m][0..1]
// (coherent).  Wave q runs canonical lanes 64 q .. 64 q + 63 of every row,
// so each lane issues all of its loads at once.
// Not inlined: it runs twice a layer in one workgroup, and its own register
// allocation keeps the kernel's (the pointers carry their address spaces so
// the accesses stay global / LDS instructions).
template <int M>
__device__ __noinline__ void norm_stats_fn(const __attribute__((address_space(1))) float* xg, uint32_t D,
                                           const __attribute__((address_space(1))) float* wg,
                                           __attribute__((address_space(1))) float* stg,
                                           __attribute__((address_space(3))) DecShared* shp,
                                           __attribute__((address_space(1))) uint64_t* trace) {
    const float* x = (const float*)xg;
    const float* w = (const float*)wg;
    float* st = (float*)stg;
    DecShared& sh = *(DecShared*)shp;
#define PF_TRN(k)                                         \
    do {                                                  \
        if (trace && threadIdx.x == 0) trace[k] = wall_clock64(); \
    } while (0)
    PF_TRN(0);
    const uint32_t t = threadIdx.x, lane = t & 63u, q = t >> 6, nk = D >> 8;   // D % 256 == 0, <= 2048
    float xv[M][8], wt[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        if ((uint32_t)k < nk) {
            const uint32_t i = 64u * q + lane + 256u * k;
            wt[k] = w[i];
#pragma unroll
            for (int m = 0; m < M; m++) xv[m][k] = ldc(x + (size_t)m * D + i);
        }
    }
#pragma unroll
    for (int m = 0; m < M; m++) {
        float part = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++)
            if ((uint32_t)k < nk) part = __builtin_fmaf(xv[m][k], xv[m][k], part);
        const float W = wave_tree_sum(part);
        if (lane == 0) sh.wsum[q][m] = W;
    }
    __syncthreads();
    PF_TRN(1);
#pragma unroll
    for (int m = 0; m < M; m++) {
        const float ss = (sh.wsum[0][m] + sh.wsum[2][m]) + (sh.wsum[1][m] + sh.wsum[3][m]);
        const float inv = 1.0f / __builtin_sqrtf(ss / (float)D + 1e-6f);
        float am = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++)
            if ((uint32_t)k < nk) am = fmaxf(am, fabsf(xv[m][k] * inv * wt[k]));
        am = wave_max(am);
        if (lane == 0) sh.wmax[q][m] = am;
    }
    __syncthreads();
    PF_TRN(2);
    if (t < (uint32_t)M) {
        const float ss = (sh.wsum[0][t] + sh.wsum[2][t]) + (sh.wsum[1][t] + sh.wsum[3][t]);
        const float inv = 1.0f / __builtin_sqrtf(ss / (float)D + 1e-6f);
        const float amax = fmaxf(fmaxf(sh.wmax[0][t], sh.wmax[1][t]), fmaxf(sh.wmax[2][t], sh.wmax[3][t]));
        stc(st + 2 * t, inv);
        stc(st + 2 * t + 1, amax);
    }
    __syncthreads();
    PF_TRN(3);
}
#undef PF_TRN

template <int M>
__device__ __forceinline__ void norm_stats(const float* x, uint32_t D, const float* w, float* st, DecShared& sh,
                                           const DecodeArgs& a, uint32_t l, uint32_t slot) {
    typedef __attribute__((address_space(1))) float gf;
    __attribute__((address_space(1))) uint64_t* tr =
        a.trace ? (__attribute__((address_space(1))) uint64_t*)(a.trace + ((size_t)l * gridDim.x + blockIdx.x) * DEC_TRACE + slot)
                : nullptr;
    norm_stats_fn<M>((const gf*)x, D, (const gf*)w, (gf*)st, (__attribute__((address_space(3))) DecShared*)&sh, tr);
}

// ------------------------------------------------------------ GEMV items

// Raw weight words of one wave's blocks: code bytes (4 dwords for Q4, 2 for
// Q2 / Q1.5) and the fp16 scales, loaded straight-line through global
// pointers so that every load of the item is in flight at once.  The wave's
// bpw blocks start at a multiple of bpw and bpw divides 8, so they lie in
// one tile: one base address with immediate offsets, and the row's scales
// of those blocks are contiguous (one load of 2 bpw bytes).
struct WRaw {
    uint32_t c[8][4];
    uint32_t s[4];     // fp16 scales of blocks 2i (low half) and 2i + 1
};

template <int FMT, int BPW>
__device__ __forceinline__ void load_raw(const uint8_t* W, uint32_t K, uint32_t tile, uint32_t b0, uint32_t lane,
                                         WRaw& w) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    typedef unsigned int v2u __attribute__((ext_vector_type(2)));
    typedef const __attribute__((address_space(1))) uint8_t gu8;
    typedef const __attribute__((address_space(1))) v4u gu128;
    typedef const __attribute__((address_space(1))) v2u gu64;
    typedef const __attribute__((address_space(1))) uint32_t gu32;
    typedef const __attribute__((address_space(1))) uint16_t gu16;
    constexpr uint32_t TB = tile_bytes(FMT);
    constexpr uint32_t CODES = TILE_ROWS * TILE_BLOCKS * code_bytes(FMT);
    gu8* tp = (gu8*)W + ((size_t)tile * (K >> 8) + (b0 >> 3)) * TB;
    const uint32_t t0 = b0 & 7u;
    if constexpr (FMT == FMT_Q4) {
        gu8* cp = tp + t0 * 1024u + lane * 16u;
#pragma unroll
        for (int k = 0; k < BPW; k++) {
            const v4u c = *(gu128*)(cp + k * 1024);
            w.c[k][0] = c.x; w.c[k][1] = c.y; w.c[k][2] = c.z; w.c[k][3] = c.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < BPW; k++) {
            const uint32_t tk = t0 + k;
            const v2u c = *(gu64*)(tp + (tk >> 1) * 1024u + lane * 16u + (tk & 1u) * 8u);
            w.c[k][0] = c.x; w.c[k][1] = c.y;
        }
    }
#pragma unroll
    for (int k = BPW; k < 8; k++) w.c[k][0] = w.c[k][1] = w.c[k][2] = w.c[k][3] = 0u;
    if constexpr (FMT != FMT_Q4) {
#pragma unroll
        for (int k = 0; k < BPW; k++) w.c[k][2] = w.c[k][3] = 0u;
    }
    w.s[0] = w.s[1] = w.s[2] = w.s[3] = 0u;
    gu8* sp = tp + CODES + lane * 16u + t0 * 2u;
    if constexpr (BPW == 8) {
        const v4u v = *(gu128*)sp;
        w.s[0] = v.x; w.s[1] = v.y; w.s[2] = v.z; w.s[3] = v.w;
    } else if constexpr (BPW == 4) {
        const v2u v = *(gu64*)sp;
        w.s[0] = v.x; w.s[1] = v.y;
    } else if constexpr (BPW == 2) {
        w.s[0] = *(gu32*)sp;
    } else {
        w.s[0] = *(gu16*)sp;
    }
}

template <int FMT>
__device__ __forceinline__ void load_raw_bpw(const uint8_t* W, uint32_t K, uint32_t tile, uint32_t b0, uint32_t bpw,
                                             uint32_t lane, WRaw& w) {
    switch (bpw) {
        case 1: load_raw<FMT, 1>(W, K, tile, b0, lane, w); break;
        case 2: load_raw<FMT, 2>(W, K, tile, b0, lane, w); break;
        case 4: load_raw<FMT, 4>(W, K, tile, b0, lane, w); break;
        default: load_raw<FMT, 8>(W, K, tile, b0, lane, w); break;
    }
}

__device__ __forceinline__ void load_w_any(int32_t fmt, const uint8_t* W, uint32_t K, uint32_t tile, uint32_t b0,
                                           uint32_t bpw, uint32_t lane, WRaw& w) {
    if (fmt == FMT_Q4) load_raw_bpw<FMT_Q4>(W, K, tile, b0, bpw, lane, w);
    else if (fmt == FMT_Q2) load_raw_bpw<FMT_Q2>(W, K, tile, b0, bpw, lane, w);
    else load_raw_bpw<FMT_Q15>(W, K, tile, b0, bpw, lane, w);
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

// Codes of the slice [0, len) of every row of src (row stride `stride`,
// len = 128 bpw <= 1024) into LDS.  With w != null the value is the normed
// x * inv[m] * w[i] (k_resid_norm_quant's order), else src itself; invq[m]
// is the row's quantization factor (quantize_activation_row,
// src/matmul_neon.cpp:16-29).  Thread t takes elements 4t .. 4t + 3 of
// every row (two coherent 8-byte loads per row, all issued first) and
// stores their codes as one dword; then the block sums of the codes
// (sdot4 against ones, exact) go to sb.
template <int M>
__device__ __forceinline__ void quant_slice(const float* src, uint32_t stride, uint32_t len, const float* w,
                                            const float* inv, const float* invq, int8_t* sa, int32_t* sb) {
    const uint32_t t = threadIdx.x, i0 = 4u * t;
    const bool live = i0 < len;
    const uint32_t ii = live ? i0 : 0u;
    uint64_t lo[M], hi[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
        const uint64_t* p = reinterpret_cast<const uint64_t*>(src + (size_t)m * stride + ii);
        lo[m] = ldc(p);
        hi[m] = ldc(p + 1);
    }
    float4 wv = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    if (w) wv = *reinterpret_cast<const float4*>(w + ii);
#pragma unroll
    for (int m = 0; m < M; m++) {
        float v[4] = {__uint_as_float((uint32_t)lo[m]), __uint_as_float((uint32_t)(lo[m] >> 32)),
                      __uint_as_float((uint32_t)hi[m]), __uint_as_float((uint32_t)(hi[m] >> 32))};
        if (w) {
            const float im = inv[m];
            v[0] = v[0] * im * wv.x;
            v[1] = v[1] * im * wv.y;
            v[2] = v[2] * im * wv.z;
            v[3] = v[3] * im * wv.w;
        }
        const float iq = invq[m];
        const uint32_t code = (uint32_t)(uint8_t)quant_code(v[0], iq) | ((uint32_t)(uint8_t)quant_code(v[1], iq) << 8) |
                              ((uint32_t)(uint8_t)quant_code(v[2], iq) << 16) |
                              ((uint32_t)(uint8_t)quant_code(v[3], iq) << 24);
        if (live) *reinterpret_cast<uint32_t*>(sa + m * 1024 + i0) = code;
    }
    __syncthreads();
    const uint32_t nb = len >> 5;
    for (uint32_t e = t; e < (uint32_t)M * nb; e += 256u) {
        const uint32_t m = e / nb, j = e - m * nb;
        const int4 a0 = *reinterpret_cast<const int4*>(sa + m * 1024 + j * 32u);
        const int4 a1 = *reinterpret_cast<const int4*>(sa + m * 1024 + j * 32u + 16u);
        const int ones = 0x01010101;
        int sum = __builtin_amdgcn_sdot4(a0.x, ones, 0, false);
        sum = __builtin_amdgcn_sdot4(a0.y, ones, sum, false);
        sum = __builtin_amdgcn_sdot4(a0.z, ones, sum, false);
        sum = __builtin_amdgcn_sdot4(a0.w, ones, sum, false);
        sum = __builtin_amdgcn_sdot4(a1.x, ones, sum, false);
        sum = __builtin_amdgcn_sdot4(a1.y, ones, sum, false);
        sum = __builtin_amdgcn_sdot4(a1.z, ones, sum, false);
        sum = __builtin_amdgcn_sdot4(a1.w, ones, sum, false);
        sb[m * 32 + j] = sum;
    }
}

// acc[m][64 tile + lane] += this item's exact block sums (the body of
// k_gemv_i8 after its loads), activation codes and block sums in LDS.
template <int M>
__device__ __forceinline__ void gemv_dots(const WRaw& w, int32_t fmt, uint32_t bpw, const int8_t* sa,
                                          const int32_t* sb, double* red, double* acc, uint32_t acc_stride,
                                          uint32_t tile) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int off = code_offset(fmt);
    double S[M];
#pragma unroll
    for (int m = 0; m < M; m++) S[m] = 0.0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        if ((uint32_t)k < bpw) {
            uint32_t u[8];
            unpack_raw(fmt, w, k, u);
            const double dk = (double)h2f((uint16_t)(w.s[k >> 1] >> (16 * (k & 1))));
            const uint32_t j = wid * bpw + k;
#pragma unroll
            for (int m = 0; m < M; m++) {
                const int4 a0 = *reinterpret_cast<const int4*>(sa + m * 1024 + j * 32u);
                const int4 a1 = *reinterpret_cast<const int4*>(sa + m * 1024 + j * 32u + 16u);
                int p = -off * sb[m * 32 + j];
                p = __builtin_amdgcn_sdot4((int)u[0], a0.x, p, false);
                p = __builtin_amdgcn_sdot4((int)u[1], a0.y, p, false);
                p = __builtin_amdgcn_sdot4((int)u[2], a0.z, p, false);
                p = __builtin_amdgcn_sdot4((int)u[3], a0.w, p, false);
                p = __builtin_amdgcn_sdot4((int)u[4], a1.x, p, false);
                p = __builtin_amdgcn_sdot4((int)u[5], a1.y, p, false);
                p = __builtin_amdgcn_sdot4((int)u[6], a1.z, p, false);
                p = __builtin_amdgcn_sdot4((int)u[7], a1.w, p, false);
                S[m] = __builtin_fma(dk, (double)p, S[m]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; m++) red[(wid * 8 + m) * 64 + lane] = S[m];
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < (uint32_t)M * 64u; t += 256u) {
        const uint32_t m = t >> 6, r = t & 63u;
        const double v = red[(0 * 8 + m) * 64 + r] + red[(1 * 8 + m) * 64 + r] + red[(2 * 8 + m) * 64 + r] +
                         red[(3 * 8 + m) * 64 + r];
        atomicAdd(acc + (size_t)m * acc_stride + (size_t)tile * 64u + r, v);
    }
}

// ------------------------------------------------------------ QKV post

// The last arrival of head h: q/k/v of the head for every row from the
// exact sums (cleared), RoPE, K/V rows stored (k_qkv_post).  Wave w takes
// rows w, w + 4.
template <int M>
__device__ __forceinline__ void qkv_post_head(const DecodeArgs& a, uint32_t layer, uint32_t h, const float* as, uint32_t pos0,
                              uint32_t pm) {
    const KvGeom& g = a.g;
    const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
    const uint32_t hd = a.hd, D = a.D, half = hd >> 1;
    const size_t plane = (size_t)layer * g.n_heads + h;
    for (uint32_t m = wv; m < (uint32_t)M; m += 4) {
        const bool act = lane < half;
        float k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
        const uint32_t pos = pos0 + m;
        if (act) {
            double* r = a.acc_qkv + (size_t)m * 3 * D;
            const float s = as[m];
            const uint32_t i0 = h * hd + 2 * lane;
            const double aq0 = ldc(r + i0), aq1 = ldc(r + i0 + 1);
            const double ak0 = ldc(r + D + i0), ak1 = ldc(r + D + i0 + 1);
            const double av0 = ldc(r + 2 * D + i0), av1 = ldc(r + 2 * D + i0 + 1);
            stc(r + i0, 0.0); stc(r + i0 + 1, 0.0);
            stc(r + D + i0, 0.0); stc(r + D + i0 + 1, 0.0);
            stc(r + 2 * D + i0, 0.0); stc(r + 2 * D + i0 + 1, 0.0);
            const float q0 = (float)(aq0 * (double)s), q1 = (float)(aq1 * (double)s);
            k0 = (float)(ak0 * (double)s); k1 = (float)(ak1 * (double)s);
            v0 = (float)(av0 * (double)s); v1 = (float)(av1 * (double)s);
            if (m < pm) {
                const float c = a.rope_c[(size_t)pos * half + lane], sn = a.rope_s[(size_t)pos * half + lane];
                const float qr0 = __builtin_fmaf(q0, c, -(q1 * sn));
                const float qr1 = __builtin_fmaf(q0, sn, q1 * c);
                const float kr0 = __builtin_fmaf(k0, c, -(k1 * sn));
                const float kr1 = __builtin_fmaf(k0, sn, k1 * c);
                k0 = kr0; k1 = kr1;
                const size_t o = (size_t)m * D + i0;
                stc(a.q + o, qr0); stc(a.q + o + 1, qr1);
                stc(a.k + o, kr0); stc(a.k + o + 1, kr1);
                stc(a.v + o, v0); stc(a.v + o + 1, v1);
            }
        }
        if (m >= pm) continue;   // wave-uniform
        // int8 K/V row of this position (store_pair's arithmetic), packed
        // four codes per coherent 32-bit store
        float ak = act ? fmaxf(fabsf(k0), fabsf(k1)) : 0.0f;
        float av = act ? fmaxf(fabsf(v0), fabsf(v1)) : 0.0f;
        ak = wave_max(ak);
        av = wave_max(av);
        const uint32_t row = kv_store_row(g, pos);
        if (row == 0xFFFFFFFFu) continue;
        const float ik = (ak == 0.0f) ? 1.0f : 127.0f / ak;
        const float iv = (av == 0.0f) ? 1.0f : 127.0f / av;
        const uint32_t kc = act ? ((uint32_t)(uint8_t)quant_code(k0, ik) | ((uint32_t)(uint8_t)quant_code(k1, ik) << 8)) : 0u;
        const uint32_t vc = act ? ((uint32_t)(uint8_t)quant_code(v0, iv) | ((uint32_t)(uint8_t)quant_code(v1, iv) << 8)) : 0u;
        const uint32_t kn = (uint32_t)__shfl_xor((int)kc, 1, 64), vn = (uint32_t)__shfl_xor((int)vc, 1, 64);
        const size_t base = (plane * g.rows + row) * hd;
        if (act && (lane & 1u) == 0u) {
            stc(reinterpret_cast<uint32_t*>(a.kv.k + base + 2 * lane), kc | (kn << 16));
            stc(reinterpret_cast<uint32_t*>(a.kv.v + base + 2 * lane), vc | (vn << 16));
        }
        if (lane == 0) {
            stc(a.kv.ks + plane * g.rows + row, (ak == 0.0f) ? 1.0f : ak / 127.0f);
            stc(a.kv.vs + plane * g.rows + row, (av == 0.0f) ? 1.0f : av / 127.0f);
        }
    }
}

// ------------------------------------------------------------ attention

// True when visible entry j of view v holds a position >= pos0 (a row
// stored earlier in this pass, read coherently).
__device__ __forceinline__ bool entry_in_pass(const KvGeom& g, const KvView& v, uint32_t j, uint32_t pos0) {
    if (j < v.sink) return j >= pos0;
    j -= v.sink;
    if (j < v.pool) return false;
    return g.sink_size + v.win_lo + (j - v.pool) >= pos0;
}

__device__ __forceinline__ int4 ldc_int4(const int8_t* p) {
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    const uint64_t lo = ldc(q), hi = ldc(q + 1);
    return make_int4((int)(uint32_t)lo, (int)(uint32_t)(lo >> 32), (int)(uint32_t)hi, (int)(uint32_t)(hi >> 32));
}

// k_attn_chunk's task (row m, head h, chunk c) with coherent loads of this
// pass's data and coherent stores of the partials.
template <int PARTS>
__device__ __forceinline__ void attn_item(const DecodeArgs& a, uint32_t layer, uint32_t m, uint32_t h, uint32_t c, uint32_t pos0,
                          uint8_t* smem) {
    constexpr uint32_t hd = 16 * PARTS;
    const KvGeom& g = a.g;
    int8_t (*vt)[144] = reinterpret_cast<int8_t (*)[144]>(smem);
    float* qs = reinterpret_cast<float*>(smem + ATT_VT);
    float* kss = qs + 128;
    float* vsc = kss + 128;
    float* pe = vsc + 256;
    float* wp = pe + 256;
    float* red = wp + 512;
    const uint32_t t = threadIdx.x;
    const uint32_t D = g.n_heads * hd;
    const KvView v = kv_view(g, pos0 + m);
    const uint32_t C = v.count(), n = C + 1, j0 = c * 256u;
    const uint32_t j = j0 + t;
    const size_t plane = (size_t)layer * g.n_heads + h;
    const size_t qrow = (size_t)m * D + h * hd;
    const uint32_t nvis = j0 < C ? min(256u, C - j0) : 0u;
    if (t < hd) {
        qs[t] = ldc(a.q + qrow + t);
        kss[t] = ldc(a.k + qrow + t);
    }
    int4 kw[PARTS];
    float ks = 0.0f, vs = 0.0f;
    if (t < nvis) {
        const size_t row = plane * g.rows + kv_row(g, v, j);
        int4 vw[PARTS];
        if (entry_in_pass(g, v, j, pos0)) {
#pragma unroll
            for (int p = 0; p < PARTS; p++) {
                kw[p] = ldc_int4(a.kv.k + row * hd + 16 * p);
                vw[p] = ldc_int4(a.kv.v + row * hd + 16 * p);
            }
            ks = ldc(a.kv.ks + row);
            vs = ldc(a.kv.vs + row);
        } else {
            const int4* kr = reinterpret_cast<const int4*>(a.kv.k + row * hd);
            const int4* vr = reinterpret_cast<const int4*>(a.kv.v + row * hd);
#pragma unroll
            for (int p = 0; p < PARTS; p++) {
                kw[p] = kr[p];
                vw[p] = vr[p];
            }
            ks = a.kv.ks[row];
            vs = a.kv.vs[row];
        }
#pragma unroll
        for (int p = 0; p < PARTS; p++) *reinterpret_cast<int4*>(&vt[t][p * 16]) = vw[p];
    }
    vsc[t] = vs;
    __syncthreads();
    { const uint32_t l = layer; PF_TR(l, 40); }
    const float scale = 1.0f / __builtin_sqrtf((float)hd);
    float s = -__builtin_inff();
    if (t < nvis) {
        float acc = 0.0f;
#pragma unroll
        for (int p = 0; p < PARTS; p++) {
            const int wv[4] = {kw[p].x, kw[p].y, kw[p].z, kw[p].w};
#pragma unroll
            for (int b = 0; b < 16; b++) {
                const int8_t cb = (int8_t)((wv[b >> 2] >> (8 * (b & 3))) & 0xFF);
                acc = __builtin_fmaf(qs[p * 16 + b], (float)cb * ks, acc);
            }
        }
        s = acc * scale;
    } else if (j == C) {
        float self = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < hd; i++) self = self + qs[i] * kss[i];
        s = self * scale;
    }
    const float mx = block_max<4>(s, red);
    const float ex = j < n ? expf_c(s - mx) : 0.0f;
    pe[t] = ex;
    const float T = block_canon_sum<4>(ex, red);
    { const uint32_t l = layer; PF_TR(l, 41); }
    const uint32_t sc = t >> 6, i0 = 2u * (t & 63u);
    if (i0 < hd) {
        float w0 = 0.0f, w1 = 0.0f;
        const uint32_t e_end = min(64u * sc + 64u, (nvis + 7u) & ~7u);
        for (uint32_t e = 64u * sc; e < e_end; e += 8) {
            float pp[8], vv[8];
            uint32_t cc[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                pp[u] = pe[e + u];
                vv[u] = vsc[e + u];
                cc[u] = *reinterpret_cast<const uint16_t*>(&vt[e + u][i0]);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                w0 = __builtin_fmaf(pp[u], (float)(int8_t)(cc[u] & 0xFFu) * vv[u], w0);
                w1 = __builtin_fmaf(pp[u], (float)(int8_t)(cc[u] >> 8) * vv[u], w1);
            }
        }
        const uint32_t js = C - j0;
        if (js < 256u && (js >> 6) == sc) {
            const float p = pe[js];
            w0 = __builtin_fmaf(p, ldc(a.v + qrow + i0), w0);
            w1 = __builtin_fmaf(p, ldc(a.v + qrow + i0 + 1), w1);
        }
        wp[sc * 128 + i0] = w0;
        wp[sc * 128 + i0 + 1] = w1;
    }
    __syncthreads();
    { const uint32_t l = layer; PF_TR(l, 42); }
    const size_t mh = (size_t)m * g.n_heads + h;
    if (t < hd) {
        float u = 0.0f;
        u = u + wp[t];
        u = u + wp[128 + t];
        u = u + wp[256 + t];
        u = u + wp[384 + t];
        stc(a.Up + (mh * a.cstride + c) * hd + t, u);
    }
    if (t == 0) {
        stc(a.S + mh * a.s_stride + 2 * c, mx);
        stc(a.S + mh * a.s_stride + 2 * c + 1, T);
    }
}

// The last arrival of head h: every row's chunks merged (max of the chunk
// maxima, f_c = exp(m_c - max), T and U fmaf chains over c in order,
// out = U * (1 / (T + 1e-10))); rows past the pass are written as 0.  The
// head's amax per row is folded into amax_o with an integer max of the
// float bits (non-negative values order as integers).  Rows go in groups
// whose chunk statistics fit in LDS; within a group every load is issued
// before the arithmetic.
template <int M>
__device__ __forceinline__ void merge_head(const DecodeArgs& a, const Ctr& cc, uint32_t h, uint32_t pos0,
                                           uint32_t pm, uint32_t NC, uint8_t* smem, DecShared& sh) {
    const KvGeom& g = a.g;
    const uint32_t hd = a.hd, H = g.n_heads, D = a.D, t = threadIdx.x;
    float* fs = reinterpret_cast<float*>(smem);        // [rows][NC] chunk maxima, then f_c
    float* ts = fs + 2048;                              // [rows][NC] chunk sums
    float* rowT = ts + 2048;                            // [8] 1 / (T + 1e-10)
    const uint32_t RG = min((uint32_t)M, 2048u / NC);   // rows per group
    for (uint32_t m0 = 0; m0 < (uint32_t)M; m0 += RG) {
        const uint32_t rows = min(RG, (uint32_t)M - m0);
        __syncthreads();
        for (uint32_t e = t; e < rows * NC; e += 256) {
            const uint32_t r = e / NC, c = e - r * NC, m = m0 + r;
            const uint32_t nc = m < pm ? (kv_view(g, pos0 + m).count() + 1 + 255) / 256 : 0u;
            if (c < nc) {
                const float* st = a.S + ((size_t)m * H + h) * a.s_stride;
                fs[e] = ldc(st + 2 * c);
                ts[e] = ldc(st + 2 * c + 1);
            }
        }
        __syncthreads();
        // per row: max, f_c and the T chain (one wave per row)
        for (uint32_t r = t >> 6; r < rows; r += 4) {
            const uint32_t m = m0 + r, lane = t & 63u;
            if (m >= pm) continue;
            const uint32_t nc = (kv_view(g, pos0 + m).count() + 1 + 255) / 256;
            float mx = -__builtin_inff();
            for (uint32_t c = lane; c < nc; c += 64) mx = fmaxf(mx, fs[r * NC + c]);
            mx = wave_max(mx);
            for (uint32_t c = lane; c < nc; c += 64) fs[r * NC + c] = expf_c(fs[r * NC + c] - mx);
            if (lane == 0) {
                float T = 0.0f;
                for (uint32_t c = 0; c < nc; c++) T = __builtin_fmaf(ts[r * NC + c], fs[r * NC + c], T);
                rowT[r] = 1.0f / (T + 1e-10f);
            }
        }
        __syncthreads();
        // U chains: output o = r * hd + i, outputs t, t + 256, ...
        const uint32_t outs = rows * hd;
        for (uint32_t o0 = 0; o0 < outs; o0 += 256) {
            const uint32_t o = o0 + t;
            const uint32_t r = o / hd, i = o - r * hd, m = m0 + r;
            const bool live = o < outs;
            const uint32_t nc = (live && m < pm) ? (kv_view(g, pos0 + m).count() + 1 + 255) / 256 : 0u;
            const float* up = a.Up + ((size_t)(live ? m : 0u) * H + h) * a.cstride * hd + i;
            float U = 0.0f;
            for (uint32_t c0 = 0; c0 < nc; c0 += 16) {
                float uv[16];
#pragma unroll
                for (int k = 0; k < 16; k++) uv[k] = ldc(up + (size_t)min(c0 + k, nc - 1u) * hd);
#pragma unroll
                for (int k = 0; k < 16; k++)
                    if (c0 + k < nc) U = __builtin_fmaf(uv[k], fs[r * NC + c0 + k], U);
            }
            const float val = nc ? U * rowT[r] : 0.0f;
            if (live) stc(a.o + (size_t)m * D + h * hd + i, val);
            // a wave holds one row (head_dim >= 64)
            const float wm = wave_max(live ? fabsf(val) : 0.0f);
            if (live && (t & 63u) == 0u) atomicMax(cc.amax_o() + m, __float_as_uint(wm));
        }
    }
}

// ------------------------------------------------------------ the kernel

// The pointer value passed through an empty asm statement: addresses built
// from it inside the layer loop are not hoisted out of the loop (where they
// would stay live in registers across every phase).
template <class T>
__device__ __forceinline__ T* opaque(T* p) {
    asm volatile("" : "+s"(p));
    return p;
}

template <int M, int PARTS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void k_decode(DecodeArgs a0) {
    __shared__ __align__(16) uint8_t smem[DEC_SMEM];
    __shared__ DecShared sh;
    int8_t* sa = reinterpret_cast<int8_t*>(smem);
    int32_t* sb = reinterpret_cast<int32_t*>(smem + DEC_SA);
    double* red = reinterpret_cast<double*>(smem + DEC_SA + DEC_SB);
    const uint32_t G = gridDim.x, wg = blockIdx.x, t = threadIdx.x, lane = t & 63u;
    const uint32_t wid = __builtin_amdgcn_readfirstlane(t >> 6);
    const KvGeom& g = a0.g;
    const uint32_t D = a0.D, F = a0.F, H = a0.H, hd = a0.hd;
    const uint32_t pos0 = a0.pd->pos0, pm = min(a0.pd->m, (uint32_t)M);
    const uint32_t TD = D / 64, TF = F / 64;
    // attention chunks of the pass (the last row has the longest list)
    const uint32_t NC = (kv_view(g, pos0 + (pm ? pm : 1u) - 1u).count() + 1 + 255) / 256;
    const uint32_t n_groups = H * NC;
    const uint32_t att_items = 8u * (uint32_t)M * ((n_groups + 7u) / 8u);

    {
        const DecodeArgs& a = a0;
        PF_TR(0, 23);
        if (wg == 0) {
            const DecodeLayer& L0 = a.layers[0];
            norm_stats<M>(a.x, D, gptr(L0.an), a.stats, sh, a, 0, 28);
            drain();
            if (t == 0) arrive(a.ctr);   // layer 0 x_ready
        }
    }

    for (uint32_t l = 0; l < a0.L; l++) {
        DecodeArgs a = a0;
        a.x = opaque(a0.x);
        a.stats = opaque(a0.stats);
        a.acc_qkv = opaque(a0.acc_qkv);
        a.acc_o = opaque(a0.acc_o);
        a.acc_gu = opaque(a0.acc_gu);
        a.acc_d = opaque(a0.acc_d);
        a.q = opaque(a0.q);
        a.k = opaque(a0.k);
        a.v = opaque(a0.v);
        a.S = opaque(a0.S);
        a.Up = opaque(a0.Up);
        a.o = opaque(a0.o);
        a.f = opaque(a0.f);
        a.ctr = opaque(a0.ctr);
        a.kv.k = opaque(a0.kv.k);
        a.kv.v = opaque(a0.kv.v);
        a.kv.ks = opaque(a0.kv.ks);
        a.kv.vs = opaque(a0.kv.vs);
        a.layers = opaque(a0.layers);
        a.rope_c = opaque(a0.rope_c);
        a.rope_s = opaque(a0.rope_s);
        const DecodeLayer& Ly = a.layers[l];
        const Ctr cc{a.ctr + (size_t)l * a.ctr_layer, H, TD, TF};
        float* st_attn = a.stats + ((size_t)l * 2 + 0) * 16;
        float* st_ffn = a.stats + ((size_t)l * 2 + 1) * 16;

        // ---------------------------------------------------------- QKV
        {
            const uint32_t K = D, bpw = a.bpw[MAT_QKV], wb = 4 * bpw, splits = (K / 32) / wb;
            const uint32_t tiles = 3 * TD, items = tiles * splits;
            const uint32_t per_head = 3 * (hd / 64) * splits;
            for (uint32_t it = wg; it < items; it += G) {
                const uint32_t tile = it / splits, s = it - tile * splits;
                WRaw w;
                load_w_any(Ly.fmt[MAT_QKV], Ly.w[MAT_QKV], K, tile, s * wb + wid * bpw, bpw, lane, w);
                PF_TR(l, 0);
                if (!wait_ge(cc.x_ready(), 1u, a, sh)) return;
                PF_TR(l, 1);
                if (t < (uint32_t)M) {
                    const float inv = ldc(st_attn + 2 * t), amax = ldc(st_attn + 2 * t + 1);
                    sh.inv[t] = inv;
                    sh.invq[t] = (amax == 0.0f) ? 1.0f : 127.0f / amax;
                    sh.as[t] = (amax == 0.0f) ? 1.0f : amax / 127.0f;
                }
                __syncthreads();
                const uint32_t k0 = s * wb * 32;
                const float* xr = a.x + k0;
                const float* wr = gptr(Ly.an) + k0;
                PF_TR(l, 35);
                quant_slice<M>(xr, D, wb * 32, wr, sh.inv, sh.invq, sa, sb);
                __syncthreads();
                PF_TR(l, 36);
                gemv_dots<M>(w, Ly.fmt[MAT_QKV], bpw, sa, sb, red, a.acc_qkv, 3 * D, tile);
                PF_TR(l, 37);
                drain();
                PF_TR(l, 2);
                const uint32_t h = (tile % TD) / (hd / 64);
                const bool last = arrive_last(cc.head_cnt(h), per_head, sh);
                PF_TR(l, 3);
                if (last) {
                    qkv_post_head<M>(a, l, h, sh.as, pos0, pm);
                    drain();
                    PF_TR(l, 4);
                    if (t == 0) stc(cc.head_flag(h), 1u);
                }
            }
        }
        // ---------------------------------------------------------- attention
        for (uint32_t it = wg; it < att_items; it += G) {
            const uint32_t xcd = it & 7u, slot = it >> 3;
            const uint32_t grp = (slot / M) * 8u + xcd, m = slot % M;
            if (grp >= n_groups) continue;
            const uint32_t h = grp % H, c = grp / H;
            PF_TR(l, 5);
            if (!wait_ge(cc.head_flag(h), 1u, a, sh)) return;
            PF_TR(l, 6);
            if (m < pm && c * 256u < kv_view(g, pos0 + m).count() + 1) attn_item<PARTS>(a, l, m, h, c, pos0, smem);
            drain();
            PF_TR(l, 7);
            if (arrive_last(cc.att_cnt(h), NC * (uint32_t)M, sh)) {
                merge_head<M>(a, cc, h, pos0, pm, NC, smem, sh);
                drain();
                PF_TR(l, 8);
                if (t == 0) arrive(cc.heads_done());
            }
        }
        // ---------------------------------------------------------- O
        {
            const uint32_t K = D, bpw = a.bpw[MAT_O], wb = 4 * bpw, splits = (K / 32) / wb;
            const uint32_t items = TD * splits;
            for (uint32_t it = wg; it < items; it += G) {
                const uint32_t tile = it / splits, s = it - tile * splits;
                WRaw w;
                load_w_any(Ly.fmt[MAT_O], Ly.w[MAT_O], K, tile, s * wb + wid * bpw, bpw, lane, w);
                PF_TR(l, 9);
                if (!wait_ge(cc.heads_done(), H, a, sh)) return;
                PF_TR(l, 10);
                if (t < (uint32_t)M) {
                    const float amax = __uint_as_float(ldc(cc.amax_o() + t));
                    sh.invq[t] = (amax == 0.0f) ? 1.0f : 127.0f / amax;
                    sh.as[t] = (amax == 0.0f) ? 1.0f : amax / 127.0f;
                }
                __syncthreads();
                const float* orow = a.o + s * wb * 32;
                quant_slice<M>(orow, D, wb * 32, nullptr, nullptr, sh.invq, sa, sb);
                __syncthreads();
                gemv_dots<M>(w, Ly.fmt[MAT_O], bpw, sa, sb, red, a.acc_o, D, tile);
                drain();
                PF_TR(l, 11);
                if (arrive_last(cc.o_tile(tile), splits, sh)) {
                    // x[m][tile] += (float)(acc * as) (k_resid_norm_quant's residual)
                    for (uint32_t e = t; e < (uint32_t)M * 64u; e += 256u) {
                        const uint32_t m = e >> 6, col = tile * 64u + (e & 63u);
                        double* ap = a.acc_o + (size_t)m * D + col;
                        float* xp = a.x + (size_t)m * D + col;
                        const float xn = ldc(xp) + (float)(ldc(ap) * (double)sh.as[m]);
                        stc(xp, xn);
                        stc(ap, 0.0);
                    }
                    drain();
                    PF_TR(l, 12);
                    if (arrive_last(cc.o_tiles(), TD, sh)) {
                        norm_stats<M>(a.x, D, gptr(Ly.fn), st_ffn, sh, a, l, 24);
                        drain();
                        PF_TR(l, 13);
                        if (t == 0) stc(cc.xmid_ready(), 1u);
                    }
                }
            }
        }
        // ---------------------------------------------------------- gate|up
        {
            const uint32_t K = D, bpw = a.bpw[MAT_GU], wb = 4 * bpw, splits = (K / 32) / wb;
            const uint32_t items = 2 * TF * splits;
            for (uint32_t it = wg; it < items; it += G) {
                const uint32_t tile = it / splits, s = it - tile * splits;
                WRaw w;
                load_w_any(Ly.fmt[MAT_GU], Ly.w[MAT_GU], K, tile, s * wb + wid * bpw, bpw, lane, w);
                PF_TR(l, 14);
                if (!wait_ge(cc.xmid_ready(), 1u, a, sh)) return;
                PF_TR(l, 15);
                if (t < (uint32_t)M) {
                    const float inv = ldc(st_ffn + 2 * t), amax = ldc(st_ffn + 2 * t + 1);
                    sh.inv[t] = inv;
                    sh.invq[t] = (amax == 0.0f) ? 1.0f : 127.0f / amax;
                    sh.as[t] = (amax == 0.0f) ? 1.0f : amax / 127.0f;
                }
                __syncthreads();
                const uint32_t k0 = s * wb * 32;
                const float* xr = a.x + k0;
                const float* wr = gptr(Ly.fn) + k0;
                PF_TR(l, 32);
                quant_slice<M>(xr, D, wb * 32, wr, sh.inv, sh.invq, sa, sb);
                __syncthreads();
                PF_TR(l, 33);
                gemv_dots<M>(w, Ly.fmt[MAT_GU], bpw, sa, sb, red, a.acc_gu, 2 * F, tile);
                PF_TR(l, 34);
                drain();
                PF_TR(l, 16);
                const uint32_t p = tile % TF;
                if (arrive_last(cc.gu_pair(p), 2 * splits, sh)) {
                    // SwiGLU of columns [64p, 64p + 64) (k_swiglu_quant's
                    // arithmetic); wave w takes rows w, w + 4
                    for (uint32_t m = wid; m < (uint32_t)M; m += 4) {
                        const uint32_t col = p * 64u + lane;
                        double* gp = a.acc_gu + (size_t)m * 2 * F + col;
                        const double ga = ldc(gp), ua = ldc(gp + F);
                        stc(gp, 0.0);
                        stc(gp + F, 0.0);
                        const double as = (double)sh.as[m];
                        const float gt = (float)(ga * as);
                        const float uu = (float)(ua * as);
                        const float sig = 1.0f / (1.0f + expf_c(-gt));
                        const float fv = gt * sig * uu;
                        stc(a.f + (size_t)m * F + col, fv);
                        const float wm = wave_max(fabsf(fv));
                        if (lane == 0) atomicMax(cc.amax_f() + m, __float_as_uint(wm));
                    }
                    drain();
                    PF_TR(l, 17);
                    if (t == 0) arrive(cc.pairs());
                }
            }
        }
        // ---------------------------------------------------------- down
        {
            const uint32_t K = F, bpw = a.bpw[MAT_DOWN], wb = 4 * bpw, splits = (K / 32) / wb;
            const uint32_t items = TD * splits;
            for (uint32_t it = wg; it < items; it += G) {
                const uint32_t tile = it / splits, s = it - tile * splits;
                WRaw w;
                load_w_any(Ly.fmt[MAT_DOWN], Ly.w[MAT_DOWN], K, tile, s * wb + wid * bpw, bpw, lane, w);
                PF_TR(l, 18);
                if (!wait_ge(cc.pairs(), TF, a, sh)) return;
                PF_TR(l, 19);
                if (t < (uint32_t)M) {
                    const float amax = __uint_as_float(ldc(cc.amax_f() + t));
                    sh.invq[t] = (amax == 0.0f) ? 1.0f : 127.0f / amax;
                    sh.as[t] = (amax == 0.0f) ? 1.0f : amax / 127.0f;
                }
                __syncthreads();
                const float* frow = a.f + s * wb * 32;
                quant_slice<M>(frow, F, wb * 32, nullptr, nullptr, sh.invq, sa, sb);
                __syncthreads();
                gemv_dots<M>(w, Ly.fmt[MAT_DOWN], bpw, sa, sb, red, a.acc_d, D, tile);
                drain();
                PF_TR(l, 20);
                if (arrive_last(cc.d_tile(tile), splits, sh)) {
                    for (uint32_t e = t; e < (uint32_t)M * 64u; e += 256u) {
                        const uint32_t m = e >> 6, col = tile * 64u + (e & 63u);
                        double* ap = a.acc_d + (size_t)m * D + col;
                        float* xp = a.x + (size_t)m * D + col;
                        const float xn = ldc(xp) + (float)(ldc(ap) * (double)sh.as[m]);
                        stc(xp, xn);
                        stc(ap, 0.0);
                    }
                    drain();
                    PF_TR(l, 21);
                    if (arrive_last(cc.d_tiles(), TD, sh) && l + 1 < a.L) {
                        const Ctr cn{a.ctr + (size_t)(l + 1) * a.ctr_layer, H, TD, TF};
                        norm_stats<M>(a.x, D, gptr(a.layers[l + 1].an), a.stats + ((size_t)(l + 1) * 2) * 16, sh, a, l, 28);
                        drain();
                        PF_TR(l, 22);
                        if (t == 0) stc(cn.x_ready(), 1u);
                    }
                }
            }
        }
    }
}

}  // namespace pf

namespace pf {

// p[0..n) = 0 (per-pass counter reset; a kernel, so that captured graphs
// hold no memset node).
__global__ void k_zero_u32(uint32_t* __restrict__ p, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

}  // namespace pf
