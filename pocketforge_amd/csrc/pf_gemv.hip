// GEMV / GEMM kernels for gfx950.
//
//  * k_gemv_i8     int8 activations x block-quantized (Q4/Q2/Q1.5, 32-wide
//                  blocks, fp16 scale) tiled matrix, M <= 8 activation rows.
//                  One lane per output row, wave-uniform activations in
//                  SGPRs, v_dot4 int32 block dots, exact fp64 accumulation of
//                  d_b * p_b, fp32 output.  HBM bound: every weight byte is
//                  read once.
//  * k_gemv_f32    fp32 activations x dequantized Q4 row-major matrix (tied
//                  unembedding, MTP heads) in the canonical 64-lane order.
//  * row prologues quantize_activation_row, residual + RMSNorm + quantize,
//                  SwiGLU + quantize, all producing int8 rows, the row scale
//                  and per-32-block sums of the codes.
//  * k_matmul_int8 / k_mm_epilogue: the reference's plain int8 matmul API.
#include "pf_device.h"

namespace pf {

// ===================================================== int8 x block GEMV

template <int FMT>
__device__ __forceinline__ void unpack_codes(const uint8_t* tile, uint32_t t, uint32_t lane,
                                             uint32_t u[8]) {
    if constexpr (FMT == FMT_Q4) {
        uint4 c = *reinterpret_cast<const uint4*>(tile + t * 1024u + lane * 16u);
        const uint32_t m = 0x0F0F0F0Fu;
        u[0] = c.x & m; u[1] = c.y & m; u[2] = c.z & m; u[3] = c.w & m;
        u[4] = (c.x >> 4) & m; u[5] = (c.y >> 4) & m; u[6] = (c.z >> 4) & m; u[7] = (c.w >> 4) & m;
    } else {
        uint2 c = *reinterpret_cast<const uint2*>(tile + (t >> 1) * 1024u + lane * 16u + (t & 1u) * 8u);
        const uint32_t m = 0x03030303u;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            u[2 * p] = (c.x >> (2 * p)) & m;
            u[2 * p + 1] = (c.y >> (2 * p)) & m;
        }
    }
}

// acc[m][n] += S_split with S = sum_b d_b * p_b over the blocks of one
// K split, p_b = sum_i a[m][32b+i] * code[n][32b+i] (int32).  Every term
// d_b * p_b is an integer multiple of the smallest block-scale ulp of the
// row and the row's scales span at most 15 binades (checked at upload), so
// all partial sums are exact in fp64: the splits meet through fp64 atomic
// adds in any order with a bit-identical result.  The consumer converts
// (float)(acc * (double)a_scale) and clears acc.
// Grid (N/64, splits), 64 WAVES threads; wave w of split s covers blocks
// [(WAVES s+w)*bpw, (WAVES s+w+1)*bpw), bpw in {1, 2, 4} with
// nb % (WAVES bpw) == 0, lane = output row.  The waves of a workgroup meet in
// LDS, so larger workgroups mean fewer K splits and fewer fp64 atomics for
// the same number of waves.  Each wave issues all its weight loads first; the
// workgroup's activation rows and block sums are staged in LDS with one
// vector load per thread (they come from another kernel, often through
// another XCD's L2).
template <int FMT, int M, bool GATED = false, int WAVES = 4>
__global__ __launch_bounds__(64 * WAVES) void k_gemv_i8(const uint8_t* __restrict__ W, uint32_t K,
                                                 const int8_t* __restrict__ act, uint32_t act_stride,
                                                 const int32_t* __restrict__ bsum, uint32_t bsum_stride,
                                                 uint32_t bpw, double* __restrict__ acc, uint32_t acc_stride,
                                                 const uint32_t* __restrict__ gate) {
    constexpr uint32_t TB = tile_bytes(FMT);
    constexpr uint32_t CODES = TILE_ROWS * TILE_BLOCKS * code_bytes(FMT);
    constexpr int OFF = code_offset(FMT);
    if constexpr (GATED)
        if (*gate == 0u) return;   // no row of the pass needs this product
    constexpr uint32_t NT = 64u * WAVES;
    __shared__ __align__(16) int32_t sa[M][WAVES * 4 * 8];  // activations of the workgroup's WAVES bpw blocks
    __shared__ int32_t sb[M][WAVES * 4];
    __shared__ double red[WAVES][M][64];
    const uint32_t g = blockIdx.x, s = blockIdx.y;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t chunks = K >> 8, wb = WAVES * bpw, wb0 = s * wb, b0 = wb0 + wid * bpw;
    const uint8_t* tiles = W + (size_t)g * chunks * TB;
    uint32_t u[4][8];
    uint16_t dh[4];        // scale bits: converted after the staging below, so that no
                           // conversion waits on a load before every load is issued
#pragma unroll
    for (uint32_t k = 0; k < 4; k++) {
        dh[k] = 0;
#pragma unroll
        for (int q = 0; q < 8; q++) u[k][q] = 0u;
        if (k < bpw) {
            const uint32_t b = b0 + k;
            const uint8_t* tile = tiles + (size_t)(b >> 3) * TB;
            unpack_codes<FMT>(tile, b & 7u, lane, u[k]);
            dh[k] = *reinterpret_cast<const uint16_t*>(tile + CODES + lane * 16u + (b & 7u) * 2u);
        }
    }
    for (uint32_t i = threadIdx.x; i < (uint32_t)M * wb * 8u; i += NT) {
        const uint32_t m = i / (wb * 8u), r = i - m * wb * 8u;
        sa[m][r] = reinterpret_cast<const int32_t*>(act + (size_t)m * act_stride)[wb0 * 8u + r];
    }
    if (threadIdx.x < (uint32_t)M * wb) {
        const uint32_t m = threadIdx.x / wb, k = threadIdx.x - m * wb;
        sb[m][k] = bsum[(size_t)m * bsum_stride + wb0 + k];
    }
    __syncthreads();
    double d[4];
#pragma unroll
    for (uint32_t k = 0; k < 4; k++) d[k] = (double)h2f(dh[k]);
    double S[M];
#pragma unroll
    for (int m = 0; m < M; m++) S[m] = 0.0;
#pragma unroll
    for (uint32_t k = 0; k < 4; k++) {
        if (k < bpw) {
            const uint32_t j = wid * bpw + k;
#pragma unroll
            for (int m = 0; m < M; m++) {
                const int4 a0 = *reinterpret_cast<const int4*>(&sa[m][j * 8u]);
                const int4 a1 = *reinterpret_cast<const int4*>(&sa[m][j * 8u + 4u]);
                int p = -OFF * sb[m][j];
                p = __builtin_amdgcn_sdot4((int)u[k][0], a0.x, p, false);
                p = __builtin_amdgcn_sdot4((int)u[k][1], a0.y, p, false);
                p = __builtin_amdgcn_sdot4((int)u[k][2], a0.z, p, false);
                p = __builtin_amdgcn_sdot4((int)u[k][3], a0.w, p, false);
                p = __builtin_amdgcn_sdot4((int)u[k][4], a1.x, p, false);
                p = __builtin_amdgcn_sdot4((int)u[k][5], a1.y, p, false);
                p = __builtin_amdgcn_sdot4((int)u[k][6], a1.z, p, false);
                p = __builtin_amdgcn_sdot4((int)u[k][7], a1.w, p, false);
                S[m] = __builtin_fma(d[k], (double)p, S[m]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; m++) red[wid][m][lane] = S[m];
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < (uint32_t)M * 64u; t += NT) {
        const uint32_t m = t >> 6, r = t & 63u;
        double v = red[0][m][r];
#pragma unroll
        for (int w = 1; w < WAVES; w++) v += red[w][m][r];
        atomicAdd(acc + (size_t)m * acc_stride + (size_t)g * 64u + r, v);
    }
}

// ===================================================== int8 x block GEMM

typedef int pf_v4i __attribute__((ext_vector_type(4)));
typedef int pf_v16i __attribute__((ext_vector_type(16)));

// Signed codes of the 16 elements 16h .. 16h + 15 of weight row r, block t,
// of a tile, packed 4 per dword in element order (MFMA B operand).  Byte
// x - OFF is formed as (x + (0x80 - OFF)) ^ 0x80 per byte (no carries: every
// byte sum is below 0x100).
// Raw code bytes of weight row r, block t (Q4: 16 bytes; Q2/Q1.5: 8 bytes in
// .x, .y), loaded one block ahead of their use.
template <int FMT>
__device__ __forceinline__ uint4 gemm_raw(const uint8_t* tile, uint32_t t, uint32_t r) {
    if constexpr (FMT == FMT_Q4) return *reinterpret_cast<const uint4*>(tile + t * 1024u + r * 16u);
    const uint2 c = *reinterpret_cast<const uint2*>(tile + (t >> 1) * 1024u + r * 16u + (t & 1u) * 8u);
    return make_uint4(c.x, c.y, 0u, 0u);
}

template <int FMT>
__device__ __forceinline__ pf_v4i gemm_unpack(uint4 c, uint32_t h) {
    constexpr uint32_t OFF = (uint32_t)code_offset(FMT);
    constexpr uint32_t ADD = (0x80u - OFF) * 0x01010101u;
    pf_v4i v;
    if constexpr (FMT == FMT_Q4) {
        const uint32_t sh = 4u * h, m = 0x0F0F0F0Fu;
        v.x = (int)((((c.x >> sh) & m) + ADD) ^ 0x80808080u);
        v.y = (int)((((c.y >> sh) & m) + ADD) ^ 0x80808080u);
        v.z = (int)((((c.z >> sh) & m) + ADD) ^ 0x80808080u);
        v.w = (int)((((c.w >> sh) & m) + ADD) ^ 0x80808080u);
    } else {
        const uint32_t sh = 4u * h, m = 0x03030303u;
        v.x = (int)((((c.x >> sh) & m) + ADD) ^ 0x80808080u);
        v.y = (int)((((c.y >> sh) & m) + ADD) ^ 0x80808080u);
        v.z = (int)((((c.x >> (sh + 2u)) & m) + ADD) ^ 0x80808080u);
        v.w = (int)((((c.y >> (sh + 2u)) & m) + ADD) ^ 0x80808080u);
    }
    return v;
}

template <int FMT>
__device__ __forceinline__ pf_v4i gemm_codes(const uint8_t* tile, uint32_t t, uint32_t r, uint32_t h) {
    constexpr uint32_t OFF = (uint32_t)code_offset(FMT);
    constexpr uint32_t ADD = (0x80u - OFF) * 0x01010101u;
    pf_v4i v;
    if constexpr (FMT == FMT_Q4) {
        const uint4 c = *reinterpret_cast<const uint4*>(tile + t * 1024u + r * 16u);
        const uint32_t sh = 4u * h, m = 0x0F0F0F0Fu;
        v.x = (int)((((c.x >> sh) & m) + ADD) ^ 0x80808080u);
        v.y = (int)((((c.y >> sh) & m) + ADD) ^ 0x80808080u);
        v.z = (int)((((c.z >> sh) & m) + ADD) ^ 0x80808080u);
        v.w = (int)((((c.w >> sh) & m) + ADD) ^ 0x80808080u);
    } else {
        const uint2 c = *reinterpret_cast<const uint2*>(tile + (t >> 1) * 1024u + r * 16u + (t & 1u) * 8u);
        const uint32_t sh = 4u * h, m = 0x03030303u;
        v.x = (int)((((c.x >> sh) & m) + ADD) ^ 0x80808080u);
        v.y = (int)((((c.y >> sh) & m) + ADD) ^ 0x80808080u);
        v.z = (int)((((c.x >> (sh + 2u)) & m) + ADD) ^ 0x80808080u);
        v.w = (int)((((c.y >> (sh + 2u)) & m) + ADD) ^ 0x80808080u);
    }
    return v;
}

// acc[m][n] += sum over the blocks [s bps, (s + 1) bps) of d[n][b] * p[m][n][b]
// for M activation rows (M > 8: verify passes of many sequences, batched
// prefill), the exact fp64 sum of k_gemv_i8.  p comes from
// v_mfma_i32_32x32x32_i8, one 32-element block per instruction: lane l
// holds activation row l % 32 and weight row l % 32, elements 16 (l / 32)
// .. + 15; result element i is activation row 8 (i / 4) + 4 (l / 32) + i % 4,
// weight row l % 32, so a lane needs one block scale per block.
// Grid (N / 32, splits), 256 threads: the block's 32 weight rows
// [32 blockIdx.x, + 32) against activation tiles w, w + 4, ... (MTW per
// wave) of 32 rows each; act holds ceil(M / 32) * 32 readable rows.
template <int FMT, int MTW, bool GATED = false>
__global__ __launch_bounds__(256) void k_gemm_i8(const uint8_t* __restrict__ W, uint32_t K, uint32_t M,
                                                 const int8_t* __restrict__ act, uint32_t act_stride, uint32_t bps,
                                                 double* __restrict__ acc, uint32_t acc_stride,
                                                 const uint32_t* __restrict__ gate) {
    constexpr uint32_t TB = tile_bytes(FMT);
    constexpr uint32_t CODES = TILE_ROWS * TILE_BLOCKS * code_bytes(FMT);
    if constexpr (GATED)
        if (*gate == 0u) return;   // no row of the pass needs this product
    const uint32_t lane = threadIdx.x & 63u, h = lane >> 5, l32 = lane & 31u;
    const uint32_t wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n0 = blockIdx.x * 32u, r = (n0 & 63u) + l32;
    const uint32_t nb = K >> 5, chunks = K >> 8, mtiles = (M + 31u) / 32u;
    const uint32_t b_begin = blockIdx.y * bps, b_end = min(b_begin + bps, nb);
    const uint8_t* tiles = W + (size_t)(n0 >> 6) * chunks * TB;
    double S[MTW][16];
#pragma unroll
    for (int j = 0; j < MTW; j++)
#pragma unroll
        for (int i = 0; i < 16; i++) S[j][i] = 0.0;
    const pf_v16i zero = {};
    // raw operands of block b: code bytes, block scale bits, activation tiles
    auto load = [&](uint32_t b, uint4& bw, uint16_t& d, pf_v4i (&a)[MTW]) {
        const uint8_t* tile = tiles + (size_t)(b >> 3) * TB;
        const uint32_t t = b & 7u;
        bw = gemm_raw<FMT>(tile, t, r);
        d = *reinterpret_cast<const uint16_t*>(tile + CODES + r * 16u + t * 2u);
        // every tile loads (a wave's tiles past the last one reload it, unused),
        // so the number of loads in flight is fixed and the waits are exact
#pragma unroll
        for (int j = 0; j < MTW; j++) {
            const uint32_t mt = min(wid + 4u * j, mtiles - 1u);
            a[j] = *reinterpret_cast<const pf_v4i*>(act + (size_t)(mt * 32u + l32) * act_stride + b * 32u + 16u * h);
        }
    };
    // the next block's operands load while this block's MFMAs and scaling run
    uint4 bw_n{};
    uint16_t d_n = 0;
    pf_v4i a_n[MTW];
    if (b_begin < b_end) load(b_begin, bw_n, d_n, a_n);
    for (uint32_t b = b_begin; b < b_end; b++) {
        const pf_v4i bw = gemm_unpack<FMT>(bw_n, h);
        const double d = (double)h2f(d_n);
        pf_v4i a[MTW];
#pragma unroll
        for (int j = 0; j < MTW; j++) a[j] = a_n[j];
        load(min(b + 1, b_end - 1), bw_n, d_n, a_n);      // unconditional: exact wait counts
        pf_v16i p[MTW];
#pragma unroll
        for (int j = 0; j < MTW; j++)
            if (wid + 4u * j < mtiles) p[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[j], bw, zero, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < MTW; j++) {
            if (wid + 4u * j < mtiles) {
#pragma unroll
                for (int i = 0; i < 16; i++) S[j][i] = __builtin_fma(d, (double)p[j][i], S[j][i]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < MTW; j++) {
        const uint32_t mt = wid + 4u * j;
        if (mt >= mtiles) continue;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t m = mt * 32u + 8u * (i / 4) + 4u * h + (i % 4);
            if (m < M) atomicAdd(acc + (size_t)m * acc_stride + n0 + l32, S[j][i]);
        }
    }
}

// y = (float)(acc * (double)as[m]); acc cleared for its next use.
__device__ __forceinline__ float take_acc(double* acc, size_t i, float as) {
    const double v = acc[i];
    acc[i] = 0.0;
    return (float)(v * (double)as);
}

// Finishes a GEMV for the kernel-level entry point.
__global__ void k_gemv_finish(double* __restrict__ acc, uint32_t N, const float* __restrict__ as,
                              float* __restrict__ y) {
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x, m = blockIdx.y;
    if (n >= N) return;
    y[(size_t)m * N + n] = take_acc(acc, (size_t)m * N + n, as[m]);
}

// acc[0..n) = 0 (one-time set-up of accumulators; a kernel, not a memset).
__global__ void k_zero_f64(double* __restrict__ p, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0;
}

// ============================================ fp32 x dequantized Q4 GEMV

// y[m][n] (+= y_in[m][n] when resid) = canonical fp32 dot of h[m] with row n:
// lane l holds block l (K <= 2048), fmaf chain over the block's elements,
// halving tree over the 64 lanes.  Each wave walks rows n = wave, wave +
// total_waves, ...
template <int M>
__global__ __launch_bounds__(256) void k_gemv_f32(const uint8_t* __restrict__ codes,
                                                  const uint16_t* __restrict__ scales,
                                                  uint32_t N, uint32_t K,
                                                  const float* __restrict__ h, uint32_t h_stride,
                                                  float* __restrict__ y, uint32_t y_stride,
                                                  const float* __restrict__ y_in) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
    const uint32_t nb = K >> 5;
    const bool live = lane < nb;
    float hv[M][32];
#pragma unroll
    for (int m = 0; m < M; m++) {
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            float4 v = live ? *reinterpret_cast<const float4*>(h + (size_t)m * h_stride + lane * 32u + i)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
            hv[m][i] = v.x; hv[m][i + 1] = v.y; hv[m][i + 2] = v.z; hv[m][i + 3] = v.w;
        }
    }
    for (uint32_t n = wave; n < N; n += nwaves) {
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; m++) acc[m] = 0.0f;
        if (live) {
            uint4 c = *reinterpret_cast<const uint4*>(codes + ((size_t)n * nb + lane) * 16u);
            float d = h2f(scales[(size_t)n * nb + lane]);
            float nd = -8.0f * d;
            uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
            for (int j = 0; j < 16; j++) {
                uint32_t byte = (cw[j >> 2] >> (8 * (j & 3))) & 0xFFu;
                float w0 = __builtin_fmaf((float)(byte & 15u), d, nd);
                float w1 = __builtin_fmaf((float)(byte >> 4), d, nd);
#pragma unroll
                for (int m = 0; m < M; m++) {
                    acc[m] = __builtin_fmaf(hv[m][2 * j], w0, acc[m]);
                    acc[m] = __builtin_fmaf(hv[m][2 * j + 1], w1, acc[m]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            float t = wave_tree_sum(acc[m]);
            if (lane == 0) {
                size_t o = (size_t)m * y_stride + n;
                y[o] = y_in ? (y_in[o] + t) : t;
            }
        }
    }
}

// y[m][n] = canonical fp32 dot of h[m] with row n of a dense fp32 matrix E
// [N][K] (an fp32 tied table handed to MTPHeads::forward): the order of
// k_gemv_f32 with the weight value itself (lane l = block l, K <= 2048).
template <int M>
__global__ __launch_bounds__(256) void k_gemv_f32_dense(const float* __restrict__ E, uint32_t N, uint32_t K,
                                                        const float* __restrict__ h, uint32_t h_stride,
                                                        float* __restrict__ y, uint32_t y_stride) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
    const bool live = lane < (K >> 5);
    float hv[M][32];
#pragma unroll
    for (int m = 0; m < M; m++) {
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            float4 v = live ? *reinterpret_cast<const float4*>(h + (size_t)m * h_stride + lane * 32u + i)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
            hv[m][i] = v.x; hv[m][i + 1] = v.y; hv[m][i + 2] = v.z; hv[m][i + 3] = v.w;
        }
    }
    for (uint32_t n = wave; n < N; n += nwaves) {
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; m++) acc[m] = 0.0f;
        if (live) {
            const float* row = E + (size_t)n * K + lane * 32u;
            float w[32];
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                float4 v = *reinterpret_cast<const float4*>(row + i);
                w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
            }
#pragma unroll
            for (int i = 0; i < 32; i++)
#pragma unroll
                for (int m = 0; m < M; m++) acc[m] = __builtin_fmaf(hv[m][i], w[i], acc[m]);
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            float t = wave_tree_sum(acc[m]);
            if (lane == 0) y[(size_t)m * y_stride + n] = t;
        }
    }
}

// MTPHeads::forward without a tied table (src/mtp.cpp:117-121): logits[v] =
// ((v * 2654435761 + head) mod V) / V.
__global__ void k_mtp_placeholder(float* __restrict__ logits, uint32_t V, uint32_t head) {
    const uint32_t v = blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= V) return;
    logits[v] = (float)(((uint64_t)v * 2654435761ULL + (uint64_t)head) % V) / (float)V;
}

// dot_product (src/matmul_neon.cpp:186-207) in the CANON(4) order: lane l of
// 256 sums a[j] * b[j] (product, then add) for j = l, l + 256, ...
__global__ __launch_bounds__(256) void k_dot_canon(const float* __restrict__ a, const float* __restrict__ b,
                                                   uint32_t n, float* __restrict__ out) {
    __shared__ float red[4];
    float p = 0.0f;
    for (uint32_t j = threadIdx.x; j < n; j += 256) p = p + a[j] * b[j];
    const float s = block_canon_sum<4>(p, red);
    if (threadIdx.x == 0) *out = s;
}

// softmax in place (src/matmul_neon.cpp:212-226): max, e = exp(x - max),
// CANON(4) sum, x = e * (1 / (sum + 1e-10)).
__global__ __launch_bounds__(256) void k_softmax_one(float* __restrict__ v, uint32_t n) {
    __shared__ float red[4];
    float mx = -__builtin_inff();
    for (uint32_t j = threadIdx.x; j < n; j += 256) mx = fmaxf(mx, v[j]);
    mx = block_max<4>(mx, red);
    float part = 0.0f;
    for (uint32_t j = threadIdx.x; j < n; j += 256) {
        const float e = expf_c(v[j] - mx);
        v[j] = e;
        part = part + e;
    }
    const float inv = 1.0f / (block_canon_sum<4>(part, red) + 1e-10f);
    for (uint32_t j = threadIdx.x; j < n; j += 256) v[j] = v[j] * inv;
}

// rmsnorm (src/matmul_neon.cpp:231-239): CANON(4) sum of squares (fmaf),
// rms = sqrt(ss / n + 1e-6), out = x * (1 / rms) * w.
__global__ __launch_bounds__(256) void k_rmsnorm_one(float* __restrict__ out, const float* __restrict__ x,
                                                     const float* __restrict__ w, uint32_t n) {
    __shared__ float red[4];
    float p = 0.0f;
    for (uint32_t j = threadIdx.x; j < n; j += 256) p = __builtin_fmaf(x[j], x[j], p);
    const float ss = block_canon_sum<4>(p, red);
    const float inv = 1.0f / __builtin_sqrtf(ss / (float)n + 1e-6f);
    for (uint32_t j = threadIdx.x; j < n; j += 256) out[j] = x[j] * inv * w[j];
}

// ============================================================ prologues

template <int PER>
__global__ __launch_bounds__(256) void k_quant_rows(const float* __restrict__ x, uint32_t x_stride,
                                                    uint32_t K, int8_t* __restrict__ q, uint32_t q_stride,
                                                    float* __restrict__ as, int32_t* __restrict__ bsum,
                                                    uint32_t bsum_stride) {
    __shared__ float red[4];
    const uint32_t m = blockIdx.x;
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        uint32_t i = threadIdx.x + 256u * k;
        v[k] = i < K ? x[(size_t)m * x_stride + i] : 0.0f;
    }
    quantize_row_block<PER, 256>(v, K, q + (size_t)m * q_stride, as + m,
                                 bsum ? bsum + (size_t)m * bsum_stride : nullptr, red);
}

// x[m] += (float)(acc[m] * as_prev[m]) (when acc != null; acc cleared),
// then the engine's RMSNorm (src/matmul_neon.cpp:231-239) with weight w in
// tile-canonical order (the sum of squares is the sequential sum over
// 64-element tiles of each tile's halving tree of x * x; normed = (x * w) *
// inv), then quantize_activation_row of the normed row.  Grid M, 1024
// threads: all loads are issued first; wave w builds the trees of tiles w,
// w + 16, ... from the row in LDS (K <= 4096, K % 64 == 0).
// Blocks past the `rows` row blocks prefetch pf (the weights of the GEMV that
// consumes the output).  SKIP instances (layer skip on): with skipm, rows
// whose flag is set take no residual
// (their FFN was skipped; acc is still cleared); with nout, the normed rows
// are also written there in fp32; with nclear, block 0 zeroes that word
// (the count of rows that run the layer's FFN, built by k_layer_skip).
template <int PER, bool SKIP = false>
__global__ __launch_bounds__(1024) void k_resid_norm_quant(float* __restrict__ x, uint32_t K,
                                                           double* __restrict__ acc,
                                                           const float* __restrict__ as_prev,
                                                           const float* __restrict__ w,
                                                           int8_t* __restrict__ q, uint32_t q_stride,
                                                           float* __restrict__ as, int32_t* __restrict__ bsum,
                                                           uint32_t bsum_stride, uint32_t rows, Prefetch pf,
                                                           const uint32_t* __restrict__ skipm,
                                                           float* __restrict__ nout, uint32_t* __restrict__ nclear) {
    __shared__ float row[4096];
    __shared__ float tree[64];
    __shared__ float red[16];
    const uint32_t m = blockIdx.x, t = threadIdx.x;
    if constexpr (SKIP)
        if (nclear && m == 0 && t == 0) *nclear = 0u;
    if (m >= rows) {
        prefetch_bytes(pf.p, pf.n, m - rows, gridDim.x - rows, pf.sink);
        return;
    }
    float xv[PER], wv[PER];
    double av[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const uint32_t i = t + 1024u * k;
        xv[k] = i < K ? x[(size_t)m * K + i] : 0.0f;
        wv[k] = i < K ? w[i] : 0.0f;
        av[k] = (acc && i < K) ? acc[(size_t)m * K + i] : 0.0;
    }
    const float ap = acc ? as_prev[m] : 0.0f;
    bool add = acc != nullptr;
    if constexpr (SKIP) add = add && !(skipm && skipm[m]);
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const uint32_t i = t + 1024u * k;
        if (acc && i < K) {
            if (add) {
                xv[k] = xv[k] + (float)(av[k] * (double)ap);
                x[(size_t)m * K + i] = xv[k];
            }
            acc[(size_t)m * K + i] = 0.0;
        }
        if (i < K) row[i] = xv[k];
    }
    __syncthreads();
    // tile trees of x * x, then their sequential sum
    const uint32_t wid = t >> 6, lane = t & 63u;
    for (uint32_t tl = wid; tl < K / 64u; tl += 16u) {
        const float v = row[64u * tl + lane];
        const float s = wave_tree_sum(v * v);
        if (lane == 0) tree[tl] = s;
    }
    __syncthreads();
    if (t == 0) {
        // sequential sum of the tile trees, 16 LDS reads in flight at a time
        float ss = 0.0f;
        for (uint32_t t0 = 0; t0 < K / 64u; t0 += 16) {
            float tv[16];
#pragma unroll
            for (int k = 0; k < 16; k++) tv[k] = tree[min(t0 + k, 63u)];
#pragma unroll
            for (int k = 0; k < 16; k++)
                if (t0 + k < K / 64u) ss = ss + tv[k];
        }
        red[0] = ss;
    }
    __syncthreads();
    const float ss = red[0];
    __syncthreads();
    const float rms = __builtin_sqrtf(ss / (float)K + 1e-6f);
    const float inv = 1.0f / rms;
#pragma unroll
    for (int k = 0; k < PER; k++) xv[k] = (xv[k] * wv[k]) * inv;
    if (SKIP && nout) {
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const uint32_t i = t + 1024u * k;
            if (i < K) nout[(size_t)m * K + i] = xv[k];
        }
    }
    __syncthreads();
    quantize_row_block<PER, 1024>(xv, K, q + (size_t)m * q_stride, as + m,
                                  bsum ? bsum + (size_t)m * bsum_stride : nullptr, red);
}

// quantize_activation_row of rows of length K <= 1024 * PER, 1024 threads.
template <int PER>
__global__ __launch_bounds__(1024) void k_quant_rows_wide(const float* __restrict__ x, uint32_t K,
                                                          int8_t* __restrict__ q, uint32_t q_stride,
                                                          float* __restrict__ as, int32_t* __restrict__ bsum,
                                                          uint32_t bsum_stride) {
    __shared__ float red[16];
    const uint32_t m = blockIdx.x;
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const uint32_t i = threadIdx.x + 1024u * k;
        v[k] = i < K ? x[(size_t)m * K + i] : 0.0f;
    }
    quantize_row_block<PER, 1024>(v, K, q + (size_t)m * q_stride, as + m,
                                  bsum ? bsum + (size_t)m * bsum_stride : nullptr, red);
}

// x[m] += (float)(acc[m] * as_prev[m]) (the last layer's down residual;
// none for rows flagged in skipm, whose acc is still cleared).
__global__ void k_resid_add(float* __restrict__ x, uint32_t K, double* __restrict__ acc,
                            const float* __restrict__ as_prev, const uint32_t* __restrict__ skipm) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x, m = blockIdx.y;
    if (i >= K) return;
    const float r = take_acc(acc, (size_t)m * K + i, as_prev[m]);
    if (!(skipm && skipm[m])) x[(size_t)m * K + i] = x[(size_t)m * K + i] + r;
}

// LayerSkipController::should_skip_ffn (src/layer_skip.cpp:22-67) at one
// layer for the rows of sequence blockIdx.x in pass order.  normed holds the
// FFN inputs of the pass's rows [M][K]; each row's delta (hidden_delta,
// src/layer_skip.cpp:105-111: sqrt of the mean squared difference, the sum in
// the tile order of the engine's RMSNorm) is taken against the input of the
// sequence's last row in this pass that ran its FFN, else against the
// sequence's cache (cache + blockIdx.x * cache_seq_stride).  flag[r] = 1:
// row r skips its FFN.  thr is the layer's adjusted threshold (< 0: the layer
// never skips).  nrun (zeroed earlier in the pass) gains the number of rows
// that run their FFN: the FFN products of a pass in which no row runs it are
// not computed.  The cache is written by k_skip_commit once it is known which
// rows count.  Rows go one after another, the 16 waves sharing each row's
// tiles.  K % 64 == 0, K <= 4096; 1024 threads.
__global__ __launch_bounds__(1024) void k_layer_skip(const PassDesc* __restrict__ pd, uint32_t M,
                                                     const float* __restrict__ normed,
                                                     const float* __restrict__ cache, size_t cache_seq_stride,
                                                     uint32_t K, float thr, uint32_t* __restrict__ flag,
                                                     uint32_t* __restrict__ nrun) {
    __shared__ float tree[64];
    __shared__ uint32_t skipped;
    const uint32_t s = blockIdx.x, t = threadIdx.x, wid = t >> 6, lane = t & 63u;
    const float* ref = cache + (size_t)s * cache_seq_stride;
    uint32_t runs = 0;
    for (uint32_t r = 0; r < M; r++) {
        if (row_seq(pd, r) != s) continue;
        const float* a = normed + (size_t)r * K;
        if (!(thr >= 0.0f)) {
            if (t == 0) flag[r] = 0;
            ref = a;
            runs++;
            continue;
        }
        for (uint32_t tl = wid; tl < K / 64u; tl += 16u) {
            const float d = a[64u * tl + lane] - ref[64u * tl + lane];
            const float sq = wave_tree_sum(d * d);
            if (lane == 0) tree[tl] = sq;
        }
        __syncthreads();
        if (t == 0) {
            float sum = 0.0f;
            for (uint32_t tl = 0; tl < K / 64u; tl++) sum = sum + tree[tl];
            const uint32_t sk = __builtin_sqrtf(sum / (float)K) < thr ? 1u : 0u;
            flag[r] = sk;
            skipped = sk;
        }
        __syncthreads();
        if (!skipped) {
            ref = a;
            runs++;
        }
    }
    if (t == 0 && runs) atomicAdd(nrun, runs);
}

// The cache update of should_skip_ffn (src/layer_skip.cpp:57-62) for the rows
// of a pass that count: per (layer blockIdx.x, sequence blockIdx.y), the
// sequence's rows j0 <= j < j1 (j numbering the sequence's rows in pass
// order), where for a verify pass (st non-null) j1 = min(accepted + 1, n_mtp)
// with the round's accepted drafts from st[sequence] -- the rows that
// src/engine.cpp:336-365 forwards.  The cache takes the FFN input of the last
// such row that ran its FFN; skips counts the rows that skipped.
// stage [L][rows][K], flags [L][rows], cache [nseq][L][K]; 256 threads.
__global__ __launch_bounds__(256) void k_skip_commit(const PassDesc* __restrict__ pd, uint32_t M,
                                                     const float* __restrict__ stage,
                                                     const uint32_t* __restrict__ flags, uint32_t rows,
                                                     float* __restrict__ cache, uint32_t L, uint32_t K, uint32_t j0,
                                                     uint32_t j1, const DecodeState* __restrict__ st,
                                                     uint32_t n_mtp, uint32_t* __restrict__ skips) {
    const uint32_t l = blockIdx.x, s = blockIdx.y;
    const uint32_t hi = st ? min(st[s].round_acc + 1u, n_mtp) : j1;
    int32_t src = -1;
    uint32_t j = 0, nskip = 0;
    for (uint32_t r = 0; r < M; r++) {
        if (row_seq(pd, r) != s) continue;
        if (j >= j0 && j < hi) {
            if (flags[(size_t)l * rows + r]) nskip++;
            else src = (int32_t)r;
        }
        j++;
    }
    if (threadIdx.x == 0 && nskip) atomicAdd(skips, nskip);
    if (src < 0) return;
    const float* a = stage + ((size_t)l * rows + (uint32_t)src) * K;
    float* c = cache + ((size_t)s * L + l) * K;
    for (uint32_t i = threadIdx.x; i < K; i += 256) c[i] = a[i];
}

// SwiGLU of src/engine.cpp:832-838 on the fused gate|up GEMV accumulators
// (row m: [0,ff) = gate, [ff, 2ff) = up; cleared), then
// quantize_activation_row of the result.  Grid M, 1024 threads.
template <int PER>
__global__ __launch_bounds__(1024) void k_swiglu_quant(double* __restrict__ acc, const float* __restrict__ as_in,
                                                       uint32_t ff,
                                                       int8_t* __restrict__ q, uint32_t q_stride,
                                                       float* __restrict__ as, int32_t* __restrict__ bsum,
                                                       uint32_t bsum_stride, uint32_t rows, Prefetch pf) {
    __shared__ float red[16];
    const uint32_t m = blockIdx.x;
    if (m >= rows) {
        prefetch_bytes(pf.p, pf.n, m - rows, gridDim.x - rows, pf.sink);
        return;
    }
    double ga[PER], ua[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const uint32_t i = threadIdx.x + 1024u * k;
        ga[k] = i < ff ? acc[(size_t)m * 2 * ff + i] : 0.0;
        ua[k] = i < ff ? acc[(size_t)m * 2 * ff + ff + i] : 0.0;
    }
    const double a = (double)as_in[m];
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const uint32_t i = threadIdx.x + 1024u * k;
        float f = 0.0f;
        if (i < ff) {
            acc[(size_t)m * 2 * ff + i] = 0.0;
            acc[(size_t)m * 2 * ff + ff + i] = 0.0;
            const float gt = (float)(ga[k] * a);
            const float u = (float)(ua[k] * a);
            const float sig = 1.0f / (1.0f + expf_c(-gt));
            f = gt * sig * u;
        }
        v[k] = f;
    }
    quantize_row_block<PER, 1024>(v, ff, q + (size_t)m * q_stride, as + m,
                                  bsum ? bsum + (size_t)m * bsum_stride : nullptr, red);
}

// dst = src (float), used instead of a copy node inside captured passes.
__global__ void k_copy_f32(const float* __restrict__ src, float* __restrict__ dst, uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

// MTP activation: a = silu(g) * u with silu(x) = x / (1 + exp(-x))
// (src/mtp.cpp:89-91, 157-159).
__global__ void k_silu_mul(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ a, uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float s = g[i] / (1.0f + expf_c(-g[i]));
    a[i] = s * u[i];
}

// Token embedding: x[m] = dequantized row tok[m] of the tied Q4 table.
__global__ void k_embed(const uint8_t* __restrict__ codes, const uint16_t* __restrict__ scales,
                        uint32_t V, uint32_t D, const PassDesc* __restrict__ pd, float* __restrict__ x) {
    uint32_t m = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (m >= pd->m || i >= D) return;
    int32_t tok = pd->tok[m];
    float val = 0.0f;
    if (tok >= 0 && (uint32_t)tok < V) {
        uint32_t nb = D >> 5, b = i >> 5, e = i & 31u;
        uint8_t byte = codes[((size_t)tok * nb + b) * 16u + (e >> 1)];
        uint32_t nib = (e & 1u) ? (byte >> 4) : (byte & 15u);
        float d = h2f(scales[(size_t)tok * nb + b]);
        val = (float)((int)nib - 8) * d;
    }
    x[(size_t)m * D + i] = val;
}

// ============================================ reference plain-int8 matmul

// C[i][j] = sum_k A[i][k] * B[j][k] (src/matmul_neon.cpp:80-144).  One
// thread per output; K handled in 4-byte steps with an exact scalar tail.
__global__ void k_matmul_int8(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                              int32_t* __restrict__ C, uint32_t M, uint32_t N, uint32_t K) {
    uint32_t j = blockIdx.x * blockDim.x + threadIdx.x, i = blockIdx.y;
    if (j >= N || i >= M) return;
    const int8_t* a = A + (size_t)i * K;
    const int8_t* b = B + (size_t)j * K;
    int acc = 0;
    uint32_t k = 0;
    if ((((uintptr_t)a | (uintptr_t)b) & 3u) == 0) {
        for (; k + 4 <= K; k += 4)
            acc = __builtin_amdgcn_sdot4(*reinterpret_cast<const int*>(a + k),
                                         *reinterpret_cast<const int*>(b + k), acc, false);
    }
    for (; k < K; k++) acc += (int)a[k] * (int)b[k];
    C[(size_t)i * N + j] = acc;
}

// matmul_quantized's given-scale activation path (src/matmul_neon.cpp:158-164).
__global__ void k_quant_div(const float* __restrict__ A, const float* __restrict__ sc,
                            int8_t* __restrict__ q, uint32_t M, uint32_t K) {
    uint32_t k = blockIdx.x * blockDim.x + threadIdx.x, i = blockIdx.y;
    if (k >= K || i >= M) return;
    q[(size_t)i * K + k] = (int8_t)(int)__builtin_roundf(A[(size_t)i * K + k] / sc[i]);
}

// C = (float)C_int * a_scale[i] * w_scale[j] (src/matmul_neon.cpp:176-180).
__global__ void k_mm_epilogue(const int32_t* __restrict__ Ci, const float* __restrict__ as,
                              const float* __restrict__ ws, float* __restrict__ C, uint32_t M, uint32_t N) {
    uint32_t j = blockIdx.x * blockDim.x + threadIdx.x, i = blockIdx.y;
    if (j >= N || i >= M) return;
    C[(size_t)i * N + j] = (float)Ci[(size_t)i * N + j] * as[i] * ws[j];
}

}  // namespace pf
