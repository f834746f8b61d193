// fp32-activation GEMV and the row kernels of the gfx950 path.
//
//  * k_gemv_f32    fp32 activations x dequantized Q4 row-major matrix (tied
//                  unembedding, MTP heads) in the canonical 64-lane order;
//                  k_gemv_f32_glu: a head's gate and up products and their
//                  SiLU product in one launch.
//  * row kernels   quantize_activation_row of whole rows, layer-skip
//                  decisions and cache commits, embedding, small copies.
//  * k_matmul_int8 / k_mm_epilogue: the reference's plain int8 matmul API.
// The int8-activation x block-quantized products are in pf_mm.hip.
#include "pf_device.h"

namespace pf {

// ============================================ fp32 x dequantized Q4 GEMV

// The M activation rows (K <= 2048 floats each) staged once per workgroup
// in LDS, then lane l's 32 elements of every row (block l) in registers
// (zeros for lanes past the row's blocks): one copy of the rows per
// workgroup from L2 instead of one per wave.
template <int M>
__device__ __forceinline__ void stage_rows(const float* __restrict__ h, uint32_t h_stride, uint32_t K, uint32_t lane,
                                           bool live, float (&hv)[M][32]) {
    __shared__ __align__(16) float hsm[M * 2048];
    const uint32_t n4 = K >> 2;
    for (uint32_t i = threadIdx.x; i < M * n4; i += blockDim.x) {
        const uint32_t m = i / n4, c = i - m * n4;
        reinterpret_cast<float4*>(hsm)[m * 512u + c] = *reinterpret_cast<const float4*>(h + (size_t)m * h_stride + 4u * c);
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; m++) {
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            const float4 v = live ? *reinterpret_cast<const float4*>(hsm + m * 2048 + lane * 32u + i)
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
            hv[m][i] = v.x; hv[m][i + 1] = v.y; hv[m][i + 2] = v.z; hv[m][i + 3] = v.w;
        }
    }
}

// y[m][n] (+= y_in[m][n] when resid) = canonical fp32 dot of h[m] with row n:
// lane l holds block l (K <= 2048), fmaf chain over the block's elements,
// halving tree over the 64 lanes.  Each wave walks rows n = wave, wave +
// total_waves, ..., loading the codes and scales of RB rows before their
// products (the tied unembedding gives each wave 8 rows).  Grid y takes
// the activation rows M at a time: slice y serves rows M y .. M y + M - 1.
// FMT: Q4 (16 code bytes per block: weight (nibble - 8) d, formed as
// fmaf(nibble, d, -8 d), exact) or Q8 (32: weight (float)code * d, exact).
template <int M, int FMT>
__global__ __launch_bounds__(256) void k_gemv_f32(const uint8_t* __restrict__ codes,
                                                  const uint16_t* __restrict__ scales,
                                                  uint32_t N, uint32_t K,
                                                  const float* __restrict__ h, uint32_t h_stride,
                                                  float* __restrict__ y, uint32_t y_stride,
                                                  const float* __restrict__ y_in) {
    h += (size_t)blockIdx.y * M * h_stride;
    y += (size_t)blockIdx.y * M * y_stride;
    if (y_in) y_in += (size_t)blockIdx.y * M * y_stride;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
    const uint32_t nb = K >> 5;
    const bool live = lane < nb;
    float hv[M][32];
    stage_rows<M>(h, h_stride, K, lane, live, hv);
    constexpr uint32_t RB = M == 1 ? 8u : (M <= 4 ? 4u : 2u);
    for (uint32_t n0 = wave; n0 < N; n0 += RB * nwaves) {
        constexpr uint32_t CB = FMT == FMT_Q8 ? 2u : 1u;   // 16-byte code words per block
        uint4 cr[RB][CB];
        float dr[RB];
#pragma unroll
        for (uint32_t q = 0; q < RB; q++) {
            const uint32_t n = n0 + q * nwaves;
#pragma unroll
            for (uint32_t u = 0; u < CB; u++) cr[q][u] = make_uint4(0u, 0u, 0u, 0u);
            dr[q] = 0.0f;
            if (live && n < N) {
#pragma unroll
                for (uint32_t u = 0; u < CB; u++)
                    cr[q][u] = *reinterpret_cast<const uint4*>(codes + ((size_t)n * nb + lane) * (16u * CB) + 16u * u);
                dr[q] = h2f(scales[(size_t)n * nb + lane]);
            }
        }
#pragma unroll
        for (uint32_t q = 0; q < RB; q++) {
            const uint32_t n = n0 + q * nwaves;
            if (n >= N) break;
            float acc[M];
#pragma unroll
            for (int m = 0; m < M; m++) acc[m] = 0.0f;
            if (live) {
                const float d = dr[q], nd = -8.0f * d;
                if constexpr (FMT == FMT_Q8) {
                    const uint32_t cw[8] = {cr[q][0].x, cr[q][0].y, cr[q][0].z, cr[q][0].w,
                                            cr[q][1].x, cr[q][1].y, cr[q][1].z, cr[q][1].w};
#pragma unroll
                    for (int j = 0; j < 32; j++) {
                        const float wj = (float)(int8_t)((cw[j >> 2] >> (8 * (j & 3))) & 0xFFu) * d;
#pragma unroll
                        for (int m = 0; m < M; m++) acc[m] = __builtin_fmaf(hv[m][j], wj, acc[m]);
                    }
                } else {
                    const uint32_t cw[4] = {cr[q][0].x, cr[q][0].y, cr[q][0].z, cr[q][0].w};
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
}

// One MTP head's gate and up products with the SiLU product fused
// (src/mtp.cpp:63-127): a[m][n] = silu(g) * u, g and u the canonical dots
// of h[m] with row n of Wg and Wu (k_gemv_f32's order), silu(g) =
// g / (1 + exp(-g)) (src/mtp.cpp:89-91, 157-159): the bits of two
// k_gemv_f32 products followed by that elementwise step.
template <int M>
__global__ __launch_bounds__(256) void k_gemv_f32_glu(const uint8_t* __restrict__ gcodes,
                                                      const uint16_t* __restrict__ gscales,
                                                      const uint8_t* __restrict__ ucodes,
                                                      const uint16_t* __restrict__ uscales, uint32_t N, uint32_t K,
                                                      const float* __restrict__ h, uint32_t h_stride,
                                                      float* __restrict__ a, uint32_t a_stride) {
    h += (size_t)blockIdx.y * M * h_stride;   // grid y: activation rows M at a time
    a += (size_t)blockIdx.y * M * a_stride;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
    const uint32_t nb = K >> 5;
    const bool live = lane < nb;
    float hv[M][32];
    stage_rows<M>(h, h_stride, K, lane, live, hv);
    for (uint32_t n = wave; n < N; n += nwaves) {
        float ag[M], au[M];
#pragma unroll
        for (int m = 0; m < M; m++) ag[m] = au[m] = 0.0f;
        if (live) {
            const uint4 cg = *reinterpret_cast<const uint4*>(gcodes + ((size_t)n * nb + lane) * 16u);
            const uint4 cu = *reinterpret_cast<const uint4*>(ucodes + ((size_t)n * nb + lane) * 16u);
            const float dg = h2f(gscales[(size_t)n * nb + lane]), du = h2f(uscales[(size_t)n * nb + lane]);
            const float ndg = -8.0f * dg, ndu = -8.0f * du;
            const uint32_t gw[4] = {cg.x, cg.y, cg.z, cg.w}, uw[4] = {cu.x, cu.y, cu.z, cu.w};
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const uint32_t bg = (gw[j >> 2] >> (8 * (j & 3))) & 0xFFu, bu = (uw[j >> 2] >> (8 * (j & 3))) & 0xFFu;
                const float g0 = __builtin_fmaf((float)(bg & 15u), dg, ndg), g1 = __builtin_fmaf((float)(bg >> 4), dg, ndg);
                const float u0 = __builtin_fmaf((float)(bu & 15u), du, ndu), u1 = __builtin_fmaf((float)(bu >> 4), du, ndu);
#pragma unroll
                for (int m = 0; m < M; m++) {
                    ag[m] = __builtin_fmaf(hv[m][2 * j], g0, ag[m]);
                    ag[m] = __builtin_fmaf(hv[m][2 * j + 1], g1, ag[m]);
                    au[m] = __builtin_fmaf(hv[m][2 * j], u0, au[m]);
                    au[m] = __builtin_fmaf(hv[m][2 * j + 1], u1, au[m]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            const float g = wave_tree_sum(ag[m]), u = wave_tree_sum(au[m]);
            if (lane == 0) {
                const float sg = g / (1.0f + expf_c(-g));
                a[(size_t)m * a_stride + n] = sg * u;
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

// dst = src (float), used instead of a copy node inside captured passes.
__global__ void k_copy_f32(const float* __restrict__ src, float* __restrict__ dst, uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

// Token embedding: x[m] = dequantized row tok[m] of the tied table (Q4 or
// Q8, fmt).
// The first kernel of every pass also advances the pass epoch `ep`, which
// names the pass in the flags of the LL words its QKV products write.
__device__ __forceinline__ void embed_elem(const uint8_t* __restrict__ codes, const uint16_t* __restrict__ scales,
                                           uint32_t V, uint32_t D, const PassDesc* __restrict__ pd,
                                           float* __restrict__ x, uint32_t* __restrict__ ep, int32_t fmt, uint32_t m,
                                           uint32_t i) {
    if (ep && m == 0 && i == 0) ep[0] += 1u;
    if (m >= pd->m || i >= D) return;
    int32_t tok = pd->tok[m];
    float val = 0.0f;
    if (tok >= 0 && (uint32_t)tok < V) {
        uint32_t nb = D >> 5, b = i >> 5, e = i & 31u;
        float d = h2f(scales[(size_t)tok * nb + b]);
        if (fmt == FMT_Q8) {
            val = (float)(int8_t)codes[((size_t)tok * nb + b) * 32u + e] * d;
        } else {
            uint8_t byte = codes[((size_t)tok * nb + b) * 16u + (e >> 1)];
            uint32_t nib = (e & 1u) ? (byte >> 4) : (byte & 15u);
            val = (float)((int)nib - 8) * d;
        }
    }
    x[(size_t)m * D + i] = val;
}
__global__ void k_embed(const uint8_t* __restrict__ codes, const uint16_t* __restrict__ scales,
                        uint32_t V, uint32_t D, const PassDesc* __restrict__ pd, float* __restrict__ x,
                        uint32_t* __restrict__ ep, int32_t fmt) {
    embed_elem(codes, scales, V, D, pd, x, ep, fmt, blockIdx.y, blockIdx.x * blockDim.x + threadIdx.x);
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
