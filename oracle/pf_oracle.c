/*
 * pf_oracle.c -- CPU restatement of the reference's MTP speculative-decoding
 * hot path.  TEST INFRASTRUCTURE ONLY: it is the checker the HIP path is
 * compared against (tests/, __graft_entry__.smoke(), bench.py cpu_baseline).
 * The product never links or loads it.
 *
 * Build: oracle/Makefile (gcc -ffp-contract=off -fopenmp).  Fused
 * multiply-adds appear only where written as fmaf().  The reference's x86
 * build (-O3 -march=native) vectorizes the products of its float-array
 * dot-product reductions and keeps the additions sequential (no FMA), keeps
 * the int8 dot of KVCache::dot_quant scalar and contracted (FMA), and
 * vectorizes and contracts the element-wise updates `out[i] += s * v[i]`.
 * The reference-order functions here follow that; the canonical ones use
 * fmaf where stated.
 *
 * Canonical orders (the reference sums sequentially; a GPU cannot):
 *   CANON(W): lane l of T = 64*W lanes accumulates x[l], x[l+T], ...
 *             sequentially from +0.0f; each 64-lane wave then reduces with a
 *             halving tree (offsets 32,16,8,4,2,1); the W wave totals are
 *             reduced with a halving tree (offsets W/2 .. 1).
 *   int8 x block GEMV: y = (float)(S * (double)a_scale) where
 *             S = sum_b (double)d_b * (double)p_b is computed EXACTLY in
 *             double (every term is an integer multiple of the smallest
 *             block-scale ulp and the row's scale spread is bounded by the
 *             quantizer), so the result does not depend on summation order.
 *   fp32 x block GEMV (tied unembed, MTP heads): lane l = b mod 64 of the
 *             64 lanes accumulates blocks b ascending, elements ascending,
 *             with fmaf(h, w, acc); then the halving tree over 64 lanes.
 *   attention (engine): chunks of 256 list entries with a chunk max, exp,
 *             CANON(4) chunk sum and sub-chunk fmaf chains, merged left to
 *             right with exp(m_c - max) factors (attn_head).
 *   KVCache::attention_weighted_sum: chunks of 64 visible entries; fmaf
 *             chain inside a chunk from 0.0f; chunk partials added left to
 *             right.
 *   sampling sums / prefix sums: 64 contiguous chunks, sequential inside
 *             a chunk, chunk totals added left to right.
 */
#include "pf_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <stdio.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ================================================================ basics */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Philox4x32-10 counter-based generator: Salmon, Moraes, Dror, Shaw,
 * "Parallel random numbers: as easy as 1, 2, 3", SC'11.  Multipliers and
 * Weyl key increments are the published constants. */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; r++) {
        if (r > 0) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        c0 = hi1 ^ c1 ^ k0;
        c1 = lo1;
        c2 = hi0 ^ c3 ^ k1;
        c3 = lo0;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* Sampling uniform for stochastic draw number `idx` (the reference draws one
 * uniform_real_distribution<float>(0,1) value per stochastic sample() call,
 * src/engine.cpp:909,952,996).  Returns a float in [0,1). */
float orc_uniform(uint64_t seed, uint64_t idx) {
    uint32_t ctr[4] = {(uint32_t)idx, (uint32_t)(idx >> 32), 0x53414D50u, 0u};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t out[4];
    orc_philox4x32_10(ctr, key, out);
    return (float)(out[0] >> 8) * 0x1p-24f;
}

/* exp(x) for float: Cody-Waite reduction x = k*ln2 + r (ln2 split in a
 * 16-bit head and a tail), degree-7 Taylor polynomial of exp(r) in Horner
 * form, scale by 2^k.  Results below 2^-124 are flushed to zero (x < -86)
 * and x > 88 returns +inf, so no subnormal result is ever formed.  The HIP
 * kernels use the same operation sequence. */
float orc_expf(float x) {
    if (x != x) return x;
    if (x < -86.0f) return 0.0f;
    if (x > 88.0f) return INFINITY;
    float kf = rintf(x * 1.44269502162933349609375f);
    float r = fmaf(kf, -0.693145751953125f, x);
    r = fmaf(kf, -1.42860676533018704503775e-06f, r);
    float p = 1.98412698412698412698e-4f;
    p = fmaf(p, r, 1.38888888888888888889e-3f);
    p = fmaf(p, r, 8.33333333333333333333e-3f);
    p = fmaf(p, r, 4.16666666666666666667e-2f);
    p = fmaf(p, r, 1.66666666666666666667e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int k = (int)kf;
    return p * u2f((uint32_t)(k + 127) << 23);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        float v = (float)m * 0x1p-24f;            /* exact */
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* float -> IEEE binary16, round to nearest even. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u);
    if (ax >= 0x477FF000u) return sign | 0x7C00u;          /* >= 65520 -> inf */
    if (ax <= 0x33000000u) return sign;                     /* <= 2^-25 -> 0 */
    uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
    if (e < 113) {                                          /* f16 subnormal */
        uint32_t shift = 126 - e;                           /* 14..24 */
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return sign | (uint16_t)q;
    }
    uint32_t q = ((e - 112u) << 10) | ((m & 0x7FFFFFu) >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return sign | (uint16_t)q;
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Threads of the OpenMP row-parallel loops from now on (1: the reference's
 * single-threaded compute).  Results do not depend on it. */
void orc_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ================================= src/matmul_neon.cpp, reference order */

/* src/matmul_neon.cpp:16-29 */
void orc_quantize_activation_row(const float* src, int8_t* dst, float* scale_out, uint32_t n) {
    float amax = 0.0f;
    for (uint32_t i = 0; i < n; i++) {
        float a = fabsf(src[i]);
        if (a > amax) amax = a;
    }
    float scale = (amax == 0.0f) ? 1.0f : 127.0f / amax;
    for (uint32_t i = 0; i < n; i++) dst[i] = (int8_t)roundf(src[i] * scale);
    *scale_out = (amax == 0.0f) ? 1.0f : amax / 127.0f;
}

/* src/matmul_neon.cpp:34-45: low nibble = element 2j, high = 2j+1, minus 8. */
void orc_dequant_q4_to_int8(const uint8_t* q4, int8_t* out, float scale, uint32_t n) {
    (void)scale;
    for (uint32_t i = 0; i < n; i += 2) {
        uint8_t b = q4[i / 2];
        out[i] = (int8_t)((int)(b & 0x0F) - 8);
        if (i + 1 < n) out[i + 1] = (int8_t)((int)((b >> 4) & 0x0F) - 8);
    }
}

/* src/matmul_neon.cpp:50-61: element 4j+t at bits 2t..2t+1, minus 2. */
void orc_dequant_q2_to_int8(const uint8_t* q2, int8_t* out, float scale, uint32_t n) {
    (void)scale;
    for (uint32_t i = 0; i < n; i += 4) {
        uint8_t b = q2[i / 4];
        for (uint32_t t = 0; t < 4 && i + t < n; t++)
            out[i + t] = (int8_t)((int)((b >> (2 * t)) & 3) - 2);
    }
}

/* src/matmul_neon.cpp:66-75: two codes per byte (bits 0-1, 2-3), LUT {-1,0,1,0}. */
void orc_dequant_ternary_to_int8(const uint8_t* t, int8_t* out, uint32_t n) {
    static const int8_t lut[4] = {-1, 0, 1, 0};
    for (uint32_t i = 0; i < n; i += 2) {
        uint8_t b = t[i / 2];
        out[i] = lut[b & 3];
        if (i + 1 < n) out[i + 1] = lut[(b >> 2) & 3];
    }
}

/* src/matmul_neon.cpp:80-144 (scalar branch :132-142). */
void orc_matmul_int8(const int8_t* A, const int8_t* B, int32_t* C,
                     uint32_t M, uint32_t N, uint32_t K) {
    for (uint32_t i = 0; i < M; i++)
        for (uint32_t j = 0; j < N; j++) {
            int32_t s = 0;
            for (uint32_t k = 0; k < K; k++) s += (int32_t)A[(size_t)i * K + k] * (int32_t)B[(size_t)j * K + k];
            C[(size_t)i * N + j] = s;
        }
}

/* src/matmul_neon.cpp:149-181. */
void orc_matmul_quantized(const float* A, const int8_t* B, float* C,
                          uint32_t M, uint32_t N, uint32_t K,
                          const float* w_scales, const float* act_scales) {
    int8_t* Aq = (int8_t*)malloc((size_t)M * K);
    float* as = (float*)malloc(sizeof(float) * (M ? M : 1));
    int32_t* Ci = (int32_t*)malloc(sizeof(int32_t) * (size_t)M * N + 4);
    for (uint32_t i = 0; i < M; i++) {
        if (act_scales) {
            as[i] = act_scales[i];
            for (uint32_t k = 0; k < K; k++)
                Aq[(size_t)i * K + k] = (int8_t)roundf(A[(size_t)i * K + k] / act_scales[i]);
        } else {
            orc_quantize_activation_row(A + (size_t)i * K, Aq + (size_t)i * K, &as[i], K);
        }
    }
    orc_matmul_int8(Aq, B, Ci, M, N, K);
    for (uint32_t i = 0; i < M; i++)
        for (uint32_t j = 0; j < N; j++)
            C[(size_t)i * N + j] = (float)Ci[(size_t)i * N + j] * as[i] * w_scales[j];
    free(Aq); free(as); free(Ci);
}

/* src/matmul_neon.cpp:186-207 (scalar branch).  The reference's x86 build
 * vectorizes the products and keeps the additions sequential, so the sum is
 * not contracted into FMAs. */
float orc_dot_product(const float* a, const float* b, uint32_t n) {
    float s = 0.0f;
    for (uint32_t i = 0; i < n; i++) s = s + a[i] * b[i];
    return s;
}

/* src/matmul_neon.cpp:212-226 with libm exp and the sequential sum. */
void orc_softmax_ref(float* v, uint32_t n) {
    float mx = v[0];
    for (uint32_t i = 1; i < n; i++) if (v[i] > mx) mx = v[i];
    float s = 0.0f;
    for (uint32_t i = 0; i < n; i++) { v[i] = expf(v[i] - mx); s += v[i]; }
    float inv = 1.0f / (s + 1e-10f);
    for (uint32_t i = 0; i < n; i++) v[i] *= inv;
}

/* src/matmul_neon.cpp:231-239 with the sequential sum of squares. */
void orc_rmsnorm_ref(float* out, const float* x, const float* w, uint32_t n) {
    float ss = 0.0f;
    for (uint32_t i = 0; i < n; i++) ss = ss + x[i] * x[i];
    float rms = sqrtf(ss / (float)n + 1e-6f);
    float inv = 1.0f / rms;
    for (uint32_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

/* ========================================== canonical reductions (CANON) */

static float canon_tree(float* P, uint32_t waves) {
    for (uint32_t w = 0; w < waves; w++) {
        float* L = P + 64 * w;
        for (uint32_t off = 32; off >= 1; off >>= 1)
            for (uint32_t l = 0; l < off; l++) L[l] = L[l] + L[l + off];
    }
    for (uint32_t off = waves / 2; off >= 1; off >>= 1)
        for (uint32_t w = 0; w < off; w++) P[64 * w] = P[64 * w] + P[64 * (w + off)];
    return P[0];
}

float orc_canon_sum(const float* x, uint32_t n, uint32_t waves) {
    uint32_t T = 64 * waves;
    float P[64 * 16];
    for (uint32_t l = 0; l < T; l++) {
        float a = 0.0f;
        for (uint32_t j = l; j < n; j += T) a = a + x[j];
        P[l] = a;
    }
    return canon_tree(P, waves);
}

float orc_canon_sumsq(const float* x, uint32_t n, uint32_t waves) {
    uint32_t T = 64 * waves;
    float P[64 * 16];
    for (uint32_t l = 0; l < T; l++) {
        float a = 0.0f;
        for (uint32_t j = l; j < n; j += T) a = fmaf(x[j], x[j], a);
        P[l] = a;
    }
    return canon_tree(P, waves);
}

/* src/matmul_neon.cpp:212-226: same formula, own exp, CANON(4) sum. */
void orc_softmax(float* v, uint32_t n) {
    float mx = v[0];
    for (uint32_t i = 1; i < n; i++) if (v[i] > mx) mx = v[i];
    for (uint32_t i = 0; i < n; i++) v[i] = orc_expf(v[i] - mx);
    float s = orc_canon_sum(v, n, 4);
    float inv = 1.0f / (s + 1e-10f);
    for (uint32_t i = 0; i < n; i++) v[i] = v[i] * inv;
}

/* src/matmul_neon.cpp:231-239: same formula, CANON(4) sum of squares. */
void orc_rmsnorm(float* out, const float* x, const float* w, uint32_t n) {
    float ss = orc_canon_sumsq(x, n, 4);
    float rms = sqrtf(ss / (float)n + 1e-6f);
    float inv = 1.0f / rms;
    for (uint32_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

/* The engine's RMSNorm (src/engine.cpp:515-523, 526-541 calling
 * src/matmul_neon.cpp:231-239): the same formula in the tile-canonical
 * order of the GPU pass.  The sum of squares is the sequential sum, tile
 * by tile, of each 64-element tile's halving tree of x * x (offsets 32, 16,
 * ..., 1); the normed value is (x * w) * inv.  n % 64 == 0.  Because
 * rounding is monotone, max |out| = fl(max |fl(x * w)| * inv), so the
 * row maximum needed by quantize_activation_row also decomposes by tile. */
void orc_engine_rmsnorm(float* out, const float* x, const float* w, uint32_t n) {
    float ss = 0.0f;
    for (uint32_t t = 0; t < n / 64; t++) {
        float L[64];
        for (uint32_t l = 0; l < 64; l++) L[l] = x[64 * t + l] * x[64 * t + l];
        for (uint32_t off = 32; off >= 1; off >>= 1)
            for (uint32_t l = 0; l < off; l++) L[l] = L[l] + L[l + off];
        ss = ss + L[0];
    }
    float rms = sqrtf(ss / (float)n + 1e-6f);
    float inv = 1.0f / rms;
    for (uint32_t i = 0; i < n; i++) out[i] = (x[i] * w[i]) * inv;
}

/* ============================================== block-quantized matrices */

uint32_t orc_block_bytes(int32_t fmt) { return fmt == ORC_Q8 ? 32u : (fmt == ORC_Q4 ? 16u : 8u); }

/* Code of element (row, col) as the signed integer multiplier of d. */
int orc_block_code(const orc_qmat* W, uint32_t row, uint32_t col) {
    uint32_t nb = W->cols / 32, b = col / 32, i = col % 32;
    const uint8_t* blk = W->codes + ((size_t)row * nb + b) * orc_block_bytes(W->fmt);
    if (W->fmt == ORC_Q8) return (int)(int8_t)blk[i];   /* Q8_0, include/forge/types.hpp:17-20 */
    if (W->fmt == ORC_Q4) {
        uint8_t byte = blk[i / 2];
        return (int)((i & 1) ? (byte >> 4) : (byte & 15)) - 8;
    }
    int c = (blk[i / 4] >> (2 * (i % 4))) & 3;
    if (W->fmt == ORC_Q2) return c - 2;
    static const int lut[4] = {-1, 0, 1, 0};
    return lut[c];
}

/* Code rules of src/quant_format.cpp:77-154 with the repairs of this build:
 * the block scale is the multiplicative d in fp16 (the reference stores the
 * inverse in fp32 and its loader drops it), and Q1.5 uses the relative
 * threshold 0.35*amax with d = mean |x| over the nonzero codes.  Blocks
 * whose fp16 exponent is more than 15 below the row maximum are zeroed so
 * that the exact-sum GEMV stays exact (see the header comment). */
void orc_quantize_matrix(const float* w, uint32_t rows, uint32_t cols, int32_t fmt,
                         uint8_t* codes, uint16_t* scales) {
    uint32_t nb = cols / 32, bb = orc_block_bytes(fmt);
    for (uint32_t r = 0; r < rows; r++) {
        int emax = 0;
        for (uint32_t b = 0; b < nb; b++) {
            const float* x = w + (size_t)r * cols + 32 * b;
            uint8_t* q = codes + ((size_t)r * nb + b) * bb;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) { float a = fabsf(x[i]); if (a > amax) amax = a; }
            memset(q, 0, bb);
            uint16_t d16 = 0;
            if (fmt == ORC_Q8) {
                /* symmetric, as the activation rows: code = round(x * 127 / amax)
                 * (the reference's round(x s + 0.5) of src/quant_format.cpp:68
                 * is kept only for codes read from its files) */
                float inv = (amax == 0.0f) ? 0.0f : 127.0f / amax;
                for (int i = 0; i < 32; i++) {
                    int v = (int)roundf(x[i] * inv);
                    q[i] = (uint8_t)(int8_t)(v < -127 ? -127 : (v > 127 ? 127 : v));
                }
                d16 = orc_f32_to_f16(amax / 127.0f);
            } else if (fmt == ORC_Q4) {
                float inv = (amax == 0.0f) ? 0.0f : 7.0f / amax;
                for (int i = 0; i < 32; i += 2) {
                    int v0 = (int)(int8_t)roundf(x[i] * inv);
                    int v1 = (int)(int8_t)roundf(x[i + 1] * inv);
                    v0 = v0 < -8 ? -8 : (v0 > 7 ? 7 : v0);
                    v1 = v1 < -8 ? -8 : (v1 > 7 ? 7 : v1);
                    q[i / 2] = (uint8_t)((v0 + 8) | ((v1 + 8) << 4));
                }
                d16 = orc_f32_to_f16(amax / 7.0f);
            } else if (fmt == ORC_Q2) {
                float inv = (amax == 0.0f) ? 0.0f : 1.0f / amax;
                for (int i = 0; i < 32; i++) {
                    int v = (int)(int8_t)roundf(x[i] * inv);
                    v = v < -2 ? -2 : (v > 1 ? 1 : v);
                    q[i / 4] |= (uint8_t)((v + 2) << (2 * (i % 4)));
                }
                d16 = orc_f32_to_f16(amax);
            } else {
                float t = 0.35f * amax, sum = 0.0f;
                uint32_t cnt = 0;
                for (int i = 0; i < 32; i++) {
                    int c = (x[i] > t) ? 2 : ((x[i] < -t) ? 0 : 1);
                    if (c != 1) { sum += fabsf(x[i]); cnt++; }
                    q[i / 4] |= (uint8_t)(c << (2 * (i % 4)));
                }
                d16 = cnt ? orc_f32_to_f16(sum / (float)cnt) : 0;
            }
            scales[(size_t)r * nb + b] = d16;
            int e = (d16 >> 10) & 31;
            if ((d16 & 0x7FFF) && e > emax) emax = e;
        }
        for (uint32_t b = 0; b < nb; b++) {
            uint16_t d16 = scales[(size_t)r * nb + b];
            int e = (d16 >> 10) & 31; if (e == 0) e = 1;
            if ((d16 & 0x7FFF) && e < emax - 15) {
                uint8_t* q = codes + ((size_t)r * nb + b) * bb;
                uint8_t zero = fmt == ORC_Q8 ? 0x00 : (fmt == ORC_Q4 ? 0x88 : (fmt == ORC_Q2 ? 0xAA : 0x55));
                memset(q, zero, bb);
                scales[(size_t)r * nb + b] = 0;
            }
        }
    }
}

/* The 32 signed codes of block b of a row. */
static void decode_block(const orc_qmat* W, uint32_t row, uint32_t b, int8_t* w) {
    uint32_t nb = W->cols / 32;
    const uint8_t* blk = W->codes + ((size_t)row * nb + b) * orc_block_bytes(W->fmt);
    if (W->fmt == ORC_Q8) {
        for (int j = 0; j < 32; j++) w[j] = (int8_t)blk[j];
    } else if (W->fmt == ORC_Q4) {
        for (int j = 0; j < 16; j++) {
            w[2 * j] = (int8_t)((blk[j] & 15) - 8);
            w[2 * j + 1] = (int8_t)((blk[j] >> 4) - 8);
        }
    } else {
        static const int8_t lut15[4] = {-1, 0, 1, 0};
        for (int j = 0; j < 8; j++)
            for (int t = 0; t < 4; t++) {
                int c = (blk[j] >> (2 * t)) & 3;
                w[4 * j + t] = W->fmt == ORC_Q2 ? (int8_t)(c - 2) : lut15[c];
            }
    }
}

/* Dequantized row: (float)code * d, exact in fp32 (8-bit x 11-bit). */
void orc_dequant_row(const orc_qmat* W, uint32_t row, float* out) {
    uint32_t nb = W->cols / 32;
    int8_t w[32];
    for (uint32_t b = 0; b < nb; b++) {
        float d = orc_f16_to_f32(W->scales[(size_t)row * nb + b]);
        decode_block(W, row, b, w);
        for (uint32_t i = 0; i < 32; i++) out[32 * b + i] = (float)w[i] * d;
    }
}

/* int8-activation x block matrix (the matmul_quantized of
 * src/matmul_neon.cpp:149-181 with per-32-block fp16 scales). */
void orc_gemv_i8(const orc_qmat* W, const int8_t* a, float a_scale, float* y) {
    uint32_t nb = W->cols / 32;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < (int64_t)W->rows; n++) {
        double S = 0.0;
        int8_t w[32];
        for (uint32_t b = 0; b < nb; b++) {
            decode_block(W, (uint32_t)n, b, w);
            int32_t p = 0;
            for (uint32_t i = 0; i < 32; i++) p += (int32_t)a[32 * b + i] * (int32_t)w[i];
            S += (double)orc_f16_to_f32(W->scales[(size_t)n * nb + b]) * (double)p;
        }
        y[n] = (float)(S * (double)a_scale);
    }
}

/* fp32-activation x dequantized block matrix: the fp32 dot of the tied
 * unembed (src/engine.cpp:575-582) and of the MTP heads
 * (src/mtp.cpp:67-119), in the canonical 64-lane order. */
void orc_gemv_f32(const orc_qmat* W, const float* h, float* y) {
    uint32_t nb = W->cols / 32;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < (int64_t)W->rows; n++) {
        float P[64];
        int8_t w[32];
        for (int l = 0; l < 64; l++) P[l] = 0.0f;
        for (uint32_t b = 0; b < nb; b++) {
            float d = orc_f16_to_f32(W->scales[(size_t)n * nb + b]);
            decode_block(W, (uint32_t)n, b, w);
            float acc = P[b % 64];
            for (uint32_t i = 0; i < 32; i++) acc = fmaf(h[32 * b + i], (float)w[i] * d, acc);
            P[b % 64] = acc;
        }
        y[n] = canon_tree(P, 1);
    }
}

/* y[n] = canonical fp32 dot of h with row n of a dense fp32 matrix
 * E [rows][cols]: the order of orc_gemv_f32 with the weight itself. */
void orc_gemv_f32_dense(const float* E, uint32_t rows, uint32_t cols, const float* h, float* y) {
    uint32_t nb = cols / 32;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < (int64_t)rows; n++) {
        float P[64];
        for (int l = 0; l < 64; l++) P[l] = 0.0f;
        for (uint32_t b = 0; b < nb; b++) {
            const float* w = E + (size_t)n * cols + 32 * b;
            float acc = P[b % 64];
            for (uint32_t i = 0; i < 32; i++) acc = fmaf(h[32 * b + i], w[i], acc);
            P[b % 64] = acc;
        }
        y[n] = canon_tree(P, 1);
    }
}

/* dot_product (src/matmul_neon.cpp:186-207) in the CANON(4) order: lane l
 * of 256 sums a[j] * b[j] (product, then add) for j = l, l + 256, ... */
float orc_dot_canon(const float* a, const float* b, uint32_t n) {
    float P[256];
    for (uint32_t l = 0; l < 256; l++) {
        float p = 0.0f;
        for (uint32_t j = l; j < n; j += 256) p = p + a[j] * b[j];
        P[l] = p;
    }
    return canon_tree(P, 4);
}

/* ================================================ src/kv_cache.cpp */

typedef struct {
    int8_t *sink_k, *sink_v; float *sink_ks, *sink_vs; uint32_t sink_count;
    int8_t *win_k, *win_v; float *win_ks, *win_vs; uint32_t* win_pos;
    uint32_t win_head, win_count;
    int8_t *pool_k, *pool_v; float *pool_ks, *pool_vs; uint32_t pool_count, pool_cap;
    double *acc_k, *acc_v; uint32_t acc_count, acc_start;
} orc_head;

struct orc_kv {
    uint32_t n_layers, n_heads, hd, sink_size, window, pool_block, max_context;
    uint32_t total_stored;
    orc_head* h;
};

/* src/kv_cache.cpp:19-28 */
static void kv_quantize_row(const float* src, int8_t* dst, float* scale_out, uint32_t n) {
    float amax = 0.0f;
    for (uint32_t i = 0; i < n; i++) { float a = fabsf(src[i]); if (a > amax) amax = a; }
    *scale_out = (amax == 0.0f) ? 1.0f : amax / 127.0f;
    float inv = (amax == 0.0f) ? 1.0f : 127.0f / amax;
    for (uint32_t i = 0; i < n; i++) dst[i] = (int8_t)roundf(src[i] * inv);
}

/* src/kv_cache.cpp:13-17.  The reference's x86 build keeps this loop
 * scalar and contracts it: sum = fma(q[i], (float)kv[i] * s, sum). */
static float kv_dot_quant(const float* q, const int8_t* kv, float s, uint32_t n) {
    float sum = 0.0f;
    for (uint32_t i = 0; i < n; i++) sum = fmaf(q[i], (float)kv[i] * s, sum);
    return sum;
}

/* src/kv_cache.cpp:32-57: window = min(window_size, max_context), pool
 * block >= 1, sink storage fixed at 8 rows. */
orc_kv* orc_kv_create(uint32_t n_layers, uint32_t n_kv_heads, uint32_t head_dim,
                      uint32_t sink_size, uint32_t window_size, uint32_t pool_block,
                      uint32_t max_context) {
    orc_kv* kv = (orc_kv*)calloc(1, sizeof(orc_kv));
    kv->n_layers = n_layers; kv->n_heads = n_kv_heads; kv->hd = head_dim;
    kv->sink_size = sink_size; kv->max_context = max_context;
    kv->window = window_size < max_context ? window_size : max_context;
    kv->pool_block = pool_block ? pool_block : 1;
    kv->h = (orc_head*)calloc((size_t)n_layers * n_kv_heads, sizeof(orc_head));
    uint32_t hd = head_dim, ws = kv->window;
    for (size_t i = 0; i < (size_t)n_layers * n_kv_heads; i++) {
        orc_head* c = &kv->h[i];
        c->sink_k = (int8_t*)calloc(8 * hd, 1); c->sink_v = (int8_t*)calloc(8 * hd, 1);
        c->sink_ks = (float*)malloc(8 * sizeof(float)); c->sink_vs = (float*)malloc(8 * sizeof(float));
        for (int j = 0; j < 8; j++) { c->sink_ks[j] = 1.0f; c->sink_vs[j] = 1.0f; }
        c->win_k = (int8_t*)calloc((size_t)ws * hd + 1, 1); c->win_v = (int8_t*)calloc((size_t)ws * hd + 1, 1);
        c->win_ks = (float*)malloc(((size_t)ws + 1) * sizeof(float));
        c->win_vs = (float*)malloc(((size_t)ws + 1) * sizeof(float));
        for (uint32_t j = 0; j < ws; j++) { c->win_ks[j] = 1.0f; c->win_vs[j] = 1.0f; }
        c->win_pos = (uint32_t*)calloc((size_t)ws + 1, sizeof(uint32_t));
        c->acc_k = (double*)calloc(hd, sizeof(double)); c->acc_v = (double*)calloc(hd, sizeof(double));
    }
    return kv;
}

void orc_kv_destroy(orc_kv* kv) {
    if (!kv) return;
    for (size_t i = 0; i < (size_t)kv->n_layers * kv->n_heads; i++) {
        orc_head* c = &kv->h[i];
        free(c->sink_k); free(c->sink_v); free(c->sink_ks); free(c->sink_vs);
        free(c->win_k); free(c->win_v); free(c->win_ks); free(c->win_vs); free(c->win_pos);
        free(c->pool_k); free(c->pool_v); free(c->pool_ks); free(c->pool_vs);
        free(c->acc_k); free(c->acc_v);
    }
    free(kv->h); free(kv);
}

static void pool_reserve(orc_head* c, uint32_t hd, uint32_t need) {
    if (need <= c->pool_cap) return;
    uint32_t cap = c->pool_cap ? c->pool_cap * 2 : 16;
    while (cap < need) cap *= 2;
    c->pool_k = (int8_t*)realloc(c->pool_k, (size_t)cap * hd);
    c->pool_v = (int8_t*)realloc(c->pool_v, (size_t)cap * hd);
    c->pool_ks = (float*)realloc(c->pool_ks, (size_t)cap * sizeof(float));
    c->pool_vs = (float*)realloc(c->pool_vs, (size_t)cap * sizeof(float));
    c->pool_cap = cap;
}

/* src/kv_cache.cpp:59-127 */
void orc_kv_store(orc_kv* kv, uint32_t layer, uint32_t head, uint32_t pos,
                  const float* key, const float* value) {
    if (layer >= kv->n_layers || head >= kv->n_heads) return;
    if (pos >= kv->max_context) return;
    orc_head* c = &kv->h[(size_t)layer * kv->n_heads + head];
    uint32_t hd = kv->hd;
    if (pos < kv->sink_size) {
        if (pos < 8) {
            kv_quantize_row(key, c->sink_k + (size_t)pos * hd, &c->sink_ks[pos], hd);
            kv_quantize_row(value, c->sink_v + (size_t)pos * hd, &c->sink_vs[pos], hd);
            if (pos >= c->sink_count) c->sink_count = pos + 1;
        }
    } else {
        uint32_t ws = kv->window;
        uint32_t slot = c->win_head;
        if (c->win_count >= ws) {
            uint32_t evict_pos = c->win_pos[slot];
            if (c->acc_count == 0) c->acc_start = evict_pos;
            for (uint32_t i = 0; i < hd; i++) {
                c->acc_k[i] += (double)c->win_k[(size_t)slot * hd + i] * (double)c->win_ks[slot];
                c->acc_v[i] += (double)c->win_v[(size_t)slot * hd + i] * (double)c->win_vs[slot];
            }
            c->acc_count++;
            if (c->acc_count >= kv->pool_block) {
                float inv = 1.0f / (float)c->acc_count;
                uint32_t p = c->pool_count++;
                pool_reserve(c, hd, c->pool_count);
                float* avg = (float*)malloc(sizeof(float) * hd);
                for (uint32_t i = 0; i < hd; i++) avg[i] = (float)(c->acc_k[i] * (double)inv);
                kv_quantize_row(avg, c->pool_k + (size_t)p * hd, &c->pool_ks[p], hd);
                for (uint32_t i = 0; i < hd; i++) avg[i] = (float)(c->acc_v[i] * (double)inv);
                kv_quantize_row(avg, c->pool_v + (size_t)p * hd, &c->pool_vs[p], hd);
                free(avg);
                memset(c->acc_k, 0, sizeof(double) * hd);
                memset(c->acc_v, 0, sizeof(double) * hd);
                c->acc_count = 0;
            }
            kv_quantize_row(key, c->win_k + (size_t)slot * hd, &c->win_ks[slot], hd);
            kv_quantize_row(value, c->win_v + (size_t)slot * hd, &c->win_vs[slot], hd);
            c->win_pos[slot] = pos;
            c->win_head = (c->win_head + 1) % ws;
        } else {
            kv_quantize_row(key, c->win_k + (size_t)slot * hd, &c->win_ks[slot], hd);
            kv_quantize_row(value, c->win_v + (size_t)slot * hd, &c->win_vs[slot], hd);
            c->win_pos[slot] = pos;
            c->win_head = (c->win_head + 1) % ws;
            c->win_count++;
        }
    }
    if (pos >= kv->total_stored) kv->total_stored = pos + 1;
}

/* Visible entry `idx` of (layer, head) in attention order: sink, pool,
 * window oldest -> newest (src/kv_cache.cpp:137-155). */
static void kv_entry(const orc_kv* kv, const orc_head* c, uint32_t idx,
                     const int8_t** k, float* ks, const int8_t** v, float* vs) {
    uint32_t hd = kv->hd;
    if (idx < c->sink_count) {
        *k = c->sink_k + (size_t)idx * hd; *ks = c->sink_ks[idx];
        *v = c->sink_v + (size_t)idx * hd; *vs = c->sink_vs[idx];
        return;
    }
    idx -= c->sink_count;
    if (idx < c->pool_count) {
        *k = c->pool_k + (size_t)idx * hd; *ks = c->pool_ks[idx];
        *v = c->pool_v + (size_t)idx * hd; *vs = c->pool_vs[idx];
        return;
    }
    idx -= c->pool_count;
    uint32_t n = c->win_count, ws = kv->window;
    uint32_t slot = (n < ws) ? idx : (c->win_head + idx) % ws;
    *k = c->win_k + (size_t)slot * hd; *ks = c->win_ks[slot];
    *v = c->win_v + (size_t)slot * hd; *vs = c->win_vs[slot];
}

static uint32_t kv_count(const orc_head* c) { return c->sink_count + c->pool_count + c->win_count; }

/* src/kv_cache.cpp:129-158 */
uint32_t orc_kv_attention_scores(orc_kv* kv, uint32_t layer, uint32_t head,
                                 const float* q, float* scores_out) {
    if (layer >= kv->n_layers || head >= kv->n_heads) return 0;
    const orc_head* c = &kv->h[(size_t)layer * kv->n_heads + head];
    uint32_t n = kv_count(c);
    for (uint32_t e = 0; e < n; e++) {
        const int8_t *k, *v; float ks, vs;
        kv_entry(kv, c, e, &k, &ks, &v, &vs);
        scores_out[e] = kv_dot_quant(q, k, ks, kv->hd);
    }
    return n;
}

/* src/kv_cache.cpp:160-198, sequential order (contracted accumulate). */
void orc_kv_attention_weighted_sum_ref(orc_kv* kv, uint32_t layer, uint32_t head,
                                       const float* scores, float* out, uint32_t count) {
    memset(out, 0, sizeof(float) * kv->hd);
    if (layer >= kv->n_layers || head >= kv->n_heads || count == 0) return;
    const orc_head* c = &kv->h[(size_t)layer * kv->n_heads + head];
    uint32_t n = kv_count(c);
    for (uint32_t e = 0; e < n && e < count; e++) {
        const int8_t *k, *v; float ks, vs;
        kv_entry(kv, c, e, &k, &ks, &v, &vs);
        for (uint32_t i = 0; i < kv->hd; i++) out[i] = fmaf(scores[e], (float)v[i] * vs, out[i]);
    }
}

/* src/kv_cache.cpp:160-198 in the canonical chunk-of-64 order. */
void orc_kv_attention_weighted_sum(orc_kv* kv, uint32_t layer, uint32_t head,
                                   const float* scores, float* out, uint32_t count) {
    uint32_t hd = kv->hd;
    memset(out, 0, sizeof(float) * hd);
    if (layer >= kv->n_layers || head >= kv->n_heads || count == 0) return;
    const orc_head* c = &kv->h[(size_t)layer * kv->n_heads + head];
    uint32_t n = kv_count(c);
    if (count < n) n = count;
    float* part = (float*)malloc(sizeof(float) * hd);
    for (uint32_t c0 = 0; c0 < n; c0 += 64) {
        for (uint32_t i = 0; i < hd; i++) part[i] = 0.0f;
        for (uint32_t e = c0; e < n && e < c0 + 64; e++) {
            const int8_t *k, *v; float ks, vs;
            kv_entry(kv, c, e, &k, &ks, &v, &vs);
            for (uint32_t i = 0; i < hd; i++) part[i] = fmaf(scores[e], (float)v[i] * vs, part[i]);
        }
        for (uint32_t i = 0; i < hd; i++) out[i] = out[i] + part[i];
    }
    free(part);
}

uint32_t orc_kv_size(const orc_kv* kv) { return kv->total_stored; }

uint32_t orc_kv_pool_count(const orc_kv* kv, uint32_t layer, uint32_t head) {
    return kv->h[(size_t)layer * kv->n_heads + head].pool_count;
}

uint32_t orc_kv_export(const orc_kv* kv, uint32_t layer, uint32_t head,
                       int8_t* k, float* ks, int8_t* v, float* vs) {
    const orc_head* c = &kv->h[(size_t)layer * kv->n_heads + head];
    uint32_t n = kv_count(c);
    for (uint32_t e = 0; e < n; e++) {
        const int8_t *kk, *vv; float s1, s2;
        kv_entry(kv, c, e, &kk, &s1, &vv, &s2);
        memcpy(k + (size_t)e * kv->hd, kk, kv->hd); ks[e] = s1;
        memcpy(v + (size_t)e * kv->hd, vv, kv->hd); vs[e] = s2;
    }
    return n;
}

/* Sets plane (layer, head) to a state given in KVCache's own terms: n_sink
 * sink rows, n_pool pooled rows, n_win window rows oldest first (the oldest
 * at position win_pos0), then n_pend evicted rows not yet folded, in
 * eviction order, whose running double sum (src/kv_cache.cpp:77-90) is
 * rebuilt here.  Rows [n][head_dim] with their scales, in that order.  A
 * full window is laid out oldest first from slot 0, the next slot to evict,
 * which is the ring state src/kv_cache.cpp:92-127 reaches up to rotation. */
void orc_kv_import(orc_kv* kv, uint32_t layer, uint32_t head, uint32_t n_sink, uint32_t n_pool, uint32_t n_win,
                   uint32_t win_pos0, uint32_t n_pend, const int8_t* k, const float* ks, const int8_t* v,
                   const float* vs) {
    orc_head* c = &kv->h[(size_t)layer * kv->n_heads + head];
    const uint32_t hd = kv->hd, ws = kv->window;
    uint32_t r = 0;
    for (uint32_t j = 0; j < n_sink && j < 8; j++, r++) {
        memcpy(c->sink_k + (size_t)j * hd, k + (size_t)r * hd, hd); c->sink_ks[j] = ks[r];
        memcpy(c->sink_v + (size_t)j * hd, v + (size_t)r * hd, hd); c->sink_vs[j] = vs[r];
    }
    c->sink_count = n_sink;
    pool_reserve(c, hd, n_pool);
    for (uint32_t j = 0; j < n_pool; j++, r++) {
        memcpy(c->pool_k + (size_t)j * hd, k + (size_t)r * hd, hd); c->pool_ks[j] = ks[r];
        memcpy(c->pool_v + (size_t)j * hd, v + (size_t)r * hd, hd); c->pool_vs[j] = vs[r];
    }
    c->pool_count = n_pool;
    for (uint32_t j = 0; j < n_win && j < ws; j++, r++) {
        memcpy(c->win_k + (size_t)j * hd, k + (size_t)r * hd, hd); c->win_ks[j] = ks[r];
        memcpy(c->win_v + (size_t)j * hd, v + (size_t)r * hd, hd); c->win_vs[j] = vs[r];
        c->win_pos[j] = win_pos0 + j;
    }
    c->win_count = n_win;
    c->win_head = n_win % ws;
    memset(c->acc_k, 0, sizeof(double) * hd);
    memset(c->acc_v, 0, sizeof(double) * hd);
    for (uint32_t j = 0; j < n_pend; j++, r++) {
        for (uint32_t i = 0; i < hd; i++) {
            c->acc_k[i] += (double)k[(size_t)r * hd + i] * (double)ks[r];
            c->acc_v[i] += (double)v[(size_t)r * hd + i] * (double)vs[r];
        }
    }
    c->acc_count = n_pend;
    c->acc_start = win_pos0 - n_pend;
}

/* src/kv_cache.cpp:200-219 */
void orc_kv_clear(orc_kv* kv) {
    for (size_t i = 0; i < (size_t)kv->n_layers * kv->n_heads; i++) {
        orc_head* c = &kv->h[i];
        c->sink_count = 0; c->win_count = 0; c->win_head = 0; c->pool_count = 0;
        memset(c->acc_k, 0, sizeof(double) * kv->hd);
        memset(c->acc_v, 0, sizeof(double) * kv->hd);
        c->acc_count = 0;
    }
    kv->total_stored = 0;
}

/* ====================================================== engine (forward) */

struct orc_engine {
    orc_model_desc d;
    orc_kv* kv;
    uint32_t pos;                 /* tokens forwarded so far (= next position) */
    int hidden_valid;
    float *h, *normed, *q, *k, *v, *attn, *o, *g, *u, *f, *last_hidden, *scores;
    int8_t* a8;
    uint32_t scores_cap;
    /* LayerSkipController state (src/layer_skip.cpp:8-20): threshold,
     * anchor interval, the normed FFN input last computed per layer */
    float skip_threshold;
    uint32_t skip_interval;
    float* skip_cache;             /* [n_layers][n_embd] */
    uint32_t skips;                /* FFN blocks skipped so far */
};

orc_engine* orc_engine_create(const orc_model_desc* d) {
    orc_engine* e = (orc_engine*)calloc(1, sizeof(orc_engine));
    e->d = *d;
    uint32_t D = d->n_embd, F = d->n_ff;
    e->kv = orc_kv_create(d->n_layers, d->n_heads, d->head_dim, d->sink_size,
                          d->window_size, d->pool_block, d->max_context);
    e->h = (float*)calloc(D, 4); e->normed = (float*)calloc(D, 4);
    e->q = (float*)calloc(D, 4); e->k = (float*)calloc(D, 4); e->v = (float*)calloc(D, 4);
    e->attn = (float*)calloc(D, 4); e->o = (float*)calloc(D, 4);
    e->g = (float*)calloc(F > D ? F : D, 4); e->u = (float*)calloc(F > D ? F : D, 4);
    e->f = (float*)calloc(F > D ? F : D, 4);
    e->last_hidden = (float*)calloc(D, 4);
    e->a8 = (int8_t*)calloc(F > D ? F : D, 1);
    e->scores_cap = d->max_context + 64;
    e->scores = (float*)calloc(e->scores_cap, 4);
    e->skip_threshold = 0.0f;      /* off: delta < 0 never holds */
    e->skip_interval = 4;          /* ModelConfig::skip_interval, include/forge/types.hpp:237 */
    e->skip_cache = (float*)calloc((size_t)d->n_layers * D, 4);
    return e;
}

/* Engine::set_layer_skip_threshold (src/engine.cpp:266-269) and the
 * controller's anchor interval (ModelConfig::skip_interval). */
void orc_engine_set_layer_skip(orc_engine* e, float threshold, uint32_t interval) {
    e->skip_threshold = threshold;
    e->skip_interval = interval;
}

uint32_t orc_engine_skip_count(const orc_engine* e) { return e->skips; }

/* LayerSkipController::hidden_delta (src/layer_skip.cpp:105-111), sqrt of
 * the mean squared difference, with the sum in the tile order of the
 * engine's RMSNorm (per 64-element tile a halving tree, tiles added in
 * order) instead of one sequential sum.  n % 64 == 0. */
float orc_skip_delta(const float* a, const float* b, uint32_t n) {
    float sum = 0.0f;
    for (uint32_t t = 0; t < n / 64; t++) {
        float L[64];
        for (uint32_t l = 0; l < 64; l++) {
            float d = a[64 * t + l] - b[64 * t + l];
            L[l] = d * d;
        }
        for (uint32_t off = 32; off >= 1; off >>= 1)
            for (uint32_t l = 0; l < off; l++) L[l] = L[l] + L[l + off];
        sum = sum + L[0];
    }
    return sqrtf(sum / (float)n);
}

/* LayerSkipController::should_skip_ffn (src/layer_skip.cpp:22-67) on the
 * FFN's normed input.  The anchor test compares tokens_since_anchor_ with
 * the interval; Engine never calls new_token() (src/layer_skip.cpp:83-87
 * has no caller), so the count stays 0 and only an interval of 0 anchors.
 * The threshold doubles for mid/2 < layer < mid + mid/2 (mid = layers / 2)
 * and the first and last two layers never skip. */
int orc_skip_decide(float* caches, uint32_t L, uint32_t D, float threshold, uint32_t interval, uint32_t l,
                    const float* normed) {
    if (l >= L) return 0;
    float* cache = caches + (size_t)l * D;
    if (interval == 0) {                                /* 0 >= interval: anchor */
        memcpy(cache, normed, sizeof(float) * D);
        return 0;
    }
    float delta = orc_skip_delta(normed, cache, D);
    uint32_t mid = L / 2;
    float thr = threshold;
    if (l > mid / 2 && l < mid + mid / 2) thr *= 2.0f;
    if (l < 2 || l >= L - 2) thr = -1.0f;
    int skip = delta < thr;
    if (!skip) memcpy(cache, normed, sizeof(float) * D);
    return skip;
}

static int skip_ffn(orc_engine* e, uint32_t l, const float* normed) {
    return orc_skip_decide(e->skip_cache, e->d.n_layers, e->d.n_embd, e->skip_threshold, e->skip_interval, l,
                           normed);
}

void orc_engine_destroy(orc_engine* e) {
    if (!e) return;
    orc_kv_destroy(e->kv);
    free(e->h); free(e->normed); free(e->q); free(e->k); free(e->v); free(e->attn);
    free(e->o); free(e->g); free(e->u); free(e->f); free(e->last_hidden); free(e->a8);
    free(e->scores); free(e->skip_cache); free(e);
}

void orc_engine_reset(orc_engine* e) {
    orc_kv_clear(e->kv);
    e->pos = 0;
    e->hidden_valid = 0;
    memset(e->skip_cache, 0, sizeof(float) * e->d.n_layers * e->d.n_embd);   /* LayerSkipController::reset */
    e->skips = 0;
}
uint32_t orc_engine_pos(const orc_engine* e) { return e->pos; }

/* After orc_kv_import of every plane: the next position and, when hidden is
 * not NULL, the last forward's hidden state (the MTP heads' input). */
void orc_engine_set_state(orc_engine* e, uint32_t pos, const float* hidden) {
    e->pos = pos;
    e->kv->total_stored = pos < e->kv->max_context ? pos : e->kv->max_context;
    if (hidden) {
        memcpy(e->last_hidden, hidden, sizeof(float) * e->d.n_embd);
        e->hidden_valid = 1;
    }
}
orc_kv* orc_engine_kv(orc_engine* e) { return e->kv; }

/* RoPE angles of src/engine.cpp:656-682 (theta 5e6) for one position:
 * cos/sin of pair t (elements 2t, 2t+1). */
void orc_rope_table(uint32_t hd, uint32_t pos, float* cos_out, float* sin_out) {
    for (uint32_t i = 0; i < hd; i += 2) {
        float freq = 1.0f / powf(5000000.0f, (float)i / (float)hd);
        float ang = (float)pos * freq;
        cos_out[i / 2] = cosf(ang);
        sin_out[i / 2] = sinf(ang);
    }
}

/* RoPE rotation of one head vector, src/engine.cpp:739-748: pair
 * (x[2t], x[2t+1]) -> (x0 c - x1 s, x0 s + x1 c) with cos/sin of pair t, in
 * the contracted form the reference's x86 build (-march=native) emits:
 * fmaf(x0, c, -(x1 s)) and fmaf(x0, s, x1 c). */
void orc_rope_rotate(float* x, uint32_t hd, const float* cos_t, const float* sin_t) {
    for (uint32_t i = 0; i < hd; i += 2) {
        float c = cos_t[i / 2], s = sin_t[i / 2];
        float x0 = x[i], x1 = x[i + 1];
        x[i] = fmaf(x0, c, -(x1 * s));
        x[i + 1] = fmaf(x0, s, x1 * c);
    }
}

/* Softmax-weighted sum of one head (src/engine.cpp:767-778 with
 * src/matmul_neon.cpp:212-226 and src/kv_cache.cpp:160-198) in the
 * canonical chunked order.  The list is the `cnt` visible entries followed
 * by the fp32 self entry (scores in e->scores[0..cnt]).  Chunks of 256
 * entries: m_c = chunk max, e_j = exp(s_j - m_c), T_c = CANON(4) sum with
 * one entry per lane, U_c = ((W0 + W1) + W2) + W3 where W_s is the fmaf
 * chain over the 64 entries of sub-chunk s of e_j * (float)v_j[i] * vs_j
 * (the self entry uses v_self).  Chunks merge left to right:
 * f_c = exp(m_c - max_c m_c), T = fmaf(T_c, f_c, T), U = fmaf(U_c, f_c, U),
 * out = U * (1 / (T + 1e-10)). */
static void attn_head(orc_kv* kv, const float* scores, uint32_t l, uint32_t hh, uint32_t cnt,
                      const float* vself, float* out) {
    const uint32_t hd = kv->hd, n = cnt + 1, nc = (n + 255) / 256;
    const orc_head* c = &kv->h[(size_t)l * kv->n_heads + hh];
    float* U = (float*)calloc(hd, sizeof(float));
    float* Uc = (float*)malloc(sizeof(float) * hd);
    float* Wv = (float*)malloc(sizeof(float) * hd);
    float* mc = (float*)malloc(sizeof(float) * nc);
    float* Tc = (float*)malloc(sizeof(float) * nc);
    float* Ucs = (float*)malloc(sizeof(float) * hd * nc);
    for (uint32_t ci = 0; ci < nc; ci++) {
        const uint32_t j0 = ci * 256, j1 = j0 + 256 < n ? j0 + 256 : n;
        float mx = scores[j0];
        for (uint32_t j = j0 + 1; j < j1; j++) if (scores[j] > mx) mx = scores[j];
        float P[256];
        float ev[256];
        for (uint32_t t = 0; t < 256; t++) {
            uint32_t j = j0 + t;
            ev[t] = j < n ? orc_expf(scores[j] - mx) : 0.0f;
            P[t] = ev[t];
        }
        Tc[ci] = canon_tree(P, 4);
        for (uint32_t i = 0; i < hd; i++) Uc[i] = 0.0f;
        for (uint32_t s = 0; s < 4; s++) {
            for (uint32_t i = 0; i < hd; i++) Wv[i] = 0.0f;
            for (uint32_t t = 64 * s; t < 64 * s + 64 && j0 + t < n; t++) {
                uint32_t j = j0 + t;
                if (j < cnt) {
                    const int8_t *k, *v; float ks, vs;
                    kv_entry(kv, c, j, &k, &ks, &v, &vs);
                    for (uint32_t i = 0; i < hd; i++) Wv[i] = fmaf(ev[t], (float)v[i] * vs, Wv[i]);
                } else {
                    for (uint32_t i = 0; i < hd; i++) Wv[i] = fmaf(ev[t], vself[i], Wv[i]);
                }
            }
            for (uint32_t i = 0; i < hd; i++) Uc[i] = Uc[i] + Wv[i];
        }
        mc[ci] = mx;
        memcpy(Ucs + (size_t)ci * hd, Uc, sizeof(float) * hd);
    }
    float M = mc[0];
    for (uint32_t ci = 1; ci < nc; ci++) if (mc[ci] > M) M = mc[ci];
    float T = 0.0f;
    for (uint32_t ci = 0; ci < nc; ci++) {
        float f = orc_expf(mc[ci] - M);
        T = fmaf(Tc[ci], f, T);
        for (uint32_t i = 0; i < hd; i++) U[i] = fmaf(Ucs[(size_t)ci * hd + i], f, U[i]);
    }
    float inv = 1.0f / (T + 1e-10f);
    for (uint32_t i = 0; i < hd; i++) out[i] = U[i] * inv;
    free(U); free(Uc); free(Wv); free(mc); free(Tc); free(Ucs);
}

/* Scores of one head's attention in the engine (src/engine.cpp:757-768):
 * the cached entries' dots, then the self entry's sequential dot with the
 * fp32 key, all times 1/sqrt(head_dim).  Returns the list length cnt + 1. */
static uint32_t attn_scores(orc_kv* kv, uint32_t l, uint32_t hh, const float* q, const float* kself, float* scores) {
    const uint32_t hd = kv->hd;
    const float scale = 1.0f / sqrtf((float)hd);
    uint32_t cnt = orc_kv_attention_scores(kv, l, hh, q, scores);
    float self = 0.0f;
    for (uint32_t i = 0; i < hd; i++) self = self + q[i] * kself[i];
    scores[cnt] = self;
    for (uint32_t i = 0; i <= cnt; i++) scores[i] *= scale;
    return cnt + 1;
}

/* One head of the engine's attention in the canonical chunked order. */
void orc_attn_head(orc_kv* kv, uint32_t layer, uint32_t head, const float* q, const float* kself,
                   const float* vself, float* out) {
    const orc_head* c = &kv->h[(size_t)layer * kv->n_heads + head];
    float* sc = (float*)malloc(sizeof(float) * (kv_count(c) + 1));
    uint32_t n = attn_scores(kv, layer, head, q, kself, sc);
    attn_head(kv, sc, layer, head, n - 1, vself, out);
    free(sc);
}

/* The same in the reference's own order (src/engine.cpp:767-778): softmax
 * with libm exp and a sequential sum, the sequential weighted sum of the
 * cached entries, then fmaf(p_self, v_self, out). */
void orc_attn_head_ref(orc_kv* kv, uint32_t layer, uint32_t head, const float* q, const float* kself,
                       const float* vself, float* out) {
    const orc_head* c = &kv->h[(size_t)layer * kv->n_heads + head];
    float* sc = (float*)malloc(sizeof(float) * (kv_count(c) + 1));
    uint32_t n = attn_scores(kv, layer, head, q, kself, sc);
    orc_softmax_ref(sc, n);
    orc_kv_attention_weighted_sum_ref(kv, layer, head, sc, out, n - 1);
    for (uint32_t i = 0; i < kv->hd; i++) out[i] = fmaf(sc[n - 1], vself[i], out[i]);
    free(sc);
}

/* Engine::forward_with_hidden, src/engine.cpp:459-589, with the weights
 * wired (src/engine.cpp:693-715, 789-796, 815-843), position = number of
 * tokens forwarded so far, and each head writing its own output slice. */
void orc_forward(orc_engine* e, int32_t token, float* logits, float* hidden) {
    const orc_model_desc* d = &e->d;
    uint32_t D = d->n_embd, H = d->n_heads, hd = d->head_dim, F = d->n_ff;
    uint32_t pos = e->pos++;
    float* h = e->h;
    /* token embedding (src/engine.cpp:476-484) */
    if (token >= 0 && (uint32_t)token < d->n_vocab) orc_dequant_row(d->emb, (uint32_t)token, h);
    else memset(h, 0, sizeof(float) * D);

    float* rc = (float*)malloc(sizeof(float) * hd / 2);
    float* rs = (float*)malloc(sizeof(float) * hd / 2);
    orc_rope_table(hd, pos, rc, rs);

    for (uint32_t l = 0; l < d->n_layers; l++) {
        const orc_qmat* W = d->layers + (size_t)l * 7;
        float as;
        /* attention block (src/engine.cpp:515-523, 646-799) */
        orc_engine_rmsnorm(e->normed, h, d->attn_norm + (size_t)l * D, D);
        orc_quantize_activation_row(e->normed, e->a8, &as, D);
        orc_gemv_i8(&W[0], e->a8, as, e->q);
        orc_gemv_i8(&W[1], e->a8, as, e->k);
        orc_gemv_i8(&W[2], e->a8, as, e->v);
        for (uint32_t hh = 0; hh < H; hh++) {              /* src/engine.cpp:732-749 */
            orc_rope_rotate(e->q + hh * hd, hd, rc, rs);
            orc_rope_rotate(e->k + hh * hd, hd, rc, rs);
        }
        for (uint32_t hh = 0; hh < H; hh++)                /* src/engine.cpp:753-779 */
            orc_attn_head(e->kv, l, hh, e->q + hh * hd, e->k + hh * hd, e->v + hh * hd, e->attn + hh * hd);
        for (uint32_t hh = 0; hh < H; hh++)                /* src/engine.cpp:782-786 */
            orc_kv_store(e->kv, l, hh, pos, e->k + hh * hd, e->v + hh * hd);
        orc_quantize_activation_row(e->attn, e->a8, &as, D); /* src/engine.cpp:789-796 */
        orc_gemv_i8(&W[3], e->a8, as, e->o);
        for (uint32_t i = 0; i < D; i++) h[i] += e->o[i];
        /* FFN block (src/engine.cpp:526-541, 805-843) */
        orc_engine_rmsnorm(e->normed, h, d->ffn_norm + (size_t)l * D, D);
        if (skip_ffn(e, l, e->normed)) {                 /* src/engine.cpp:529-534 */
            e->skips++;
            continue;
        }
        orc_quantize_activation_row(e->normed, e->a8, &as, D);
        orc_gemv_i8(&W[4], e->a8, as, e->g);
        orc_gemv_i8(&W[5], e->a8, as, e->u);
        for (uint32_t i = 0; i < F; i++) {
            float gi = e->g[i];
            float sig = 1.0f / (1.0f + orc_expf(-gi));
            e->f[i] = gi * sig * e->u[i];
        }
        orc_quantize_activation_row(e->f, e->a8, &as, F);
        orc_gemv_i8(&W[6], e->a8, as, e->o);
        for (uint32_t i = 0; i < D; i++) h[i] += e->o[i];
    }
    free(rc); free(rs);
    memcpy(e->last_hidden, h, sizeof(float) * D);       /* src/engine.cpp:550 */
    e->hidden_valid = 1;
    if (hidden) memcpy(hidden, h, sizeof(float) * D);
    /* logits from the pre-norm hidden state (src/engine.cpp:571-582) */
    if (logits) orc_gemv_f32(d->emb, h, logits);
}

/* MTPHeads::forward, src/mtp.cpp:47-129, tied unembed. */
void orc_mtp_forward(orc_engine* e, const float* hidden, float* logits) {
    const orc_model_desc* d = &e->d;
    uint32_t D = d->n_embd;
    float* cur = (float*)malloc(sizeof(float) * D);
    float* g = (float*)malloc(sizeof(float) * D);
    float* u = (float*)malloc(sizeof(float) * D);
    float* a = (float*)malloc(sizeof(float) * D);
    float* dn = (float*)malloc(sizeof(float) * D);
    memcpy(cur, hidden, sizeof(float) * D);
    for (uint32_t k = 0; k < d->n_mtp; k++) {
        const orc_qmat* M = d->mtp + (size_t)k * 3;
        orc_gemv_f32(&M[0], cur, g);
        orc_gemv_f32(&M[1], cur, u);
        for (uint32_t j = 0; j < D; j++) {                 /* src/mtp.cpp:89-91, 157-159 */
            float s = g[j] / (1.0f + orc_expf(-g[j]));
            a[j] = s * u[j];
        }
        orc_gemv_f32(&M[2], a, dn);
        for (uint32_t i = 0; i < D; i++) cur[i] += dn[i];  /* src/mtp.cpp:105-107 */
        orc_gemv_f32(d->emb, cur, logits + (size_t)k * d->n_vocab);
    }
    free(cur); free(g); free(u); free(a); free(dn);
}

/* MTPHeads::forward (src/mtp.cpp:47-129) of n_heads chained heads (each
 * gate, up, down: d x d block-quantized, fp32 activations in the canonical
 * order) with an fp32 tied table [V][d], or the placeholder logits
 * ((v * 2654435761 + head) mod V) / V when table is NULL (src/mtp.cpp:117-121). */
void orc_mtp_heads_forward(const orc_qmat* heads, uint32_t n_heads, uint32_t d, uint32_t V,
                           const float* table, const float* hidden, float* logits) {
    float* cur = (float*)malloc(sizeof(float) * d);
    float* g = (float*)malloc(sizeof(float) * d);
    float* u = (float*)malloc(sizeof(float) * d);
    float* a = (float*)malloc(sizeof(float) * d);
    float* dn = (float*)malloc(sizeof(float) * d);
    memcpy(cur, hidden, sizeof(float) * d);
    for (uint32_t k = 0; k < n_heads; k++) {
        const orc_qmat* M = heads + (size_t)k * 3;
        orc_gemv_f32(&M[0], cur, g);
        orc_gemv_f32(&M[1], cur, u);
        for (uint32_t j = 0; j < d; j++) {
            float sg = g[j] / (1.0f + orc_expf(-g[j]));
            a[j] = sg * u[j];
        }
        orc_gemv_f32(&M[2], a, dn);
        for (uint32_t i = 0; i < d; i++) cur[i] += dn[i];
        float* lk = logits + (size_t)k * V;
        if (table) orc_gemv_f32_dense(table, V, d, cur, lk);
        else
            for (uint32_t v = 0; v < V; v++)
                lk[v] = (float)(((uint64_t)v * 2654435761ULL + (uint64_t)k) % V) / (float)V;
    }
    free(cur); free(g); free(u); free(a); free(dn);
}

/* ============================================================ sampling */

/* MTPHeads::argmax / Engine::sample_greedy (src/mtp.cpp:145-155,
 * src/engine.cpp:918-928): first index of the maximum. */
int32_t orc_argmax(const float* x, uint32_t n) {
    int32_t best = 0; float bv = x[0];
    for (uint32_t i = 1; i < n; i++) if (x[i] > bv) { bv = x[i]; best = (int32_t)i; }
    return best;
}

/* Sum of x[0..n) over 64 contiguous chunks: sequential inside a chunk,
 * chunk totals added left to right. */
static float chunk64_sum(const float* x, uint32_t n) {
    uint32_t cl = (n + 63) / 64;
    float tot = 0.0f;
    for (uint32_t b = 0; b < 64; b++) {
        float t = 0.0f;
        for (uint32_t i = b * cl; i < n && i < (b + 1) * cl; i++) t = t + x[i];
        tot = tot + t;
    }
    return tot;
}

/* Inclusive prefix sums in the same chunk structure: chunk b starts from
 * the left-to-right sum of the previous chunk totals. */
static void chunk64_scan(const float* x, uint32_t n, float* cum) {
    uint32_t cl = (n + 63) / 64;
    float off = 0.0f;
    for (uint32_t b = 0; b < 64; b++) {
        float t = 0.0f, c = off;
        for (uint32_t i = b * cl; i < n && i < (b + 1) * cl; i++) { t = t + x[i]; c = c + x[i]; cum[i] = c; }
        off = off + t;
    }
}

typedef struct { float v; int32_t i; } orc_pair;
static int pair_desc(const void* a, const void* b) {
    const orc_pair* x = (const orc_pair*)a; const orc_pair* y = (const orc_pair*)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return (x->i < y->i) ? -1 : (x->i > y->i);
}

/* Engine::sample dispatch (src/engine.cpp:881-916), sample_top_k
 * (:930-959) and sample_top_p (:961-1003).  Ties in the sorts are broken by
 * ascending index. */
int32_t orc_sample(const float* logits, uint32_t V, const orc_sampling* cfg,
                   uint64_t seed, uint64_t* draw_idx) {
    if (cfg->greedy || cfg->temperature <= 0.0f) return orc_argmax(logits, V);
    float temp = cfg->temperature > 0.001f ? cfg->temperature : 0.001f;
    if (cfg->top_p < 1.0f && cfg->top_p > 0.0f) {
        orc_pair* s = (orc_pair*)malloc(sizeof(orc_pair) * V);
        for (uint32_t i = 0; i < V; i++) { s[i].v = logits[i]; s[i].i = (int32_t)i; }
        qsort(s, V, sizeof(orc_pair), pair_desc);
        float mx = s[0].v;
        float* pr = (float*)malloc(sizeof(float) * V);
        float* cum = (float*)malloc(sizeof(float) * V);
        for (uint32_t i = 0; i < V; i++) pr[i] = orc_expf((s[i].v - mx) / temp);
        float sum = chunk64_sum(pr, V);
        for (uint32_t i = 0; i < V; i++) pr[i] = pr[i] / sum;
        chunk64_scan(pr, V, cum);
        uint32_t cutoff = V;
        for (uint32_t i = 0; i < V; i++) if (cum[i] >= cfg->top_p) { cutoff = i + 1; break; }
        float r = orc_uniform(seed, (*draw_idx)++);
        int32_t res = s[cutoff - 1].i;
        for (uint32_t i = 0; i < cutoff; i++) if (r <= cum[i]) { res = s[i].i; break; }
        free(s); free(pr); free(cum);
        return res;
    }
    if (cfg->top_k > 0 && cfg->top_k < V) {
        uint32_t k = cfg->top_k;
        orc_pair* s = (orc_pair*)malloc(sizeof(orc_pair) * V);
        for (uint32_t i = 0; i < V; i++) { s[i].v = logits[i]; s[i].i = (int32_t)i; }
        qsort(s, V, sizeof(orc_pair), pair_desc);
        float mx = s[0].v, sum = 0.0f;
        float* pr = (float*)malloc(sizeof(float) * k);
        for (uint32_t i = 0; i < k; i++) { pr[i] = orc_expf((s[i].v - mx) / temp); sum += pr[i]; }
        float r = orc_uniform(seed, (*draw_idx)++);
        float cum = 0.0f; int32_t res = s[k - 1].i;
        for (uint32_t i = 0; i < k; i++) { cum += pr[i] / sum; if (r <= cum) { res = s[i].i; break; } }
        free(s); free(pr);
        return res;
    }
    float mx = logits[0];
    for (uint32_t i = 1; i < V; i++) if (logits[i] > mx) mx = logits[i];
    float* sc = (float*)malloc(sizeof(float) * V);
    float* cum = (float*)malloc(sizeof(float) * V);
    for (uint32_t i = 0; i < V; i++) sc[i] = orc_expf((logits[i] - mx) / temp);
    float sum = chunk64_sum(sc, V);
    for (uint32_t i = 0; i < V; i++) sc[i] = sc[i] / sum;
    chunk64_scan(sc, V, cum);
    float r = orc_uniform(seed, (*draw_idx)++);
    int32_t res = (int32_t)V - 1;
    for (uint32_t i = 0; i < V; i++) if (r <= cum[i]) { res = (int32_t)i; break; }
    free(sc); free(cum);
    return res;
}

/* ============================================================ generate */

#include <time.h>
static double g_last_decode_seconds = 0.0;
static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}
/* Wall time of the decode loop (after the prompt) of the last orc_generate. */
double orc_last_decode_seconds(void) { return g_last_decode_seconds; }

/* Engine::generate, src/engine.cpp:276-396 (MTP branch :304-373, fallback
 * :377-386) over an abstract model (orc_gen_ops), so that the same control
 * flow runs on the oracle engine and on scripted logits.  The sampling
 * configuration is passed explicitly (the reference can only use its
 * defaults, :311, 324, 355, 383).  Returns 0, or -1 when tokens_cap is too
 * small. */
/* The decode loop of Engine::generate (src/engine.cpp:294-389) from the
 * current token `cur`, appending to tokens[*n_io ..]; -1 once `cap` tokens
 * would be exceeded. */
static int32_t gen_loop(const orc_gen_ops* ops, int32_t cur, uint32_t max_new, const orc_sampling* cfg,
                        uint64_t seed, int32_t* tokens, uint32_t cap, uint32_t* n_io, int32_t* mtp_accepted,
                        int32_t* mtp_rejected) {
    uint32_t V = ops->n_vocab, NH = ops->n_mtp;
    uint64_t draw = 0;
    uint32_t nt = *n_io;
    int32_t acc_total = 0, rej_total = 0;
    float* logits = (float*)malloc(sizeof(float) * V);
    float* mtp_logits = (float*)malloc(sizeof(float) * V * (NH ? NH : 1));
    int32_t* preds = (int32_t*)malloc(sizeof(int32_t) * (NH ? NH : 1));
#define PUSH(t) do { if (nt >= cap) { nt = cap + 1; goto done; } tokens[nt++] = (t); } while (0)
    double t_dec = now_s();
    uint32_t n_gen = 0;
    while (n_gen < max_new) {
        /* :304-305: MTP heads present, a hidden state, and n + 4 <= N */
        if (NH > 0 && ops->hidden_valid(ops->ctx) && n_gen + 4 <= max_new) {
            ops->forward(ops->ctx, cur, logits);                          /* :308 */
            int32_t T1 = orc_sample(logits, V, cfg, seed, &draw);         /* :311 */
            PUSH(T1); n_gen++;
            ops->mtp(ops->ctx, NULL, mtp_logits);                         /* :318-319 */
            for (uint32_t k = 0; k < NH; k++) preds[k] = orc_sample(mtp_logits + (size_t)k * V, V, cfg, seed, &draw);
            int accepted = 0, rejected = 0;
            for (uint32_t k = 0; k < NH; k++) {                           /* :332-366 */
                int32_t in = (k == 0) ? T1 : preds[k - 1];
                ops->forward(ops->ctx, in, logits);
                int32_t main_pred = orc_argmax(logits, V);
                if (main_pred == preds[k]) {
                    PUSH(preds[k]); n_gen++; accepted++;
                } else {
                    int32_t corr = orc_sample(logits, V, cfg, seed, &draw);
                    if (corr != preds[k]) { PUSH(corr); n_gen++; rejected++; }   /* :357-363 */
                    break;
                }
            }
            acc_total += accepted; rej_total += rejected;
            cur = tokens[nt - 1];                                         /* :372 */
            continue;
        }
        ops->forward(ops->ctx, cur, logits);                              /* :378 */
        cur = orc_sample(logits, V, cfg, seed, &draw);
        PUSH(cur); n_gen++;
    }
done:
#undef PUSH
    g_last_decode_seconds = now_s() - t_dec;
    free(logits); free(mtp_logits); free(preds);
    *n_io = nt > cap ? cap : nt;
    *mtp_accepted = acc_total; *mtp_rejected = rej_total;
    return nt > cap ? -1 : 0;
}

int32_t orc_generate_ops(const orc_gen_ops* ops, const int32_t* prompt, uint32_t n_prompt,
                         uint32_t max_new, const orc_sampling* cfg, uint64_t seed,
                         int32_t* tokens, uint32_t cap, uint32_t* n_tokens,
                         int32_t* mtp_accepted, int32_t* mtp_rejected) {
    for (uint32_t i = 0; i < n_prompt; i++) ops->forward(ops->ctx, prompt[i], NULL);   /* :286-290 */
    uint32_t nt = 0;
    for (uint32_t i = 0; i < n_prompt; i++) {
        if (nt >= cap) { *n_tokens = cap; *mtp_accepted = 0; *mtp_rejected = 0; return -1; }
        tokens[nt++] = prompt[i];
    }
    int32_t cur = n_prompt ? prompt[n_prompt - 1] : 0;                     /* :294 */
    int32_t rc = gen_loop(ops, cur, max_new, cfg, seed, tokens, cap, &nt, mtp_accepted, mtp_rejected);
    *n_tokens = nt;
    return rc;
}

/* Engine::step_mtp, src/engine.cpp:402-448, over an abstract model: drafts
 * sampled from the heads on `hidden`, each verified by one greedy forward.
 * Without heads (or with no table, has_table == 0) it is one plain forward
 * of current_token (:413-416).  On a rejection the reference returns the
 * rejecting forward's logits and leaves mtp_accepted_out at 0 (:437-440);
 * when every draft is accepted the logits are empty (:443-447).  Returns the
 * accepted count; *n_logits is V when logits_out was written, else 0.  The
 * draw counter advances once per stochastic sample. */
int32_t orc_step_mtp_ops(const orc_gen_ops* ops, int32_t current_token, const float* hidden, int32_t has_table,
                         const orc_sampling* cfg, uint64_t seed, uint64_t* draw, float* logits_out,
                         uint32_t* n_logits, int32_t* acc_out, int32_t* rej_out) {
    uint32_t V = ops->n_vocab, NH = ops->n_mtp;
    *acc_out = 0; *rej_out = 0; *n_logits = 0;
    if (NH == 0 || !has_table) {
        ops->forward(ops->ctx, current_token, logits_out);
        *n_logits = V;
        return 0;
    }
    float* mtp_logits = (float*)malloc(sizeof(float) * V * NH);
    int32_t* preds = (int32_t*)malloc(sizeof(int32_t) * NH);
    ops->mtp(ops->ctx, hidden, mtp_logits);
    for (uint32_t k = 0; k < NH; k++) preds[k] = orc_sample(mtp_logits + (size_t)k * V, V, cfg, seed, draw);
    int32_t accepted = 0;
    for (uint32_t k = 0; k < NH; k++) {
        int32_t in = (k == 0) ? current_token : preds[k - 1];
        ops->forward(ops->ctx, in, logits_out);
        if (orc_argmax(logits_out, V) == preds[k]) {
            accepted++;
        } else {
            *rej_out = (int32_t)NH - accepted;
            *n_logits = V;
            free(mtp_logits); free(preds);
            return accepted;
        }
    }
    *acc_out = accepted;
    free(mtp_logits); free(preds);
    return accepted;
}

/* The oracle engine as an orc_gen_ops model: forward = orc_forward,
 * hidden_valid = Engine::hidden_valid_ (set by every forward,
 * src/engine.cpp:551), heads = MTPHeads::forward on the given hidden state
 * or on the last forward's (last_hidden_, :550) with the tied table. */
static void eng_forward(void* ctx, int32_t token, float* logits) { orc_forward((orc_engine*)ctx, token, logits, NULL); }
static int32_t eng_hidden_valid(void* ctx) { return ((orc_engine*)ctx)->hidden_valid; }
static void eng_mtp(void* ctx, const float* hidden, float* logits) {
    orc_engine* e = (orc_engine*)ctx;
    orc_mtp_forward(e, hidden ? hidden : e->last_hidden, logits);
}
static orc_gen_ops engine_ops(orc_engine* e) {
    orc_gen_ops o = {e, e->d.n_vocab, e->d.n_mtp, eng_forward, eng_hidden_valid, eng_mtp};
    return o;
}

int32_t orc_generate(orc_engine* e, const int32_t* prompt, uint32_t n_prompt,
                     uint32_t max_new, const orc_sampling* cfg, uint64_t seed,
                     int32_t* tokens, uint32_t cap, uint32_t* n_tokens,
                     int32_t* mtp_accepted, int32_t* mtp_rejected) {
    orc_gen_ops o = engine_ops(e);
    return orc_generate_ops(&o, prompt, n_prompt, max_new, cfg, seed, tokens, cap, n_tokens, mtp_accepted,
                            mtp_rejected);
}

int32_t orc_generate_continue(orc_engine* e, int32_t cur, uint32_t max_new, const orc_sampling* cfg,
                              uint64_t seed, int32_t* tokens, uint32_t cap, uint32_t* n_tokens,
                              int32_t* mtp_accepted, int32_t* mtp_rejected) {
    orc_gen_ops o = engine_ops(e);
    uint32_t nt = 0;
    int32_t rc = gen_loop(&o, cur, max_new, cfg, seed, tokens, cap, &nt, mtp_accepted, mtp_rejected);
    *n_tokens = nt;
    return rc;
}

int32_t orc_step_mtp(orc_engine* e, int32_t current_token, const float* hidden, int32_t has_table,
                     const orc_sampling* cfg, uint64_t seed, uint64_t* draw, float* logits_out,
                     uint32_t* n_logits, int32_t* acc_out, int32_t* rej_out) {
    orc_gen_ops o = engine_ops(e);
    return orc_step_mtp_ops(&o, current_token, hidden, has_table, cfg, seed, draw, logits_out, n_logits, acc_out,
                            rej_out);
}
