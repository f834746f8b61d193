// 3-tier int8 KV cache and verify attention for gfx950.
//
// A pass of M rows at consecutive positions p0..p0+M-1 runs, per layer
// (after the Q/K/V product, whose epilogue applies RoPE, pf_mm.hip):
//   k_kv_store_pass  (passes of more than 8 rows) int8 K/V rows of each pass
//                  row written to the plane row of its position (sink slot
//                  or ring slot; the ring has slack, so pending rows of a
//                  verify pass never overwrite a visible entry)
//   k_attn_group   per (head, 256-entry chunk, group of rows whose lists
//                  extend each other): scores, chunk max, exp, chunk sum and
//                  chunk-weighted V of each row; passes of at most 8 rows
//                  also quantize and store their own K/V rows here
//   k_attn_chunk   the same per (row, head, chunk), for batched passes of
//                  more than 8 rows
//   k_attn_seq     the same per (head, chunk, group of a sequence's rows)
//                  for batched verify passes, whose rows' windows may slide
//   k_attn_merge_quant  per row: chunks rescaled to the row max and merged,
//                  then the O projection's quantize_activation_row
// The KVCache API (raw scores; weighted sum of caller probabilities) runs
// k_attn_scores and k_attn_wsum.
// k_pool_rows folds evicted window entries into pooled rows
// (src/kv_cache.cpp:77-109) before a pass needs them.
#include "pf_device.h"

namespace pf {

__device__ __forceinline__ size_t plane_index(const KvGeom& g, uint32_t seq, uint32_t layer, uint32_t head) {
    return ((size_t)seq * g.n_layers + layer) * g.n_heads + head;
}

// View of row m of a pass: from its position, or from explicit counts when
// view_sink >= 0 (the KVCache API, whose planes advance independently).
__device__ __forceinline__ KvView pass_view(const KvGeom& g, const PassDesc* pd, uint32_t m,
                                            int32_t view_sink, uint32_t view_nw) {
    if (view_sink >= 0) return kv_view_counts(g, (uint32_t)view_sink, view_nw);
    return kv_view(g, row_pos(pd, m));
}

// ------------------------------------------------------------ store side

// Quantizes one head's key and value (src/kv_cache.cpp:19-28) and writes
// them to plane row `row`.  Called by one wave; element pair (2t, 2t+1) per
// lane, head_dim <= 128.
__device__ __forceinline__ void store_pair(const KvGeom& g, KvPlanes kv, size_t plane, uint32_t row,
                                           uint32_t t, bool act, float k0, float k1, float v0, float v1) {
    float ak = act ? fmaxf(fabsf(k0), fabsf(k1)) : 0.0f;
    float av = act ? fmaxf(fabsf(v0), fabsf(v1)) : 0.0f;
    ak = wave_max(ak);
    av = wave_max(av);
    if (row == 0xFFFFFFFFu) return;
    const uint32_t hd = g.head_dim;
    const float ik = (ak == 0.0f) ? 1.0f : 127.0f / ak;
    const float iv = (av == 0.0f) ? 1.0f : 127.0f / av;
    size_t base = (plane * g.rows + row) * hd;
    if (act) {
        kv.k[base + 2 * t] = quant_code(k0, ik);
        kv.k[base + 2 * t + 1] = quant_code(k1, ik);
        kv.v[base + 2 * t] = quant_code(v0, iv);
        kv.v[base + 2 * t + 1] = quant_code(v1, iv);
    }
    if (t == 0) {
        kv.ks[plane * g.rows + row] = (ak == 0.0f) ? 1.0f : ak / 127.0f;
        kv.vs[plane * g.rows + row] = (av == 0.0f) ? 1.0f : av / 127.0f;
    }
}

// KVCache::store (src/kv_cache.cpp:59-127) of every row of a pass: grid
// (M, heads), 64 threads; k and v [M][D] hold the rows' keys (after RoPE) and
// values in fp32.
__global__ __launch_bounds__(64) void k_kv_store_pass(const PassDesc* __restrict__ pd, KvGeom g, KvPlanes kv,
                                                      uint32_t layer, const float* __restrict__ k,
                                                      const float* __restrict__ v) {
    const uint32_t m = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    if (m >= pd->m) return;
    const uint32_t hd = g.head_dim, D = g.n_heads * hd, half = hd >> 1;
    const uint32_t pos = row_pos(pd, m);
    const bool act = t < half;
    float k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
    if (act) {
        const size_t o = (size_t)m * D + h * hd + 2 * t;
        k0 = k[o]; k1 = k[o + 1];
        v0 = v[o]; v1 = v[o + 1];
    }
    store_pair(g, kv, plane_index(g, row_seq(pd, m), layer, h), kv_store_row(g, pos), t, act, k0, k1, v0, v1);
}

// KVCache::store of one (layer, head) row given fp32 key/value (the
// reference API).  64 threads.
__global__ __launch_bounds__(64) void k_kv_store_row(KvGeom g, KvPlanes kv, uint32_t layer, uint32_t head,
                                                     uint32_t row, const float* __restrict__ key,
                                                     const float* __restrict__ val) {
    const uint32_t t = threadIdx.x, half = g.head_dim >> 1;
    const bool act = t < half;
    float k0 = act ? key[2 * t] : 0.f, k1 = act ? key[2 * t + 1] : 0.f;
    float v0 = act ? val[2 * t] : 0.f, v1 = act ? val[2 * t + 1] : 0.f;
    store_pair(g, kv, plane_index(g, 0, layer, head), row, t, act, k0, k1, v0, v1);
}

// Pooled row r of one plane: the mean of pool_block consecutive window
// entries accumulated in double in eviction order, scaled by
// (double)(1.0f/P), then requantized (src/kv_cache.cpp:83-104).
// 64 or 128 threads (head_dim <= 128).
__device__ void pool_row(const KvGeom& g, KvPlanes kv, size_t plane, uint32_t r) {
    __shared__ float red[4];
    const uint32_t i = threadIdx.x, hd = g.head_dim, P = g.pool_block;
    const bool act = i < hd;
    const float inv = 1.0f / (float)P;
    const size_t prow = plane * g.rows;
    const uint32_t dst = KV_SINK_ROWS + g.ring + r;
    for (int which = 0; which < 2; which++) {
        const int8_t* src = which ? kv.v : kv.k;
        const float* srs = which ? kv.vs : kv.ks;
        double acc = 0.0;
        if (act) {
            for (uint32_t e = 0; e < P; e++) {
                uint32_t slot = KV_SINK_ROWS + (r * P + e) % g.ring;
                acc += (double)src[(prow + slot) * hd + i] * (double)srs[prow + slot];
            }
        }
        float avg = act ? (float)(acc * (double)inv) : 0.0f;
        float w = wave_max(fabsf(avg));
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = w;
        __syncthreads();
        const float amax = (blockDim.x > 64) ? fmaxf(red[0], red[1]) : red[0];
        __syncthreads();
        const float qi = (amax == 0.0f) ? 1.0f : 127.0f / amax;
        int8_t* d8 = which ? kv.v : kv.k;
        float* ds = which ? kv.vs : kv.ks;
        if (act) d8[(prow + dst) * hd + i] = quant_code(avg, qi);
        if (i == 0) ds[prow + dst] = (amax == 0.0f) ? 1.0f : amax / 127.0f;
    }
}

// One pooled row of plane `plane` (the KVCache API, which folds a block as
// soon as its last entry is evicted).
__global__ __launch_bounds__(128) void k_pool_row_one(KvGeom g, KvPlanes kv, uint32_t plane, uint32_t r) {
    pool_row(g, kv, plane, r);
}

// Pooled rows a pass can see and earlier passes may not have folded, from
// the pass descriptor; refolding a row rewrites the same values.  Grid
// (layers * heads, y), y over the rows [pool(p0 - 1), pool(p0 + M - 1)) of
// a single-sequence pass, or over the pass rows of a batched pass: row m at
// position p folds [pool(p - 1), pool(p)), at most one row, since the
// pooled count grows by at most one per position.
__device__ __forceinline__ void pool_rows_block(const KvGeom& g, const KvPlanes& kv, const PassDesc* __restrict__ pd,
                                                uint32_t bx, uint32_t y) {
    uint32_t p_first, p_last, seq;
    if (pd->batch) {
        if (y >= pd->m) return;
        p_first = p_last = pd->rpos[y];
        seq = pd->rseq[y];
        y = 0;
    } else {
        p_first = pd->pos0;
        p_last = pd->pos0 + pd->m - 1;
        seq = pd->seq0;
    }
    const uint32_t r_lo = kv_view(g, p_first > 0 ? p_first - 1 : 0).pool;
    const uint32_t r_hi = kv_view(g, p_last).pool;
    const uint32_t r = r_lo + y;
    if (r >= r_hi || r >= g.pool_cap) return;
    pool_row(g, kv, (size_t)seq * g.n_layers * g.n_heads + bx, r);
}
__global__ __launch_bounds__(128) void k_pool_rows(KvGeom g, KvPlanes kv, const PassDesc* __restrict__ pd) {
    pool_rows_block(g, kv, pd, blockIdx.x, blockIdx.y);
}

// ------------------------------------------------------------ attention

// S[(m*H + y)*s_stride + j]: scores of the visible entries (j < C) and of
// the fp32 self key (j == C), multiplied by 1/sqrt(head_dim) when `scaled`
// (src/engine.cpp:757-768; KVCache::attention_scores returns them raw).
// Grid (M, H, ceil((Cmax+1)/256)); head = blockIdx.y unless head_override
// >= 0 (then q, kself and S are indexed with y = 0).
__global__ __launch_bounds__(256) void k_attn_scores(const PassDesc* __restrict__ pd, KvGeom g, KvPlanes kv,
                                                     uint32_t layer, int32_t view_sink, uint32_t view_nw,
                                                     int32_t head_override,
                                                     const float* __restrict__ q, const float* __restrict__ kself,
                                                     float* __restrict__ S, uint32_t s_stride, int32_t scaled) {
    __shared__ float qs[128];
    const uint32_t m = blockIdx.x, y = blockIdx.y;
    const uint32_t h = head_override >= 0 ? (uint32_t)head_override : y;
    if (m >= pd->m) return;
    const uint32_t hd = g.head_dim, D = g.n_heads * hd;
    const KvView v = pass_view(g, pd, m, view_sink, view_nw);
    const uint32_t C = v.count();
    const uint32_t j = blockIdx.z * 256u + threadIdx.x;
    if (blockIdx.z * 256u > C) return;
    const uint32_t qrow = head_override >= 0 ? 0u : (uint32_t)m * D + y * hd;
    for (uint32_t i = threadIdx.x; i < hd; i += 256) qs[i] = q[qrow + i];
    __syncthreads();
    const float scale = scaled ? 1.0f / __builtin_sqrtf((float)hd) : 1.0f;
    float* out = S + ((size_t)m * g.n_heads + y) * s_stride;
    if (j < C) {
        const size_t plane = plane_index(g, row_seq(pd, m), layer, h);
        const uint32_t row = kv_row(g, v, j);
        const int8_t* kr = kv.k + (plane * g.rows + row) * hd;
        const float ks = kv.ks[plane * g.rows + row];
        float acc = 0.0f;
        if ((hd & 15u) == 0) {
            for (uint32_t i = 0; i < hd; i += 16) {
                int4 w = *reinterpret_cast<const int4*>(kr + i);
                int wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int b = 0; b < 16; b++) {
                    int8_t c = (int8_t)((wv[b >> 2] >> (8 * (b & 3))) & 0xFF);
                    acc = __builtin_fmaf(qs[i + b], (float)c * ks, acc);
                }
            }
        } else {
            for (uint32_t i = 0; i < hd; i++) acc = __builtin_fmaf(qs[i], (float)kr[i] * ks, acc);
        }
        out[j] = scaled ? acc * scale : acc;
    } else if (j == C) {
        const float* kk = kself + qrow;
        float self = 0.0f;
        for (uint32_t i = 0; i < hd; i++) self = self + qs[i] * kk[i];
        out[C] = scaled ? self * scale : self;
    }
}

// Wp[((m*H + y)*cstride + c)*hd + i] = fmaf chain over the visible entries
// [64c, min(64c+64, C, limit)) of p_j * ((float)v_j[i] * vs_j)
// (src/kv_cache.cpp:173-197, contracted as the reference build does).  The
// chunk's V rows, row scales and probabilities are staged in LDS first.
// Grid (M, H, chunks), 128 threads (head_dim <= 128).
__global__ __launch_bounds__(128) void k_attn_wsum(const PassDesc* __restrict__ pd, KvGeom g, KvPlanes kv,
                                                   uint32_t layer, int32_t view_sink, uint32_t view_nw,
                                                   int32_t head_override, uint32_t limit,
                                                   const float* __restrict__ S, uint32_t s_stride,
                                                   float* __restrict__ Wp, uint32_t cstride) {
    __shared__ __align__(16) int8_t vt[64][128];
    __shared__ float vsc[64], pp[64];
    const uint32_t m = blockIdx.x, y = blockIdx.y, c = blockIdx.z, i = threadIdx.x;
    const uint32_t h = head_override >= 0 ? (uint32_t)head_override : y;
    if (m >= pd->m) return;
    const uint32_t hd = g.head_dim;
    const KvView v = pass_view(g, pd, m, view_sink, view_nw);
    const uint32_t C = min(v.count(), limit);
    if (c * 64u >= C) return;
    const size_t plane = plane_index(g, row_seq(pd, m), layer, h);
    const float* p = S + ((size_t)m * g.n_heads + y) * s_stride;
    const uint32_t j0 = c * 64u, n = min(64u, C - j0);
    if ((hd & 15u) == 0) {
        const uint32_t parts = hd >> 4;
        for (uint32_t idx = i; idx < n * parts; idx += blockDim.x) {
            const uint32_t e = idx / parts, q = idx % parts;
            const uint32_t row = kv_row(g, v, j0 + e);
            *reinterpret_cast<int4*>(&vt[e][q * 16]) =
                *reinterpret_cast<const int4*>(kv.v + (plane * g.rows + row) * hd + q * 16);
        }
    } else {
        for (uint32_t idx = i; idx < n * hd; idx += blockDim.x) {
            const uint32_t e = idx / hd, q = idx % hd;
            vt[e][q] = kv.v[(plane * g.rows + kv_row(g, v, j0 + e)) * hd + q];
        }
    }
    for (uint32_t e = i; e < n; e += blockDim.x) {
        vsc[e] = kv.vs[plane * g.rows + kv_row(g, v, j0 + e)];
        pp[e] = p[j0 + e];
    }
    __syncthreads();
    if (i >= hd) return;
    float acc = 0.0f;
    for (uint32_t e = 0; e < n; e++) acc = __builtin_fmaf(pp[e], (float)vt[e][i] * vsc[e], acc);
    Wp[(((size_t)m * g.n_heads + y) * cstride + c) * hd + i] = acc;
}

// One head's chunk partials added left to right (the KVCache API path).
__global__ void k_wsum_combine_one(const float* __restrict__ Wp, uint32_t nch, uint32_t hd, float* __restrict__ out) {
    const uint32_t i = threadIdx.x;
    if (i >= hd) return;
    float o = 0.0f;
    for (uint32_t c = 0; c < nch; c++) o = o + Wp[(size_t)c * hd + i];
    out[i] = o;
}

// Engine attention, first stage.  Task (row m, head h, chunk c) covers list
// entries [256c, 256c + 256) of row m; the list is the C visible entries
// followed by the fp32 self entry (index C).  Scores as in
// src/engine.cpp:757-768 (cached entries: sequential fmaf dot of q with
// (float)k * k_scale; self entry: sequential mul+add dot with the fp32 key;
// both times 1/sqrt(head_dim)), then the chunk max m_c, e_j = exp(s_j - m_c),
// the CANON(4) chunk sum T_c (one entry per thread) and the chunk's weighted
// sum U_c = (((0 + W0) + W1) + W2) + W3, where W_s is the fmaf chain from
// 0.0f over the entries of sub-chunk s (64 entries) of e_j * ((float)v_j *
// v_scale_j), or of e_j * v_self for the self entry.  Writes
// S[(m*H + h)*s_stride + 2c] = m_c, [.. + 2c + 1] = T_c and
// Up[((m*H + h)*cstride + c)*hd + i] = U_c[i].

// Per-row attention, for batched passes of more than 8 rows (many
// sequences, a few rows each): one block per (row, head, chunk) with the
// first stage's arithmetic, every thread loading its own entry's K and V
// rows.  Shared memory of one block (bytes): V rows of the chunk first,
// VROW = 136 bytes each (8 bytes of padding), which keeps the block under
// 40 KB, so four blocks fit in a CU's 160 KB.
constexpr uint32_t att_vt(uint32_t vrow) { return 256 * vrow; }
constexpr uint32_t att_smem(uint32_t vrow) { return att_vt(vrow) + (128 + 128 + 256 + 256 + 512 + 4) * 4; }

template <int PARTS, uint32_t VROW = 144>
__device__ __forceinline__ void attn_one_row(const PassHead& pd, const KvGeom& g, const KvPlanes& kv,
                                             uint32_t layer, uint32_t m, uint32_t h, uint32_t c,
                                             const float* __restrict__ q, const float* __restrict__ kself,
                                             const float* __restrict__ vself, float* __restrict__ S,
                                             uint32_t s_stride, float* __restrict__ Up, uint32_t cstride,
                                             uint8_t* smem) {
    constexpr uint32_t hd = 16 * PARTS;
    int8_t (*vt)[VROW] = reinterpret_cast<int8_t (*)[VROW]>(smem);
    float* qs = reinterpret_cast<float*>(smem + att_vt(VROW));
    float* kss = qs + 128;
    float* vsc = kss + 128;
    float* pe = vsc + 256;
    float* wp = pe + 256;                           // [4][128]
    float* red = wp + 512;
    const uint32_t t = threadIdx.x;
    const uint32_t D = g.n_heads * hd;
    const KvView v = kv_view(g, row_pos(pd, m));
    const uint32_t C = v.count(), n = C + 1, j0 = c * 256u;
    if (j0 >= n) return;
    const uint32_t j = j0 + t;
    const size_t plane = plane_index(g, row_seq(pd, m), layer, h);
    const size_t qrow = (size_t)m * D + h * hd;
    const uint32_t nvis = j0 < C ? min(256u, C - j0) : 0u;
    // every load first: the query, the fp32 self key, this thread's K and V rows
    if (t < hd) {
        qs[t] = q[qrow + t];
        kss[t] = kself[qrow + t];
    }
    int4 kw[PARTS];
    float ks = 0.0f, vs = 0.0f;
    if (t < nvis) {
        const size_t row = plane * g.rows + kv_row(g, v, j);
        const int4* kr = reinterpret_cast<const int4*>(kv.k + row * hd);
        const int4* vr = reinterpret_cast<const int4*>(kv.v + row * hd);
        int4 vw[PARTS];
#pragma unroll
        for (int p = 0; p < PARTS; p++) {
            kw[p] = kr[p];
            vw[p] = vr[p];
        }
        ks = kv.ks[row];
        vs = kv.vs[row];
#pragma unroll
        for (int p = 0; p < PARTS; p++) {
            if constexpr (VROW % 16 == 0) {
                *reinterpret_cast<int4*>(&vt[t][p * 16]) = vw[p];
                continue;
            }
            *reinterpret_cast<int2*>(&vt[t][p * 16]) = make_int2(vw[p].x, vw[p].y);
            *reinterpret_cast<int2*>(&vt[t][p * 16 + 8]) = make_int2(vw[p].z, vw[p].w);
        }
    }
    vsc[t] = vs;                 // 0 past the visible entries: their terms below add exactly 0
    __syncthreads();
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
    const float T = block_canon_sum<4>(ex, red);       // its barriers publish pe
    const uint32_t sc = t >> 6, i0 = 2u * (t & 63u);
    if (i0 < hd) {
        float w0 = 0.0f, w1 = 0.0f;
        // entries [64sc, min(64sc + 64, nvis)) in groups of 8; the padding
        // entries up to the next multiple of 8 have v_scale 0 and finite
        // codes and weights, so fmaf(e, code * 0, w) == w
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
        const uint32_t js = C - j0;                     // list index of the self entry in the chunk
        if (js < 256u && (js >> 6) == sc) {
            const float p = pe[js];
            w0 = __builtin_fmaf(p, vself[qrow + i0], w0);
            w1 = __builtin_fmaf(p, vself[qrow + i0 + 1], w1);
        }
        wp[sc * 128 + i0] = w0;
        wp[sc * 128 + i0 + 1] = w1;
    }
    __syncthreads();
    const size_t mh = (size_t)m * g.n_heads + h;
    if (t < hd) {
        float u = 0.0f;
        u = u + wp[t];
        u = u + wp[128 + t];
        u = u + wp[256 + t];
        u = u + wp[384 + t];
        Up[(mh * cstride + c) * hd + t] = u;
    }
    if (t == 0) {
        S[mh * s_stride + 2 * c] = mx;
        S[mh * s_stride + 2 * c + 1] = T;
    }
}

// 1-D grid of 8 * M * ceil(G / 8) blocks, G = H * chunks, task group
// grp = c * H + h.  Blocks are dealt to the 8 XCDs round-robin, so block b
// runs on XCD b mod 8: group grp's M rows get blocks with b mod 8 = grp mod
// 8, and after the first row a chunk's K/V rows come from that XCD's L2.
// 256 threads; head_dim = 16 * PARTS; V rows of VROW bytes in LDS.
template <int PARTS, uint32_t VROW>
__global__ __launch_bounds__(256) void k_attn_chunk(const PassDesc* __restrict__ pd, KvGeom g, KvPlanes kv,
                                                    uint32_t layer, uint32_t M, uint32_t n_groups,
                                                    const float* __restrict__ q, const float* __restrict__ kself,
                                                    const float* __restrict__ vself, float* __restrict__ S,
                                                    uint32_t s_stride, float* __restrict__ Up, uint32_t cstride) {
    __shared__ __align__(16) uint8_t smem[att_smem(VROW)];
    const uint32_t xcd = blockIdx.x & 7u, slot = blockIdx.x >> 3;
    const uint32_t grp = (slot / M) * 8u + xcd, m = slot % M;
    const PassHead ph = pass_head(pd);
    if (grp >= n_groups || m >= ph.m) return;
    attn_one_row<PARTS, VROW>(ph, g, kv, layer, m, grp % g.n_heads, grp / g.n_heads, q, kself, vself, S, s_stride,
                              Up, cstride, smem);
}

// ------------------------------------------- sequence-group attention

// LDS of k_attn_seq (bytes): K and V tiles of AS_TILE entries (the K tile
// is reused after the dots for the dots [NR][AS_TILE], the probabilities
// [NR][256] and the V partials [NR][4][128]), the tile's scales [2][AS_TILE],
// queries and self keys [NR][128] fp32 each, wave maxima and sums [2][NR][4],
// self scores and self weights [2][NR].
constexpr uint32_t AS_EXTRA = 16;                  // extra tile entries for the rows' shifts
constexpr uint32_t AS_TILE = 256 + AS_EXTRA;
constexpr uint32_t AS_NR = 5;                      // rows of one group at most
constexpr uint32_t as_smem() {
    return 2u * AS_TILE * 128u + (2u * AS_TILE + 2u * AS_NR * 128u + 8u * AS_NR + 2u * AS_NR) * 4u;
}
static_assert((AS_NR * AS_TILE + AS_NR * 256u + AS_NR * 4u * 128u) * 4u <= AS_TILE * 128u, "K tile reuse");
// Over AS_NR consecutive positions the sink count, the pooled count and the
// oldest window entry each move by at most one per position, so a row's
// shift D_r stays within the tile's extra entries.
static_assert(3u * (AS_NR - 1u) <= AS_EXTRA, "row shifts fit the tile");

// Engine attention (the first stage above) of batched passes whose rows
// come in groups of gsize (<= AS_NR) consecutive positions of one
// sequence (a batched verify pass: each sequence's n_mtp + 1 rows).  Unlike
// k_attn_group the rows' lists need not extend each other: when the window
// slides (or a pooled row completes, or the sink fills) between the rows,
// row r's list index j names a different entry than row 0's.  The block
// for (head h, chunk c, group y) therefore loads the union of the rows'
// chunk-c entries once, in a unified order: the S_max sink entries, the
// pool_max pooled rows, then the window from the first row's oldest entry
// (the counts of the group's last row are the largest).  Row r's entry j
// sits at unified index u = j + shift_r(j), shift 0 in the sink part,
// S_max - S_r in the pooled part, and D_r = (S_max - S_r) + (pool_max -
// pool_r) + (win_lo_r - win_lo_0) in the window part, so chunk c of every
// row lies in unified [256 c, 256 c + 256 + max D_r) (D_r <= 12 for 5
// consecutive positions).  Each row's arithmetic is k_attn_group's: the
// per-entry fmaf dot, the self score as a sequential mul+add, chunk max,
// exp, CANON(4) sum, and 64-entry V chains in list order (zero-weight
// terms past a row's list are left out, which changes no bit).  The K/V
// conversions of the dots are shared by the rows.  Grid (heads * chunks,
// ceil(M / gsize)), 512 threads: waves 0-4 compute the tile's dots (one
// entry per thread), wave 7 the self dots; for the softmax and V chains
// waves 0-3 serve rows 0-2 and waves 4-7 rows 3-4.
template <int PARTS>
__global__ __launch_bounds__(512) void k_attn_seq(const PassDesc* __restrict__ pd, KvGeom g, KvPlanes kv,
                                                  uint32_t layer, uint32_t M, uint32_t gsize,
                                                  const float* __restrict__ q, const float* __restrict__ kself,
                                                  const float* __restrict__ vself, float* __restrict__ S,
                                                  uint32_t s_stride, float* __restrict__ Up, uint32_t cstride) {
    constexpr uint32_t hd = 16 * PARTS, NR = AS_NR;
    __shared__ __align__(16) uint8_t smem[as_smem()];
    int4* kt = reinterpret_cast<int4*>(smem);                                // [PARTS][AS_TILE], swizzled
    int8_t (*vt)[128] = reinterpret_cast<int8_t (*)[128]>(smem + AS_TILE * 128u);
    float* ksc = reinterpret_cast<float*>(smem + 2u * AS_TILE * 128u);     // [AS_TILE]
    float* vsc = ksc + AS_TILE;                                             // [AS_TILE]
    float* qs = vsc + AS_TILE;                                              // [NR][128]
    float* kss = qs + NR * 128;                                             // [NR][128]
    float* rmx = kss + NR * 128;                                            // [NR][4]
    float* rsm = rmx + NR * 4;                                              // [NR][4]
    float* selfs = rsm + NR * 4;                                            // [NR] self dots
    float* pself = selfs + NR;                                              // [NR]
    float* dot = reinterpret_cast<float*>(smem);                            // [NR][AS_TILE], after the dots
    float* pe = dot + NR * AS_TILE;                                         // [NR][256]
    float* wp = pe + NR * 256;                                              // [NR][4][128]

    const uint32_t H = g.n_heads, h = blockIdx.x % H, c = blockIdx.x / H;
    const uint32_t t = threadIdx.x, lane = t & 63u, wid = t >> 6;
    const PassHead ph = pass_head(pd);
    const uint32_t Mp = min(M, ph.m), mb = blockIdx.y * gsize;
    if (mb >= Mp) return;
    const uint32_t G = min(min(gsize, NR), Mp - mb);
    // the rows' views (positions consecutive, so every count is nondecreasing)
    uint32_t Sr[NR], Pr[NR], Cr[NR], Dr[NR];
    const KvView v0 = kv_view(g, row_pos(ph, mb));
    const KvView vl = kv_view(g, row_pos(ph, mb + G - 1u));
    const uint32_t Smax = vl.sink, Pmax = vl.pool, wl0 = v0.win_lo;
    uint32_t Cmax = 0, Dmax = 0;
#pragma unroll
    for (uint32_t r = 0; r < NR; r++) {
        const KvView v = kv_view(g, row_pos(ph, mb + min(r, G - 1u)));
        Sr[r] = v.sink;
        Pr[r] = v.pool;
        Cr[r] = v.count();
        Dr[r] = (Smax - v.sink) + (Pmax - v.pool) + (v.win_lo - wl0);
        Cmax = max(Cmax, Cr[r]);
        Dmax = max(Dmax, Dr[r]);
    }
    const uint32_t j0 = 256u * c;
    if (j0 > Cmax) return;                                   // past every row's self entry
    const uint32_t U = Smax + Pmax + (vl.win_hi - wl0);      // unified entries
    const uint32_t ntile = U > j0 ? min(min(AS_TILE, 256u + Dmax), U - j0) : 0u;
    const uint32_t D = H * hd, seq = row_seq(ph, mb);
    const size_t plane = plane_index(g, seq, layer, h);
    const uint32_t wb0 = wl0 % g.ring;
    // physical row of unified entry u
    auto urow = [&](uint32_t u) -> uint32_t {
        if (u < Smax) return u;
        if (u < Smax + Pmax) return KV_SINK_ROWS + g.ring + (u - Smax);
        uint32_t x = wb0 + (u - Smax - Pmax);
        x = x >= g.ring ? x - g.ring : x;
        return KV_SINK_ROWS + x;
    };

    // ---- loads, all issued before any is used
    constexpr uint32_t QPT = (NR * hd + 511u) / 512u;
    float qv[QPT], kvv[QPT];
#pragma unroll
    for (uint32_t k = 0; k < QPT; k++) {
        const uint32_t i = t + 512u * k, r = i / hd, d = i - r * hd;
        qv[k] = 0.0f;
        kvv[k] = 0.0f;
        if (r < G) {
            const size_t o = (size_t)(mb + r) * D + h * hd + d;
            qv[k] = q[o];
            kvv[k] = kself[o];
        }
    }
    // K and V of the tile: 16-byte piece pi = t + 512 i is part pi % PARTS
    // of tile entry pi / PARTS
    constexpr uint32_t LPT = (AS_TILE * PARTS + 511u) / 512u;
    int4 kw[LPT], vw[LPT];
#pragma unroll
    for (uint32_t i = 0; i < LPT; i++) {
        const uint32_t pi = t + 512u * i, e = pi / PARTS, part = pi % PARTS;
        kw[i] = make_int4(0, 0, 0, 0);
        vw[i] = make_int4(0, 0, 0, 0);
        if (e < ntile) {
            const size_t row = plane * g.rows + urow(j0 + e);
            kw[i] = reinterpret_cast<const int4*>(kv.k + row * hd)[part];
            vw[i] = reinterpret_cast<const int4*>(kv.v + row * hd)[part];
        }
    }
    float ks = 0.0f, vs = 0.0f;
    if (t < ntile) {
        const size_t row = plane * g.rows + urow(j0 + t);
        ks = kv.ks[row];
        vs = kv.vs[row];
    }

    // ---- LDS
#pragma unroll
    for (uint32_t k = 0; k < QPT; k++) {
        const uint32_t i = t + 512u * k, r = i / hd, d = i - r * hd;
        if (r < NR) {
            qs[r * 128 + d] = qv[k];
            kss[r * 128 + d] = kvv[k];
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < LPT; i++) {
        const uint32_t pi = t + 512u * i, e = pi / PARTS, part = pi % PARTS;
        if (e < AS_TILE) {
            kt[part * AS_TILE + (e ^ part)] = kw[i];
            *reinterpret_cast<int4*>(&vt[e][16 * part]) = vw[i];
        }
    }
    if (t < AS_TILE) {
        ksc[t] = ks;                                         // 0 past the tile: those terms add exactly 0
        vsc[t] = vs;
    }
    __syncthreads();

    // ---- dots of tile entry t (waves 0-4) with every row's query (the
    // converted key shared by the rows); wave 7 lane r: row r's self dot
    float acc[NR];
#pragma unroll
    for (uint32_t r = 0; r < NR; r++) acc[r] = 0.0f;
    if (t < ntile) {
        const float ksv = ksc[t];
        const float* qo = lds_opaque(qs);
#pragma unroll
        for (int p = 0; p < PARTS; p++) {
            const int4 w4 = kt[p * AS_TILE + (t ^ (uint32_t)p)];
            const int wv4[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
            for (int b4 = 0; b4 < 4; b4++) {
                float qc[NR][4];
#pragma unroll
                for (uint32_t r = 0; r < NR; r++) {
                    const float4 q4 = *reinterpret_cast<const float4*>(&qo[r * 128 + p * 16 + 4 * b4]);
                    qc[r][0] = q4.x;
                    qc[r][1] = q4.y;
                    qc[r][2] = q4.z;
                    qc[r][3] = q4.w;
                }
#pragma unroll
                for (int bb = 0; bb < 4; bb++) {
                    const float kf = (float)(int8_t)((wv4[b4] >> (8 * bb)) & 0xFF) * ksv;
#pragma unroll
                    for (uint32_t r = 0; r < NR; r++) acc[r] = __builtin_fmaf(qc[r][bb], kf, acc[r]);
                }
            }
        }
    }
    {
        const uint32_t rs = wid == 7u ? lane : NR;
        if (rs < G) {
            float sd = 0.0f;
#pragma unroll 16
            for (uint32_t i = 0; i < hd; i++) sd = sd + qs[rs * 128 + i] * kss[rs * 128 + i];
            selfs[rs] = sd;
        }
    }
    __syncthreads();                                         // the K tile is read; dot reuses it
    if (t < AS_TILE)
#pragma unroll
        for (uint32_t r = 0; r < NR; r++) dot[r * AS_TILE + t] = acc[r];
    __syncthreads();

    // ---- per row: scores by list index j = j0 + tt, chunk max, exp and the
    // CANON(4) chunk sum; waves 0-3 serve rows 0-2, waves 4-7 rows 3-4
    // (wave w & 3 holds list indices 64 (w & 3) ..)
    const float scale = 1.0f / __builtin_sqrtf((float)hd);
    const uint32_t half = wid >> 2, tt = t & 255u, wq = wid & 3u;
    const uint32_t j = j0 + tt;
    float sc[NR];
#pragma unroll
    for (uint32_t r = 0; r < NR; r++) {
        sc[r] = -__builtin_inff();
        if ((r >= 3u ? 1u : 0u) != half) continue;
        if (r < G) {
            if (j < Cr[r]) {
                const uint32_t sh = j < Sr[r] ? 0u : (j < Sr[r] + Pr[r] ? Smax - Sr[r] : Dr[r]);
                sc[r] = dot[r * AS_TILE + tt + sh] * scale;
            } else if (j == Cr[r]) {
                sc[r] = selfs[r] * scale;
            }
        }
        const float w = wave_max(sc[r]);
        if (lane == 0) rmx[r * 4 + wq] = w;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t r = 0; r < NR; r++) {
        if ((r >= 3u ? 1u : 0u) != half) continue;
        const float* rr = rmx + r * 4;
        const float mx = fmaxf(fmaxf(rr[0], rr[1]), fmaxf(rr[2], rr[3]));
        const bool in = r < G && j <= Cr[r];
        const float ex = in ? expf_c(sc[r] - mx) : 0.0f;
        pe[r * 256 + tt] = r < G && j < Cr[r] ? ex : 0.0f;
        if (in && j == Cr[r]) pself[r] = ex;
        const float w = wave_tree_sum(ex);
        if (lane == 0) rsm[r * 4 + wq] = w;
    }
    __syncthreads();

    // ---- V: per row and 64-entry sub-chunk an fmaf chain in list order
    // (entries in groups of 8, the rows' chains interleaved; entries past a
    // row's list up to the next multiple of 8 have weight 0 and read finite
    // tile values, so fmaf(0, a, w) == w)
    const uint32_t sub = wq, i0 = 2u * lane;
    if (i0 < hd) {
        float w0[NR], w1[NR];
        uint32_t e_end[NR], b1[NR], b2[NR];
        uint32_t e_max = 64u * sub;
#pragma unroll
        for (uint32_t r = 0; r < NR; r++) {
            w0[r] = 0.0f;
            w1[r] = 0.0f;
            const bool mine = (r >= 3u ? 1u : 0u) == half;
            const uint32_t nvis = mine && r < G && j0 < Cr[r] ? min(256u, Cr[r] - j0) : 0u;
            e_end[r] = min(64u * sub + 64u, (nvis + 7u) & ~7u);
            e_max = max(e_max, e_end[r]);
            b1[r] = Sr[r] > j0 ? Sr[r] - j0 : 0u;                    // first pooled offset
            b2[r] = Sr[r] + Pr[r] > j0 ? Sr[r] + Pr[r] - j0 : 0u;    // first window offset
        }
        // rows whose chunk lies in the window part with shift D_r = r (the
        // window sliding by one entry per row, no pooled row completed in
        // the group) read slots e + u + r: the conversions of slots e ..
        // are shared by the rows
        bool fast = true;
#pragma unroll
        for (uint32_t r = 0; r < NR; r++)
            if (r < G && (r >= 3u ? 1u : 0u) == half) fast = fast && Dr[r] == r && b2[r] == 0u;
#define PF_ATTN_SEQ_VFAST(R0, NRH)                                                                         \
    for (uint32_t e = 64u * sub; e < e_max; e += 8) {                                                      \
        float a0[8 + NRH - 1], a1[8 + NRH - 1];                                                            \
        _Pragma("unroll") for (uint32_t k = 0; k < 8u + NRH - 1u; k++) {                                   \
            const uint32_t sl = e + R0 + k;                                                                \
            const uint32_t cc = *reinterpret_cast<const uint16_t*>(&vt[sl][i0]);                           \
            const float vv = vsc[sl];                                                                      \
            a0[k] = (float)(int8_t)(cc & 0xFFu) * vv;                                                      \
            a1[k] = (float)(int8_t)(cc >> 8) * vv;                                                         \
        }                                                                                                  \
        _Pragma("unroll") for (uint32_t rr = 0; rr < NRH; rr++) {                                          \
            const uint32_t r = R0 + rr;                                                                    \
            if (e >= e_end[r]) continue;                                                                   \
            const float4 p0 = *reinterpret_cast<const float4*>(&pe[r * 256 + e]);                          \
            const float4 p1 = *reinterpret_cast<const float4*>(&pe[r * 256 + e + 4]);                      \
            const float pp[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};                          \
            _Pragma("unroll") for (uint32_t u = 0; u < 8; u++) {                                           \
                w0[r] = __builtin_fmaf(pp[u], a0[u + rr], w0[r]);                                          \
                w1[r] = __builtin_fmaf(pp[u], a1[u + rr], w1[r]);                                          \
            }                                                                                              \
        }                                                                                                  \
    }
        if (fast && half == 0u) {
            PF_ATTN_SEQ_VFAST(0u, 3u)
        } else if (fast) {
            PF_ATTN_SEQ_VFAST(3u, 2u)
        } else
        for (uint32_t e = 64u * sub; e < e_max; e += 8) {
#pragma unroll
            for (uint32_t r = 0; r < NR; r++) {
                if (e >= e_end[r]) continue;
                uint32_t sl[8];
                if (e >= b2[r]) {
#pragma unroll
                    for (int u = 0; u < 8; u++) sl[u] = e + u + Dr[r];
                } else {
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        const uint32_t x = e + u;
                        sl[u] = x + (x < b1[r] ? 0u : (x < b2[r] ? Smax - Sr[r] : Dr[r]));
                    }
                }
                float vv[8];
                uint32_t cc[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    cc[u] = *reinterpret_cast<const uint16_t*>(&vt[sl[u]][i0]);
                    vv[u] = vsc[sl[u]];
                }
                const float4 p0 = *reinterpret_cast<const float4*>(&pe[r * 256 + e]);
                const float4 p1 = *reinterpret_cast<const float4*>(&pe[r * 256 + e + 4]);
                const float pp[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    w0[r] = __builtin_fmaf(pp[u], (float)(int8_t)(cc[u] & 0xFFu) * vv[u], w0[r]);
                    w1[r] = __builtin_fmaf(pp[u], (float)(int8_t)(cc[u] >> 8) * vv[u], w1[r]);
                }
            }
        }
#pragma unroll
        for (uint32_t r = 0; r < NR; r++) {
            if (r >= G) break;
            if ((r >= 3u ? 1u : 0u) != half) continue;
            const uint32_t js = Cr[r] - j0;                  // the row's self entry in the chunk
            if (js < 256u && (js >> 6) == sub) {
                const float ps = pself[r];
                const size_t o = (size_t)(mb + r) * D + h * hd + i0;
                w0[r] = __builtin_fmaf(ps, vself[o], w0[r]);
                w1[r] = __builtin_fmaf(ps, vself[o + 1], w1[r]);
            }
            wp[(r * 4 + sub) * 128 + i0] = w0[r];
            wp[(r * 4 + sub) * 128 + i0 + 1] = w1[r];
        }
#undef PF_ATTN_SEQ_VFAST
    }
    __syncthreads();
    // ---- outputs of the rows whose list reaches this chunk
    for (uint32_t i = t; i < G * hd; i += 512u) {
        const uint32_t r = i / hd, d = i - r * hd;
        if (j0 > Cr[r]) continue;
        const size_t mh = (size_t)(mb + r) * H + h;
        float u = 0.0f;
        u = u + wp[(r * 4 + 0) * 128 + d];
        u = u + wp[(r * 4 + 1) * 128 + d];
        u = u + wp[(r * 4 + 2) * 128 + d];
        u = u + wp[(r * 4 + 3) * 128 + d];
        Up[(mh * cstride + c) * hd + d] = u;
    }
    if (t < G && j0 <= Cr[t]) {
        const float* mm = rmx + t * 4;
        const float* ss = rsm + t * 4;
        const size_t mh = (size_t)(mb + t) * H + h;
        S[mh * s_stride + 2 * c] = fmaxf(fmaxf(mm[0], mm[1]), fmaxf(mm[2], mm[3]));
        S[mh * s_stride + 2 * c + 1] = (ss[0] + ss[2]) + (ss[1] + ss[3]);   // CANON(4) over the wave totals
    }
}

// ------------------------------------------------- grouped attention

// Rows b = a + 1 of one sequence whose lists extend each other: b sees a's
// entries plus one more, the store of a's position (same sink and pooled
// counts, same oldest window entry).  Chunk c then holds the same entries
// for both, so one block serves both rows.
__device__ __forceinline__ bool rows_aligned(const KvGeom& g, const PassHead& pd, uint32_t a, uint32_t b) {
    if (row_seq(pd, a) != row_seq(pd, b)) return false;
    const uint32_t pa = row_pos(pd, a), pb = row_pos(pd, b);
    if (pb != pa + 1u) return false;
    // kv_view without the pooled count (equal win_lo gives equal counts)
    const uint32_t s_eff = min(g.sink_size, KV_SINK_ROWS);
    const uint32_t na = min(pa, g.max_context), nb = min(pb, g.max_context);
    const uint32_t wa = na > g.sink_size ? na - g.sink_size : 0u, wb = nb > g.sink_size ? nb - g.sink_size : 0u;
    const uint32_t la = wa > g.window ? wa - g.window : 0u, lb = wb > g.window ? wb - g.window : 0u;
    return min(na, s_eff) == min(nb, s_eff) && la == lb && wb == wa + 1u;
}

// Position of visible entry j of a view (sink slot j holds position j,
// window entry w position sink_size + w); pooled rows have none (UINT32_MAX).
__device__ __forceinline__ uint32_t entry_pos(const KvGeom& g, const KvView& v, uint32_t j) {
    if (j < v.sink) return j;
    j -= v.sink;
    if (j < v.pool) return 0xFFFFFFFFu;
    return g.sink_size + v.win_lo + (j - v.pool);
}

// List index of position P in view v, or UINT32_MAX when v does not show it.
__device__ __forceinline__ uint32_t list_index(const KvGeom& g, const KvView& v, uint32_t P) {
    if (P < g.sink_size) return P < v.sink ? P : 0xFFFFFFFFu;
    const uint32_t w = P - g.sink_size;
    if (w < v.win_lo || w >= v.win_hi) return 0xFFFFFFFFu;
    return v.sink + v.pool + (w - v.win_lo);
}

// kv_row for the entries j >= wstart of one chunk, wstart = max(j0,
// sink + pool) and wb = kv_row's ring index of entry wstart (one division
// per block instead of one per entry).
__device__ __forceinline__ uint32_t chunk_row(const KvGeom& g, const KvView& v, uint32_t j, uint32_t wstart,
                                              uint32_t wb) {
    if (j < v.sink) return j;
    if (j < wstart) return KV_SINK_ROWS + g.ring + (j - v.sink);
    uint32_t x = wb + (j - wstart);
    x = g.ring >= 256u ? (x >= g.ring ? x - g.ring : x) : x % g.ring;
    return KV_SINK_ROWS + x;
}

constexpr uint32_t AG_MAX_ROWS = 8;   // rows of one attention group

// LDS of k_attn_group (bytes): K and V rows of the chunk, 32 KB each, their
// scales [2][256], the group's queries and self keys [NR][128] fp32 each,
// probabilities [NR][256], wave maxima and sums [2][NR][4], self weights
// [NR].  The V partials [NR][4][128] reuse the K rows.  K is stored by
// 16-byte part: part p of entry e at slot p * 256 + (e ^ p), so that the
// 8 lanes writing one row and the lanes reading part p of consecutive rows
// both fall on distinct banks.  V rows are plain [256][128].
constexpr uint32_t ag_smem(uint32_t nr) { return 2u * 256u * 128u + (512u + nr * (256u + 256u + 8u + 1u)) * 4u; }
// With the rows' q/k/v taken from LL words, their self values [NR][128]
// follow (the V stage reads them from LDS).
constexpr uint32_t ag_smem_ll(uint32_t nr) { return ag_smem(nr) + nr * 128u * 4u; }

// Engine attention of every row of a pass (the first stage above), one
// block per (head h, 256-entry chunk c, share of a group of rows), with the
// chunk's K and V rows loaded once, coalesced, into LDS for all the rows
// the block serves.
//
// Groups are the runs of aligned rows inside each 8-row slice of the pass
// (rows 8s .. 8s + 7); the lists of a group's rows are prefixes of its last
// row's list: row r of the group sees C + r entries (C the count of its
// first row), then its fp32 self entry at list index C + r.  A group of n
// rows is served by ceil(n / NR) blocks of at most NR rows each.
// Grid (heads * chunks, M), 512 threads (waves 4-7 join only the V chains,
// one element each): block (x, m) serves share
// m - m0 of the group led by row m0 (if that share exists).  With pf.p set
// the grid has one more row of blocks, which load pf's groups (the next
// kernel's weights) into the L2 of the XCDs that will read them instead.
//
// FUSED (passes of at most 8 rows): the pass's own K/V rows are not yet in
// the cache.  Entries at positions of this pass are quantized here from the
// fp32 k / v rows (KVCache::quantize_row arithmetic, as store_pair), and the
// block whose chunk holds row r's self entry writes row r's K/V to the
// cache (src/kv_cache.cpp:59-127).  The ring's slack keeps those rows out
// of every list of the pass, so blocks still reading other chunks never see
// them change.  Otherwise k_kv_store_pass has stored the pass's rows.
//
// LL: the pass's q/k/v rows come from LL words written by the QKV
// workgroups of the same launch (k_qkv_attn); the cached K/V rows, which do
// not depend on them, are loaded first.  attn_group_body is block (bx, by)
// of a grid gx wide, linear workgroup id lin.
template <int PARTS, bool FUSED, int NR, bool LL>
__device__ __forceinline__ void attn_group_body(const PassDesc* __restrict__ pd, const KvGeom& g, const KvPlanes& kv,
                                                uint32_t layer, uint32_t M, const float* __restrict__ q,
                                                const float* __restrict__ kself, const float* __restrict__ vself,
                                                float* __restrict__ S, uint32_t s_stride, float* __restrict__ Up,
                                                uint32_t cstride, const Prefetch& pf, const LLIn& lli, uint32_t bx,
                                                uint32_t by, uint32_t lin, uint32_t gx, uint8_t* smem) {
    constexpr uint32_t hd = 16 * PARTS;
    if (by >= M) {
        prefetch_groups(pf, lin, bx, gx);
        return;
    }
    const uint32_t epoch = LL ? ll_epoch(lli.ep) : 0u;
    int4* kt = reinterpret_cast<int4*>(smem);                       // [PARTS][256], swizzled
    int8_t (*vt)[128] = reinterpret_cast<int8_t (*)[128]>(smem + 256u * 128u);
    float* ksc = reinterpret_cast<float*>(smem + 512u * 128u);      // [256]
    float* vsc = ksc + 256;                                         // [256]
    float* qs = vsc + 256;                                          // [NR][128]
    float* kss = qs + NR * 128;                                     // [NR][128]
    float* pe = kss + NR * 128;                                     // [NR][256]
    float* rmx = pe + NR * 256;                                     // [NR][4] wave maxima
    float* rsm = rmx + NR * 4;                                      // [NR][4] wave sums
    float* pself = rsm + NR * 4;                                    // [NR]
    float* vss = pself + NR;                                        // LL: [NR][128] self values
    float* wp = reinterpret_cast<float*>(smem);                     // [NR][4][128], after the scores

    const uint32_t H = g.n_heads, h = bx % H, c = bx / H, m0 = by;
    const uint32_t t = threadIdx.x, lane = t & 63u, wid = t >> 6;
    const bool hi = t >= 256u;   // waves 4-7 join the V chains only
    const PassHead ph = pass_head(pd);
    const uint32_t Mp = min(M, ph.m);
    if (m0 >= Mp) return;
    // lane l < 8: row base + l starts a group (not aligned with row base + l - 1)
    const uint32_t base = m0 & ~7u;
    bool st = true;
    if (lane >= 1u && lane < 8u && base + lane < Mp) st = !rows_aligned(g, ph, base + lane - 1u, base + lane);
    const uint32_t starts = (uint32_t)__ballot(st) & 0xFFu;
    const uint32_t k = m0 - base;                                   // this block's row in the slice
    const uint32_t lead = 31u - (uint32_t)__builtin_clz(starts & ((2u << k) - 1u));
    const uint32_t after = starts & ~((2u << lead) - 1u);           // starts of the later groups
    const uint32_t glen = min(after ? (uint32_t)__builtin_ctz(after) : 8u, Mp - base) - lead;
    const uint32_t nsh = (glen + NR - 1u) / NR, share = k - lead;
    if (share >= nsh) return;                                       // no share for this block
    const uint32_t per = (glen + nsh - 1u) / nsh;
    const uint32_t mb = base + lead + share * per;                  // first row of this block
    const uint32_t G = min(per, glen - share * per);
    const KvView vL = kv_view(g, row_pos(ph, mb + G - 1u));         // the longest list
    const uint32_t CL = vL.count(), C0 = CL - (G - 1u), j0 = 256u * c;
    if (j0 > CL) return;                                            // past the last row's self entry
    const uint32_t D = H * hd, seq = row_seq(ph, mb);
    const size_t plane = plane_index(g, seq, layer, h);
    const uint32_t nvis = j0 < CL ? min(256u, CL - j0) : 0u;
    const uint32_t wstart = max(j0, vL.sink + vL.pool), wb = (vL.win_lo + (wstart - vL.sink - vL.pool)) % g.ring;
    // FUSED: the sequence's first row in the pass; entries at its position
    // or later are the pass's own rows
    uint32_t first = mb, p_first = 0xFFFFFFFFu;
    if constexpr (FUSED) {
        while (first > 0 && row_seq(ph, first - 1u) == seq) first--;
        p_first = row_pos(ph, first);
    }

    // ---- loads, all issued before any is used
    // the group's queries and self keys: element i = t + 256 k of [NR][hd]
    constexpr uint32_t QPT = (NR * hd + 255u) / 256u;
    float qv[QPT], kvv[QPT], vvv[QPT];
#pragma unroll
    for (uint32_t k = 0; k < QPT; k++) {
        const uint32_t i = t + 256u * k, r = i / hd, d = i - r * hd;
        qv[k] = 0.0f;
        kvv[k] = 0.0f;
        vvv[k] = 0.0f;
        if (!LL && !hi && r < G) {
            const size_t o = (size_t)(mb + r) * D + h * hd + d;
            qv[k] = q[o];
            kvv[k] = kself[o];
        }
    }
    // FUSED: wave w quantizes pass rows first + w and first + w + 4 (at most
    // 8 rows in the pass), two elements per lane
    const uint32_t nq = FUSED ? mb + G - first : 0u;
    float fk[2][2], fv[2][2];
#pragma unroll
    for (uint32_t u = 0; u < 2; u++) {
        const uint32_t i = wid + 4u * u;
        fk[u][0] = fk[u][1] = fv[u][0] = fv[u][1] = 0.0f;
        if (!LL && !hi && i < nq && 2u * lane < hd) {
            const size_t o = (size_t)(first + i) * D + h * hd + 2u * lane;
            fk[u][0] = kself[o];
            fk[u][1] = kself[o + 1];
            fv[u][0] = vself[o];
            fv[u][1] = vself[o + 1];
        }
    }
    // K and V rows: 16-byte piece pi = t + 256 i is part pi % PARTS of
    // entry pi / PARTS, so a wave reads 64 / PARTS whole rows per load
    // (waves 0-3 only).  Every load of a wave is issued unconditionally:
    // list index j0 + e past the visible entries still names a valid row of
    // the plane (chunk_row stays inside the sink, pooled or ring rows), and
    // the staging below keeps only the entries it needs, so no wait
    // separates the loads.
    if constexpr (LL) {
        if (lli.gate) {   // the K/V loads wait for an earlier stage's word
            const uint32_t go[1] = {lli.gate_off};
            float gv[1];
            if (wid == 0) ll_wait<1>(lli.gate, go, gv, epoch * lli.fmul + lli.fadd - lli.gate_back, lli.err);
            __syncthreads();
        }
    }
    int4 kw[PARTS], vw[PARTS];
#pragma unroll
    for (uint32_t i = 0; i < (uint32_t)PARTS; i++) kw[i] = vw[i] = make_int4(0, 0, 0, 0);
    float ks = 0.0f, vs = 0.0f;
    bool pend = false;
    if (!hi) {
#pragma unroll
        for (uint32_t i = 0; i < (uint32_t)PARTS; i++) {
            const uint32_t pi = t + 256u * i, e = pi / PARTS, part = pi % PARTS;
            const size_t row = plane * g.rows + chunk_row(g, vL, j0 + e, wstart, wb);
            kw[i] = reinterpret_cast<const int4*>(kv.k + row * hd)[part];
            vw[i] = reinterpret_cast<const int4*>(kv.v + row * hd)[part];
        }
        const uint32_t pos = FUSED ? entry_pos(g, vL, j0 + t) : 0xFFFFFFFFu;
        pend = t < nvis && pos != 0xFFFFFFFFu && pos >= p_first;
        const size_t row = plane * g.rows + chunk_row(g, vL, j0 + t, wstart, wb);
        ks = kv.ks[row];
        vs = kv.vs[row];
    }
    // the cached rows into LDS (pass rows quantized here take other slots)
    auto stage_cached = [&]() {
#pragma unroll
        for (uint32_t i = 0; i < (uint32_t)PARTS; i++) {
            const uint32_t pi = t + 256u * i, e = pi / PARTS, part = pi % PARTS;
            if (!hi && e < nvis) {
                const uint32_t pos = FUSED ? entry_pos(g, vL, j0 + e) : 0xFFFFFFFFu;
                if (pos == 0xFFFFFFFFu || pos < p_first) {
                    kt[part * 256u + (e ^ part)] = kw[i];
                    *reinterpret_cast<int4*>(&vt[e][16 * part]) = vw[i];
                }
            }
        }
        if (!hi && !pend) {               // 0 past the visible entries: their terms below add exactly 0
            ksc[t] = t < nvis ? ks : 0.0f;
            vsc[t] = t < nvis ? vs : 0.0f;
        }
    };
    if constexpr (LL) {
        // staged before the wait, so that no register holds them meanwhile
        stage_cached();
        // the rows' q, self k and self v (element i = t + 256 k of [G][hd]),
        // and for FUSED the k / v of pass rows first + w, first + w + 4
        // (elements 2 lane, 2 lane + 1), once their QKV workgroups wrote them
        constexpr int NW = 3 * (int)QPT + 8;
        uint32_t wa[NW];
        float wv_[NW];
        const uint32_t rs3 = 3u * D;
#pragma unroll
        for (uint32_t k = 0; k < QPT; k++) {
            const uint32_t i = t + 256u * k, r = i / hd, d = i - r * hd;
            const bool use = !hi && r < G;
            const uint32_t b = (mb + r) * rs3 + h * hd + d;
            wa[3 * k] = use ? b : LL_NONE;
            wa[3 * k + 1] = use ? b + D : LL_NONE;
            wa[3 * k + 2] = use ? b + 2u * D : LL_NONE;
        }
#pragma unroll
        for (uint32_t u = 0; u < 2; u++) {
            const uint32_t i = wid + 4u * u;
            const bool use = !hi && i < nq && 2u * lane < hd;
            const uint32_t b = (first + i) * rs3 + D + h * hd + 2u * lane;
            wa[3 * QPT + 4 * u] = use ? b : LL_NONE;
            wa[3 * QPT + 4 * u + 1] = use ? b + 1u : LL_NONE;
            wa[3 * QPT + 4 * u + 2] = use ? b + D : LL_NONE;
            wa[3 * QPT + 4 * u + 3] = use ? b + D + 1u : LL_NONE;
        }
        // wave 0 first waits for one word of the head's v rows (every lane
        // loads the same word: one request per round) while the other waves
        // wait at a barrier, so that the block does not keep the memory
        // system busy with its polls; then each wave waits for its own words
        const uint32_t flag = epoch * lli.fmul + lli.fadd;
        const uint32_t sp[1] = {mb * rs3 + 2u * D + h * hd + hd - 1u};
        float sv_[1];
        if (wid == 0) ll_wait<1>(lli.ll, sp, sv_, flag, lli.err);
        __syncthreads();
        ll_wait<NW>(lli.ll, wa, wv_, flag, lli.err);
#pragma unroll
        for (uint32_t k = 0; k < QPT; k++) {
            qv[k] = wv_[3 * k];
            kvv[k] = wv_[3 * k + 1];
            vvv[k] = wv_[3 * k + 2];
        }
#pragma unroll
        for (uint32_t u = 0; u < 2; u++) {
            fk[u][0] = wv_[3 * QPT + 4 * u];
            fk[u][1] = wv_[3 * QPT + 4 * u + 1];
            fv[u][0] = wv_[3 * QPT + 4 * u + 2];
            fv[u][1] = wv_[3 * QPT + 4 * u + 3];
        }
    }

    // ---- LDS: queries, self keys, pass rows quantized here, cached rows
#pragma unroll
    for (uint32_t k = 0; k < QPT; k++) {
        const uint32_t i = t + 256u * k, r = i / hd, d = i - r * hd;
        if (!hi && r < (uint32_t)NR) {
            qs[r * 128 + d] = qv[k];
            kss[r * 128 + d] = kvv[k];
            if (LL) vss[r * 128 + d] = vvv[k];
        }
    }
    if constexpr (FUSED) {
#pragma unroll
        for (uint32_t u = 0; u < 2; u++) {
            const uint32_t i = wid + 4u * u;
            if (hi || i >= nq) continue;
            const float ak = wave_max(fmaxf(fabsf(fk[u][0]), fabsf(fk[u][1])));
            const float av = wave_max(fmaxf(fabsf(fv[u][0]), fabsf(fv[u][1])));
            const float ik = ak == 0.0f ? 1.0f : 127.0f / ak, iv = av == 0.0f ? 1.0f : 127.0f / av;
            const float sk = ak == 0.0f ? 1.0f : ak / 127.0f, sv = av == 0.0f ? 1.0f : av / 127.0f;
            const uint16_t ck = (uint16_t)(uint8_t)quant_code(fk[u][0], ik) |
                                (uint16_t)((uint16_t)(uint8_t)quant_code(fk[u][1], ik) << 8);
            const uint16_t cv = (uint16_t)(uint8_t)quant_code(fv[u][0], iv) |
                                (uint16_t)((uint16_t)(uint8_t)quant_code(fv[u][1], iv) << 8);
            const uint32_t P = p_first + i;
            // an entry of this chunk for the group's later rows
            const uint32_t jl = list_index(g, vL, P) - j0;
            if (jl < nvis) {
                if (2u * lane < hd) {
                    const uint32_t pp = lane >> 3;
                    *reinterpret_cast<uint16_t*>(reinterpret_cast<int8_t*>(&kt[pp * 256u + (jl ^ pp)]) +
                                                 2u * (lane & 7u)) = ck;
                    *reinterpret_cast<uint16_t*>(&vt[jl][2 * lane]) = cv;
                }
                if (lane == 0) {
                    ksc[jl] = sk;
                    vsc[jl] = sv;
                }
            }
            // the store of a group row whose self entry is in this chunk
            const uint32_t r = first + i - mb;
            if (r < G && C0 + r - j0 < 256u) {
                const uint32_t dst = kv_store_row(g, P);
                if (dst != 0xFFFFFFFFu) {
                    const size_t base = (plane * g.rows + dst) * hd;
                    if (2u * lane < hd) {
                        *reinterpret_cast<uint16_t*>(kv.k + base + 2u * lane) = ck;
                        *reinterpret_cast<uint16_t*>(kv.v + base + 2u * lane) = cv;
                    }
                    if (lane == 0) {
                        kv.ks[plane * g.rows + dst] = sk;
                        kv.vs[plane * g.rows + dst] = sv;
                    }
                }
            }
        }
    }
    if constexpr (!LL) stage_cached();
    __syncthreads();

    // ---- scores: per row an fmaf chain over the converted key
    const uint32_t j = j0 + t;
    const float scale = 1.0f / __builtin_sqrtf((float)hd);
    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) acc[r] = 0.0f;
    if (t < nvis) {
        // part p + 1's key words and query elements are read from LDS while
        // part p's fmaf steps run (the order of the steps is unchanged)
        const float ksv = ksc[t];
        int4 wn = kt[t];
        const float* qo = lds_opaque(qs);
        float4 qn[NR][4];
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) qn[r][i] = *reinterpret_cast<const float4*>(&qo[r * 128 + 4 * i]);
#pragma unroll
        for (int p = 0; p < PARTS; p++) {
            const int4 w4 = wn;
            float qc[NR][16];
#pragma unroll
            for (int r = 0; r < NR; r++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    qc[r][4 * i] = qn[r][i].x;
                    qc[r][4 * i + 1] = qn[r][i].y;
                    qc[r][4 * i + 2] = qn[r][i].z;
                    qc[r][4 * i + 3] = qn[r][i].w;
                }
            if (p + 1 < PARTS) {
                wn = kt[(p + 1) * 256u + (t ^ (uint32_t)(p + 1))];
#pragma unroll
                for (int r = 0; r < NR; r++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        qn[r][i] = *reinterpret_cast<const float4*>(&qo[r * 128 + (p + 1) * 16 + 4 * i]);
            }
            const int wv4[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
            for (int b = 0; b < 16; b++) {
                const float kf = (float)(int8_t)((wv4[b >> 2] >> (8 * (b & 3))) & 0xFF) * ksv;
#pragma unroll
                for (int r = 0; r < NR; r++) acc[r] = __builtin_fmaf(qc[r][b], kf, acc[r]);
            }
        }
    }
    // the self score of row j - C0, when this thread holds that row's self entry
    float selfd = 0.0f;
    const uint32_t rs = j - C0;
    if (!hi && rs < G) {
#pragma unroll 16
        for (uint32_t i = 0; i < hd; i++) selfd = selfd + qs[rs * 128 + i] * kss[rs * 128 + i];
    }
    float sc[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const uint32_t Cr = C0 + r;
        sc[r] = -__builtin_inff();
        if ((uint32_t)r < G) sc[r] = j < Cr ? acc[r] * scale : (j == Cr ? selfd * scale : -__builtin_inff());
    }
    // ---- chunk max, exp and CANON(4) chunk sum per row
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const float w = wave_max(sc[r]);
        if (!hi && lane == 0) rmx[r * 4 + wid] = w;
    }
    __syncthreads();
    float ex[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const float* rr = rmx + r * 4;
        const float mx = fmaxf(fmaxf(rr[0], rr[1]), fmaxf(rr[2], rr[3]));
        const bool in = !hi && (uint32_t)r < G && j <= C0 + r;
        ex[r] = in ? expf_c(sc[r] - mx) : 0.0f;
        // the V chains take cached and pending entries; the self term is added apart
        if (!hi) pe[r * 256 + t] = j < C0 + r ? ex[r] : 0.0f;
        if (in && j == C0 + r) pself[r] = ex[r];
        const float w = wave_tree_sum(ex[r]);
        if (!hi && lane == 0) rsm[r * 4 + wid] = w;
    }
    __syncthreads();
    // ---- V: per row and 64-entry sub-chunk an fmaf chain; wave w takes
    // sub-chunk w & 3 and element lane + 64 (w >> 2) of every row
    const uint32_t sub = wid & 3u, iv = lane + 64u * (wid >> 2);
    if (iv < hd) {
        float w0[NR];
#pragma unroll
        for (int r = 0; r < NR; r++) w0[r] = 0.0f;
        // entries [64 sub, min(64 sub + 64, nvis)) in groups of 8; entries
        // past nvis up to the next multiple of 8 have v_scale 0 and finite
        // codes, and entries past a row's list have weight 0
        const uint32_t e_end = min(64u * sub + 64u, (nvis + 7u) & ~7u);   // both multiples of 8
        // the next group's scales, codes and weights are read from LDS while
        // the current group's fmaf steps run (the order of the steps is
        // unchanged; a group past e_end reads in-bounds slots it never uses)
        float4 ns0, ns1, np0[NR], np1[NR];
        int nb[8];
        auto load_group = [&](uint32_t e) {
            ns0 = *reinterpret_cast<const float4*>(&vsc[e]);
            ns1 = *reinterpret_cast<const float4*>(&vsc[e + 4]);
#pragma unroll
            for (int u = 0; u < 8; u++) nb[u] = vt[e + u][iv];
#pragma unroll
            for (int r = 0; r < NR; r++) {
                np0[r] = *reinterpret_cast<const float4*>(&pe[r * 256 + e]);
                np1[r] = *reinterpret_cast<const float4*>(&pe[r * 256 + e + 4]);
            }
        };
        load_group(min(64u * sub, 248u));
        for (uint32_t e = 64u * sub; e < e_end; e += 8) {
            const float vv[8] = {ns0.x, ns0.y, ns0.z, ns0.w, ns1.x, ns1.y, ns1.z, ns1.w};
            int cb[8];
#pragma unroll
            for (int u = 0; u < 8; u++) cb[u] = nb[u];
            float pc[NR][8];
#pragma unroll
            for (int r = 0; r < NR; r++) {
                pc[r][0] = np0[r].x; pc[r][1] = np0[r].y; pc[r][2] = np0[r].z; pc[r][3] = np0[r].w;
                pc[r][4] = np1[r].x; pc[r][5] = np1[r].y; pc[r][6] = np1[r].z; pc[r][7] = np1[r].w;
            }
            load_group(min(e + 8u, 248u));
            float a0[8];
#pragma unroll
            for (int u = 0; u < 8; u++) a0[u] = (float)cb[u] * vv[u];
#pragma unroll
            for (int r = 0; r < NR; r++)
#pragma unroll
                for (int u = 0; u < 8; u++) w0[r] = __builtin_fmaf(pc[r][u], a0[u], w0[r]);
        }
#pragma unroll
        for (int r = 0; r < NR; r++) {
            if ((uint32_t)r >= G) continue;
            const uint32_t js = C0 + r - j0;          // row r's self entry in the chunk
            if (js < 256u && (js >> 6) == sub) {
                const float ps = pself[r];
                const size_t o = (size_t)(mb + r) * D + h * hd + iv;
                w0[r] = __builtin_fmaf(ps, LL ? vss[r * 128 + iv] : vself[o], w0[r]);
            }
            wp[(r * 4 + sub) * 128 + iv] = w0[r];
        }
    }
    __syncthreads();
    // ---- outputs of the rows whose list reaches this chunk
    for (uint32_t i = t; i < G * hd; i += 512u) {
        const uint32_t r = i / hd, d = i - r * hd;
        if (j0 > C0 + r) continue;
        const size_t mh = (size_t)(mb + r) * H + h;
        float u = 0.0f;
        u = u + wp[(r * 4 + 0) * 128 + d];
        u = u + wp[(r * 4 + 1) * 128 + d];
        u = u + wp[(r * 4 + 2) * 128 + d];
        u = u + wp[(r * 4 + 3) * 128 + d];
        if (LL && lli.out) ll_store(lli.out + lli.sreg + (mh * cstride + c) * hd + d, u, epoch * lli.fmul + lli.fadd);
        else Up[(mh * cstride + c) * hd + d] = u;
    }
    if (t < G && j0 <= C0 + t) {
        const float* mm = rmx + t * 4;
        const float* ss = rsm + t * 4;
        const size_t mh = (size_t)(mb + t) * H + h;
        const float smx = fmaxf(fmaxf(mm[0], mm[1]), fmaxf(mm[2], mm[3]));
        const float ssm = (ss[0] + ss[2]) + (ss[1] + ss[3]);   // CANON(4) over the wave totals
        if (LL && lli.out) {
            const uint32_t flag = epoch * lli.fmul + lli.fadd;
            ll_store(lli.out + mh * s_stride + 2 * c, smx, flag);
            ll_store(lli.out + mh * s_stride + 2 * c + 1, ssm, flag);
        } else {
            S[mh * s_stride + 2 * c] = smx;
            S[mh * s_stride + 2 * c + 1] = ssm;
        }
    }
}

template <int PARTS, bool FUSED, int NR>
__global__ __launch_bounds__(512) void k_attn_group(const PassDesc* __restrict__ pd, KvGeom g, KvPlanes kv,
                                                    uint32_t layer, uint32_t M, const float* __restrict__ q,
                                                    const float* __restrict__ kself, const float* __restrict__ vself,
                                                    float* __restrict__ S, uint32_t s_stride,
                                                    float* __restrict__ Up, uint32_t cstride, Prefetch pf) {
    __shared__ __align__(16) uint8_t smem[ag_smem(NR)];
    attn_group_body<PARTS, FUSED, NR, false>(pd, g, kv, layer, M, q, kself, vself, S, s_stride, Up, cstride, pf,
                                             LLIn{}, blockIdx.x, blockIdx.y, blockIdx.x + blockIdx.y * gridDim.x,
                                             gridDim.x, smem);
}

// Engine attention, second stage: the chunks of (row m, head h) merged left
// to right with f_c = exp(m_c - max_c m_c): T = fmaf(T_c, f_c, T),
// U = fmaf(U_c, f_c, U), out = U * (1 / (T + 1e-10)) (the softmax
// normalisation of src/matmul_neon.cpp:212-226 applied after the weighted
// sum; each head writes its own slice, src/engine.cpp:771-778).
// Grid (M, H), 128 threads.
__global__ __launch_bounds__(128) void k_attn_merge_chunks(const PassDesc* __restrict__ pd, KvGeom g,
                                                           const float* __restrict__ S, uint32_t s_stride,
                                                           const float* __restrict__ Up, uint32_t cstride,
                                                           float* __restrict__ out) {
    __shared__ float fs[128], ts[128];
    const uint32_t m = blockIdx.x, h = blockIdx.y, i = threadIdx.x;
    if (m >= pd->m) return;
    const uint32_t hd = g.head_dim, D = g.n_heads * hd;
    const uint32_t nc = (kv_view(g, row_pos(pd, m)).count() + 1 + 255) / 256;
    const size_t mh = (size_t)m * g.n_heads + h;
    const float* st = S + mh * s_stride;
    float mx = st[0];
#pragma unroll 8
    for (uint32_t c = 1; c < nc; c++) mx = fmaxf(mx, st[2 * c]);
    const float* up = Up + mh * cstride * hd + (i < hd ? i : 0u);
    float T = 0.0f, U = 0.0f;
    for (uint32_t cb = 0; cb < nc; cb += 128) {
        const uint32_t nb = min(128u, nc - cb);
        __syncthreads();
        if (i < nb) {
            fs[i] = expf_c(st[2 * (cb + i)] - mx);
            ts[i] = st[2 * (cb + i) + 1];
        }
        __syncthreads();
#pragma unroll 8
        for (uint32_t k = 0; k < nb; k++) {
            const float f = fs[k];
            T = __builtin_fmaf(ts[k], f, T);
            U = __builtin_fmaf(up[(size_t)(cb + k) * hd], f, U);
        }
    }
    if (i < hd) out[(size_t)m * D + h * hd + i] = U * (1.0f / (T + 1e-10f));
}

// Second stage of the engine's attention fused with the O projection's
// quantize_activation_row (src/engine.cpp:789-796): per row m, every head's
// chunks merged exactly as k_attn_merge_chunks does (max over the chunk
// maxima, f_c = exp(m_c - max), T and U fmaf chains over c in order,
// out = U * (1 / (T + 1e-10))), then the row quantized.  NT threads;
// element i = t + NT k; heads * chunks <= 2048 (checked when the engine is
// created).  fs and ts hold 2048 floats each, hmax and hinv 128, red 16.
template <int PER, int NT>
__device__ __forceinline__ void merge_quant_row(const PassDesc* __restrict__ pd, const KvGeom& g, uint32_t m,
                                                const float* __restrict__ S, uint32_t s_stride,
                                                const float* __restrict__ Up, uint32_t cstride,
                                                int8_t* __restrict__ q, uint32_t q_stride, float* __restrict__ as,
                                                int32_t* __restrict__ bsum, uint32_t bsum_stride, float* fs,
                                                float* ts, float* hmax, float* hinv, float* red) {
    const uint32_t t = threadIdx.x;
    const uint32_t H = g.n_heads, hd = g.head_dim, D = H * hd;
    const uint32_t nc = (kv_view(g, row_pos(pd, m)).count() + 1 + 255) / 256;
    const float* st = S + (size_t)m * H * s_stride;
    for (uint32_t i = t; i < H * nc; i += NT) {
        const uint32_t h = i / nc, c = i - h * nc;
        fs[i] = st[(size_t)h * s_stride + 2 * c];
        ts[i] = st[(size_t)h * s_stride + 2 * c + 1];
    }
    __syncthreads();
    if (t < H) {
        float mx = fs[t * nc];
        for (uint32_t c = 1; c < nc; c++) mx = fmaxf(mx, fs[t * nc + c]);
        hmax[t] = mx;
    }
    __syncthreads();
    for (uint32_t i = t; i < H * nc; i += NT) fs[i] = expf_c(fs[i] - hmax[i / nc]);
    __syncthreads();
    if (t < H) {
        float T = 0.0f;
        for (uint32_t c = 0; c < nc; c++) T = __builtin_fmaf(ts[t * nc + c], fs[t * nc + c], T);
        hinv[t] = 1.0f / (T + 1e-10f);
    }
    __syncthreads();
    // U chains over c in order per element; the loads of 8 chunks of all
    // PER elements are issued before their FMAs
    float v[PER];
    const float* up[PER];
    const float* f[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const uint32_t i = t + (uint32_t)NT * k;
        const uint32_t h = i < D ? i / hd : 0u, l = i < D ? i - h * hd : 0u;
        up[k] = Up + ((size_t)m * H + h) * cstride * hd + l;
        f[k] = fs + h * nc;
        v[k] = 0.0f;
    }
    for (uint32_t c0 = 0; c0 < nc; c0 += 8) {
        const uint32_t nb = min(8u, nc - c0);
        float uc[PER][8];
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const bool in = t + (uint32_t)NT * k < D;
#pragma unroll
            for (uint32_t u = 0; u < 8; u++) {
                const float* a = up[k] + (size_t)(c0 + u) * hd;
                uc[k][u] = (in && u < nb) ? *a : 0.0f;
            }
        }
#pragma unroll
        for (int k = 0; k < PER; k++) {
#pragma unroll
            for (uint32_t u = 0; u < 8; u++)
                if (u < nb) v[k] = __builtin_fmaf(uc[k][u], f[k][c0 + u], v[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const uint32_t i = t + (uint32_t)NT * k;
        v[k] = i < D ? v[k] * hinv[i / hd] : 0.0f;
    }
    quantize_row_block<PER, NT>(v, D, q + (size_t)m * q_stride, as + m,
                                bsum ? bsum + (size_t)m * bsum_stride : nullptr, red);
}

// Grid M + prefetch blocks, 1024 threads: merge_quant_row per row.
template <int PER>
__global__ __launch_bounds__(1024) void k_attn_merge_quant(const PassDesc* __restrict__ pd, KvGeom g,
                                                           const float* __restrict__ S, uint32_t s_stride,
                                                           const float* __restrict__ Up, uint32_t cstride,
                                                           int8_t* __restrict__ q, uint32_t q_stride,
                                                           float* __restrict__ as, int32_t* __restrict__ bsum,
                                                           uint32_t bsum_stride, uint32_t rows, Prefetch pf) {
    __shared__ float fs[2048], ts[2048];
    __shared__ float hmax[128], hinv[128];
    __shared__ float red[16];
    const uint32_t m = blockIdx.x;
    if (m >= rows) {
        prefetch_groups(pf, m, m - rows, gridDim.x - rows);
        return;
    }
    if (m >= pd->m) return;
    merge_quant_row<PER, 1024>(pd, g, m, S, s_stride, Up, cstride, q, q_stride, as, bsum, bsum_stride, fs, ts,
                                      hmax, hinv, red);
}

}  // namespace pf
