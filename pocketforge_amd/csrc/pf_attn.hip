// 3-tier int8 KV cache and verify attention for gfx950.
//
// A pass of M rows at consecutive positions p0..p0+M-1 runs, per layer
// (after the Q/K/V product, whose epilogue applies RoPE, pf_mm.hip):
//   k_kv_store_pass  int8 K/V rows of each pass row written to the plane row
//                  of its position (sink slot or ring slot; the ring has
//                  slack, so pending rows of a verify pass never overwrite a
//                  visible entry)
//   k_attn_chunk   per (row, head, 256-entry chunk of the row's list):
//                  scores, chunk max, exp, chunk sum and chunk-weighted V
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
__global__ __launch_bounds__(128) void k_pool_rows(KvGeom g, KvPlanes kv, const PassDesc* __restrict__ pd) {
    uint32_t p_first, p_last, seq, y = blockIdx.y;
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
    pool_row(g, kv, (size_t)seq * g.n_layers * g.n_heads + blockIdx.x, r);
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

// Shared memory of one attention block (bytes): V rows of the chunk first,
// VROW bytes each.  VROW = 136 (8 bytes of padding) keeps the block under
// 40 KB, so four blocks fit in a CU's 160 KB: passes of many rows.  VROW =
// 144 (16-byte rows, one 16-byte store per part) for passes of a few rows,
// whose grids do not fill the CUs anyway.
constexpr uint32_t att_vt(uint32_t vrow) { return 256 * vrow; }
constexpr uint32_t att_smem(uint32_t vrow) { return att_vt(vrow) + (128 + 128 + 256 + 256 + 512 + 4) * 4; }

template <int PARTS, uint32_t VROW = 144>
__device__ __forceinline__ void attn_one_row(const PassDesc* __restrict__ pd, const KvGeom& g, const KvPlanes& kv,
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
    if (grp >= n_groups || m >= pd->m) return;
    attn_one_row<PARTS, VROW>(pd, g, kv, layer, m, grp % g.n_heads, grp / g.n_heads, q, kself, vself, S, s_stride,
                              Up, cstride, smem);
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
        prefetch_bytes(pf.p, pf.n, m - rows, gridDim.x - rows, pf.sink);
        return;
    }
    if (m >= pd->m) return;
    merge_quant_row<PER, 1024>(pd, g, m, S, s_stride, Up, cstride, q, q_stride, as, bsum, bsum_stride, fs, ts,
                                      hmax, hinv, red);
}

}  // namespace pf
