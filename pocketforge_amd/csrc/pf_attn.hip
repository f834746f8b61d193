// 3-tier int8 KV cache and verify attention for gfx950.
//
// A pass of M rows at consecutive positions p0..p0+M-1 runs, per layer:
//   k_qkv_post     Q/K/V from the fused GEMV partials, RoPE, int8 K/V rows
//                  written to the plane row of each position (sink slot or
//                  ring slot; the ring has slack, so pending rows of a
//                  verify pass never overwrite a visible entry)
//   k_attn_scores  one thread per visible entry: the reference's sequential
//                  dot over head_dim, and the fp32 self score
//   k_attn_softmax per (row, head): max, exp, CANON(4) sum, normalise
//   k_attn_wsum    per (row, head, 64-entry chunk): fmaf chain over entries
//   k_attn_combine per row: chunk partials left to right + self term, then
//                  quantize_activation_row for the O projection
// k_pool_rows folds evicted window entries into pooled rows
// (src/kv_cache.cpp:77-109) before a pass needs them.
#include "pf_device.h"

namespace pf {

__device__ __forceinline__ size_t plane_index(const KvGeom& g, uint32_t layer, uint32_t head) {
    return (size_t)layer * g.n_heads + head;
}

// View of row m of a pass: from its position, or from explicit counts when
// view_sink >= 0 (the KVCache API, whose planes advance independently).
__device__ __forceinline__ KvView pass_view(const KvGeom& g, const PassDesc* pd, uint32_t m,
                                            int32_t view_sink, uint32_t view_nw) {
    if (view_sink >= 0) return kv_view_counts(g, (uint32_t)view_sink, view_nw);
    return kv_view(g, pd->pos0 + m);
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

// Grid (M, heads), 64 threads.  part = fused QKV GEMV partials ([s][M][3D]).
// RoPE of src/engine.cpp:732-749 with the host-computed angle tables
// (cos/sin [position][head_dim/2]).
__global__ __launch_bounds__(64) void k_qkv_post(const double* __restrict__ part, uint32_t splits, uint32_t M,
                                                 const float* __restrict__ as, const PassDesc* __restrict__ pd,
                                                 const float* __restrict__ rc, const float* __restrict__ rs,
                                                 KvGeom g, KvPlanes kv, uint32_t layer,
                                                 float* __restrict__ q_out, float* __restrict__ k_out,
                                                 float* __restrict__ v_out) {
    const uint32_t m = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    if (m >= pd->m) return;
    const uint32_t hd = g.head_dim, D = g.n_heads * hd, N = 3 * D, half = hd >> 1;
    const uint32_t pos = pd->pos0 + m;
    const bool act = t < half;
    float k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
    if (act) {
        const float a = as[m];
        const uint32_t i0 = h * hd + 2 * t;
        float q0 = gemv_out(part, splits, M, N, m, i0, a), q1 = gemv_out(part, splits, M, N, m, i0 + 1, a);
        k0 = gemv_out(part, splits, M, N, m, D + i0, a); k1 = gemv_out(part, splits, M, N, m, D + i0 + 1, a);
        v0 = gemv_out(part, splits, M, N, m, 2 * D + i0, a); v1 = gemv_out(part, splits, M, N, m, 2 * D + i0 + 1, a);
        const float c = rc[(size_t)pos * half + t], s = rs[(size_t)pos * half + t];
        float qr0 = __builtin_fmaf(q0, c, -(q1 * s));
        float qr1 = __builtin_fmaf(q0, s, q1 * c);
        float kr0 = __builtin_fmaf(k0, c, -(k1 * s));
        float kr1 = __builtin_fmaf(k0, s, k1 * c);
        k0 = kr0; k1 = kr1;
        size_t o = (size_t)m * D + i0;
        q_out[o] = qr0; q_out[o + 1] = qr1;
        k_out[o] = kr0; k_out[o + 1] = kr1;
        v_out[o] = v0; v_out[o + 1] = v1;
    }
    store_pair(g, kv, plane_index(g, layer, h), kv_store_row(g, pos), t, act, k0, k1, v0, v1);
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
    store_pair(g, kv, plane_index(g, layer, head), row, t, act, k0, k1, v0, v1);
}

// Pooled rows [r_lo, r_lo + gridDim.y) of every plane in [plane_lo,
// plane_lo + gridDim.x): the mean of pool_block consecutive window entries
// accumulated in double in eviction order, scaled by (double)(1.0f/P), then
// requantized (src/kv_cache.cpp:83-104).  head_dim threads (<= 128).
__global__ __launch_bounds__(128) void k_pool_rows(KvGeom g, KvPlanes kv, uint32_t plane_lo, uint32_t r_lo) {
    __shared__ float red[4];
    const size_t plane = plane_lo + blockIdx.x;
    const uint32_t r = r_lo + blockIdx.y, i = threadIdx.x, hd = g.head_dim, P = g.pool_block;
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
        float amax = fabsf(avg);
        // head_dim <= 128: at most two waves
        float w = wave_max(amax);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = w;
        __syncthreads();
        amax = (blockDim.x > 64) ? fmaxf(red[0], red[1]) : red[0];
        __syncthreads();
        const float qi = (amax == 0.0f) ? 1.0f : 127.0f / amax;
        int8_t* d8 = which ? kv.v : kv.k;
        float* ds = which ? kv.vs : kv.ks;
        if (act) d8[(prow + dst) * hd + i] = quant_code(avg, qi);
        if (i == 0) ds[prow + dst] = (amax == 0.0f) ? 1.0f : amax / 127.0f;
    }
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
        const size_t plane = plane_index(g, layer, h);
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

// In place: S <- softmax(S[0..C]) (src/matmul_neon.cpp:212-226 with the
// CANON(4) sum).  Grid (M, H), 256 threads.
__global__ __launch_bounds__(256) void k_attn_softmax(const PassDesc* __restrict__ pd, KvGeom g,
                                                      int32_t view_sink, uint32_t view_nw,
                                                      float* __restrict__ S, uint32_t s_stride) {
    __shared__ float red[4];
    const uint32_t m = blockIdx.x, h = blockIdx.y;
    if (m >= pd->m) return;
    const uint32_t n = pass_view(g, pd, m, view_sink, view_nw).count() + 1;
    float* s = S + ((size_t)m * g.n_heads + h) * s_stride;
    float mx = -__builtin_inff();
    for (uint32_t j = threadIdx.x; j < n; j += 256) mx = fmaxf(mx, s[j]);
    mx = block_max<4>(mx, red);
    float part = 0.0f;
    for (uint32_t j = threadIdx.x; j < n; j += 256) {
        float e = expf_c(s[j] - mx);
        s[j] = e;
        part = part + e;
    }
    const float sum = block_canon_sum<4>(part, red);
    const float inv = 1.0f / (sum + 1e-10f);
    for (uint32_t j = threadIdx.x; j < n; j += 256) s[j] = s[j] * inv;
}

// Wp[((m*H + y)*cstride + c)*hd + i] = fmaf chain over the visible entries
// [64c, min(64c+64, C, limit)) of p_j * ((float)v_j[i] * vs_j)
// (src/kv_cache.cpp:173-197, contracted as the reference build does).
// Grid (M, H, chunks), 128 threads (head_dim <= 128).
__global__ __launch_bounds__(128) void k_attn_wsum(const PassDesc* __restrict__ pd, KvGeom g, KvPlanes kv,
                                                   uint32_t layer, int32_t view_sink, uint32_t view_nw,
                                                   int32_t head_override, uint32_t limit,
                                                   const float* __restrict__ S, uint32_t s_stride,
                                                   float* __restrict__ Wp, uint32_t cstride) {
    const uint32_t m = blockIdx.x, y = blockIdx.y, c = blockIdx.z, i = threadIdx.x;
    const uint32_t h = head_override >= 0 ? (uint32_t)head_override : y;
    if (m >= pd->m) return;
    const uint32_t hd = g.head_dim;
    const KvView v = pass_view(g, pd, m, view_sink, view_nw);
    const uint32_t C = min(v.count(), limit);
    if (c * 64u >= C || i >= hd) return;
    const size_t plane = plane_index(g, layer, h);
    const float* p = S + ((size_t)m * g.n_heads + y) * s_stride;
    const uint32_t j1 = min(C, c * 64u + 64u);
    float acc = 0.0f;
    for (uint32_t j = c * 64u; j < j1; j++) {
        uint32_t row = kv_row(g, v, j);
        float vv = (float)kv.v[(plane * g.rows + row) * hd + i] * kv.vs[plane * g.rows + row];
        acc = __builtin_fmaf(p[j], vv, acc);
    }
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

// Per row m: attention output element e = h*hd + i as chunk partials added
// left to right, then fmaf(p_self, v_self, .).  Writes the fp32 output
// (when out != null) and its quantize_activation_row codes for the O
// projection.  Grid M, 256 threads, D <= 256 * PER.
template <int PER>
__global__ __launch_bounds__(256) void k_attn_combine(const PassDesc* __restrict__ pd, KvGeom g,
                                                      int32_t view_sink, uint32_t view_nw,
                                                      const float* __restrict__ S, uint32_t s_stride,
                                                      const float* __restrict__ Wp, uint32_t cstride,
                                                      const float* __restrict__ vself, float* __restrict__ out,
                                                      int8_t* __restrict__ q, uint32_t q_stride,
                                                      float* __restrict__ as, int32_t* __restrict__ bsum,
                                                      uint32_t bsum_stride) {
    __shared__ float red[4];
    const uint32_t m = blockIdx.x;
    if (m >= pd->m) return;
    const uint32_t hd = g.head_dim, D = g.n_heads * hd;
    const uint32_t C = pass_view(g, pd, m, view_sink, view_nw).count();
    const uint32_t nch = (C + 63u) / 64u;
    float x[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        uint32_t e = threadIdx.x + 256u * k;
        float o = 0.0f;
        if (e < D) {
            uint32_t h = e / hd, i = e % hd;
            const float* wp = Wp + ((size_t)m * g.n_heads + h) * cstride * hd + i;
            for (uint32_t c = 0; c < nch; c++) o = o + wp[(size_t)c * hd];
            float ps = S[((size_t)m * g.n_heads + h) * s_stride + C];
            o = __builtin_fmaf(ps, vself[(size_t)m * D + e], o);
            if (out) out[(size_t)m * D + e] = o;
        }
        x[k] = o;
    }
    if (q) quantize_row_block<PER>(x, D, q + (size_t)m * q_stride, as + m,
                                   bsum ? bsum + (size_t)m * bsum_stride : nullptr, red);
}

}  // namespace pf
