// Device-side helpers shared by the gfx950 kernels.
//
// Float results of the hot path must be bit-identical to the CPU restatement,
// so every reduction here has one fixed association order and every fused
// multiply-add is written explicitly (the library is compiled with
// -ffp-contract=off).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pf_layout.h"

#define PF_WAVE 64

namespace pf {

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// exp(x): Cody-Waite reduction x = k*ln2 + r with ln2 split into a 16-bit
// head and a tail, degree-7 Taylor polynomial of exp(r) in Horner form,
// scaling by 2^k through the exponent field.  x < -86 gives 0 and x > 88
// gives +inf, so no subnormal result is formed.
__device__ __forceinline__ float expf_c(float x) {
    if (x != x) return x;
    if (x < -86.0f) return 0.0f;
    if (x > 88.0f) return __builtin_inff();
    float kf = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(kf, -0.693145751953125f, x);
    r = __builtin_fmaf(kf, -1.42860676533018704503775e-06f, r);
    float p = 1.98412698412698412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-3f);
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-2f);
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    int k = (int)kf;
    return p * u2f((uint32_t)(k + 127) << 23);
}

// IEEE binary16 bits -> float: v_cvt_f32_f16, exact for every finite value
// (subnormal halves included: this code is built without denormal flushing).
__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// Philox4x32-10 (Salmon et al., SC'11).
__device__ __forceinline__ void philox(uint32_t c[4], uint32_t k0, uint32_t k1) {
    for (int r = 0; r < 10; r++) {
        if (r > 0) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        uint32_t lo0 = 0xD2511F53u * c[0], hi0 = __umulhi(0xD2511F53u, c[0]);
        uint32_t lo1 = 0xCD9E8D57u * c[2], hi1 = __umulhi(0xCD9E8D57u, c[2]);
        uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
    }
}

// Uniform in [0,1) for stochastic draw number idx of a run seeded `seed`.
__device__ __forceinline__ float uniform(uint64_t seed, uint64_t idx) {
    uint32_t c[4] = {(uint32_t)idx, (uint32_t)(idx >> 32), 0x53414D50u, 0u};
    philox(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    return (float)(c[0] >> 8) * 0x1p-24f;
}

// ---------------------------------------------------------------- waves

__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, PF_WAVE); }
__device__ __forceinline__ double shfl_xor(double v, int m) { return __shfl_xor(v, m, PF_WAVE); }

// Value of lane (lane & ~15) | ((lane & 15) - n) mod 16 (DPP row_ror:n), or a
// quad permutation (DPP quad_perm), without the LDS path.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
constexpr int DPP_ROR4 = 0x124, DPP_ROR8 = 0x128, DPP_ROR12 = 0x12C, DPP_XOR2 = 0x4E, DPP_XOR1 = 0xB1;

// The butterfly steps of offsets 8, 4, 2, 1 inside each row of 16 lanes:
// lane i adds the value of lane i ^ off (row_ror:8 is xor 8; xor 4 takes
// row_ror:4 or row_ror:12 by bit 2 of the lane).
__device__ __forceinline__ float row16_tree_sum(float v) {
    v = v + dpp_mov<DPP_ROR8>(v);
    const float a = v + dpp_mov<DPP_ROR4>(v), b = v + dpp_mov<DPP_ROR12>(v);
    v = (threadIdx.x & 4u) ? a : b;
    v = v + dpp_mov<DPP_XOR2>(v);
    v = v + dpp_mov<DPP_XOR1>(v);
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_mov<DPP_ROR8>(v));
    v = fmaxf(v, dpp_mov<DPP_ROR4>(v));
    v = fmaxf(v, dpp_mov<DPP_XOR2>(v));
    v = fmaxf(v, dpp_mov<DPP_XOR1>(v));
    return v;
}

// Halving tree over the 64 lanes of a wave: after the butterfly every lane
// holds ((P0+P32)+(P16+P48)) ... in the order offsets 32,16,8,4,2,1 (the
// offsets below 16 stay inside a row of 16 lanes and use DPP; additions are
// commutative, so every lane's sum has the same bits).
__device__ __forceinline__ float wave_tree_sum(float v) {
    v = v + shfl_xor(v, 32);
    v = v + shfl_xor(v, 16);
    return row16_tree_sum(v);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, shfl_xor(v, 32));
    v = fmaxf(v, shfl_xor(v, 16));
    return row16_max(v);
}

// Canonical sum over a block of W waves where each thread has already
// accumulated its strided partial: wave trees, then a halving tree over the
// wave totals (offsets W/2 .. 1).  `red` is __shared__ float[W].  All threads
// return the total.
template <int W>
__device__ __forceinline__ float block_canon_sum(float part, float* red) {
    float w = wave_tree_sum(part);
    int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wid] = w;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t[W];
#pragma unroll
        for (int i = 0; i < W; i++) t[i] = red[i];
#pragma unroll
        for (int off = W / 2; off >= 1; off >>= 1)
#pragma unroll
            for (int i = 0; i < off; i++) t[i] = t[i] + t[i + off];
        red[0] = t[0];
    }
    __syncthreads();
    float r = red[0];
    __syncthreads();
    return r;
}

template <int W>
__device__ __forceinline__ float block_max(float v, float* red) {
    float w = wave_max(v);
    int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wid] = w;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < W; i++) m = fmaxf(m, red[i]);
    __syncthreads();
    return m;
}

// quantize_activation_row / KVCache::quantize_row arithmetic for one value.
__device__ __forceinline__ int8_t quant_code(float x, float inv) {
    return (int8_t)(int)__builtin_roundf(x * inv);
}

// ------------------------------------------------------- 3-tier KV views

// Visible entries of a query, from the plane's sink count and the number of
// window stores so far (src/kv_cache.cpp:59-127 keeps exactly this state
// per (layer, head)): sink rows, pooled rows, window entries oldest ->
// newest (src/kv_cache.cpp:137-155).
struct KvView {
    uint32_t sink, pool, win_lo, win_hi;
    __device__ __host__ uint32_t count() const { return sink + pool + (win_hi - win_lo); }
};

__device__ __host__ __forceinline__ KvView kv_view_counts(const KvGeom& g, uint32_t sink, uint32_t nw) {
    KvView v;
    v.sink = sink;
    v.win_hi = nw;
    v.win_lo = nw > g.window ? nw - g.window : 0u;
    v.pool = v.win_lo / g.pool_block;
    return v;
}

// The engine stores every position once, in order, in every plane: a query
// at position p sees the stores of positions [0, min(p, max_context)).
__device__ __host__ __forceinline__ KvView kv_view(const KvGeom& g, uint32_t p) {
    uint32_t n = p < g.max_context ? p : g.max_context;
    uint32_t s_eff = g.sink_size < KV_SINK_ROWS ? g.sink_size : KV_SINK_ROWS;
    uint32_t nw = n > g.sink_size ? n - g.sink_size : 0u;
    return kv_view_counts(g, n < s_eff ? n : s_eff, nw);
}

// Destination row of the store of position p, or UINT32_MAX when the
// reference stores nothing (p >= max_context, or a sink position >= 8).
__device__ __host__ __forceinline__ uint32_t kv_store_row(const KvGeom& g, uint32_t p) {
    if (p >= g.max_context) return 0xFFFFFFFFu;
    if (p < g.sink_size) return p < KV_SINK_ROWS ? p : 0xFFFFFFFFu;
    return KV_SINK_ROWS + (p - g.sink_size) % g.ring;
}

// Position and sequence of row m of a pass.
__device__ __forceinline__ uint32_t row_pos(const PassDesc* pd, uint32_t m) {
    return pd->batch ? pd->rpos[m] : pd->pos0 + m;
}
__device__ __forceinline__ uint32_t row_seq(const PassDesc* pd, uint32_t m) {
    return pd->batch ? pd->rseq[m] : pd->seq0;
}

// The descriptor's first four words (pos0, m, batch, seq0) read with one
// 16-byte load at a kernel's start, so that the positions and sequences of
// a single-sequence pass's rows need no further memory round trip (each
// dependent descriptor read costs one on the kernel's critical path).
struct PassHead {
    uint32_t pos0, m, batch, seq0;
    const PassDesc* pd;
};
__device__ __forceinline__ PassHead pass_head(const PassDesc* pd) {
    const uint4 w = *reinterpret_cast<const uint4*>(pd);
    return PassHead{w.x, w.y, w.z, w.w, pd};
}
// The same words with vector loads, for a kernel that needs them only after
// its main loads: a scalar load issued early would hold up every later
// kernel-argument read (scalar loads return out of order, so a wait for one
// is a wait for all).
__device__ __forceinline__ PassHead pass_head_late(const PassDesc* pd) {
    const unsigned long long* q = reinterpret_cast<const unsigned long long*>(pd);
    const unsigned long long a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return PassHead{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32), pd};
}
__device__ __forceinline__ uint32_t row_pos(const PassHead& p, uint32_t m) {
    return p.batch ? p.pd->rpos[m] : p.pos0 + m;
}
__device__ __forceinline__ uint32_t row_seq(const PassHead& p, uint32_t m) {
    return p.batch ? p.pd->rseq[m] : p.seq0;
}

// Row index (within one (layer, head) plane) of visible entry j.
__device__ __forceinline__ uint32_t kv_row(const KvGeom& g, const KvView& v, uint32_t j) {
    if (j < v.sink) return j;
    j -= v.sink;
    if (j < v.pool) return KV_SINK_ROWS + g.ring + j;
    j -= v.pool;
    return KV_SINK_ROWS + (v.win_lo + j) % g.ring;
}

// ---------------------------------------------------------- prefetch

// The weights of the next kernel in the stream, loaded by extra blocks of
// the current one so that the next kernel finds them in its L2.  The matrix
// is stored as `groups` contiguous runs of `gbytes` bytes (the 32-row groups
// of the tiled layout) and the next kernel's workgroup g reads group g.
// Every dispatch deals its workgroups to the 8 XCDs round-robin from XCD 0
// (workgroup b runs on XCD b mod 8, measured with the XCC_ID register on
// consecutive dispatches and graph replays), and each XCD has its own L2:
// group g is wanted in the L2 of XCD g mod 8.
struct Prefetch {
    const uint8_t* p;   // null: nothing to prefetch
    uint32_t gbytes;    // bytes per group, a multiple of 16
    uint32_t groups;
    uint32_t blocks;    // prefetch workgroups a GEMV launch adds to its grid
    uint32_t* sink;
    uint32_t xoff;      // the consumer reads group g on XCD (g + xoff) mod 8
};

// Prefetch block x of T, whose linear block id is lin (the prefetch blocks
// of a launch have consecutive ids), loads the groups g with
// g + xoff = lin (mod 8) into its XCD's L2, sharing them with the other
// prefetch blocks of that XCD (those with the same x mod 8).  The loaded
// words feed a value that is stored only if it equals a constant, so the
// loads stay.
__device__ __forceinline__ void prefetch_groups(const Prefetch& pf, uint32_t lin, uint32_t x, uint32_t T) {
    const uint32_t g0 = (lin - pf.xoff) & 7u;
    if (!pf.p || g0 >= pf.groups) return;
    const uint32_t rank = x >> 3, cnt = (T - (x & 7u) + 7u) >> 3;
    const uint32_t gb16 = pf.gbytes >> 4, n16 = ((pf.groups - g0 + 7u) >> 3) * gb16;
    const uint32_t stride = cnt * blockDim.x;
    const uint4* q = reinterpret_cast<const uint4*>(pf.p);
    uint32_t acc = 0;
    for (uint32_t u = rank * blockDim.x + threadIdx.x; u < n16; u += 4u * stride) {
        uint4 v[4];
#pragma unroll
        for (uint32_t k = 0; k < 4; k++) {
            const uint32_t w = min(u + k * stride, n16 - 1u), i = w / gb16;   // i-th group of this XCD
            v[k] = q[(size_t)(g0 + 8u * i) * gb16 + (w - i * gb16)];
        }
        acc ^= v[0].x ^ v[1].y ^ v[2].z ^ v[3].w;
    }
    if (acc == 0x7A5C3E1Fu) pf.sink[0] = acc;
}

// ------------------------------------------------------ quantized rows

// Block sums of int8 codes over 32-element blocks for a 256-thread block
// where thread t handles elements t, t+256, ...: the 32 elements of a block
// sit in 32 consecutive lanes of one wave.
__device__ __forceinline__ int half_wave_isum(int v) {
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Quantize one row held by a block of NT threads (thread t has elements
// t, t+NT, ...) with the arithmetic of src/matmul_neon.cpp:16-29.  Writes
// the codes, the row scale and (when bsum != null) the sums of the codes
// of each 32-element block: a block's elements sit in 32 consecutive lanes.
template <int PER, int NT>
__device__ __forceinline__ void quantize_row_block(const float (&x)[PER], uint32_t K, int8_t* q,
                                                   float* scale_out, int32_t* bsum, float* red) {
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        uint32_t i = threadIdx.x + (uint32_t)NT * k;
        if (i < K) amax = fmaxf(amax, fabsf(x[k]));
    }
    amax = block_max<NT / 64>(amax, red);
    const float inv = (amax == 0.0f) ? 1.0f : 127.0f / amax;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        uint32_t i = threadIdx.x + (uint32_t)NT * k;
        int code = 0;
        if (i < K) {
            int8_t c = quant_code(x[k], inv);
            q[i] = c;
            code = c;
        }
        if (bsum) {
            int s = half_wave_isum(code);
            if (i < K && (i & 31u) == 0) bsum[i >> 5] = s;
        }
    }
    if (threadIdx.x == 0) *scale_out = (amax == 0.0f) ? 1.0f : amax / 127.0f;
}

// An LDS pointer (16-byte aligned) whose address sits in a VGPR the
// compiler cannot fold: reads at constant offsets from it carry the offset
// in the instruction instead of materialising each address in a register of
// its own.
template <typename T>
__device__ __forceinline__ const T* lds_opaque(const T* p) {
    uint32_t z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return reinterpret_cast<const T*>(__builtin_assume_aligned(reinterpret_cast<const uint8_t*>(p) + z, 16));
}

// ------------------------------------------------------------- LL words
// Values handed from workgroups of one launch to later workgroups of the
// same launch: 8-byte words (value bits, flag) written with one device-scope
// store each, flag = ep[0] * fmul + fadd (the pass epoch kept in device
// memory and the layer), so a reader that sees the flag sees the value and
// a word of an earlier pass or layer is never taken for the current one.  A
// reader loads its words with device-scope loads and loads again the ones
// whose flag is not yet the current one.  A wait longer than LL_SPIN_MAX
// rounds sets *err (the host reports it) and goes on, so every workgroup
// ends.
struct LLIn {
    const unsigned long long* ll;
    const uint32_t* ep;
    uint32_t fmul, fadd;
    uint32_t* err;
    // a word of the input that an early producer writes: a waiting wave
    // polls it alone (one request per round) before it polls its own words,
    // which keeps the memory traffic of long waits small
    uint32_t sent;
    // attention blocks with out set write their chunk results as LL words:
    // S pairs at out[(row H + h) s_stride + 2 c ..], U at
    // out[sreg + ((row H + h) cstride + c) hd + d]
    unsigned long long* out;
    uint32_t sreg;
    // LL_GATE (GEMV), or attention blocks with gate set: the word
    // gate[gate_off] a workgroup waits for before its weight (or cached K/V)
    // loads, flagged gate_back layers before the workgroup's own
    const unsigned long long* gate;
    uint32_t gate_off, gate_back;
};
constexpr uint32_t LL_SPIN_MAX = 1u << 20;

// The pass epoch, with a vector load: it is needed only when the first LL
// word is written or checked, after the kernel's main loads are issued.
__device__ __forceinline__ uint32_t ll_epoch(const uint32_t* ep) {
    return __hip_atomic_load(ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long ll_load(const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void ll_store(unsigned long long* p, float v, uint32_t flag) {
    __hip_atomic_store(p, ((unsigned long long)flag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Values of the N words base[off[i]] (off[i] == LL_NONE: 0) once each
// carries `flag`.
constexpr uint32_t LL_NONE = 0xFFFFFFFFu;
//
// One word per thread (a sentinel) is polled with two rounds of loads in
// flight: while the older round is checked the newer one travels, so the
// word is seen about half a memory round trip after it lands instead of up
// to a whole one.  A round issued later sees every word an earlier round saw
// (a word, once written for this pass and layer, keeps its flag until the
// launch ends), so the newest completed round decides.
template <int N>
__device__ __forceinline__ void ll_wait(const unsigned long long* base, const uint32_t (&off)[N], float (&out)[N],
                                        uint32_t flag, uint32_t* err) {
    unsigned long long w[N];
    const unsigned long long done = (unsigned long long)flag << 32;
#pragma unroll
    for (int i = 0; i < N; i++) w[i] = off[i] != LL_NONE ? ll_load(base + off[i]) : done;
    if constexpr (N == 1) {
        unsigned long long v[N];
        __builtin_amdgcn_s_sleep(8);
#pragma unroll
        for (int i = 0; i < N; i++) v[i] = off[i] != LL_NONE ? ll_load(base + off[i]) : done;
        for (uint32_t spins = 0;; spins++) {
            bool ok = true;
#pragma unroll
            for (int i = 0; i < N; i++) ok = ok && (uint32_t)(w[i] >> 32) == flag;
            if (ok) break;
#pragma unroll
            for (int i = 0; i < N; i++) w[i] = off[i] != LL_NONE ? ll_load(base + off[i]) : done;
            ok = true;
#pragma unroll
            for (int i = 0; i < N; i++) ok = ok && (uint32_t)(v[i] >> 32) == flag;
            if (ok) {
#pragma unroll
                for (int i = 0; i < N; i++) out[i] = __uint_as_float((uint32_t)v[i]);
                return;
            }
            if (spins >= LL_SPIN_MAX) {
                atomicOr(err, 1u);
                break;
            }
#pragma unroll
            for (int i = 0; i < N; i++) v[i] = off[i] != LL_NONE ? ll_load(base + off[i]) : done;
        }
#pragma unroll
        for (int i = 0; i < N; i++) out[i] = __uint_as_float((uint32_t)w[i]);
        return;
    }
    for (uint32_t spins = 0;; spins++) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < N; i++) ok = ok && (uint32_t)(w[i] >> 32) == flag;
        if (ok) break;
        if (spins >= LL_SPIN_MAX) {
            atomicOr(err, 1u);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int i = 0; i < N; i++)
            if ((uint32_t)(w[i] >> 32) != flag) w[i] = ll_load(base + off[i]);
    }
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __uint_as_float((uint32_t)w[i]);
}

}  // namespace pf
