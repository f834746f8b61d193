// Sampling, acceptance and decode-round control on the device.
//
// Engine::sample's dispatch (src/engine.cpp:881-916): greedy when
// cfg.greedy or temperature <= 0; else top-p when 0 < top_p < 1 (top-k is
// then ignored); else top-k when 0 < top_k < V; else full-vocabulary
// temperature sampling.  One uniform per stochastic call, drawn from
// Philox4x32-10 keyed by the run seed with the draw index as counter.
//
// The decode round (src/engine.cpp:304-373) runs as: sample T1 from the
// base logits, sample one draft per MTP head, verify [T1, d0..d{n-1}] in
// one or two passes (segments), greedy argmax of every verify row, accept
// the longest matching prefix, sample the corrective from the first
// mismatching row.  Row j of the verify rows checks draft j (row n, fed
// d{n-1}, is the next round's F(cur)).  A segment covers rows k0 .. k0+m-1;
// the reference verifies one row at a time and stops at the first
// mismatch, so a segment that ends with a mismatch has done all the work
// the reference does, and one that accepts every row it checked leaves the
// rest to the next segment.  Every token decision is made here; the host
// reads one 32-bit word per segment (accepted count | corrective pushed << 8
// | next segment needed << 9).
#include "pf_device.h"

#include <rocprim/block/block_radix_sort.hpp>

namespace pf {

struct ArgBest { float v; int32_t i; };

__device__ __forceinline__ ArgBest arg_better(ArgBest a, ArgBest b) {
    if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
    return a;
}

// First index of the maximum (src/engine.cpp:918-928) of a row, computed by
// a 1024-thread block.  Result valid in thread 0.
__device__ ArgBest block_argmax(const float* __restrict__ x, uint32_t V) {
    __shared__ float sv[16];
    __shared__ int32_t si[16];
    ArgBest b{-__builtin_inff(), 0x7FFFFFFF};
    // 16-byte loads, four per thread in flight (the whole row at V = 16384),
    // then the elements past the last aligned quad; arg_better picks the
    // same element in any order
    const uint32_t V4 = ((uintptr_t)x & 15u) == 0u ? V / 4u : 0u;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    for (uint32_t i0 = threadIdx.x; i0 < V4; i0 += 4u * blockDim.x) {
        float4 v[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; u++) {
            const uint32_t i = i0 + u * blockDim.x;
            v[u] = x4[i < V4 ? i : V4 - 1u];
        }
#pragma unroll
        for (uint32_t u = 0; u < 4; u++) {
            const uint32_t i = i0 + u * blockDim.x;
            if (i < V4) {
                b = arg_better(b, ArgBest{v[u].x, (int32_t)(4u * i)});
                b = arg_better(b, ArgBest{v[u].y, (int32_t)(4u * i + 1u)});
                b = arg_better(b, ArgBest{v[u].z, (int32_t)(4u * i + 2u)});
                b = arg_better(b, ArgBest{v[u].w, (int32_t)(4u * i + 3u)});
            }
        }
    }
    for (uint32_t i = 4u * V4 + threadIdx.x; i < V; i += blockDim.x) b = arg_better(b, ArgBest{x[i], (int32_t)i});
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        ArgBest o{__shfl_xor(b.v, off, 64), __shfl_xor(b.i, off, 64)};
        b = arg_better(b, o);
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = b.v; si[threadIdx.x >> 6] = b.i; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < blockDim.x / 64; w++) b = arg_better(b, ArgBest{sv[w], si[w]});
        if (b.i == 0x7FFFFFFF) b.i = 0;
    }
    __syncthreads();
    return b;
}

// MTPHeads::argmax (src/mtp.cpp:145-155) of one row: first index of the
// maximum.  One block of 1024 threads.
__global__ __launch_bounds__(1024) void k_argmax_one(const float* __restrict__ x, uint32_t n,
                                                     int32_t* __restrict__ out) {
    ArgBest b = block_argmax(x, n);
    if (threadIdx.x == 0) *out = b.i;
}

// ----------------------------------------------------- stochastic sampler

__device__ __forceinline__ uint32_t ord_f(float f) {
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// LDS arena for the sampler: 16384 64-bit slots (128 KiB).
constexpr uint32_t SAMPLE_MAX_V = 16384;
constexpr uint32_t SAMPLE_IPT = SAMPLE_MAX_V / 1024;   // items per thread of the 1024-thread sampler

// Stable radix sort of 16384 32-bit keys with their indices (rocPRIM's
// block radix sort with the blocked-order rank algorithm): thread t holds
// positions 16 t .. 16 t + 15 before and after, and equal keys keep their
// order of positions.
typedef rocprim::block_radix_sort<uint32_t, 1024, SAMPLE_IPT, uint32_t, 1, 1, 8,
                                  rocprim::block_radix_rank_algorithm::basic_memoize>
    SampleSort;
static_assert(sizeof(SampleSort::storage_type) <= SAMPLE_MAX_V * sizeof(uint64_t),
              "sampler sort storage must fit the arena");

// Sorted (logit desc, index asc) order into `a` (hi = ~ord bits, lo = idx):
// a stable ascending sort of ~ord(x) over the indices in ascending order,
// so equal logits keep ascending indices.  Slots past V hold ~0 keys and
// sort last.  1024 threads; `a` doubles as the sort's scratch.
// The sort itself, leaving sorted positions 16 t .. 16 t + 15 in thread t's
// registers (`a` is the sort's scratch, free again after the call).
__device__ void sort_desc_regs(const float* __restrict__ x, uint32_t V, uint64_t* a, uint32_t (&key)[SAMPLE_IPT],
                               uint32_t (&idx)[SAMPLE_IPT]) {
#pragma unroll
    for (uint32_t j = 0; j < SAMPLE_IPT; j++) {
        const uint32_t i = threadIdx.x * SAMPLE_IPT + j;
        key[j] = i < V ? ~ord_f(x[i]) : ~0u;
        idx[j] = i;
    }
    SampleSort().sort(key, idx, *reinterpret_cast<SampleSort::storage_type*>(a));
    __syncthreads();
}

__device__ uint32_t sort_desc(const float* __restrict__ x, uint32_t V, uint64_t* a) {
    uint32_t key[SAMPLE_IPT], idx[SAMPLE_IPT];
    sort_desc_regs(x, V, a, key, idx);
#pragma unroll
    for (uint32_t j = 0; j < SAMPLE_IPT; j++)
        a[threadIdx.x * SAMPLE_IPT + j] = ((uint64_t)key[j] << 32) | idx[j];
    __syncthreads();
    return SAMPLE_MAX_V;
}

__device__ __forceinline__ float key_val(uint64_t k) {
    uint32_t o = ~(uint32_t)(k >> 32);
    uint32_t u = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
    return __uint_as_float(u);
}

// Chunk-of-64 sum and scan (the canonical order of the oracle's sampler):
// element s of n belongs to chunk L = s / cl (cl = ceil(n / 64)); each chunk
// is summed left to right from 0, the chunk totals left to right; the scan
// runs from the chunk's offset (the totals before it, left to right).  The
// scan returns the first index with cum >= thr1 (or n) and the first index
// with thr2 <= cum (or n).
struct ScanHit { uint32_t first_ge1, first_ge2; };

// The values live transposed in LDS: element s at (s - L cl) * 64 + L, so
// that the 64 lanes of wave 0, one per chunk, read consecutive words (in the
// plain layout every lane's word falls in the same bank).
__device__ __forceinline__ uint32_t tpos(uint32_t s, uint32_t cl) {
    const uint32_t L = s / cl;
    return (s - L * cl) * 64u + L;
}
// tpos for s = s0 + j (j < 16) from the chunk of s0, cl >= 16: consecutive
// positions cross at most one chunk boundary.
__device__ __forceinline__ uint32_t tpos_next(uint32_t s, uint32_t L0, uint32_t cl) {
    const uint32_t L = s >= (L0 + 1u) * cl ? L0 + 1u : L0;
    return (s - L * cl) * 64u + L;
}
// Chunk of element s with a float reciprocal of cl, corrected to the exact
// quotient (s < 2^24).
__device__ __forceinline__ uint32_t tpos_r(uint32_t s, uint32_t cl, float rcl) {
    uint32_t L = (uint32_t)((float)s * rcl);
    L -= L * cl > s ? 1u : 0u;
    L += (L + 1u) * cl <= s ? 1u : 0u;
    return (s - L * cl) * 64u + L;
}
__device__ __forceinline__ uint32_t chunk_len(uint32_t lane, uint32_t n, uint32_t cl) {
    return lane * cl < n ? min(cl, n - lane * cl) : 0u;
}
__device__ float chunk64_total_t(const float* P, uint32_t n, float* tot_lds) {
    const uint32_t lane = threadIdx.x, cl = (n + 63u) / 64u, len = chunk_len(lane, n, cl);
    float t = 0.0f;
    for (uint32_t o = 0; o < len; o++) t = t + P[o * 64u + lane];
    tot_lds[lane] = t;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float s = 0.0f;
    for (uint32_t b = 0; b < 64; b++) s = s + tot_lds[b];
    return s;
}
__device__ ScanHit chunk64_scan_t(const float* P, uint32_t n, float thr1, float thr2, float* tot_lds) {
    const uint32_t lane = threadIdx.x, cl = (n + 63u) / 64u, len = chunk_len(lane, n, cl);
    float t = 0.0f;
    for (uint32_t o = 0; o < len; o++) t = t + P[o * 64u + lane];
    tot_lds[lane] = t;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float off = 0.0f;
    for (uint32_t b = 0; b < lane; b++) off = off + tot_lds[b];
    uint32_t h1 = n, h2 = n;
    float c = off;
    for (uint32_t o = 0; o < len; o++) {
        c = c + P[o * 64u + lane];
        if (h1 == n && c >= thr1) h1 = lane * cl + o;
        if (h2 == n && thr2 <= c) h2 = lane * cl + o;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        h1 = min(h1, (uint32_t)__shfl_xor((int)h1, o, 64));
        h2 = min(h2, (uint32_t)__shfl_xor((int)h2, o, 64));
    }
    return ScanHit{h1, h2};
}

// Engine::sample of one logits row.  1024 threads.  Returns the token in
// thread 0.  `draw` is the draw index to use for a stochastic call.
__device__ int32_t sample_row(const float* __restrict__ x, uint32_t V, const SamplingCfg& cfg, uint64_t seed,
                              uint64_t draw, bool* used_draw) {
    __shared__ __align__(16) uint64_t arena[SAMPLE_MAX_V];
    __shared__ float tot[64];
    __shared__ float bcast[2];
    *used_draw = false;
    if (cfg.greedy || cfg.temperature <= 0.0f) return block_argmax(x, V).i;
    *used_draw = true;
    const float temp = cfg.temperature > 0.001f ? cfg.temperature : 0.001f;
    const float r = uniform(seed, draw);
    int32_t result = 0;
    if (cfg.top_p < 1.0f && cfg.top_p > 0.0f) {            // src/engine.cpp:961-1003
        // sorted positions 16 t + j in thread t's registers; then the
        // probabilities of the sorted order in the transposed chunk layout
        // P (at most 16,448 words) and the sorted indices IX (16-bit, V <=
        // 16384) in the arena
        uint32_t key[SAMPLE_IPT], idx[SAMPLE_IPT];
        sort_desc_regs(x, V, arena, key, idx);
        float* P = reinterpret_cast<float*>(arena);
        uint16_t* IX = reinterpret_cast<uint16_t*>(P + SAMPLE_MAX_V + 64u);
        const uint32_t cl = (V + 63u) / 64u;
        if (threadIdx.x == 0) bcast[1] = key_val(((uint64_t)key[0]) << 32);
        __syncthreads();
        const float mx = bcast[1];
        // this thread's positions' slots in P (one division per thread)
        uint32_t ps[SAMPLE_IPT];
        {
            const uint32_t s0 = threadIdx.x * SAMPLE_IPT, L0 = s0 / cl;
#pragma unroll
            for (uint32_t j = 0; j < SAMPLE_IPT; j++) ps[j] = cl >= SAMPLE_IPT ? tpos_next(s0 + j, L0, cl) : tpos(s0 + j, cl);
        }
        float pv[SAMPLE_IPT];
#pragma unroll
        for (uint32_t j = 0; j < SAMPLE_IPT; j++) {
            const uint32_t sp = threadIdx.x * SAMPLE_IPT + j;
            pv[j] = expf_c((key_val(((uint64_t)key[j]) << 32) - mx) / temp);
            if (sp < V) {
                P[ps[j]] = pv[j];
                IX[sp] = (uint16_t)idx[j];
            }
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            float sum = chunk64_total_t(P, V, tot);
            if (threadIdx.x == 0) bcast[0] = sum;
        }
        __syncthreads();
        const float sum = bcast[0];
#pragma unroll
        for (uint32_t j = 0; j < SAMPLE_IPT; j++) {
            const uint32_t sp = threadIdx.x * SAMPLE_IPT + j;
            if (sp < V) P[ps[j]] = pv[j] / sum;
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            ScanHit h = chunk64_scan_t(P, V, cfg.top_p, r, tot);
            uint32_t cutoff = h.first_ge1 < V ? h.first_ge1 + 1 : V;
            uint32_t pick = h.first_ge2 < cutoff ? h.first_ge2 : cutoff - 1;
            if (threadIdx.x == 0) result = (int32_t)IX[pick];
        }
    } else if (cfg.top_k > 0 && cfg.top_k < V) {           // src/engine.cpp:930-959
        sort_desc(x, V, arena);
        if (threadIdx.x == 0) {
            const uint32_t k = cfg.top_k;
            const float mx = key_val(arena[0]);
            float sum = 0.0f;
            for (uint32_t i = 0; i < k; i++) sum = sum + expf_c((key_val(arena[i]) - mx) / temp);
            float cum = 0.0f;
            result = (int32_t)(uint32_t)arena[k - 1];
            for (uint32_t i = 0; i < k; i++) {
                cum = cum + expf_c((key_val(arena[i]) - mx) / temp) / sum;
                if (r <= cum) { result = (int32_t)(uint32_t)arena[i]; break; }
            }
        }
    } else {                                               // src/engine.cpp:895-915
        float* fa = reinterpret_cast<float*>(arena);
        float mx = -__builtin_inff();
        {
            ArgBest b = block_argmax(x, V);
            if (threadIdx.x == 0) bcast[1] = b.v;
            __syncthreads();
            mx = bcast[1];
        }
        // index order: element i = t + 1024 k in thread t's registers and in
        // the transposed chunk layout
        const uint32_t cl = (V + 63u) / 64u;
        const float rcl = 1.0f / (float)cl;
        uint32_t ps[SAMPLE_IPT];
        float pv[SAMPLE_IPT];
#pragma unroll
        for (uint32_t k = 0; k < SAMPLE_IPT; k++) {
            const uint32_t i = threadIdx.x + 1024u * k;
            ps[k] = tpos_r(i, cl, rcl);
            pv[k] = i < V ? expf_c((x[i] - mx) / temp) : 0.0f;
            if (i < V) fa[ps[k]] = pv[k];
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            float sum = chunk64_total_t(fa, V, tot);
            if (threadIdx.x == 0) bcast[0] = sum;
        }
        __syncthreads();
        const float sum = bcast[0];
#pragma unroll
        for (uint32_t k = 0; k < SAMPLE_IPT; k++) {
            const uint32_t i = threadIdx.x + 1024u * k;
            if (i < V) fa[ps[k]] = pv[k] / sum;
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            ScanHit h = chunk64_scan_t(fa, V, 2.0f, r, tot);
            if (threadIdx.x == 0) result = h.first_ge2 < V ? (int32_t)h.first_ge2 : (int32_t)V - 1;
        }
    }
    __syncthreads();
    return result;
}

// Roles of a sample call inside the decode round.
enum SampleRole : int32_t {
    ROLE_PLAIN = 0,       // write the token to *out
    ROLE_T1 = 1,          // push; it is row 0 of the verify pass
    ROLE_DRAFT = 2,       // draft of head `k`: row k+1 of the verify pass
    ROLE_CORRECTIVE = 3,  // corrective of the first mismatching verify row
    ROLE_FALLBACK = 4,    // single-token path: push, becomes `cur`
};

__device__ __forceinline__ void push_token(DecodeState* st, int32_t* tokens, uint32_t cap, int32_t t) {
    if (st->n_tokens < cap) tokens[st->n_tokens] = t;
    st->n_tokens++;
    st->n_gen++;
    st->cur = t;
}

// One Engine::sample call outside the round's first samples (the
// corrective, the single-token fallback, a plain call).  Row `row` of
// `logits` (row < 0: the verify row of the first mismatch, st->round_acc).
// Grid 1, 1024 threads.
__global__ __launch_bounds__(1024) void k_sample(const float* __restrict__ logits, uint32_t stride, int32_t row,
                                                 uint32_t V, SamplingCfg cfg, uint64_t seed, DecodeState* st,
                                                 int32_t* tokens, uint32_t cap, int32_t role, int32_t* out) {
    __shared__ uint32_t skip;
    if (threadIdx.x == 0)
        skip = (role == ROLE_CORRECTIVE && (st->round_acc >= st->n_mtp || st->more)) ? 1u : 0u;
    // a row given by the caller is ranked while thread 0 reads the skip
    // condition; a row chosen by the round's acceptance waits for it
    if (row < 0) {
        __syncthreads();
        if (skip) return;
    }
    const uint32_t r = row >= 0 ? (uint32_t)row : st->round_acc;
    bool used = false;
    const int32_t t = sample_row(logits + (size_t)r * stride, V, cfg, seed, st->draw, &used);
    if (row >= 0) {
        __syncthreads();
        if (skip) return;
    }
    if (threadIdx.x != 0) return;
    if (used) st->draw++;
    switch (role) {
        case ROLE_CORRECTIVE: {
            uint32_t a = st->round_acc;
            uint32_t pushed = 0;
            if (t != st->draft[a]) { push_token(st, tokens, cap, t); st->rejected++; pushed = 1; }
            st->round_word = a | (pushed << 8);
            break;
        }
        case ROLE_FALLBACK:
            push_token(st, tokens, cap, t);
            break;
        default:
            if (out) *out = t;
    }
}

// The first samples of an MTP round in one launch: block 0 samples T1 from
// the base row (ROLE_T1: pushed, row 0 of the verify pass, `h` rows in its
// first segment), block 1 + k the draft of head k from its logits
// (ROLE_DRAFT), every block on its own CU at once.  Draw indices follow the
// reference's order, T1 then the drafts by head (src/engine.cpp:311, 318-330):
// block j draws st->draw + j when sampling is stochastic, and the last block
// to finish (every block has read st->draw by then) advances it past them.
// Grid 1 + n_mtp, 1024 threads; or the same samples in two launches, T1
// (grid 1, j0 = 0, advance = 0) and then the drafts (grid n_mtp, j0 = 1,
// advance = 1), which read the same st->draw and take the same draws.
__global__ __launch_bounds__(1024) void k_sample_round(const float* __restrict__ base_logits,
                                                       const float* __restrict__ mlogits, uint32_t V, SamplingCfg cfg,
                                                       uint64_t seed, DecodeState* st, int32_t* tokens, uint32_t cap,
                                                       PassDesc* pdB, int32_t h, uint32_t j0, int32_t advance) {
    __shared__ uint64_t base_s;
    if (threadIdx.x == 0) base_s = st->draw;
    __syncthreads();
    const uint64_t base = base_s;
    const uint32_t j = blockIdx.x + j0;
    bool used = false;
    const float* row = j == 0 ? base_logits : mlogits + (size_t)(j - 1u) * V;
    const int32_t t = sample_row(row, V, cfg, seed, base + j, &used);
    if (threadIdx.x != 0) return;
    if (j == 0) {
        push_token(st, tokens, cap, t);
        pdB->tok[0] = t;
        pdB->pos0 = st->pos;
        pdB->m = (uint32_t)h;
        pdB->batch = 0;
        pdB->seq0 = 0;
        st->seg_k0 = 0;
        st->more = 0;
    } else {
        st->draft[j - 1u] = t;
        pdB->tok[j] = t;
    }
    const uint32_t done = __hip_atomic_fetch_add(&st->blocks_done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (done == gridDim.x - 1u) {
        if (used && advance) st->draw = base + j0 + gridDim.x;
        st->blocks_done = 0u;
    }
}

// Engine::step_mtp's samples (src/engine.cpp:418-423): block j samples head
// j's logits with draw st->draw + j when sampling is stochastic (the order of
// the reference's calls), keeps it as draft j and, for j < n - 1, makes it
// row j + 1 of the verify pass `pd`; the last block to finish advances the
// draw counter.  Grid n_mtp, 1024 threads.
__global__ __launch_bounds__(1024) void k_step_drafts(const float* __restrict__ mlogits, uint32_t V, SamplingCfg cfg,
                                                      uint64_t seed, DecodeState* st, PassDesc* pd) {
    __shared__ uint64_t base_s;
    if (threadIdx.x == 0) base_s = st->draw;
    __syncthreads();
    const uint64_t base = base_s;
    const uint32_t j = blockIdx.x;
    bool used = false;
    const int32_t t = sample_row(mlogits + (size_t)j * V, V, cfg, seed, base + j, &used);
    if (threadIdx.x != 0) return;
    st->draft[j] = t;
    if (j + 1u < gridDim.x) pd->tok[j + 1u] = t;
    const uint32_t done = __hip_atomic_fetch_add(&st->blocks_done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (done == gridDim.x - 1u) {
        if (used) st->draw = base + gridDim.x;
        st->blocks_done = 0u;
    }
}

// Engine::step_mtp's verification (src/engine.cpp:426-447) of the pass over
// [current, d0 .. d{n-2}]: block r ranks row r (the first index of its
// maximum, sample_greedy); the last block to finish counts the rows whose
// argmax equals draft r up to the first mismatch into round_word.  Grid
// n_mtp, 1024 threads.
__global__ __launch_bounds__(1024) void k_step_accept(const float* __restrict__ logits, uint32_t V, DecodeState* st) {
    const ArgBest b = block_argmax(logits + (size_t)blockIdx.x * V, V);
    if (threadIdx.x != 0) return;
    st->row_argmax[blockIdx.x] = b.i;
    const uint32_t done = __hip_atomic_fetch_add(&st->blocks_done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (done != gridDim.x - 1u) return;
    st->blocks_done = 0u;
    uint32_t a = 0;
    while (a < gridDim.x && st->row_argmax[a] == st->draft[a]) a++;
    st->round_word = a;
}

// Pass A setup: forward `cur` at the next position.
__global__ void k_ctl_pass_a(DecodeState* st, PassDesc* pdA) {
    pdA->pos0 = st->pos;
    pdA->m = 1;
    pdA->batch = 0;
    pdA->seq0 = 0;
    pdA->tok[0] = st->cur;
    st->pos += 1;
    st->have_row4 = 0;
}

// The last verify row already holds F(cur) at position st->pos.
// The round word into the pinned host word the host reads after a decode
// segment (fine-grained host memory, one system-scope store), as the
// segment's last command.
__global__ void k_word_out(const DecodeState* st, uint32_t* out) {
    if (threadIdx.x == 0) __hip_atomic_store(out, st->round_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ void k_ctl_reuse_row(DecodeState* st) {
    st->pos += 1;
    st->have_row4 = 0;
}

// Acceptance (src/engine.cpp:333-365) of one verify segment in one launch:
// block r ranks verify row r (the first index of its maximum) into
// row_argmax, row r checking draft seg_k0 + r; the last block to finish
// (counted with a device-scope atomic; every block's row is visible to it)
// pushes the drafts while the rows' argmax equal them, commits the
// positions of the rows the reference would have forwarded, sets the next
// segment, and with greedy sampling also
// takes the corrective: Engine::sample of the first mismatching row is its
// argmax, pushed when it differs from the draft (k_sample's corrective
// without a draw).  Grid rows of the segment's largest height, 1024 threads.
__global__ __launch_bounds__(1024) void k_verify_accept(const float* __restrict__ logits, uint32_t stride, uint32_t V,
                                                        DecodeState* st, const PassDesc* __restrict__ pdB,
                                                        int32_t* tokens, uint32_t cap, int32_t greedy) {
    const uint32_t m = pdB->m, rb = blockIdx.x;
    if (rb < m) {
        const ArgBest b = block_argmax(logits + (size_t)rb * stride, V);
        if (threadIdx.x == 0) st->row_argmax[rb] = b.i;
    }
    if (threadIdx.x != 0) return;
    const uint32_t done = __hip_atomic_fetch_add(&st->blocks_done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (done != gridDim.x - 1u) return;
    st->blocks_done = 0u;
    const uint32_t n_mtp = st->n_mtp, k0 = st->seg_k0;
    uint32_t a = k0, r = 0;
    while (r < m && a < n_mtp && st->row_argmax[r] == st->draft[a]) {
        push_token(st, tokens, cap, st->draft[a]);
        a++;
        r++;
    }
    st->round_acc = a;
    st->accepted += a - k0;
    st->more = 0;
    st->have_row4 = 0;
    if (a < n_mtp && r < m) {         // mismatch at row r: rows 0..r were forwarded
        st->pos = pdB->pos0 + r + 1;
    } else if (a < n_mtp) {           // every row accepted, drafts remain: next segment
        st->pos = pdB->pos0 + m;
        st->seg_k0 = a;
        st->more = 1;
    } else if (r < m) {               // all drafts accepted; row r holds F(last draft)
        st->pos = pdB->pos0 + r;
        st->have_row4 = 1;
    } else {                          // all drafts accepted by the segment's last row
        st->pos = pdB->pos0 + m;
    }
    st->round_word = a | (st->more << 9);
    if (greedy && a < n_mtp && r < m) {   // the corrective of row r (draft a)
        const int32_t t = st->row_argmax[r];
        uint32_t pushed = 0;
        if (t != st->draft[a]) { push_token(st, tokens, cap, t); st->rejected++; pushed = 1; }
        st->round_word = a | (pushed << 8);
    }
}

// Setup of a verify segment that continues a round: rows check drafts
// k0 .. n_mtp - 1 (inputs d{k0-1} .. d{n-2}) and end with F(d{n-1}).
__global__ void k_ctl_segment(DecodeState* st, PassDesc* pdB) {
    const uint32_t k0 = st->seg_k0, m = st->n_mtp - k0 + 1;
    pdB->pos0 = st->pos;
    pdB->m = m;
    pdB->batch = 0;
    pdB->seq0 = 0;
    for (uint32_t r = 0; r < m; r++) pdB->tok[r] = st->draft[k0 - 1 + r];
}

// ------------------------------------------- multi-sequence decode rounds
//
// A batched round runs the round above for n independent sequences at
// once: row i of the base pass is sequence sel[i] (state st[sel[i]], token
// buffer tokens + sel[i] * cap, seed seeds[sel[i]]); the first nm of them
// run the MTP round and own verify rows [R i, R i + R), R = n_mtp + 1, the
// rest take the single-token step.  Every decision per sequence is the
// single-sequence one; the base pass always runs (a verify row that already
// holds F(cur) is recomputed bit for bit).

// Base pass of a batched round: row i forwards sequence sel[i]'s current
// token at its next position.  One block.
__global__ void k_bctl_pass_a(DecodeState* st, const uint32_t* __restrict__ sel, uint32_t n, PassDesc* pdA) {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        DecodeState* S = st + sel[i];
        pdA->rpos[i] = S->pos;
        pdA->rseq[i] = sel[i];
        pdA->tok[i] = S->cur;
        S->pos += 1;
        S->have_row4 = 0;
    }
    if (threadIdx.x == 0) {
        pdA->m = n;
        pdA->batch = 1;
        pdA->pos0 = 0;
        pdA->seq0 = 0;
    }
}

// Engine::sample for row i of a batched round, block i.  Roles as k_sample:
// T1 (row i of `logits`; sets up verify rows [R i, R i + R)), DRAFT k (row
// i), CORRECTIVE (verify row R i + round_acc), FALLBACK (row i).
__global__ __launch_bounds__(1024) void k_bsample(const float* __restrict__ logits, uint32_t stride, uint32_t V,
                                                  SamplingCfg cfg, const uint64_t* __restrict__ seeds,
                                                  DecodeState* st, const uint32_t* __restrict__ sel,
                                                  uint32_t row0, int32_t* tokens, uint32_t cap, PassDesc* pdB,
                                                  uint32_t R, int32_t role, int32_t k) {
    const uint32_t i = row0 + blockIdx.x, s = sel[i];
    DecodeState* S = st + s;
    __shared__ uint32_t skip;
    if (threadIdx.x == 0) skip = (role == ROLE_CORRECTIVE && S->round_acc >= R - 1) ? 1u : 0u;
    __syncthreads();
    if (skip) return;
    const uint32_t r = role == ROLE_CORRECTIVE ? R * i + S->round_acc : i;
    bool used = false;
    const int32_t t = sample_row(logits + (size_t)r * stride, V, cfg, seeds[s], S->draw, &used);
    if (threadIdx.x != 0) return;
    if (used) S->draw++;
    int32_t* tk = tokens + (size_t)s * cap;
    switch (role) {
        case ROLE_T1:
            push_token(S, tk, cap, t);
            pdB->tok[R * i] = t;
            for (uint32_t j = 0; j < R; j++) {
                pdB->rpos[R * i + j] = S->pos + j;
                pdB->rseq[R * i + j] = s;
            }
            if (blockIdx.x == 0) {
                pdB->m = R * gridDim.x;
                pdB->batch = 1;
                pdB->pos0 = 0;
                pdB->seq0 = 0;
            }
            break;
        case ROLE_DRAFT:
            S->draft[k] = t;
            pdB->tok[R * i + k + 1] = t;
            break;
        case ROLE_CORRECTIVE: {
            uint32_t a = S->round_acc;
            uint32_t pushed = 0;
            if (t != S->draft[a]) { push_token(S, tk, cap, t); S->rejected++; pushed = 1; }
            S->round_word = a | (pushed << 8);
            break;
        }
        case ROLE_FALLBACK:
            push_token(S, tk, cap, t);
            break;
        default:
            break;
    }
}

// Greedy argmax of every verify row of a batched round: row r is sequence
// sel[r / R], verify row r % R.  Grid rows, 1024 threads.
__global__ __launch_bounds__(1024) void k_bargmax_rows(const float* __restrict__ logits, uint32_t V, uint32_t R,
                                                       const uint32_t* __restrict__ sel, DecodeState* st) {
    const uint32_t r = blockIdx.x;
    ArgBest b = block_argmax(logits + (size_t)r * V, V);
    if (threadIdx.x == 0) st[sel[r / R]].row_argmax[r % R] = b.i;
}

// Acceptance of k_verify_accept for the nm MTP sequences of a batched round.
__global__ void k_bctl_accept(DecodeState* st, const uint32_t* __restrict__ sel, uint32_t nm,
                              const PassDesc* __restrict__ pdB, uint32_t R, int32_t* tokens, uint32_t cap) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nm) return;
    const uint32_t s = sel[i], n_mtp = R - 1, pos0 = pdB->rpos[R * i];
    DecodeState* S = st + s;
    int32_t* tk = tokens + (size_t)s * cap;
    uint32_t a = 0;
    while (a < n_mtp && S->row_argmax[a] == S->draft[a]) {
        push_token(S, tk, cap, S->draft[a]);
        a++;
    }
    S->round_acc = a;
    S->accepted += a;
    if (a < n_mtp) {
        S->pos = pos0 + a + 1;
        S->have_row4 = 0;
    } else {
        S->pos = pos0 + n_mtp;
        S->have_row4 = 1;
    }
    S->round_word = a;
}

}  // namespace pf
