// One-launch stages of a decode pass (at most 8 rows), for gfx950: the
// Q/K/V product with the attention, and the chunk merge with the O, gate|up
// and down products.
//
// The attention of a one-row pass reads about 9.5 MB of cached K/V rows per
// layer at the 1B model's 2K context, and none of them depends on the pass's
// own q/k/v.  In separate launches the attention kernel can only start
// loading them after the QKV product has finished; here the attention blocks
// run beside the QKV workgroups, load their chunk's cached rows into LDS
// while the product runs, and then wait for their head's q/k/v only.
//
// Workgroups [0, nq) are the QKV GEMV's (gemv_body, pf_mm.hip, RMSNorm +
// quantize prologue and RoPE epilogue as in k_gemv), whose epilogue writes
// the rows as LL words: 8 bytes of (value bits, flag) stored with one
// device-scope store each, the flag naming the pass and the layer.  The next
// tasks * M workgroups are attention blocks (attn_group_body, pf_attn.hip,
// block (x mod tasks, x / tasks)); a block polls only the words it needs
// (its rows' q, self k and self v in its head, and the pass rows' k and v it
// quantizes) until every flag is the pass's, so a word it sees is a word
// written in this pass.  The last `tasks` workgroups load the next launch's
// weights (b.pf, b.pf2, b.pf3: O, and with k_o_ffn gate|up and down) into
// the L2 of the XCDs that will read them.
//
// Progress: each XCD receives its workgroups in id order, and the QKV
// workgroups (the lowest ids) never wait, so every QKV workgroup is running
// or finished before any attention block on its XCD can occupy its slot.  A
// wait is nevertheless bounded (LL_SPIN_MAX rounds, then *err is set for the
// host and the block goes on), so the launch always ends.
//
// Included by pf_runtime.hip after pf_mm.hip and pf_attn.hip.

namespace pf {

struct AttnGroupArgs {
    const PassDesc* pd;
    KvGeom g;
    KvPlanes kv;
    uint32_t layer, M;
    float* S;
    uint32_t s_stride;
    float* Up;
    uint32_t cstride;
    Prefetch pf;
    LLIn lli;
    Prefetch pf2, pf3;   // more weights the prefetch blocks load after pf's
};

// LDS of k_qkv_attn: the larger of the two roles' needs.
__host__ __device__ constexpr uint32_t qkv_attn_smem(uint32_t M, uint32_t K, uint32_t nr) {
    return gemv_smem(M, K) > ag_smem_ll(nr) ? gemv_smem(M, K) : ag_smem_ll(nr);
}

// Two blocks per CU (at most 128 VGPRs: 4 waves per SIMD), so that the
// attention blocks are resident beside the QKV workgroups.
template <int FMT, int MR, int PARTS, int NR>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void k_qkv_attn(uint32_t nq, uint32_t tasks, const PassDesc* pd, const uint8_t* W, const float* xr,
                                      const float* nw, GemvArgs a, AttnGroupArgs b) {
    extern __shared__ __align__(16) uint8_t smem[];
    if (blockIdx.x < nq) {
        // the operands of its first loads come preloaded into SGPRs
        gemv_body<FMT, PRO_NORM, EPI_QKV, false, 1, MR>(a, blockIdx.x, nq, smem, W, xr, nw);
        return;
    }
    const uint32_t x = blockIdx.x - nq;
    if (x / tasks >= b.M) {
        // the prefetch row: the next launch's weights into L2, once the QKV
        // product is done (its last word written), so that these loads run
        // beside the attention's arithmetic rather than its K/V loads
        const uint32_t last[1] = {3u * b.g.n_heads * b.g.head_dim - 1u};
        float lv[1];
        ll_wait<1>(b.lli.ll, last, lv, ll_epoch(b.lli.ep) * b.lli.fmul + b.lli.fadd, b.lli.err);
        prefetch_groups(b.pf, blockIdx.x, x % tasks, tasks);
        prefetch_groups(b.pf2, blockIdx.x, x % tasks, tasks);
        prefetch_groups(b.pf3, blockIdx.x, x % tasks, tasks);
        return;
    }
    attn_group_body<PARTS, true, NR, true>(pd, b.g, b.kv, b.layer, b.M, nullptr, nullptr, nullptr, b.S,
                                           b.s_stride, b.Up, b.cstride, b.pf, b.lli, x % tasks, x / tasks,
                                           blockIdx.x, tasks, smem);
}

// LDS of k_o_ffn for M rows: the largest of its GEMV roles' needs.
__host__ __device__ constexpr uint32_t o_ffn_smem(uint32_t M, uint32_t D, uint32_t F) {
    return gemv_smem(M, D) > gemv_smem(M, F) ? gemv_smem(M, D) : gemv_smem(M, F);
}

// The chunk merge of a decode pass's attention output for the columns
// 512 cb .. 512 cb + 511 of row `row`, one column per thread, as LL words to
// a.lli.ll[row D ..]: for column j of head h, with the chunks' maxima m_c, sums T_c
// and weighted values U_c (the attention's S and Up), f_c = exp(m_c - max_c
// m_c), T and U fmaf chains over c in order, U * (1 / (T + 1e-10)), the
// arithmetic of merge_quant_row before its quantization.  Loads cover
// ncap chunks (a.ncap, the buffers' capacity) so they issue before the
// pass descriptor gives the count nc; lists of more than MC chunks load the
// later chunks MC at a time (one round trip per group for the maximum and
// one for the chains).
// The inputs its loads need come as separate kernel arguments (preloaded
// into SGPRs), the rest from a.
__device__ __forceinline__ void merge_cols_ll(const GemvArgs& a, uint32_t row, uint32_t cb, const float* S,
                                              const float* Up, const uint32_t* ep, const PassDesc* pd,
                                              uint32_t s_stride, uint32_t cstride, uint32_t D, uint32_t hd,
                                              uint32_t ncap) {
    constexpr uint32_t MC = 16;
    const uint32_t hs = (uint32_t)__builtin_ctz(hd), H = D >> hs;
    const uint32_t j0 = 512u * cb + threadIdx.x, j = min(j0, D - 1u), h = j >> hs, e = j & (hd - 1u);
    const uint32_t epoch = ll_epoch(ep);
    const float* sp = S + ((size_t)row * H + h) * s_stride;
    const float* up = Up + ((size_t)row * H + h) * cstride * hd + e;
    const uint32_t ncl = ncap;
    float m[MC], ts[MC], u[MC];
#pragma unroll
    for (uint32_t c = 0; c < MC; c++) {
        const uint32_t cc = min(c, ncl - 1u);
        m[c] = sp[2u * cc];
        ts[c] = sp[2u * cc + 1u];
        u[c] = up[(size_t)cc * hd];
    }
    const uint32_t nc = (kv_view(a.g, row_pos(pass_head_late(pd), row)).count() + 1u + 255u) / 256u;
    const uint32_t flag = epoch * a.lli.fmul + a.lli.fadd;
    // the maximum over the chunk maxima (exact in any order), later groups of
    // MC chunks loaded together, one round trip per group
    float mx = m[0];
#pragma unroll
    for (uint32_t c = 1; c < MC; c++)
        if (c < nc) mx = fmaxf(mx, m[c]);
    for (uint32_t c0 = MC; c0 < nc; c0 += MC) {
        float mm[MC];
#pragma unroll
        for (uint32_t k = 0; k < MC; k++) mm[k] = sp[2u * min(c0 + k, nc - 1u)];
#pragma unroll
        for (uint32_t k = 0; k < MC; k++) mx = fmaxf(mx, mm[k]);
    }
    // T and U chains over c in order
    float T = 0.0f, U = 0.0f;
#pragma unroll
    for (uint32_t c = 0; c < MC; c++) {
        if (c < nc) {
            const float f = expf_c(m[c] - mx);
            T = __builtin_fmaf(ts[c], f, T);
            U = __builtin_fmaf(u[c], f, U);
        }
    }
    for (uint32_t c0 = MC; c0 < nc; c0 += MC) {
#pragma unroll
        for (uint32_t k = 0; k < MC; k++) {
            const uint32_t cc = min(c0 + k, nc - 1u);
            m[k] = sp[2u * cc];
            ts[k] = sp[2u * cc + 1u];
            u[k] = up[(size_t)cc * hd];
        }
#pragma unroll
        for (uint32_t k = 0; k < MC; k++) {
            if (c0 + k < nc) {
                const float f = expf_c(m[k] - mx);
                T = __builtin_fmaf(ts[k], f, T);
                U = __builtin_fmaf(u[k], f, U);
            }
        }
    }
    if (j0 < D)
        ll_store(const_cast<unsigned long long*>(a.lli.ll) + (size_t)row * D + j0, U * (1.0f / (T + 1e-10f)), flag);
}

// The rest of a decode pass's layer after the attention (M <= MR rows), in
// one launch: workgroups [0, n_mg) merge the attention's chunks into the
// rows (ceil(D / 512) per row; LL words at o.lli.ll), [n_mg, n_mg + n_o)
// are the O product's (quantize prologue over the merged rows, residual
// epilogue), the next n_gu the gate|up product's (RMSNorm + quantize
// prologue, SwiGLU epilogue), the last N / 32 the down product's (quantize
// prologue, residual epilogue).  Stage outputs are LL words: O writes the
// updated residual rows to o.e.ll ([M][D] words), gate|up its SwiGLU rows
// to gu.e.ll ([M][F] words); gate|up reads the residual rows and down
// reads both (passes of several rows stop after gate|up, which then writes
// plain rows and row maxima for a separate down launch).  The GEMV
// workgroups issue their weight loads as they start, before they wait, so
// the weights stream in while the earlier stages run; the O workgroups, once done, load the next layer's QKV
// weights (o.nx) into the L2 of the XCDs whose workgroups will read them.
// Only down writes the residual row itself (dn.e.y) and the pass's hidden
// output.
//
// Progress, as for k_qkv_attn: each XCD receives its workgroups in id order
// and a workgroup waits only for workgroups of earlier stages (lower ids),
// and the first stage waits for nothing; every wait is bounded.
template <int FMT, int CPWD, int MR>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void k_o_ffn(uint32_t n_mg, uint32_t n_o, uint32_t n_gu, const float* mS, const float* mUp, uint32_t s_stride,
             uint32_t cstride, uint32_t D, uint32_t hd, uint32_t ncap, const uint32_t* ep, const PassDesc* pd,
             GemvArgs o, GemvArgs gu, GemvArgs dn) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t b = blockIdx.x;
    if (b < n_mg) {
        const uint32_t nmr = (D + 511u) / 512u;   // merge workgroups per row (at most 4)
        uint32_t row = 0, cb = b;
        while (cb >= nmr) {   // at most 8 rows: no division on the merge's critical path
            cb -= nmr;
            row++;
        }
        merge_cols_ll(o, row, cb, mS, mUp, ep, pd, s_stride, cstride, D, hd, ncap);
    } else if (b < n_mg + n_o) {
        // several rows: O also stores the residual rows for the down launch
        constexpr int LO = MR == 1 ? (LL_IN | LL_OUT) : (LL_IN | LL_OUT | LL_COPY);
        gemv_body<FMT, PRO_QUANT, EPI_RESID, false, 1, MR, LO>(o, b - n_mg, n_o, smem, o.W, o.x, o.nw);
        prefetch_groups(o.nx, b, b - n_mg, n_o);
    } else if constexpr (MR == 1) {
        if (b < n_mg + n_o + n_gu) {
            gemv_body<FMT, PRO_NORM, EPI_SWIGLU, false, 1, 1, LL_IN | LL_OUT>(gu, b - n_mg - n_o, n_gu, smem, gu.W,
                                                                              gu.x, gu.nw);
        } else {
            const uint32_t x = b - n_mg - n_o - n_gu;
            gemv_body<FMT, PRO_QUANT, EPI_RESID, false, CPWD, 1, LL_IN | LL_OLD>(dn, x, dn.N / 32u, smem, dn.W, dn.x,
                                                                                 dn.nw);
        }
    } else {
        // several rows: the gate|up workgroups write the SwiGLU rows and their
        // row maxima to memory for a separate down launch (the down role's
        // rows and weights together exceed the registers of two workgroups
        // per CU)
        gemv_body<FMT, PRO_NORM, EPI_SWIGLU, false, 1, MR, LL_IN>(gu, b - n_mg - n_o, n_gu, smem, gu.W, gu.x, gu.nw);
    }
}

// The chunk merge of a one-row pass from the attention blocks of the same
// launch (k_layer): their chunk results are LL words at ain (S pairs, then U
// from ain + sreg), the arithmetic that of merge_cols_ll.  Lane L of a wave
// (the wave's 64 columns lie in one head) waits for chunk L's maximum and sum
// and its column's U of the first UC chunks in one round of polls; the
// maximum over the chunk maxima is a wave reduction (exact in any order) and
// the T and U chains take chunk c's f_c and sum from lane c in order.  At
// most 64 chunks.  Written to a.lli.ll like merge_cols_ll's row.
__device__ __forceinline__ void merge_cols_poll(const GemvArgs& a, uint32_t cb, const unsigned long long* ain,
                                                uint32_t sreg, uint32_t s_stride, uint32_t cstride, uint32_t D,
                                                uint32_t hd, const uint32_t* ep, const PassDesc* pd,
                                                uint32_t lay = 0u) {
    constexpr uint32_t UC = 16;
    const uint32_t lane = threadIdx.x & 63u, hs = (uint32_t)__builtin_ctz(hd);
    const uint32_t j0 = 512u * cb + threadIdx.x, j = min(j0, D - 1u), h = j >> hs, e = j & (hd - 1u);
    const uint32_t flag = ll_epoch(ep) * a.lli.fmul + a.lli.fadd + lay;
    const uint32_t nc = (kv_view(a.g, row_pos(pass_head_late(pd), 0)).count() + 1u + 255u) / 256u;
    uint32_t off[2 + UC];
    float v[2 + UC];
    const uint32_t cl = min(lane, nc - 1u);
    off[0] = h * s_stride + 2u * cl;
    off[1] = off[0] + 1u;
#pragma unroll
    for (uint32_t k = 0; k < UC; k++) off[2 + k] = sreg + (h * cstride + min(k, nc - 1u)) * hd + e;
    ll_wait<2 + UC>(ain, off, v, flag, a.lli.err);
    const float mx = wave_max(lane < nc ? v[0] : -__builtin_inff());
    const int fL = __float_as_int(expf_c(v[0] - mx)), tL = __float_as_int(v[1]);
    float uc[UC];
#pragma unroll
    for (uint32_t k = 0; k < UC; k++) uc[k] = v[2 + k];
    float T = 0.0f, U = 0.0f;
    for (uint32_t c0 = 0; c0 < nc; c0 += UC) {
        if (c0) {   // lists of more than UC chunks: the next UC chunks' U
            uint32_t o2[UC];
#pragma unroll
            for (uint32_t k = 0; k < UC; k++) o2[k] = sreg + (h * cstride + min(c0 + k, nc - 1u)) * hd + e;
            ll_wait<UC>(ain, o2, uc, flag, a.lli.err);
        }
#pragma unroll
        for (uint32_t k = 0; k < UC; k++) {
            if (c0 + k < nc) {
                const float fc = __int_as_float(__builtin_amdgcn_readlane(fL, c0 + k));
                const float tc = __int_as_float(__builtin_amdgcn_readlane(tL, c0 + k));
                T = __builtin_fmaf(tc, fc, T);
                U = __builtin_fmaf(uc[k], fc, U);
            }
        }
    }
    if (j0 < D) ll_store(const_cast<unsigned long long*>(a.lli.ll) + j0, U * (1.0f / (T + 1e-10f)), flag);
}

// One launch for a whole layer of a one-row pass: workgroups [0, nq) are
// k_qkv_attn's QKV GEMV, the next `tasks` its attention blocks (their chunk
// results as LL words at b.lli.out), then k_o_ffn's roles for one row with
// the merge reading those words (merge_cols_poll): n_mg merge, n_o O, n_gu
// gate|up, the rest down.  The O, gate|up and down workgroups wait for the
// QKV product's last word (LL_GATE) before their weight loads, so that those
// run beside the attention's arithmetic rather than its K/V loads.  At most
// 64 chunks per list.  Progress as for k_qkv_attn and k_o_ffn: every wait is
// for workgroups of lower ids, and bounded.
template <int FMT, int PARTS, int CPWD>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void k_layer(
    uint32_t nq, uint32_t tasks, uint32_t n_mg, uint32_t n_o, uint32_t n_gu, const PassDesc* pd, const uint8_t* W,
    const float* xr, const float* nw, GemvArgs a, AttnGroupArgs b, GemvArgs o, GemvArgs gu, GemvArgs dn) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t bid = blockIdx.x;
    if (bid < nq) {
        gemv_body<FMT, PRO_NORM, EPI_QKV, false, 1, 1>(a, bid, nq, smem, W, xr, nw);
        return;
    }
    uint32_t x = bid - nq;
    if (x < tasks) {
        attn_group_body<PARTS, true, 1, true>(pd, b.g, b.kv, b.layer, b.M, nullptr, nullptr, nullptr, b.S,
                                              b.s_stride, b.Up, b.cstride, b.pf, b.lli, x, 0, bid, tasks, smem);
        return;
    }
    x -= tasks;
    if (x < n_mg) {
        merge_cols_poll(o, x, b.lli.out, b.lli.sreg, b.s_stride, b.cstride, o.K, o.e.hd, o.lli.ep, pd);
        return;
    }
    x -= n_mg;
    if (x < n_o) {
        gemv_body<FMT, PRO_QUANT, EPI_RESID, false, 1, 1, LL_IN | LL_OUT | LL_GATE>(o, x, n_o, smem, o.W, o.x, o.nw);
        prefetch_groups(o.nx, bid, x, n_o);
        return;
    }
    x -= n_o;
    if (x < n_gu) {
        gemv_body<FMT, PRO_NORM, EPI_SWIGLU, false, 1, 1, LL_IN | LL_OUT | LL_GATE>(gu, x, n_gu, smem, gu.W, gu.x,
                                                                                    gu.nw);
        return;
    }
    x -= n_gu;
    gemv_body<FMT, PRO_QUANT, EPI_RESID, false, CPWD, 1, LL_IN | LL_OLD | LL_GATE>(dn, x, dn.N / 32u, smem, dn.W,
                                                                                   dn.x, dn.nw);
}

// A pass's first launch: the pooled rows it can see (k_pool_rows, blocks
// [0, n_pool): layers * heads per pooled-row slot ny) and its embedded rows
// with the epoch advance (k_embed, 128 columns per block), two independent
// jobs in one launch.  128 threads.
__global__ __launch_bounds__(128) void k_pass_prep(KvGeom g, KvPlanes kv, const PassDesc* __restrict__ pd,
                                                   uint32_t n_pool, const uint8_t* __restrict__ codes,
                                                   const uint16_t* __restrict__ scales, uint32_t V, uint32_t D,
                                                   float* __restrict__ x, uint32_t* __restrict__ ep, int32_t fmt) {
    const uint32_t b = blockIdx.x, lh = g.n_layers * g.n_heads;
    if (b < n_pool) {
        pool_rows_block(g, kv, pd, b % lh, b / lh);
        return;
    }
    const uint32_t e = b - n_pool, nbx = (D + 127u) / 128u, m = e / nbx;
    embed_elem(codes, scales, V, D, pd, x, ep, fmt, m, (e - m * nbx) * 128u + threadIdx.x);
}

// Per-layer operands of k_stack.
struct StackLayer {
    const uint8_t *qkv, *o, *gu, *dn;   // packed matrices
    const float *an, *fn;               // attention and FFN norm weights [D]
};

// The gate|up and down formats k_stack is built for: all Q4, or Q2 gate|up
// with Q1.5 down (the QKV and O matrices Q4 in both).
inline bool stack_fmts(int32_t fg, int32_t fd) {
    return (fg == FMT_Q4 && fd == FMT_Q4) || (fg == FMT_Q2 && fd == FMT_Q15);
}

// Every layer of a one-row pass in one launch: layer l's workgroups are
// [l G, (l + 1) G), laid out as k_layer's (QKV, attention, merge, O,
// gate|up, down).  Layer l's down product hands the updated residual row to
// layer l + 1 as LL words (dn.e.ll, flagged for layer l + 1): its QKV
// workgroups read them as the prologue's input and its O workgroups as the
// residual; layer 0 reads the embedded row a.x / o.e.y from memory and the
// last layer's down writes dn.e.y (and dn.e.y2) to memory.  A layer's
// workgroups start while the layer before runs, so their weight loads (and
// the attention's cached K/V loads) overlap its arithmetic.  Flags are
// epoch * layers + layer (the args carry fadd = 0; each role adds its layer).
// Progress as for k_layer: every wait is for workgroups of lower ids (the
// layer before, or earlier roles of the layer), and bounded.  FMT is the
// format of the QKV and O matrices, FG of gate|up, FD of down.
template <int FMT, int FG, int FD, int PARTS, int CPWD>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void k_stack(
    uint32_t nq, uint32_t tasks, uint32_t n_mg, uint32_t n_o, uint32_t n_gu, uint32_t G, const PassDesc* pd,
    const StackLayer* lw, GemvArgs a, AttnGroupArgs b, GemvArgs o, GemvArgs gu, GemvArgs dn) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t bid = blockIdx.x, l = bid / G;
    uint32_t x = bid - l * G;
    const StackLayer& w = lw[l];
    if (x < nq) {
        if (l == 0) gemv_body<FMT, PRO_NORM, EPI_QKV, false, 1, 1>(a, x, nq, smem, w.qkv, a.x, w.an, 0u);
        else gemv_body<FMT, PRO_NORM, EPI_QKV, false, 1, 1, LL_IN | LL_GATE>(a, x, nq, smem, w.qkv, a.x, w.an, l);
        return;
    }
    x -= nq;
    if (x < tasks) {
        LLIn li = b.lli;
        li.fadd = l;
        if (l == 0) li.gate = nullptr;
        attn_group_body<PARTS, true, 1, true>(pd, b.g, b.kv, l, b.M, nullptr, nullptr, nullptr, b.S, b.s_stride,
                                              b.Up, b.cstride, b.pf, li, x, 0, bid, tasks, smem);
        return;
    }
    x -= tasks;
    if (x < n_mg) {
        merge_cols_poll(o, x, b.lli.out, b.lli.sreg, b.s_stride, b.cstride, o.K, o.e.hd, o.lli.ep, pd, l);
        return;
    }
    x -= n_mg;
    if (x < n_o) {
        if (l == 0)
            gemv_body<FMT, PRO_QUANT, EPI_RESID, false, 1, 1, LL_IN | LL_OUT | LL_GATE>(o, x, n_o, smem, w.o, o.x,
                                                                                        o.nw, 0u);
        else
            gemv_body<FMT, PRO_QUANT, EPI_RESID, false, 1, 1, LL_IN | LL_OLD | LL_OUT | LL_GATE>(o, x, n_o, smem, w.o,
                                                                                                 o.x, o.nw, l);
        return;
    }
    x -= n_o;
    if (x < n_gu) {
        gemv_body<FG, PRO_NORM, EPI_SWIGLU, false, 1, 1, LL_IN | LL_OUT | LL_GATE>(gu, x, n_gu, smem, w.gu, gu.x,
                                                                                   w.fn, l);
        return;
    }
    x -= n_gu;
    if (l + 1 < a.e.fmul)
        gemv_body<FD, PRO_QUANT, EPI_RESID, false, CPWD, 1, LL_IN | LL_OLD | LL_OUT | LL_NEXT | LL_GATE>(
            dn, x, dn.N / 32u, smem, w.dn, dn.x, dn.nw, l);
    else
        gemv_body<FD, PRO_QUANT, EPI_RESID, false, CPWD, 1, LL_IN | LL_OLD | LL_GATE>(dn, x, dn.N / 32u, smem, w.dn,
                                                                                      dn.x, dn.nw, l);
}

// LDS of k_layer and k_stack: the attention blocks' need is the largest.
__host__ __device__ constexpr uint32_t layer_smem(uint32_t D, uint32_t F) {
    return qkv_attn_smem(1, D, 1) > o_ffn_smem(1, D, F) ? qkv_attn_smem(1, D, 1) : o_ffn_smem(1, D, F);
}

}  // namespace pf
