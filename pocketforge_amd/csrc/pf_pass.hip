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

}  // namespace pf
