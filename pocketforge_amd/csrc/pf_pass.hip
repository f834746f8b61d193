// One launch for a decode pass's Q/K/V product and its attention (passes of
// at most 8 rows), for gfx950.
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
// written in this pass.  The last `tasks` workgroups load the O weights into
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
};

// LDS of k_qkv_attn: the larger of the two roles' needs.
__host__ __device__ constexpr uint32_t qkv_attn_smem(uint32_t M, uint32_t K, uint32_t nr) {
    return gemv_smem(M, K) > ag_smem_ll(nr) ? gemv_smem(M, K) : ag_smem_ll(nr);
}

// Two blocks per CU (at most 128 VGPRs: 4 waves per SIMD), so that the
// attention blocks are resident beside the QKV workgroups.
template <int FMT, int MR, int PARTS, int NR>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void k_qkv_attn(GemvArgs a, AttnGroupArgs b, uint32_t nq, uint32_t tasks) {
    extern __shared__ __align__(16) uint8_t smem[];
    if (blockIdx.x < nq) {
        gemv_body<FMT, PRO_NORM, EPI_QKV, false, 1, MR>(a, blockIdx.x, nq, smem);
        return;
    }
    const uint32_t x = blockIdx.x - nq;
    attn_group_body<PARTS, true, NR, true>(b.pd, b.g, b.kv, b.layer, b.M, nullptr, nullptr, nullptr, b.S,
                                           b.s_stride, b.Up, b.cstride, b.pf, b.lli, x % tasks, x / tasks,
                                           blockIdx.x, tasks, smem);
}

}  // namespace pf
