// Host runtime of libpocketforge_amd.so: implements include/pf_gpu.h on
// top of the gfx950 kernels (single translation unit with the kernels).
#include "pf_gemv.hip"
#include "pf_mm.hip"
#include "pf_attn.hip"
#include "pf_pass.hip"
#include "pf_ctl.hip"

#include <hip/hip_ext.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/pf_gpu.h"

using namespace pf;

// ================================================================ context

struct pf_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    size_t bytes = 0;
    // growable scratch for the kernel-level entry points
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
};

static pf_status fail(const pf_ctx* c, pf_status s, const std::string& msg) {
    if (c) const_cast<pf_ctx*>(c)->err = msg;
    return s;
}

#define PF_HIP(ctx, call)                                                                        \
    do {                                                                                         \
        hipError_t e_ = (call);                                                                  \
        if (e_ != hipSuccess)                                                                    \
            return fail(ctx, PF_ERR_HIP, std::string(#call) + " failed: " + hipGetErrorString(e_)); \
    } while (0)

#define PF_LAUNCHED(ctx) PF_HIP(ctx, hipGetLastError())

static pf_status dalloc(pf_ctx* c, void** p, size_t bytes) {
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) return fail(c, PF_ERR_HIP, "hipMalloc(" + std::to_string(bytes) + ") failed: " + hipGetErrorString(e));
    c->bytes += bytes;
    return PF_OK;
}

static void dfree(pf_ctx* c, void* p, size_t bytes) {
    if (!p) return;
    (void)hipFree(p);
    if (bytes == 0) bytes = 256;
    c->bytes -= std::min(c->bytes, bytes);
}

template <class T>
static pf_status dalloc_t(pf_ctx* c, T** p, size_t n) {
    return dalloc(c, reinterpret_cast<void**>(p), n * sizeof(T));
}

static pf_status ctx_scratch(pf_ctx* c, size_t bytes, void** out) {
    if (bytes > c->scratch_bytes) {
        if (c->scratch) {
            PF_HIP(c, hipStreamSynchronize(c->stream));
            dfree(c, c->scratch, c->scratch_bytes);
            c->scratch = nullptr;
            c->scratch_bytes = 0;
        }
        pf_status s = dalloc(c, &c->scratch, bytes);
        if (s) return s;
        c->scratch_bytes = bytes;
    }
    *out = c->scratch;
    return PF_OK;
}

static std::string g_init_error;

// Fixed scratch of pf_gemv_q_noalloc: the int8 activation rows of its
// M > 8 path (ceil(M / 32) * 32 rows of K codes) followed by their M fp32
// scales.  Each GPU holds its own copy until the process ends; host code
// reaches a GPU's copy only through the address that hipGetSymbolAddress
// gave for that GPU (g_scratch_dev), resolved once per device by pf_init.
constexpr size_t NOALLOC_ACT_BYTES = (size_t)1 << 20;
constexpr size_t NOALLOC_SCALE_BYTES = 512 * 4;
static __device__ __align__(256) uint8_t scratch[NOALLOC_ACT_BYTES + NOALLOC_SCALE_BYTES];
constexpr int MAX_DEVICES = 64;
static void* g_scratch_dev[MAX_DEVICES];
static std::mutex g_scratch_mu;

// With `device` current: the device address of its scratch copy.
static hipError_t resolve_scratch(int device) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_dev[device]) return hipSuccess;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_dev[device] = p;
    return hipSuccess;
}

extern "C" pf_status pf_init(int device, pf_ctx** out) {
    if (!out) return PF_ERR_ARG;
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) { g_init_error = std::string("hipGetDeviceCount: ") + hipGetErrorString(e); return PF_ERR_HIP; }
    if (device < 0 || device >= n) { g_init_error = "device index out of range"; return PF_ERR_ARG; }
    e = hipSetDevice(device);
    if (e != hipSuccess) { g_init_error = std::string("hipSetDevice: ") + hipGetErrorString(e); return PF_ERR_HIP; }
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) { g_init_error = std::string("hipGetDeviceProperties: ") + hipGetErrorString(e); return PF_ERR_HIP; }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        g_init_error = std::string("device is ") + prop.gcnArchName + ", not gfx950";
        return PF_ERR_UNSUPPORTED;
    }
    if (device >= MAX_DEVICES) { g_init_error = "device index beyond the library's table"; return PF_ERR_ARG; }
    e = resolve_scratch(device);
    if (e != hipSuccess) { g_init_error = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e); return PF_ERR_HIP; }
    pf_ctx* c = new pf_ctx();
    c->device = device;
    e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        g_init_error = std::string("hipStreamCreateWithFlags: ") + hipGetErrorString(e);
        delete c;
        return PF_ERR_HIP;
    }
    *out = c;
    return PF_OK;
}

extern "C" void pf_destroy(pf_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    if (c->scratch) (void)hipFree(c->scratch);
    (void)hipStreamDestroy(c->stream);
    delete c;
}

extern "C" const char* pf_last_error(const pf_ctx* c) { return c ? c->err.c_str() : g_init_error.c_str(); }

extern "C" pf_status pf_malloc(pf_ctx* c, size_t bytes, void** out) {
    if (!c || !out) return PF_ERR_ARG;
    return dalloc(c, out, bytes);
}

extern "C" pf_status pf_free(pf_ctx* c, void* p, size_t bytes) {
    if (!c) return PF_ERR_ARG;
    PF_HIP(c, hipStreamSynchronize(c->stream));
    dfree(c, p, bytes);
    return PF_OK;
}

extern "C" pf_status pf_memcpy(pf_ctx* c, void* dst, const void* src, size_t bytes, int32_t kind) {
    if (!c || (!dst && bytes) || (!src && bytes)) return PF_ERR_ARG;
    hipMemcpyKind k = kind == 0 ? hipMemcpyHostToDevice : (kind == 1 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice);
    PF_HIP(c, hipMemcpyAsync(dst, src, bytes, k, c->stream));
    PF_HIP(c, hipStreamSynchronize(c->stream));
    return PF_OK;
}

extern "C" pf_status pf_device_info(pf_ctx* c, char* name, size_t len, int* cus) {
    if (!c) return PF_ERR_ARG;
    hipDeviceProp_t prop;
    PF_HIP(c, hipGetDeviceProperties(&prop, c->device));
    if (name && len) std::snprintf(name, len, "%s (%s)", prop.name, prop.gcnArchName);
    if (cus) *cus = prop.multiProcessorCount;
    return PF_OK;
}

extern "C" pf_status pf_synchronize(pf_ctx* c) {
    if (!c) return PF_ERR_ARG;
    PF_HIP(c, hipStreamSynchronize(c->stream));
    return PF_OK;
}

extern "C" size_t pf_device_bytes(const pf_ctx* c) { return c ? c->bytes : 0; }

// ============================================================== matrices

struct pf_matrix {
    pf_ctx* ctx = nullptr;
    int32_t fmt = 0;
    uint32_t rows = 0, cols = 0;
    bool rowmajor = false;
    bool ilv = false;           // halves [0, rows/2) and [rows/2, rows) interleaved by 16 rows
    uint8_t* data = nullptr;    // 32-row group tiles; row-major: codes
    uint16_t* scales = nullptr; // row-major only
    uint8_t* xmin = nullptr;    // tiled only: per device row, smallest binade of its nonzero block scales
    std::vector<uint8_t> xmin_host;
    size_t bytes = 0;
};

// Smallest binade max(biased exponent, 1) of a row's nonzero fp16 block
// scales (1 for a row of zero scales): the unit of the GEMM's integer sums.
static uint8_t row_xmin(const uint16_t* sc, uint32_t nb) {
    int xm = 31;
    for (uint32_t b = 0; b < nb; b++) {
        if ((sc[b] & 0x7FFF) == 0) continue;
        const int e = (sc[b] >> 10) & 31;
        xm = std::min(xm, e ? e : 1);
    }
    return (uint8_t)(xm == 31 ? 1 : xm);
}

static uint32_t interchange_code(int fmt, const uint8_t* blk, uint32_t e) {
    if (fmt == FMT_Q4) return (e & 1u) ? (blk[e >> 1] >> 4) : (blk[e >> 1] & 15u);
    return (blk[e >> 2] >> (2 * (e & 3u))) & 3u;
}

// Checks the exact-sum condition of one row: nonzero block scales within 15
// binades of each other; Q1.5 codes in {0,1,2}.
static pf_status check_row(const pf_ctx* c, int fmt, const uint8_t* codes, const uint16_t* sc, uint32_t nb,
                           uint32_t row) {
    int emax = -1, emin = 99;
    for (uint32_t b = 0; b < nb; b++) {
        uint16_t h = sc[b];
        if ((h & 0x7FFF) == 0) continue;
        int e = (h >> 10) & 31;
        if (e == 31) return fail(c, PF_ERR_RANGE, "row " + std::to_string(row) + ": non-finite block scale");
        if (e == 0) e = 1;
        emax = std::max(emax, e);
        emin = std::min(emin, e);
    }
    if (emax >= 0 && emax - emin > 15)
        return fail(c, PF_ERR_RANGE, "row " + std::to_string(row) +
                                         ": block scales span more than 15 binades (exact fp64 block sums would not hold)");
    if (fmt == FMT_Q15) {
        for (uint32_t b = 0; b < nb * 8; b++)
            for (int t = 0; t < 4; t++)
                if (((codes[b] >> (2 * t)) & 3u) == 3u)
                    return fail(c, PF_ERR_RANGE, "row " + std::to_string(row) + ": Q1.5 code 3 is not a ternary code");
    }
    return PF_OK;
}

// Device row of logical row r (pf_layout.h: the fused gate|up matrix
// interleaves its halves by 16 rows).
static uint32_t device_row(const pf_matrix* M, uint32_t r) {
    if (!M->ilv) return r;
    const uint32_t half = M->rows / 2, hi = r >= half ? 1u : 0u, j = r - hi * half;
    return 32u * (j / 16u) + 16u * hi + (j % 16u);
}

// Writes one interchange row (codes [cols/32][code_bytes], fp16 scales
// [cols/32]) as row r of a 32-row group whose tiles start at gtiles.
static void pack_row(int fmt, uint32_t cols, const uint8_t* codes, const uint16_t* scales, uint32_t r,
                     uint8_t* gtiles) {
    const uint32_t nb = cols / 32, bb = code_bytes(fmt), TB = g32_tile_bytes(fmt), CODES = g32_code_bytes(fmt);
    for (uint32_t b = 0; b < nb; b++) {
        uint8_t* tile = gtiles + (size_t)(b / 8) * TB;
        const uint32_t t = b % 8;
        const uint8_t* blk = codes + (size_t)b * bb;
        std::memcpy(tile + CODES + r * 16 + t * 2, &scales[b], 2);
        for (uint32_t h = 0; h < 2; h++) {
            const uint32_t lane = r + 32 * h;
            if (fmt == FMT_Q8) {
                std::memcpy(tile + t * 1024 + lane * 16, blk + 16 * h, 16);
            } else if (fmt == FMT_Q4) {
                uint8_t* dst = tile + (t >> 1) * 1024 + lane * 16 + (t & 1) * 8;
                for (uint32_t j = 0; j < 8; j++)
                    dst[j] = (uint8_t)(interchange_code(fmt, blk, 16 * h + j) |
                                       (interchange_code(fmt, blk, 16 * h + j + 8) << 4));
            } else {
                uint8_t* dst = tile + (t >> 2) * 1024 + lane * 16 + (t & 3) * 4;
                for (uint32_t j = 0; j < 4; j++) {
                    uint32_t v = 0;
                    for (uint32_t u = 0; u < 4; u++) v |= interchange_code(fmt, blk, 16 * h + 4 * u + j) << (2 * u);
                    dst[j] = (uint8_t)v;
                }
            }
        }
    }
}

static pf_status matrix_alloc(pf_ctx* c, int32_t fmt, uint32_t rows, uint32_t cols, bool rowmajor, pf_matrix** out,
                              bool ilv = false) {
    if (fmt != FMT_Q4 && fmt != FMT_Q2 && fmt != FMT_Q15 && fmt != FMT_Q8) return fail(c, PF_ERR_ARG, "unknown format");
    if (cols % 256 || rows % 64 || rows == 0 || cols == 0)
        return fail(c, PF_ERR_UNSUPPORTED, "matrix shape must have rows % 64 == 0 and cols % 256 == 0");
    if (rowmajor && ((fmt != FMT_Q4 && fmt != FMT_Q8) || cols > 2048))
        return fail(c, PF_ERR_UNSUPPORTED, "fp32-activation matrices must be Q4 or Q8 with cols <= 2048");
    if (!rowmajor && cols > 8192) return fail(c, PF_ERR_UNSUPPORTED, "int8-activation matrices need cols <= 8192");
    pf_matrix* M = new pf_matrix();
    M->ctx = c; M->fmt = fmt; M->rows = rows; M->cols = cols; M->rowmajor = rowmajor; M->ilv = ilv;
    const uint32_t nb = cols / 32;
    if (rowmajor) {
        M->bytes = (size_t)rows * nb * code_bytes(fmt);
        pf_status s = dalloc_t(c, &M->data, M->bytes);
        if (!s) s = dalloc_t(c, &M->scales, (size_t)rows * nb);
        if (s) { delete M; return s; }
    } else {
        M->bytes = (size_t)(rows / 32) * (cols / 256) * g32_tile_bytes(fmt);
        pf_status s = dalloc_t(c, &M->data, M->bytes);
        if (!s) s = dalloc_t(c, &M->xmin, rows);
        if (s) {
            if (M->data) dfree(c, M->data, M->bytes);
            delete M;
            return s;
        }
        M->xmin_host.assign(rows, 1);
    }
    *out = M;
    return PF_OK;
}

// Uploads interchange rows [r0, r0 + n) of a matrix.  A 32-row group that
// the upload covers only in part keeps its other rows (its tiles are read
// back, patched and written).
static pf_status matrix_put(pf_matrix* M, uint32_t r0, uint32_t n, const uint8_t* codes, const uint16_t* scales) {
    pf_ctx* c = M->ctx;
    const uint32_t nb = M->cols / 32, bb = code_bytes(M->fmt);
    if (n == 0) return PF_OK;
    if ((uint64_t)r0 + n > M->rows) return fail(c, PF_ERR_ARG, "rows beyond the matrix");
    for (uint32_t r = 0; r < n; r++) {
        pf_status s = check_row(c, M->fmt, codes + (size_t)r * nb * bb, scales + (size_t)r * nb, nb, r0 + r);
        if (s) return s;
    }
    if (M->rowmajor) {
        PF_HIP(c, hipMemcpy(M->data + (size_t)r0 * nb * bb, codes, (size_t)n * nb * bb, hipMemcpyHostToDevice));
        PF_HIP(c, hipMemcpy(M->scales + (size_t)r0 * nb, scales, (size_t)n * nb * 2, hipMemcpyHostToDevice));
        return PF_OK;
    }
    const size_t gbytes = (size_t)(M->cols / 256) * g32_tile_bytes(M->fmt);
    uint32_t g_lo = UINT32_MAX, g_hi = 0;
    for (uint32_t r = r0; r < r0 + n; r++) {
        const uint32_t g = device_row(M, r) / 32;
        g_lo = std::min(g_lo, g);
        g_hi = std::max(g_hi, g);
    }
    std::vector<uint8_t> buf((size_t)(g_hi - g_lo + 1) * gbytes);
    const bool whole = !M->ilv && r0 % 32 == 0 && n % 32 == 0;
    if (!whole) PF_HIP(c, hipMemcpy(buf.data(), M->data + g_lo * gbytes, buf.size(), hipMemcpyDeviceToHost));
    for (uint32_t r = r0; r < r0 + n; r++) {
        const uint32_t dr = device_row(M, r);
        pack_row(M->fmt, M->cols, codes + (size_t)(r - r0) * nb * bb, scales + (size_t)(r - r0) * nb, dr % 32,
                 buf.data() + (size_t)(dr / 32 - g_lo) * gbytes);
        M->xmin_host[dr] = row_xmin(scales + (size_t)(r - r0) * nb, nb);
    }
    PF_HIP(c, hipMemcpy(M->data + g_lo * gbytes, buf.data(), buf.size(), hipMemcpyHostToDevice));
    PF_HIP(c, hipMemcpy(M->xmin, M->xmin_host.data(), M->rows, hipMemcpyHostToDevice));
    return PF_OK;
}

extern "C" pf_status pf_matrix_upload(pf_ctx* c, int32_t fmt, uint32_t rows, uint32_t cols, const uint8_t* codes,
                                      const uint16_t* scales, int32_t rowmajor, pf_matrix** out) {
    if (!c || !codes || !scales || !out) return PF_ERR_ARG;
    pf_matrix* M = nullptr;
    pf_status s = matrix_alloc(c, fmt, rows, cols, rowmajor != 0, &M);
    if (s) return s;
    s = matrix_put(M, 0, rows, codes, scales);
    if (s) { pf_matrix_free(M); return s; }
    *out = M;
    return PF_OK;
}

extern "C" void pf_matrix_free(pf_matrix* M) {
    if (!M) return;
    dfree(M->ctx, M->data, M->bytes);
    if (M->scales) dfree(M->ctx, M->scales, (size_t)M->rows * (M->cols / 32) * 2);
    if (M->xmin) dfree(M->ctx, M->xmin, M->rows);
    delete M;
}

// ------------------------------------------------------- kernel launches

// Instances of k_gemv / k_gemm in use: (prologue, epilogue, gated).
enum MmKind : int {
    MM_QKV = 0,       // NORM -> QKV                 (attention input)
    MM_O = 1,         // INT8 -> RESID               (O projection)
    MM_GU = 2,        // NORM -> SWIGLU              (gate|up)
    MM_GU_SKIP = 3,   // QUANT -> SWIGLU, gated      (gate|up on staged normed rows, layer skip)
    MM_DOWN = 4,      // QPART -> RESID              (down)
    MM_DOWN_SKIP = 5, // QPART -> RESID, gated       (down, layer skip)
    MM_STORE = 6,     // QUANT -> STORE              (kernel-level entry point)
    MM_O_MERGE = 7,   // MERGE -> RESID              (O projection of a one-row pass, chunk merge fused)
};

template <int F, int PRO, int EPI, bool G, int CPW, int MR>
static void gemv_one(hipStream_t st, const GemvArgs& a, hipEvent_t ev0, hipEvent_t ev1) {
    const uint32_t smem = gemv_smem(a.M, a.K) + (PRO == PRO_MERGE ? GEMV_MERGE_SMEM : 0u);
    static bool attr = false;   // LDS beyond 64 KiB is granted per kernel
    if (!attr) {
        (void)hipFuncSetAttribute((const void*)k_gemv<F, PRO, EPI, G, CPW, MR>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, gemv_smem(GEMV_MAX_M, 8192));
        attr = true;
    }
    const dim3 grid(a.N / 32 + (a.nx.p ? a.nx.blocks : 0u));
    if (ev0)
        hipExtLaunchKernelGGL((k_gemv<F, PRO, EPI, G, CPW, MR>), grid, dim3(64 * GEMV_WAVES), smem, st, ev0, ev1, 0, a);
    else
        hipLaunchKernelGGL((k_gemv<F, PRO, EPI, G, CPW, MR>), grid, dim3(64 * GEMV_WAVES), smem, st, a);
}

// Rows held in registers: 1 (base passes), 5 (verify passes of four
// heads), else 8.
template <int F, int PRO, int EPI, bool G, int CPW>
static void gemv_mr(hipStream_t st, const GemvArgs& a, hipEvent_t ev0, hipEvent_t ev1) {
    if (a.M == 1) gemv_one<F, PRO, EPI, G, CPW, 1>(st, a, ev0, ev1);
    else if (a.M <= 5) gemv_one<F, PRO, EPI, G, CPW, 5>(st, a, ev0, ev1);
    else gemv_one<F, PRO, EPI, G, CPW, 8>(st, a, ev0, ev1);
}

// Chunks per wave of a K-column product: products over n_embd (<= 2048)
// take one, those over n_ff up to four.
template <int F, int PRO, int EPI, bool G>
static void gemv_cpw(hipStream_t st, const GemvArgs& a, hipEvent_t ev0, hipEvent_t ev1) {
    const uint32_t cpw = (a.K / 256 + GEMV_WAVES - 1) / GEMV_WAVES;
    if (cpw <= 1) gemv_mr<F, PRO, EPI, G, 1>(st, a, ev0, ev1);
    else if (cpw == 2) gemv_mr<F, PRO, EPI, G, 2>(st, a, ev0, ev1);
    else if (cpw == 3) gemv_mr<F, PRO, EPI, G, 3>(st, a, ev0, ev1);
    else gemv_mr<F, PRO, EPI, G, 4>(st, a, ev0, ev1);
}

template <int F, int EPI, bool G, int MW, int NW, int KW, int DI>
static void gemm_tiled(hipStream_t st, const GemmArgs& a, hipEvent_t ev0, hipEvent_t ev1) {
    const dim3 grid((a.N / 32 + NW - 1) / NW, (a.M + 32 * MW - 1) / (32 * MW));
    if (ev0) hipExtLaunchKernelGGL((k_gemm<F, EPI, G, MW, NW, KW, DI>), grid, dim3(512), 0, st, ev0, ev1, 0, a);
    else hipLaunchKernelGGL((k_gemm<F, EPI, G, MW, NW, KW, DI>), grid, dim3(512), 0, st, a);
}

// Workgroup shapes measured at M = 320 on the 1B products: matrices of at
// least 4096 rows take 32 activation rows x 8 row groups per workgroup;
// narrower ones split K over two wave sets (32 x 4 x 2) so that the chip
// still gets enough workgroups.  Every wave issues its chunk's 8 MFMAs
// before their integer scaling.
template <int F, int EPI, bool G>
static void gemm_one(hipStream_t st, const GemmArgs& a, hipEvent_t ev0, hipEvent_t ev1) {
    if (a.N >= 4096) gemm_tiled<F, EPI, G, 1, 8, 1, 8>(st, a, ev0, ev1);
    else gemm_tiled<F, EPI, G, 1, 4, 2, 8>(st, a, ev0, ev1);
}

#define PF_MM_FMT(fmt, CALL)                                  \
    switch (fmt) {                                            \
        case FMT_Q4: { constexpr int F = FMT_Q4; CALL; } break; \
        case FMT_Q2: { constexpr int F = FMT_Q2; CALL; } break; \
        case FMT_Q8: { constexpr int F = FMT_Q8; CALL; } break; \
        default: { constexpr int F = FMT_Q15; CALL; } break;    \
    }

// M <= 8 rows: one workgroup per 32-row group over all of K (products over
// n_embd hold one chunk per wave).
static void launch_gemv(hipStream_t st, const pf_matrix* W, MmKind kind, const GemvArgs& a, hipEvent_t ev0 = nullptr,
                        hipEvent_t ev1 = nullptr) {
    switch (kind) {
        case MM_QKV: PF_MM_FMT(W->fmt, (gemv_mr<F, PRO_NORM, EPI_QKV, false, 1>(st, a, ev0, ev1))) break;
        case MM_O: PF_MM_FMT(W->fmt, (gemv_mr<F, PRO_INT8, EPI_RESID, false, 1>(st, a, ev0, ev1))) break;
        case MM_O_MERGE: PF_MM_FMT(W->fmt, (gemv_one<F, PRO_MERGE, EPI_RESID, false, 1, 1>(st, a, ev0, ev1))) break;
        case MM_GU: PF_MM_FMT(W->fmt, (gemv_mr<F, PRO_NORM, EPI_SWIGLU, false, 1>(st, a, ev0, ev1))) break;
        case MM_GU_SKIP: PF_MM_FMT(W->fmt, (gemv_mr<F, PRO_QUANT, EPI_SWIGLU, true, 1>(st, a, ev0, ev1))) break;
        case MM_DOWN: PF_MM_FMT(W->fmt, (gemv_cpw<F, PRO_QPART, EPI_RESID, false>(st, a, ev0, ev1))) break;
        case MM_DOWN_SKIP: PF_MM_FMT(W->fmt, (gemv_cpw<F, PRO_QPART, EPI_RESID, true>(st, a, ev0, ev1))) break;
        default:
            PF_MM_FMT(W->fmt, ({
                          const uint32_t cpw = (a.K / 256 + GEMV_WAVES - 1) / GEMV_WAVES;
                          if (cpw <= 1) gemv_one<F, PRO_QUANT, EPI_STORE, false, 1, 8>(st, a, ev0, ev1);
                          else if (cpw == 2) gemv_one<F, PRO_QUANT, EPI_STORE, false, 2, 8>(st, a, ev0, ev1);
                          else if (cpw == 3) gemv_one<F, PRO_QUANT, EPI_STORE, false, 3, 8>(st, a, ev0, ev1);
                          else gemv_one<F, PRO_QUANT, EPI_STORE, false, 4, 8>(st, a, ev0, ev1);
                      }))
            break;
    }
}

// M > 8 rows: activation rows quantized beforehand (int8 + scales).
static void launch_gemm(hipStream_t st, const pf_matrix* W, MmKind kind, GemmArgs a, hipEvent_t ev0 = nullptr,
                        hipEvent_t ev1 = nullptr) {
    a.xmin = W->xmin;
    switch (kind) {
        case MM_QKV: PF_MM_FMT(W->fmt, (gemm_one<F, EPI_QKV, false>(st, a, ev0, ev1))) break;
        case MM_O:
        case MM_DOWN: PF_MM_FMT(W->fmt, (gemm_one<F, EPI_RESID, false>(st, a, ev0, ev1))) break;
        case MM_GU: PF_MM_FMT(W->fmt, (gemm_one<F, EPI_SWIGLU, false>(st, a, ev0, ev1))) break;
        case MM_GU_SKIP: PF_MM_FMT(W->fmt, (gemm_one<F, EPI_SWIGLU, true>(st, a, ev0, ev1))) break;
        case MM_DOWN_SKIP: PF_MM_FMT(W->fmt, (gemm_one<F, EPI_RESID, true>(st, a, ev0, ev1))) break;
        default: PF_MM_FMT(W->fmt, (gemm_one<F, EPI_STORE, false>(st, a, ev0, ev1))) break;
    }
}

constexpr uint32_t MAX_GEMM_ROWS = 512;
static_assert(NOALLOC_SCALE_BYTES >= MAX_GEMM_ROWS * 4, "one scale per GEMM row");

// y[m] (+= y_in[m]) = h[m] x dequantized rows, any M (launches of up to 8
// rows; each row's result does not depend on the rows beside it).
// Rows per slice of the fp32 GEMVs: 4 staged rows (128 VGPRs) leave room
// for two waves per SIMD, where 8 rows (256 VGPRs) run one (64 sequences x
// 4 MTP heads: 49.2 -> 46.6 ms per round); the weights are read once per
// slice, from L2.
constexpr uint32_t F32_GROUP = 4;

static void launch_gemv_f32(hipStream_t st, const pf_matrix* W, uint32_t M, const float* h, uint32_t h_stride,
                            float* y, uint32_t y_stride, const float* y_in, uint32_t max_waves = 4096) {
    uint32_t waves = std::min<uint32_t>(W->rows, max_waves);
    // whole groups of F32_GROUP rows in one launch (grid y), then the rest
    constexpr uint32_t GR = F32_GROUP;
    for (uint32_t r0 = 0; r0 < M;) {
        const uint32_t mb = std::min(GR, M - r0);
        const dim3 grid((waves + 3) / 4, mb == GR ? (M - r0) / GR : 1u);
        const float* hr = h + (size_t)r0 * h_stride;
        float* yr = y + (size_t)r0 * y_stride;
        const float* yi = y_in ? y_in + (size_t)r0 * y_stride : nullptr;
#define PF_F32_CASE(MM)                                                                                       \
    case MM:                                                                                                  \
        if (W->fmt == FMT_Q8)                                                                                 \
            hipLaunchKernelGGL((k_gemv_f32<MM, FMT_Q8>), grid, dim3(256), 0, st, W->data, W->scales, W->rows,   \
                               W->cols, hr, h_stride, yr, y_stride, yi);                                      \
        else                                                                                                  \
            hipLaunchKernelGGL((k_gemv_f32<MM, FMT_Q4>), grid, dim3(256), 0, st, W->data, W->scales, W->rows,   \
                               W->cols, hr, h_stride, yr, y_stride, yi);                                      \
        break;
        switch (mb) {
            PF_F32_CASE(1) PF_F32_CASE(2) PF_F32_CASE(3) PF_F32_CASE(4)
            PF_F32_CASE(5) PF_F32_CASE(6) PF_F32_CASE(7) PF_F32_CASE(8)
        }
#undef PF_F32_CASE
        r0 += mb * grid.y;
    }
}

// Gate and up products of one MTP head with the SiLU product fused:
// a[m] = silu(Wg h[m]) * (Wu h[m]), rows in chunks of 8.
static void launch_gemv_f32_glu(hipStream_t st, const pf_matrix* Wg, const pf_matrix* Wu, uint32_t M, const float* h,
                                uint32_t h_stride, float* a, uint32_t a_stride, uint32_t max_waves = 2048) {
    uint32_t waves = std::min<uint32_t>(Wg->rows, max_waves);
    constexpr uint32_t GR = F32_GROUP;
    for (uint32_t r0 = 0; r0 < M;) {
        const uint32_t mb = std::min(GR, M - r0);
        const dim3 grid((waves + 3) / 4, mb == GR ? (M - r0) / GR : 1u);
        const float* hr = h + (size_t)r0 * h_stride;
        float* ar = a + (size_t)r0 * a_stride;
#define PF_GLU_CASE(MM)                                                                                          \
    case MM:                                                                                                     \
        hipLaunchKernelGGL(k_gemv_f32_glu<MM>, grid, dim3(256), 0, st, Wg->data, Wg->scales, Wu->data, Wu->scales, \
                           Wg->rows, Wg->cols, hr, h_stride, ar, a_stride);                                      \
        break;
        switch (mb) {
            PF_GLU_CASE(1) PF_GLU_CASE(2) PF_GLU_CASE(3) PF_GLU_CASE(4)
            PF_GLU_CASE(5) PF_GLU_CASE(6) PF_GLU_CASE(7) PF_GLU_CASE(8)
        }
#undef PF_GLU_CASE
        r0 += mb * grid.y;
    }
}

static int per_for(uint32_t K) {
    uint32_t per = (K + 255) / 256;
    for (int p : {4, 8, 12, 16, 24, 32})
        if ((uint32_t)p >= per) return p;
    return 0;
}

#define PF_PER_SWITCH(K, CALL)                           \
    switch (per_for(K)) {                                \
        case 4: { constexpr int PER = 4; CALL; } break;   \
        case 8: { constexpr int PER = 8; CALL; } break;   \
        case 12: { constexpr int PER = 12; CALL; } break; \
        case 16: { constexpr int PER = 16; CALL; } break; \
        case 24: { constexpr int PER = 24; CALL; } break; \
        case 32: { constexpr int PER = 32; CALL; } break; \
    }

#define PF_PER1024_SWITCH(K, CALL)                     \
    switch (((K) + 1023) / 1024 <= 2 ? 2 : (((K) + 1023) / 1024 <= 4 ? 4 : 8)) { \
        case 2: { constexpr int PER = 2; CALL; } break;   \
        case 4: { constexpr int PER = 4; CALL; } break;   \
        case 8: { constexpr int PER = 8; CALL; } break;   \
    }

// Engine attention of a pass (head_dim 64 or 128, checked at model
// creation): one block per (head, 256-entry chunk, share of a group of
// aligned rows), grid (heads * chunks, M); groups of more than 3 rows are
// split over two or three blocks (two blocks fit on a CU), so that the
// chip's CUs share the work.  Batched passes of more than 8 rows take the
// sequence-group kernel (rows in groups of 2-5 consecutive positions) or the
// per-row kernel.  Passes of at most 8 rows quantize and store their own K/V
// rows inside the attention kernel (FUSED); taller passes have them stored by
// k_kv_store_pass first.
static bool attn_fused(uint32_t M) { return M <= AG_MAX_ROWS; }
static void launch_attn(hipStream_t st, uint32_t hd, uint32_t M, uint32_t tasks, const PassDesc* pd,
                        const KvGeom& g, const KvPlanes& kv, uint32_t l, const float* q, const float* k,
                        const float* v, float* S, uint32_t s_stride, float* Wp, uint32_t cstride, Prefetch pf,
                        bool batch, uint32_t gsize, hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr) {
    if (batch && M > AG_MAX_ROWS && gsize >= 2 && gsize <= AS_NR) {
        // groups of gsize consecutive positions of one sequence (a batched
        // verify pass): one block per (head, chunk, group) loads the union
        // of the rows' chunk entries once
        const dim3 grid(tasks, (M + gsize - 1) / gsize);
        if (hd == 64) {
            if (ev0)
                hipExtLaunchKernelGGL((k_attn_seq<4>), grid, dim3(512), 0, st, ev0, ev1, 0, pd, g, kv, l, M, gsize, q,
                                      k, v, S, s_stride, Wp, cstride);
            else
                hipLaunchKernelGGL((k_attn_seq<4>), grid, dim3(512), 0, st, pd, g, kv, l, M, gsize, q, k, v, S,
                                   s_stride, Wp, cstride);
        } else {
            if (ev0)
                hipExtLaunchKernelGGL((k_attn_seq<8>), grid, dim3(512), 0, st, ev0, ev1, 0, pd, g, kv, l, M, gsize, q,
                                      k, v, S, s_stride, Wp, cstride);
            else
                hipLaunchKernelGGL((k_attn_seq<8>), grid, dim3(512), 0, st, pd, g, kv, l, M, gsize, q, k, v, S,
                                   s_stride, Wp, cstride);
        }
        return;
    }
    if (batch && M > AG_MAX_ROWS) {
        // many sequences of a few rows each: one block per (row, head, chunk),
        // the M rows of one (head, chunk) on one XCD (blocks b with equal b mod 8)
        const uint32_t blocks = 8 * M * ((tasks + 7) / 8);
        if (hd == 64) {
            if (ev0)
                hipExtLaunchKernelGGL((k_attn_chunk<4, 136u>), dim3(blocks), dim3(256), 0, st, ev0, ev1, 0, pd, g, kv,
                                      l, M, tasks, q, k, v, S, s_stride, Wp, cstride);
            else
                hipLaunchKernelGGL((k_attn_chunk<4, 136u>), dim3(blocks), dim3(256), 0, st, pd, g, kv, l, M, tasks, q,
                                   k, v, S, s_stride, Wp, cstride);
        } else {
            if (ev0)
                hipExtLaunchKernelGGL((k_attn_chunk<8, 136u>), dim3(blocks), dim3(256), 0, st, ev0, ev1, 0, pd, g, kv,
                                      l, M, tasks, q, k, v, S, s_stride, Wp, cstride);
            else
                hipLaunchKernelGGL((k_attn_chunk<8, 136u>), dim3(blocks), dim3(256), 0, st, pd, g, kv, l, M, tasks, q,
                                   k, v, S, s_stride, Wp, cstride);
        }
        return;
    }
    const uint32_t gy = M + (pf.p ? 1u : 0u);   // one more row of blocks prefetches pf
#define PF_ATTN_LAUNCH(P, F, NR)                                                                              \
    do {                                                                                                      \
        if (ev0)                                                                                              \
            hipExtLaunchKernelGGL((k_attn_group<P, F, NR>), dim3(tasks, gy), dim3(512), 0, st, ev0, ev1, 0, pd, \
                                  g, kv, l, M, q, k, v, S, s_stride, Wp, cstride, pf);                       \
        else                                                                                                  \
            hipLaunchKernelGGL((k_attn_group<P, F, NR>), dim3(tasks, gy), dim3(512), 0, st, pd, g, kv, l, M, q, \
                               k, v, S, s_stride, Wp, cstride, pf);                                           \
    } while (0)
#define PF_ATTN_ROWS(P)                              \
    switch (M) {                                     \
        case 1: PF_ATTN_LAUNCH(P, true, 1); break;   \
        case 2: PF_ATTN_LAUNCH(P, true, 2); break;   \
        case 3: PF_ATTN_LAUNCH(P, true, 3); break;   \
        case 4: PF_ATTN_LAUNCH(P, true, 2); break;   \
        case 5: PF_ATTN_LAUNCH(P, true, 2); break;   \
        case 6: PF_ATTN_LAUNCH(P, true, 3); break;   \
        case 7: PF_ATTN_LAUNCH(P, true, 4); break;   \
        case 8: PF_ATTN_LAUNCH(P, true, 4); break;   \
        default: PF_ATTN_LAUNCH(P, false, 4); break; \
    }
    if (hd == 64) {
        PF_ATTN_ROWS(4);
    } else {
        PF_ATTN_ROWS(8);
    }
#undef PF_ATTN_ROWS
#undef PF_ATTN_LAUNCH
}

// The QKV product and the attention of a pass of at most 8 rows in one
// launch (k_qkv_attn, pf_pass.hip), for Q4 attention matrices: rows held
// per QKV workgroup as gemv_mr chooses (1, 5 or 8), attention rows per
// block as launch_attn's table (M = 1 -> 1, 2 -> 2, 3 -> 3, 4-5 -> 2,
// 6 -> 3, 7-8 -> 4).
template <int MR, int P, int NR>
static void qkv_attn_one(hipStream_t st, const GemvArgs& a, const AttnGroupArgs& b, uint32_t tasks, hipEvent_t ev0,
                         hipEvent_t ev1) {
    const uint32_t nq = a.N / 32;
    static bool attr = false;   // LDS beyond 64 KiB is granted per kernel
    if (!attr) {
        (void)hipFuncSetAttribute((const void*)k_qkv_attn<FMT_Q4, MR, P, NR>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, qkv_attn_smem(GEMV_MAX_M, 2048, NR));
        attr = true;
    }
    const uint32_t smem = qkv_attn_smem(a.M, a.K, NR);
    const dim3 grid(nq + tasks * (b.M + (b.pf.p ? 1u : 0u)));
    if (ev0)
        hipExtLaunchKernelGGL((k_qkv_attn<FMT_Q4, MR, P, NR>), grid, dim3(512), smem, st, ev0, ev1, 0, nq, tasks, b.pd,
                              a.W, a.x, a.nw, a, b);
    else
        hipLaunchKernelGGL((k_qkv_attn<FMT_Q4, MR, P, NR>), grid, dim3(512), smem, st, nq, tasks, b.pd, a.W, a.x, a.nw,
                           a, b);
}

template <int P>
static void qkv_attn_rows(hipStream_t st, const GemvArgs& a, const AttnGroupArgs& b, uint32_t tasks, hipEvent_t ev0,
                          hipEvent_t ev1) {
    switch (a.M) {
        case 1: qkv_attn_one<1, P, 1>(st, a, b, tasks, ev0, ev1); break;
        case 2: case 4: qkv_attn_one<5, P, 2>(st, a, b, tasks, ev0, ev1); break;
        case 3: case 5: qkv_attn_one<5, P, 3>(st, a, b, tasks, ev0, ev1); break;   // 5 rows: groups of 3 and 2
        case 6: qkv_attn_one<8, P, 3>(st, a, b, tasks, ev0, ev1); break;
        default: qkv_attn_one<8, P, 4>(st, a, b, tasks, ev0, ev1); break;
    }
}

extern "C" pf_status pf_quantize_activation_rows(pf_ctx* c, const float* src, int8_t* dst, float* scales,
                                                 uint32_t M, uint32_t K) {
    if (!c || !src || !dst || !scales || M == 0) return PF_ERR_ARG;
    if (!per_for(K)) return fail(c, PF_ERR_UNSUPPORTED, "K > 8192");
    PF_PER_SWITCH(K, hipLaunchKernelGGL(k_quant_rows<PER>, dim3(M), dim3(256), 0, c->stream, src, K, K, dst, K,
                                        scales, (int32_t*)nullptr, 0u));
    PF_LAUNCHED(c);
    return PF_OK;
}

extern "C" pf_status pf_matmul_int8(pf_ctx* c, const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N,
                                    uint32_t K) {
    if (!c || !A || !B || !C) return PF_ERR_ARG;
    if (M == 0 || N == 0) return PF_OK;
    hipLaunchKernelGGL(k_matmul_int8, dim3((N + 255) / 256, M), dim3(256), 0, c->stream, A, B, C, M, N, K);
    PF_LAUNCHED(c);
    return PF_OK;
}

extern "C" pf_status pf_matmul_quantized(pf_ctx* c, const float* A, const int8_t* B, float* C, uint32_t M,
                                         uint32_t N, uint32_t K, const float* ws, const float* as_in) {
    if (!c || !A || !B || !C || !ws) return PF_ERR_ARG;
    if (M == 0 || N == 0) return PF_OK;
    size_t need = (size_t)M * K + 256 + (size_t)M * 4 + 256 + (size_t)M * N * 4 + 256;
    void* s = nullptr;
    pf_status st = ctx_scratch(c, need, &s);
    if (st) return st;
    int8_t* Aq = (int8_t*)s;
    float* as = (float*)((char*)s + (((size_t)M * K + 255) & ~(size_t)255));
    int32_t* Ci = (int32_t*)((char*)as + (((size_t)M * 4 + 255) & ~(size_t)255));
    if (as_in) {
        hipLaunchKernelGGL(k_quant_div, dim3((K + 255) / 256, M), dim3(256), 0, c->stream, A, as_in, Aq, M, K);
        PF_HIP(c, hipMemcpyAsync(as, as_in, M * 4, hipMemcpyDeviceToDevice, c->stream));
    } else {
        if (!per_for(K)) return fail(c, PF_ERR_UNSUPPORTED, "K > 8192");
        PF_PER_SWITCH(K, hipLaunchKernelGGL(k_quant_rows<PER>, dim3(M), dim3(256), 0, c->stream, A, K, K, Aq, K,
                                            as, (int32_t*)nullptr, 0u));
    }
    hipLaunchKernelGGL(k_matmul_int8, dim3((N + 255) / 256, M), dim3(256), 0, c->stream, Aq, B, Ci, M, N, K);
    hipLaunchKernelGGL(k_mm_epilogue, dim3((N + 255) / 256, M), dim3(256), 0, c->stream, Ci, as, ws, C, M, N);
    PF_LAUNCHED(c);
    return PF_OK;
}

// pf_gemv_q and pf_gemv_q_noalloc: M <= 8 runs the GEMV, which quantizes
// x itself; larger M quantizes x into act / as (ceil(M / 32) * 32 rows of
// K codes, M scales) and runs the int8 MFMA GEMM.
static pf_status gemv_q_check(pf_ctx* c, const pf_matrix* W, const float* x, float* y, uint32_t M) {
    if (!c || !W || !x || !y || M == 0 || M > MAX_GEMM_ROWS) return PF_ERR_ARG;
    if (W->rowmajor) return fail(c, PF_ERR_ARG, "pf_gemv_q needs an int8-activation (tiled) matrix");
    if (M > GEMV_MAX_M && !per_for(W->cols)) return fail(c, PF_ERR_UNSUPPORTED, "K > 8192");
    return PF_OK;
}
static size_t gemv_q_act_bytes(uint32_t M, uint32_t K) {
    return ((size_t)((M + 31) / 32 * 32) * K + 255) & ~(size_t)255;
}
static pf_status gemv_q_run(pf_ctx* c, const pf_matrix* W, const float* x, float* y, uint32_t M, int8_t* act,
                            float* as) {
    const uint32_t K = W->cols, N = W->rows;
    MmEpi e{};
    e.y = y;
    e.y_stride = N;
    e.ilv = W->ilv ? 1u : 0u;
    if (M <= GEMV_MAX_M) {
        GemvArgs a{};
        a.W = W->data; a.N = N; a.K = K; a.M = M; a.x = x; a.xs = K; a.e = e;
        launch_gemv(c->stream, W, MM_STORE, a);
        PF_LAUNCHED(c);
        return PF_OK;
    }
    PF_PER_SWITCH(K, hipLaunchKernelGGL(k_quant_rows<PER>, dim3(M), dim3(256), 0, c->stream, x, K, K, act, K, as,
                                        (int32_t*)nullptr, 0u));
    GemmArgs g{};
    g.W = W->data; g.N = N; g.K = K; g.M = M; g.act = act; g.act_stride = K; g.as = as; g.e = e;
    launch_gemm(c->stream, W, MM_STORE, g);
    PF_LAUNCHED(c);
    return PF_OK;
}

extern "C" pf_status pf_gemv_q(pf_ctx* c, const pf_matrix* W, const float* x, float* y, uint32_t M) {
    if (pf_status st = gemv_q_check(c, W, x, y, M)) return st;
    if (M <= GEMV_MAX_M) return gemv_q_run(c, W, x, y, M, nullptr, nullptr);
    const size_t a_bytes = gemv_q_act_bytes(M, W->cols);
    void* s = nullptr;
    pf_status st = ctx_scratch(c, a_bytes + (size_t)M * 4, &s);
    if (st) return st;
    return gemv_q_run(c, W, x, y, M, (int8_t*)s, (float*)((char*)s + a_bytes));
}

// The same without allocating: the M > 8 path's activation rows and scales
// live in the GPU's copy of `scratch`.  Every buffer byte the GEMM reads is
// written first by the quantize kernel, except the padding rows up to a
// multiple of 32, which feed only outputs the GEMM discards; nothing needs
// clearing.  Calls that overlap on one GPU (other streams or contexts)
// share the array and race.
extern "C" pf_status pf_gemv_q_noalloc(pf_ctx* c, const pf_matrix* W, const float* x, float* y, uint32_t M) {
    if (pf_status st = gemv_q_check(c, W, x, y, M)) return st;
    if (M <= GEMV_MAX_M) return gemv_q_run(c, W, x, y, M, nullptr, nullptr);
    if (gemv_q_act_bytes(M, W->cols) > NOALLOC_ACT_BYTES)
        return fail(c, PF_ERR_CAPACITY,
                    "pf_gemv_q_noalloc: ceil(M / 32) * 32 * cols = " +
                        std::to_string((size_t)((M + 31) / 32 * 32) * W->cols) +
                        " activation bytes, beyond its fixed scratch of 1 MiB");
    uint8_t* p = (uint8_t*)g_scratch_dev[c->device];
    if (!p) return fail(c, PF_ERR_STATE, "scratch address not resolved for this device");
    return gemv_q_run(c, W, x, y, M, (int8_t*)p, (float*)(p + NOALLOC_ACT_BYTES));
}
extern "C" pf_status pf_gemv_f32(pf_ctx* c, const pf_matrix* W, const float* x, float* y, uint32_t M) {
    if (!c || !W || !x || !y || M == 0 || M > 8) return PF_ERR_ARG;
    if (!W->rowmajor) return fail(c, PF_ERR_ARG, "pf_gemv_f32 needs a row-major matrix");
    launch_gemv_f32(c->stream, W, M, x, W->cols, y, W->rows, nullptr);
    PF_LAUNCHED(c);
    return PF_OK;
}

// dot_product / softmax / rmsnorm / argmax of include/forge/matmul_neon.hpp
// and src/mtp.cpp on device buffers.
extern "C" pf_status pf_dot_product(pf_ctx* c, const float* a, const float* b, uint32_t n, float* out) {
    if (!c || !a || !b || !out) return PF_ERR_ARG;
    hipLaunchKernelGGL(k_dot_canon, dim3(1), dim3(256), 0, c->stream, a, b, n, out);
    PF_LAUNCHED(c);
    return PF_OK;
}

extern "C" pf_status pf_softmax(pf_ctx* c, float* v, uint32_t n) {
    if (!c || !v || n == 0) return PF_ERR_ARG;
    hipLaunchKernelGGL(k_softmax_one, dim3(1), dim3(256), 0, c->stream, v, n);
    PF_LAUNCHED(c);
    return PF_OK;
}

extern "C" pf_status pf_rmsnorm(pf_ctx* c, float* out, const float* x, const float* w, uint32_t n) {
    if (!c || !out || !x || !w || n == 0) return PF_ERR_ARG;
    hipLaunchKernelGGL(k_rmsnorm_one, dim3(1), dim3(256), 0, c->stream, out, x, w, n);
    PF_LAUNCHED(c);
    return PF_OK;
}

extern "C" pf_status pf_argmax(pf_ctx* c, const float* x, uint32_t n, int32_t* out) {
    if (!c || !x || !out || n == 0) return PF_ERR_ARG;
    hipLaunchKernelGGL(k_argmax_one, dim3(1), dim3(1024), 0, c->stream, x, n, out);
    PF_LAUNCHED(c);
    return PF_OK;
}

// ============================================================ MTP heads
// A standalone MTPHeads (include/forge/mtp.hpp:31-53): its own head
// matrices and, optionally, an fp32 tied table handed in by the caller.

struct pf_mtp {
    pf_ctx* c = nullptr;
    uint32_t H = 0, D = 0, V = 0;
    std::vector<pf_matrix*> mats;     // [H][3]: gate, up, down (row-major Q4)
    float* table = nullptr;           // [V][D] fp32, or null
    float *cur = nullptr, *g = nullptr, *u = nullptr, *a = nullptr, *logits = nullptr;
};

extern "C" void pf_mtp_destroy(pf_mtp* m) {
    if (!m) return;
    pf_ctx* c = m->c;
    (void)hipStreamSynchronize(c->stream);
    for (pf_matrix* M : m->mats) pf_matrix_free(M);
    dfree(c, m->table, (size_t)m->V * m->D * 4);
    dfree(c, m->cur, (size_t)m->D * 4);
    dfree(c, m->g, (size_t)m->D * 4);
    dfree(c, m->u, (size_t)m->D * 4);
    dfree(c, m->a, (size_t)m->D * 4);
    dfree(c, m->logits, (size_t)m->H * m->V * 4);
    delete m;
}

extern "C" pf_status pf_mtp_create(pf_ctx* c, uint32_t n_heads, uint32_t n_embd, uint32_t n_vocab, pf_mtp** out) {
    if (!c || !out || n_heads == 0 || n_vocab == 0) return PF_ERR_ARG;
    *out = nullptr;
    if (n_embd % 256 || n_embd == 0 || n_embd > 2048)
        return fail(c, PF_ERR_UNSUPPORTED, "MTP heads need n_embd a multiple of 256 up to 2048");
    pf_mtp* m = new pf_mtp();
    m->c = c; m->H = n_heads; m->D = n_embd; m->V = n_vocab;
    m->mats.assign((size_t)n_heads * 3, nullptr);
    pf_status s = PF_OK;
    for (uint32_t i = 0; i < n_heads * 3 && !s; i++) s = matrix_alloc(c, FMT_Q4, n_embd, n_embd, true, &m->mats[i]);
    if (!s) s = dalloc_t(c, &m->cur, n_embd);
    if (!s) s = dalloc_t(c, &m->g, n_embd);
    if (!s) s = dalloc_t(c, &m->u, n_embd);
    if (!s) s = dalloc_t(c, &m->a, n_embd);
    if (!s) s = dalloc_t(c, &m->logits, (size_t)n_heads * n_vocab);
    if (s) { pf_mtp_destroy(m); return s; }
    *out = m;
    return PF_OK;
}

extern "C" pf_status pf_mtp_set_head(pf_mtp* m, uint32_t head, int32_t which, const uint8_t* codes,
                                     const uint16_t* scales) {
    if (!m || !codes || !scales || head >= m->H || which < 0 || which > 2) return PF_ERR_ARG;
    return matrix_put(m->mats[(size_t)head * 3 + which], 0, m->D, codes, scales);
}

extern "C" pf_status pf_mtp_set_table(pf_mtp* m, const float* table) {
    if (!m) return PF_ERR_ARG;
    pf_ctx* c = m->c;
    if (!table) {
        PF_HIP(c, hipStreamSynchronize(c->stream));
        dfree(c, m->table, (size_t)m->V * m->D * 4);
        m->table = nullptr;
        return PF_OK;
    }
    if (!m->table) {
        pf_status s = dalloc_t(c, &m->table, (size_t)m->V * m->D);
        if (s) return s;
    }
    PF_HIP(c, hipMemcpyAsync(m->table, table, (size_t)m->V * m->D * 4, hipMemcpyHostToDevice, c->stream));
    PF_HIP(c, hipStreamSynchronize(c->stream));
    return PF_OK;
}

extern "C" pf_status pf_mtp_heads_forward(pf_mtp* m, const float* hidden, float* logits) {
    if (!m || !hidden || !logits) return PF_ERR_ARG;
    pf_ctx* c = m->c;
    hipStream_t st = c->stream;
    const uint32_t D = m->D, V = m->V;
    PF_HIP(c, hipMemcpyAsync(m->cur, hidden, (size_t)D * 4, hipMemcpyHostToDevice, st));
    for (uint32_t k = 0; k < m->H; k++) {            // src/mtp.cpp:63-127
        launch_gemv_f32_glu(st, m->mats[k * 3 + 0], m->mats[k * 3 + 1], 1, m->cur, D, m->a, D);
        launch_gemv_f32(st, m->mats[k * 3 + 2], 1, m->a, D, m->cur, D, m->cur);
        float* lk = m->logits + (size_t)k * V;
        if (m->table)
            hipLaunchKernelGGL(k_gemv_f32_dense<1>, dim3((std::min<uint32_t>(V, 2048) + 3) / 4), dim3(256), 0, st,
                               (const float*)m->table, V, D, (const float*)m->cur, D, lk, V);
        else
            hipLaunchKernelGGL(k_mtp_placeholder, dim3((V + 255) / 256), dim3(256), 0, st, lk, V, k);
    }
    PF_LAUNCHED(c);
    PF_HIP(c, hipMemcpyAsync(logits, m->logits, (size_t)m->H * V * 4, hipMemcpyDeviceToHost, st));
    PF_HIP(c, hipStreamSynchronize(st));
    return PF_OK;
}

extern "C" size_t pf_mtp_memory(const pf_mtp* m) {
    if (!m) return 0;
    size_t b = 0;
    for (const pf_matrix* M : m->mats) b += M->bytes + (size_t)M->rows * (M->cols / 32) * 2;
    if (m->table) b += (size_t)m->V * m->D * 4;
    return b;
}

// ================================================================= KV cache

static pf_status kv_geom(const pf_ctx* c, uint32_t L, uint32_t H, uint32_t hd, uint32_t sink, uint32_t win,
                         uint32_t pool, uint32_t maxc, uint32_t slack, KvGeom* g) {
    if (L == 0 || H == 0 || hd == 0 || hd % 2 || hd > 128 || maxc == 0)
        return fail(c, PF_ERR_UNSUPPORTED, "KV cache needs even head_dim <= 128 and max_context > 0");
    g->n_layers = L; g->n_heads = H; g->head_dim = hd;
    g->sink_size = sink;
    g->window = std::min(win, maxc);                 // src/kv_cache.cpp:33
    g->pool_block = std::max(1u, pool);              // src/kv_cache.cpp:34
    g->max_context = maxc;
    if (g->window < MAX_PASS_ROWS) return fail(c, PF_ERR_UNSUPPORTED, "window must hold at least 8 entries");
    g->ring = g->window + g->pool_block + slack;
    uint32_t evictable = maxc > sink + g->window ? maxc - sink - g->window : 0;
    g->pool_cap = evictable / g->pool_block + 1;
    g->rows = KV_SINK_ROWS + g->ring + g->pool_cap;
    g->n_seq = 1;
    return PF_OK;
}

static pf_status kv_alloc(pf_ctx* c, const KvGeom& g, KvPlanes* p, size_t* bytes) {
    size_t planes = (size_t)g.n_seq * g.n_layers * g.n_heads, rows = planes * g.rows;
    pf_status s = dalloc_t(c, &p->k, rows * g.head_dim);
    if (!s) s = dalloc_t(c, &p->v, rows * g.head_dim);
    if (!s) s = dalloc_t(c, &p->ks, rows);
    if (!s) s = dalloc_t(c, &p->vs, rows);
    if (s) return s;
    PF_HIP(c, hipMemset(p->k, 0, rows * g.head_dim));
    PF_HIP(c, hipMemset(p->v, 0, rows * g.head_dim));
    *bytes = 2 * rows * g.head_dim + 2 * rows * 4;
    return PF_OK;
}

static void kv_free(pf_ctx* c, const KvGeom& g, KvPlanes* p) {
    size_t rows = (size_t)g.n_seq * g.n_layers * g.n_heads * g.rows;
    dfree(c, p->k, rows * g.head_dim);
    dfree(c, p->v, rows * g.head_dim);
    dfree(c, p->ks, rows * 4);
    dfree(c, p->vs, rows * 4);
}

struct pf_kv {
    pf_ctx* ctx = nullptr;
    KvGeom g{};
    KvPlanes p{};
    size_t bytes = 0;
    std::vector<uint32_t> sink_count, nw;
    uint32_t total_stored = 0;
    float* io = nullptr;      // staging: key, value, query, scores
    float* S = nullptr;       // scores for weighted sum
    float* Wp = nullptr;      // chunk partials
    PassDesc* pd = nullptr;
    uint32_t cap = 0;         // max visible entries
};

extern "C" pf_status pf_kv_create(pf_ctx* c, const pf_kv_config* cfg, pf_kv** out) {
    if (!c || !cfg || !out) return PF_ERR_ARG;
    pf_kv* kv = new pf_kv();
    kv->ctx = c;
    pf_status s = kv_geom(c, cfg->n_layers, cfg->n_kv_heads, cfg->head_dim, cfg->sink_size, cfg->window_size,
                          cfg->pool_block, cfg->max_context, MAX_PASS_ROWS, &kv->g);
    if (!s) s = kv_alloc(c, kv->g, &kv->p, &kv->bytes);
    kv->cap = KV_SINK_ROWS + kv->g.pool_cap + kv->g.window + 1;
    if (!s) s = dalloc_t(c, &kv->io, 4 * 128);
    if (!s) s = dalloc_t(c, &kv->S, kv->cap + 64);
    if (!s) s = dalloc_t(c, &kv->Wp, (size_t)((kv->cap + 63) / 64 + 1) * 128);
    if (!s) s = dalloc_t(c, &kv->pd, 1);
    if (s) { delete kv; return s; }
    PassDesc pd{};
    pd.m = 1;
    PF_HIP(c, hipMemcpy(kv->pd, &pd, sizeof(pd), hipMemcpyHostToDevice));
    size_t planes = (size_t)kv->g.n_layers * kv->g.n_heads;
    kv->sink_count.assign(planes, 0);
    kv->nw.assign(planes, 0);
    *out = kv;
    return PF_OK;
}

extern "C" void pf_kv_destroy(pf_kv* kv) {
    if (!kv) return;
    pf_ctx* c = kv->ctx;
    (void)hipStreamSynchronize(c->stream);
    kv_free(c, kv->g, &kv->p);
    dfree(c, kv->io, 4 * 128 * 4);
    dfree(c, kv->S, (kv->cap + 64) * 4);
    dfree(c, kv->Wp, (size_t)((kv->cap + 63) / 64 + 1) * 128 * 4);
    dfree(c, kv->pd, sizeof(PassDesc));
    delete kv;
}

// src/kv_cache.cpp:59-127 on per-plane counters; a pooled row is folded as
// soon as its last entry is evicted, as the reference does.
extern "C" pf_status pf_kv_store(pf_kv* kv, uint32_t layer, uint32_t head, uint32_t pos, const float* key,
                                 const float* value) {
    if (!kv || !key || !value) return PF_ERR_ARG;
    pf_ctx* c = kv->ctx;
    const KvGeom& g = kv->g;
    if (layer >= g.n_layers || head >= g.n_heads) return PF_OK;   // silent, src/kv_cache.cpp:61
    if (pos >= g.max_context) return PF_OK;                        // src/kv_cache.cpp:62
    const size_t pl = (size_t)layer * g.n_heads + head;
    uint32_t row = 0xFFFFFFFFu;
    if (pos < g.sink_size) {
        if (pos < KV_SINK_ROWS) {
            row = pos;
            kv->sink_count[pl] = std::max(kv->sink_count[pl], pos + 1);
        }
    } else {
        const uint32_t w = kv->nw[pl];
        if (w >= g.window) {
            const uint32_t ev = w - g.window;                      // evicted window index
            if ((ev + 1) % g.pool_block == 0) {
                const uint32_t r = ev / g.pool_block;
                if (r >= g.pool_cap) return fail(c, PF_ERR_CAPACITY, "pooled rows exceed capacity");
                hipLaunchKernelGGL(k_pool_row_one, dim3(1), dim3(g.head_dim <= 64 ? 64 : 128), 0, c->stream, g,
                                   kv->p, (uint32_t)pl, r);
            }
        }
        row = KV_SINK_ROWS + w % g.ring;
        kv->nw[pl] = w + 1;
    }
    if (row != 0xFFFFFFFFu) {
        PF_HIP(c, hipMemcpyAsync(kv->io, key, g.head_dim * 4, hipMemcpyHostToDevice, c->stream));
        PF_HIP(c, hipMemcpyAsync(kv->io + 128, value, g.head_dim * 4, hipMemcpyHostToDevice, c->stream));
        hipLaunchKernelGGL(k_kv_store_row, dim3(1), dim3(64), 0, c->stream, g, kv->p, layer, head, row, kv->io,
                           kv->io + 128);
        PF_LAUNCHED(c);
        PF_HIP(c, hipStreamSynchronize(c->stream));
    }
    if (pos >= kv->total_stored) kv->total_stored = pos + 1;
    return PF_OK;
}

extern "C" pf_status pf_kv_attention_scores(pf_kv* kv, uint32_t layer, uint32_t head, const float* q, float* out,
                                            uint32_t* count) {
    if (!kv || !q || !out || !count) return PF_ERR_ARG;
    pf_ctx* c = kv->ctx;
    const KvGeom& g = kv->g;
    *count = 0;
    if (layer >= g.n_layers || head >= g.n_heads) return PF_OK;
    const size_t pl = (size_t)layer * g.n_heads + head;
    const KvView v = kv_view_counts(g, kv->sink_count[pl], kv->nw[pl]);
    const uint32_t C = v.count();
    PF_HIP(c, hipMemcpyAsync(kv->io + 256, q, g.head_dim * 4, hipMemcpyHostToDevice, c->stream));
    // the kernel reads a full head row of q per head index: place q at head `head`
    KvGeom g1 = g;
    hipLaunchKernelGGL(k_attn_scores, dim3(1, 1, (C + 1 + 255) / 256), dim3(256), 0, c->stream, kv->pd, g1, kv->p,
                       layer, (int32_t)kv->sink_count[pl], kv->nw[pl], (int32_t)head, kv->io + 256,
                       kv->io + 256, kv->S, 0u, 0);
    PF_LAUNCHED(c);
    if (C) PF_HIP(c, hipMemcpyAsync(out, kv->S, (size_t)C * 4, hipMemcpyDeviceToHost, c->stream));
    PF_HIP(c, hipStreamSynchronize(c->stream));
    *count = C;
    return PF_OK;
}

extern "C" pf_status pf_kv_attention_weighted_sum(pf_kv* kv, uint32_t layer, uint32_t head, const float* scores,
                                                  float* output, uint32_t count) {
    if (!kv || !output) return PF_ERR_ARG;
    pf_ctx* c = kv->ctx;
    const KvGeom& g = kv->g;
    std::memset(output, 0, g.head_dim * 4);
    if (layer >= g.n_layers || head >= g.n_heads || count == 0) return PF_OK;
    if (!scores) return PF_ERR_ARG;
    const size_t pl = (size_t)layer * g.n_heads + head;
    const KvView v = kv_view_counts(g, kv->sink_count[pl], kv->nw[pl]);
    const uint32_t n = std::min(count, v.count());
    if (n == 0) return PF_OK;
    PF_HIP(c, hipMemcpyAsync(kv->S, scores, (size_t)n * 4, hipMemcpyHostToDevice, c->stream));
    const uint32_t nch = (n + 63) / 64;
    hipLaunchKernelGGL(k_attn_wsum, dim3(1, 1, nch), dim3(128), 0, c->stream, kv->pd, g, kv->p, layer,
                       (int32_t)kv->sink_count[pl], kv->nw[pl], (int32_t)head, n, kv->S, 0u, kv->Wp, nch);
    hipLaunchKernelGGL(k_wsum_combine_one, dim3(1), dim3(128), 0, c->stream, kv->Wp, nch, g.head_dim, kv->io + 384);
    PF_LAUNCHED(c);
    PF_HIP(c, hipMemcpyAsync(output, kv->io + 384, g.head_dim * 4, hipMemcpyDeviceToHost, c->stream));
    PF_HIP(c, hipStreamSynchronize(c->stream));
    return PF_OK;
}

extern "C" uint32_t pf_kv_size(const pf_kv* kv) { return kv ? kv->total_stored : 0; }

extern "C" pf_status pf_kv_clear(pf_kv* kv) {
    if (!kv) return PF_ERR_ARG;
    std::fill(kv->sink_count.begin(), kv->sink_count.end(), 0u);
    std::fill(kv->nw.begin(), kv->nw.end(), 0u);
    kv->total_stored = 0;
    return PF_OK;
}

extern "C" size_t pf_kv_memory_usage(const pf_kv* kv) { return kv ? kv->bytes : 0; }

// ================================================================== model

struct pf_model {
    pf_ctx* ctx = nullptr;
    pf_model_desc d{};
    std::vector<pf_matrix*> qkv, o, gu, down, mtp;
    pf_matrix* emb = nullptr;
    float* attn_norm = nullptr;
    float* ffn_norm = nullptr;
    std::vector<uint32_t> set_mask;   // per layer: bit id for matrices 0..6
    std::vector<uint32_t> mtp_mask;
    bool emb_set = false;
};

extern "C" pf_status pf_model_create(pf_ctx* c, const pf_model_desc* d, pf_model** out) {
    if (!c || !d || !out) return PF_ERR_ARG;
    if (d->n_heads * d->head_dim != d->n_embd)
        return fail(c, PF_ERR_UNSUPPORTED, "n_heads * head_dim must equal n_embd (multi-head attention)");
    if (d->n_embd % 256 || d->n_ff % 256 || d->n_vocab % 64 || d->n_embd > 2048 || d->n_ff > 8192)
        return fail(c, PF_ERR_UNSUPPORTED, "n_embd and n_ff must be multiples of 256 (n_embd <= 2048, n_ff <= 8192), "
                                           "n_vocab a multiple of 64");
    if (d->head_dim != 64 && d->head_dim != 128) return fail(c, PF_ERR_UNSUPPORTED, "head_dim must be 64 or 128");
    if (d->n_mtp + 1 > MAX_PASS_ROWS) return fail(c, PF_ERR_UNSUPPORTED, "at most 7 MTP heads");
    if (d->n_vocab > SAMPLE_MAX_V) return fail(c, PF_ERR_UNSUPPORTED, "n_vocab > 16384");
    pf_model* m = new pf_model();
    m->ctx = c;
    m->d = *d;
    m->qkv.assign(d->n_layers, nullptr);
    m->o.assign(d->n_layers, nullptr);
    m->gu.assign(d->n_layers, nullptr);
    m->down.assign(d->n_layers, nullptr);
    m->mtp.assign((size_t)d->n_mtp * 3, nullptr);
    m->set_mask.assign(d->n_layers, 0);
    m->mtp_mask.assign(d->n_mtp, 0);
    size_t nn = (size_t)std::max(1u, d->n_layers) * d->n_embd;
    pf_status s = dalloc_t(c, &m->attn_norm, nn);
    if (!s) s = dalloc_t(c, &m->ffn_norm, nn);
    if (s) { delete m; return s; }
    std::vector<float> ones(nn, 1.0f);   // src/engine.cpp:171-173 fallback
    PF_HIP(c, hipMemcpy(m->attn_norm, ones.data(), nn * 4, hipMemcpyHostToDevice));
    PF_HIP(c, hipMemcpy(m->ffn_norm, ones.data(), nn * 4, hipMemcpyHostToDevice));
    *out = m;
    return PF_OK;
}

extern "C" void pf_model_destroy(pf_model* m) {
    if (!m) return;
    for (auto* v : {&m->qkv, &m->o, &m->gu, &m->down, &m->mtp})
        for (pf_matrix* x : *v) pf_matrix_free(x);
    pf_matrix_free(m->emb);
    size_t nn = (size_t)std::max(1u, m->d.n_layers) * m->d.n_embd;
    dfree(m->ctx, m->attn_norm, nn * 4);
    dfree(m->ctx, m->ffn_norm, nn * 4);
    delete m;
}

extern "C" pf_status pf_model_set_matrix(pf_model* m, uint32_t layer, int32_t id, int32_t fmt, const uint8_t* codes,
                                         const uint16_t* scales) {
    if (!m || !codes || !scales || layer >= m->d.n_layers || id < 0 || id > 6) return PF_ERR_ARG;
    pf_ctx* c = m->ctx;
    const uint32_t D = m->d.n_embd, F = m->d.n_ff;
    pf_matrix** slot;
    uint32_t rows_total, cols, row0, rows;
    if (id <= 2) { slot = &m->qkv[layer]; rows_total = 3 * D; cols = D; row0 = id * D; rows = D; }
    else if (id == 3) { slot = &m->o[layer]; rows_total = D; cols = D; row0 = 0; rows = D; }
    else if (id <= 5) { slot = &m->gu[layer]; rows_total = 2 * F; cols = D; row0 = (id - 4) * F; rows = F; }
    else { slot = &m->down[layer]; rows_total = D; cols = F; row0 = 0; rows = D; }
    if (!*slot) {
        pf_status s = matrix_alloc(c, fmt, rows_total, cols, false, slot, id == 4 || id == 5);
        if (s) return s;
    } else if ((*slot)->fmt != fmt) {
        return fail(c, PF_ERR_ARG, "Q/K/V (and gate/up) of a layer must share one format");
    }
    pf_status s = matrix_put(*slot, row0, rows, codes, scales);
    if (s) return s;
    m->set_mask[layer] |= 1u << id;
    return PF_OK;
}

extern "C" pf_status pf_model_set_embedding_fmt(pf_model* m, int32_t fmt, const uint8_t* codes,
                                                 const uint16_t* scales) {
    if (!m || !codes || !scales) return PF_ERR_ARG;
    if (fmt != FMT_Q4 && fmt != FMT_Q8) return fail(m->ctx, PF_ERR_UNSUPPORTED, "the embedding table must be Q4 or Q8");
    if (m->emb && m->emb->fmt != fmt) {
        pf_matrix_free(m->emb);
        m->emb = nullptr;
        m->emb_set = false;
    }
    if (!m->emb) {
        pf_status s = matrix_alloc(m->ctx, fmt, m->d.n_vocab, m->d.n_embd, true, &m->emb);
        if (s) return s;
    }
    pf_status s = matrix_put(m->emb, 0, m->d.n_vocab, codes, scales);
    if (s) return s;
    m->emb_set = true;
    return PF_OK;
}

extern "C" pf_status pf_model_set_embedding(pf_model* m, const uint8_t* codes, const uint16_t* scales) {
    return pf_model_set_embedding_fmt(m, FMT_Q4, codes, scales);
}

extern "C" pf_status pf_model_set_mtp(pf_model* m, uint32_t head, int32_t which, const uint8_t* codes,
                                      const uint16_t* scales) {
    if (!m || !codes || !scales || head >= m->d.n_mtp || which < 0 || which > 2) return PF_ERR_ARG;
    pf_matrix*& M = m->mtp[(size_t)head * 3 + which];
    if (!M) {
        pf_status s = matrix_alloc(m->ctx, FMT_Q4, m->d.n_embd, m->d.n_embd, true, &M);
        if (s) return s;
    }
    pf_status s = matrix_put(M, 0, m->d.n_embd, codes, scales);
    if (s) return s;
    m->mtp_mask[head] |= 1u << which;
    return PF_OK;
}

extern "C" pf_status pf_model_set_norm(pf_model* m, uint32_t layer, int32_t which, const float* w) {
    if (!m || !w || layer >= m->d.n_layers || (which != 7 && which != 8)) return PF_ERR_ARG;
    float* dst = (which == 7 ? m->attn_norm : m->ffn_norm) + (size_t)layer * m->d.n_embd;
    PF_HIP(m->ctx, hipMemcpy(dst, w, m->d.n_embd * 4, hipMemcpyHostToDevice));
    return PF_OK;
}

static bool model_complete(const pf_model* m) {
    if (!m->emb_set) return false;
    for (uint32_t l = 0; l < m->d.n_layers; l++)
        if (m->set_mask[l] != 0x7Fu) return false;
    for (uint32_t k = 0; k < m->d.n_mtp; k++)
        if (m->mtp_mask[k] != 0x7u) return false;
    return true;
}

// ================================================================= engine

struct TimedPass { hipEvent_t a, b; bool verify; };

struct pf_engine {
    pf_model* m = nullptr;
    pf_ctx* c = nullptr;
    KvGeom g{};
    KvPlanes kv{};
    size_t kv_bytes = 0;
    float* rope_c = nullptr;
    float* rope_s = nullptr;
    uint32_t rope_pos = 0;
    // pass scratch
    float* x = nullptr;         // residual stream [rows][D]
    int8_t* act = nullptr;      // quantized activation rows [rows][kmax]
    float* as = nullptr;        // their row scales [4][rows]
    float *q = nullptr, *k = nullptr, *v = nullptr;   // [rows][D] after RoPE
    float* sg = nullptr;        // SwiGLU output [rows][F]
    float* pmax = nullptr;      // its per-workgroup row maxima [8][2F / 32] (decode passes)
    float* S = nullptr;
    float* Wp = nullptr;
    uint32_t s_stride = 0, cstride = 0, kmax = 0;
    uint32_t cmax = 0;            // longest attention list (sink + pool + window)
    uint32_t prefill_rows = 8;    // rows of a prompt pass
    PassDesc pd_host{};           // staging of the prompt passes' descriptors
    float *logitsA = nullptr, *hiddenA = nullptr, *logitsB = nullptr, *hiddenB = nullptr;
    float *mcur = nullptr, *ma = nullptr, *mlogits = nullptr;
    PassDesc *pdA = nullptr, *pdB = nullptr, *pdP = nullptr;
    DecodeState* st = nullptr;
    int32_t* tokens = nullptr;
    uint32_t tok_cap = 0;         // token-buffer capacity of each sequence
    size_t tok_alloc = 0;         // elements allocated (nseq * tok_cap)
    uint32_t* word = nullptr;   // pinned readback (fine-grained), written by k_word_out
    uint32_t* word_dev = nullptr;   // its device address
    // multi-sequence engines (pf_batch_*): nseq sequences, each with its own
    // KV planes, decode state (st[s]) and token buffer (tokens + s * tok_cap)
    uint32_t nseq = 1;
    uint32_t rows = MAX_PREFILL_ROWS;   // rows of the pass buffers
    std::vector<uint32_t> spos;         // host mirror of each sequence's position
    uint64_t* seeds = nullptr;          // [nseq] sampling seed of each sequence
    uint32_t* sel = nullptr;            // [nseq] row -> sequence of a batched round
    float* mlogb = nullptr;             // [nseq][V] draft logits of one head
    std::vector<std::pair<void*, size_t>> owned;
    // host mirrors
    uint32_t pos = 0;
    uint32_t pool_rows_max = 1;
    bool hidden_valid = false;
    size_t max_memory = 0;
    uint32_t pf_blocks = 128;     // blocks of the attention merge that prefetch the O weights (PF_PREFETCH_BLOCKS)
    uint32_t l2_blocks = 64;      // blocks of a decode GEMV that prefetch the next product's weights (PF_L2_BLOCKS)
    uint32_t* sink = nullptr;     // 4 bytes the prefetch loops never write in practice
    bool mtp_enabled = true;      // ModelConfig::mtp_enabled, include/forge/types.hpp
    // layer skip (LayerSkipController, src/layer_skip.cpp): on while the
    // threshold is > 0; caches [nseq][L][D], FFN inputs of the last pass
    // [L][rows][D], skip flags [L][rows], skipped-row counter
    bool skip_on = false;
    float skip_thr = 0.0f;
    uint32_t skip_interval = 4;
    float* skip_cache = nullptr;
    float* skip_stage = nullptr;
    uint32_t* skip_flags = nullptr;
    uint32_t* skip_ctr = nullptr;
    uint32_t* skip_nrun = nullptr;     // [L] rows of the current pass that run the layer's FFN
    // timing
    std::vector<TimedPass> timed;
    size_t timed_used = 0;
    // captured decode rounds: [reuse][mtp] -> graph exec, for one sampling
    // configuration / seed / profiling mode
    // [reuse][mtp][first verify segment: 1 row, or all n_mtp + 1 rows]
    hipGraphExec_t round_exec[2][2][2] = {};
    hipGraphExec_t cont_exec = nullptr;   // the verify segment that continues a round (drafts 1..n_mtp-1)
    bool verify_full = false;             // always verify all drafts in one segment
    uint32_t round_ev[2][2][4] = {};   // pass-event and GEMV-event slot ranges of each variant
    hipEvent_t rev0 = nullptr, rev1 = nullptr;
    double round_us = 0;
    uint32_t round_n = 0;
    // HIP events around every decode segment of pf_generate, for
    // pf_engine_round_time (off: about 10 us less per round)
    bool round_timing = false;
    SamplingCfg graph_cfg{};
    uint64_t graph_seed = 0;
    int32_t graph_profile = 0;
    bool graphs_valid = false;
    bool capturing = false;
    bool use_graphs = true;
    // profiling mode: 0 off (captured graphs), 1 kernels one by one with
    // pass events and per-dispatch events on the verify passes' GEMVs and
    // attention, 2 kernels one by one with pass events only
    int32_t profile = 0;
    bool in_verify = false;
    uint32_t batch_group = 0;     // batched pass: rows come in groups of this many consecutive positions of one sequence
    std::vector<TimedPass> kev;
    std::vector<double> kev_bytes;
    size_t kev_used = 0;
    std::vector<TimedPass> aev;        // attention launches of verify passes (profiling mode)
    size_t aev_used = 0;
    double aev_us = 0;
    uint32_t aev_n = 0;
    double kev_us = 0, kev_bytes_sum = 0;
    uint32_t kev_n = 0;
    std::map<double, std::pair<double, uint32_t>> kev_by_size;   // bytes -> (us sum, launches)
    double verify_us = 0, base_us = 0;
    uint32_t verify_n = 0, base_n = 0;
    // one launch for the QKV product and the attention of passes of at most
    // 8 rows (k_qkv_attn, pf_pass.hip): the rows' q/k/v as LL words
    // [MAX_PASS_ROWS][3 D], the pass epoch k_embed advances, and the flag a
    // timed-out wait sets.  PF_QKV_ATTN=0 launches the two separately.
    unsigned long long* ll = nullptr;
    uint32_t* ep = nullptr;
    uint32_t* ll_err = nullptr;
    bool qkv_attn = true;
    // one launch for the O, gate|up and down products of one-row passes
    // (k_o_ffn, pf_pass.hip): the residual rows after O [8][D], the SwiGLU
    // rows [8][F] and the merged attention rows [8][D], as LL words.
    // PF_O_FFN=0 launches them separately.
    unsigned long long* llt = nullptr;
    bool o_ffn = true;
    // one launch per layer of a one-row pass (k_layer, pf_pass.hip): the
    // attention's chunk results as LL words (one row: S pairs [H][s_stride],
    // then U [H][cstride][hd]).  PF_LAYER=0 keeps the two launches.
    unsigned long long* lla = nullptr;
    bool layer_fuse = true;
    // one launch for every layer of a one-row pass (k_stack, pf_pass.hip):
    // the per-layer operand table, whether every layer suits the fused
    // roles, and PF_STACK=0 to keep one launch per layer (k_layer)
    StackLayer* lw = nullptr;
    bool stack_ok = false;
    bool stack = true;
    // a second stream for the MTP head chain beside a one-row verify pass
    // (fork and join events), its launches limited to mtp_side_waves waves
    // so that they leave the CUs to the verify pass (PF_MTP_SIDE_WAVES);
    // PF_MTP_OVERLAP=0 keeps them in sequence
    hipStream_t st2 = nullptr;
    hipEvent_t evf = nullptr, evj = nullptr;
    bool mtp_overlap = true;
    uint32_t mtp_side_waves = 256;
    // continuous batching (pf_batch_open / admit / step / take, pf_batch.hip):
    // per sequence slot its state (0 free, 1 generating, 2 finished), token
    // budget, generated count, verify-row reuse, memory-guard stop, counters
    // and the last device state read back
    bool bs_open = false;
    SamplingCfg bs_cfg{};
    std::vector<uint8_t> bs_state, bs_have, bs_oom;
    std::vector<uint32_t> bs_ngen, bs_lim;
    std::vector<pf_gen_result> bs_res;
    std::vector<DecodeState> bs_hs;
};

template <class T>
static pf_status ealloc(pf_engine* e, T** p, size_t n) {
    pf_status s = dalloc_t(e->c, p, n);
    if (!s) e->owned.push_back({(void*)*p, n * sizeof(T)});
    return s;
}

// RoPE tables of src/engine.cpp:656-682 (theta 5e6): cos/sin of pos * freq
// for pair t, freq = 1 / pow(theta, 2t / head_dim), computed with the host
// C library in float as the reference does.
static void rope_tables(uint32_t hd, uint32_t npos, std::vector<float>& cs, std::vector<float>& sn) {
    const uint32_t half = hd / 2;
    cs.resize((size_t)npos * half);
    sn.resize((size_t)npos * half);
    std::vector<float> freq(half);
    for (uint32_t t = 0; t < half; t++) freq[t] = 1.0f / powf(5000000.0f, (float)(2 * t) / (float)hd);
    for (uint32_t p = 0; p < npos; p++)
        for (uint32_t t = 0; t < half; t++) {
            float ang = (float)p * freq[t];
            cs[(size_t)p * half + t] = cosf(ang);
            sn[(size_t)p * half + t] = sinf(ang);
        }
}

static pf_status engine_create(pf_model* m, const pf_cache_desc* cd, uint32_t nseq, pf_engine** out) {
    if (!m || !cd || !out || nseq == 0) return PF_ERR_ARG;
    pf_ctx* c = m->ctx;
    if (!model_complete(m)) return fail(c, PF_ERR_STATE, "model has unset matrices");
    const pf_model_desc& d = m->d;
    const uint32_t R = d.n_mtp + 1;
    if (nseq > MAX_SEQS || R * nseq > MAX_ROWS)
        return fail(c, PF_ERR_UNSUPPORTED, "sequences x (n_mtp + 1) verify rows exceed 512, or more than 128 sequences");
    pf_engine* e = new pf_engine();
    e->m = m;
    e->c = c;
    e->nseq = nseq;
    pf_status s = kv_geom(c, d.n_layers, d.n_heads, d.head_dim, cd->sink_size, cd->window_size, cd->pool_block,
                          cd->max_context, MAX_PREFILL_ROWS, &e->g);
    e->g.n_seq = nseq;
    if (!s) s = kv_alloc(c, e->g, &e->kv, &e->kv_bytes);
    if (s) { delete e; return s; }
    const uint32_t D = d.n_embd, F = d.n_ff, V = d.n_vocab, H = d.n_heads, hd = d.head_dim;
    // rows of the pass buffers: prompt passes, or a batched verify pass
    // (the MFMA GEMM reads whole 32-row activation tiles)
    const uint32_t PR = std::max(MAX_PREFILL_ROWS, (R * nseq + 31) / 32 * 32);
    const uint32_t MR = std::max(MAX_PASS_ROWS, R * nseq);   // rows of pass-B outputs
    const uint32_t MA = std::max(MAX_PASS_ROWS, nseq);       // rows of pass-A outputs
    e->rows = PR;
    e->spos.assign(nseq, 0);
    e->rope_pos = cd->max_context + 2 * PR;
    {
        std::vector<float> cs, sn;
        rope_tables(hd, e->rope_pos, cs, sn);
        s = ealloc(e, &e->rope_c, cs.size());
        if (!s) s = ealloc(e, &e->rope_s, sn.size());
        if (s) { pf_engine_destroy(e); return s; }
        PF_HIP(c, hipMemcpy(e->rope_c, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
        PF_HIP(c, hipMemcpy(e->rope_s, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    }
    e->kmax = std::max(D, F);
    e->pool_rows_max = (MAX_PREFILL_ROWS + e->g.pool_block - 1) / e->g.pool_block + 1;
    // prompt passes: at most one window of rows, so that every pooled row a
    // pass sees was folded from entries stored before the pass
    e->prefill_rows = std::min(PR, e->g.window);
    const uint32_t cmax = KV_SINK_ROWS + e->g.pool_cap + e->g.window;
    if (H > 128 || (uint64_t)H * ((cmax + 1 + 255) / 256) > 2048) {
        pf_engine_destroy(e);
        return fail(c, PF_ERR_UNSUPPORTED, "heads x attention chunks exceeds 2048 (context too long for the merge)");
    }
    e->cmax = cmax;
    e->s_stride = 2 * ((cmax + 1 + 255) / 256) + 8;    // per (row, head): chunk max and sum
    e->cstride = (cmax + 1 + 255) / 256 + 1;          // per (row, head): chunk partials
    if (const char* v = std::getenv("PF_PREFETCH_BLOCKS")) e->pf_blocks = (uint32_t)std::strtoul(v, nullptr, 10);
    if (const char* v = std::getenv("PF_L2_BLOCKS")) e->l2_blocks = 8u * ((uint32_t)std::strtoul(v, nullptr, 10) / 8u);
    if (!s) s = ealloc(e, &e->sink, 1);
    if (!s) s = ealloc(e, &e->x, (size_t)PR * D);
    if (!s) s = ealloc(e, &e->act, (size_t)PR * e->kmax);
    if (!s) s = ealloc(e, &e->as, 4 * PR);
    if (!s) s = ealloc(e, &e->q, (size_t)PR * D);
    if (!s) s = ealloc(e, &e->k, (size_t)PR * D);
    if (!s) s = ealloc(e, &e->v, (size_t)PR * D);
    if (!s) s = ealloc(e, &e->S, (size_t)PR * H * e->s_stride);
    if (!s) s = ealloc(e, &e->Wp, (size_t)PR * H * e->cstride * hd);
    if (!s) s = ealloc(e, &e->sg, (size_t)PR * F);
    if (!s) s = ealloc(e, &e->pmax, (size_t)GEMV_MAX_M * (2 * F / 32));
    if (!s) s = ealloc(e, &e->logitsA, (size_t)MA * V);
    if (!s) s = ealloc(e, &e->hiddenA, (size_t)MA * D);
    if (!s) s = ealloc(e, &e->logitsB, (size_t)MR * V);
    if (!s) s = ealloc(e, &e->hiddenB, (size_t)MR * D);
    if (!s) s = ealloc(e, &e->mcur, (size_t)std::max(nseq, d.n_mtp) * D);
    if (!s) s = ealloc(e, &e->ma, (size_t)nseq * D);
    if (!s) s = ealloc(e, &e->mlogits, (size_t)std::max(1u, d.n_mtp) * V);
    if (!s) s = ealloc(e, &e->mlogb, (size_t)nseq * V);
    if (!s) s = ealloc(e, &e->seeds, nseq);
    if (!s) s = ealloc(e, &e->sel, nseq);
    if (!s) s = ealloc(e, &e->pdA, 1);
    if (!s) s = ealloc(e, &e->pdB, 1);
    if (!s) s = ealloc(e, &e->pdP, 1);
    if (!s) s = ealloc(e, &e->st, nseq);
    if (!s) s = ealloc(e, &e->ll, (size_t)MAX_PASS_ROWS * 3 * D);
    if (!s) s = ealloc(e, &e->ep, 2);
    if (!s) s = ealloc(e, &e->llt, (size_t)MAX_PASS_ROWS * (2 * D + d.n_ff));
    if (!s) s = ealloc(e, &e->lla, (size_t)d.n_heads * (e->s_stride + (size_t)e->cstride * d.head_dim));
    if (!s) s = ealloc(e, &e->lw, std::max(1u, d.n_layers));
    if (s) { pf_engine_destroy(e); return s; }
    {
        const pf_model* m = e->m;
        std::vector<StackLayer> lw(d.n_layers);
        bool ok = d.n_layers > 0 && D <= 2048 && (hd == 64 || hd == 128);
        for (uint32_t l = 0; l < d.n_layers; l++) {
            lw[l] = StackLayer{m->qkv[l]->data, m->o[l]->data, m->gu[l]->data, m->down[l]->data,
                               m->attn_norm + (size_t)l * D, m->ffn_norm + (size_t)l * D};
            ok = ok && m->qkv[l]->fmt == FMT_Q4 && m->o[l]->fmt == FMT_Q4 && m->gu[l]->fmt == m->gu[0]->fmt &&
                 m->down[l]->fmt == m->down[0]->fmt;
        }
        ok = ok && stack_fmts(m->gu[0]->fmt, m->down[0]->fmt);
        e->stack_ok = ok && F % 256 == 0 && F <= 6144 && e->cstride - 1 <= 64;
        if (d.n_layers)
            PF_HIP(c, hipMemcpy(e->lw, lw.data(), lw.size() * sizeof(StackLayer), hipMemcpyHostToDevice));
    }
    e->ll_err = e->ep + 1;
    PF_HIP(c, hipMemset(e->ll, 0, (size_t)MAX_PASS_ROWS * 3 * D * 8));
    PF_HIP(c, hipMemset(e->llt, 0, (size_t)MAX_PASS_ROWS * (2 * D + d.n_ff) * 8));
    PF_HIP(c, hipMemset(e->lla, 0, (size_t)d.n_heads * (e->s_stride + (size_t)e->cstride * d.head_dim) * 8));
    PF_HIP(c, hipMemset(e->ep, 0, 8));
    if (const char* v = std::getenv("PF_QKV_ATTN")) e->qkv_attn = !(v[0] == '0');
    if (const char* v = std::getenv("PF_O_FFN")) e->o_ffn = !(v[0] == '0');
    if (const char* v = std::getenv("PF_LAYER")) e->layer_fuse = !(v[0] == '0');
    if (const char* v = std::getenv("PF_STACK")) e->stack = !(v[0] == '0');
    if (hipHostMalloc((void**)&e->word, 64, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
        hipHostGetDevicePointer((void**)&e->word_dev, e->word, 0) != hipSuccess) {
        pf_engine_destroy(e);
        return fail(c, PF_ERR_HIP, "hipHostMalloc failed");
    }
    if (const char* ng = std::getenv("PF_NO_GRAPHS")) e->use_graphs = !(ng[0] == '1');
    PF_HIP(c, hipEventCreate(&e->rev0));
    PF_HIP(c, hipEventCreate(&e->rev1));
    PF_HIP(c, hipStreamCreateWithFlags(&e->st2, hipStreamNonBlocking));   // default priority
    PF_HIP(c, hipEventCreateWithFlags(&e->evf, hipEventDisableTiming));
    PF_HIP(c, hipEventCreateWithFlags(&e->evj, hipEventDisableTiming));
    if (const char* v = std::getenv("PF_MTP_OVERLAP")) e->mtp_overlap = !(v[0] == '0');
    if (const char* v = std::getenv("PF_MTP_SIDE_WAVES")) e->mtp_side_waves = std::max(4u, (uint32_t)std::strtoul(v, nullptr, 10));
    // every field of the pass descriptors defined (single-sequence passes of
    // sequence 0) before any kernel reads them
    PassDesc pb{};
    PF_HIP(c, hipMemcpy(e->pdA, &pb, sizeof(pb), hipMemcpyHostToDevice));
    PF_HIP(c, hipMemcpy(e->pdP, &pb, sizeof(pb), hipMemcpyHostToDevice));
    pb.m = d.n_mtp + 1;
    PF_HIP(c, hipMemcpy(e->pdB, &pb, sizeof(pb), hipMemcpyHostToDevice));
    std::vector<DecodeState> st0(nseq);
    PF_HIP(c, hipMemcpy(e->st, st0.data(), nseq * sizeof(DecodeState), hipMemcpyHostToDevice));
    *out = e;
    return PF_OK;
}

extern "C" pf_status pf_engine_create(pf_model* m, const pf_cache_desc* cd, pf_engine** out) {
    return engine_create(m, cd, 1, out);
}

extern "C" void pf_engine_destroy(pf_engine* e) {
    if (!e) return;
    (void)hipStreamSynchronize(e->c->stream);
    for (auto& t : e->timed) { (void)hipEventDestroy(t.a); (void)hipEventDestroy(t.b); }
    for (auto& t : e->kev) { (void)hipEventDestroy(t.a); (void)hipEventDestroy(t.b); }
    for (auto& t : e->aev) { (void)hipEventDestroy(t.a); (void)hipEventDestroy(t.b); }
    for (auto& row : e->round_exec)
        for (auto& col : row)
            for (auto& g : col)
                if (g) (void)hipGraphExecDestroy(g);
    if (e->cont_exec) (void)hipGraphExecDestroy(e->cont_exec);
    if (e->rev0) (void)hipEventDestroy(e->rev0);
    if (e->rev1) (void)hipEventDestroy(e->rev1);
    if (e->st2) {
        (void)hipStreamSynchronize(e->st2);
        (void)hipStreamDestroy(e->st2);
    }
    if (e->evf) (void)hipEventDestroy(e->evf);
    if (e->evj) (void)hipEventDestroy(e->evj);
    for (auto& p : e->owned) dfree(e->c, p.first, p.second);
    if (e->tokens) dfree(e->c, e->tokens, e->tok_alloc * 4);
    kv_free(e->c, e->g, &e->kv);
    if (e->word) (void)hipHostFree(e->word);
    delete e;
}

extern "C" pf_status pf_engine_reset(pf_engine* e) {
    if (!e) return PF_ERR_ARG;
    e->pos = 0;
    std::fill(e->spos.begin(), e->spos.end(), 0u);
    e->hidden_valid = false;
    if (e->skip_cache) {
        // LayerSkipController::reset (src/layer_skip.cpp:89-99)
        const pf_model_desc& d = e->m->d;
        PF_HIP(e->c, hipMemset(e->skip_cache, 0, (size_t)e->nseq * d.n_layers * d.n_embd * 4));
        PF_HIP(e->c, hipMemset(e->skip_ctr, 0, 4));
    }
    return PF_OK;
}

// Engine::set_layer_skip_threshold (src/engine.cpp:266-269) with the
// controller's anchor interval (ModelConfig::skip_interval).  The controller
// runs while threshold > 0; switching it on starts from zeroed caches (a new
// controller's state).
extern "C" pf_status pf_engine_set_layer_skip(pf_engine* e, float threshold, uint32_t interval) {
    if (!e) return PF_ERR_ARG;
    pf_ctx* c = e->c;
    if (!(threshold == threshold)) return fail(c, PF_ERR_ARG, "layer-skip threshold is NaN");
    const pf_model_desc& d = e->m->d;
    const bool on = threshold > 0.0f && d.n_layers > 0;
    if (on && (d.n_embd % 64 || d.n_embd > 4096))
        return fail(c, PF_ERR_ARG, "layer skip needs n_embd % 64 == 0 and n_embd <= 4096");
    if (on && !e->skip_cache) {
        const size_t LD = (size_t)d.n_layers * d.n_embd;
        if (pf_status s = ealloc(e, &e->skip_cache, e->nseq * LD)) return s;
        if (pf_status s = ealloc(e, &e->skip_stage, (size_t)e->rows * LD)) return s;
        if (pf_status s = ealloc(e, &e->skip_flags, (size_t)e->rows * d.n_layers)) return s;
        if (pf_status s = ealloc(e, &e->skip_ctr, 1)) return s;
        if (pf_status s = ealloc(e, &e->skip_nrun, d.n_layers)) return s;
        PF_HIP(c, hipMemset(e->skip_flags, 0, (size_t)e->rows * d.n_layers * 4));
        PF_HIP(c, hipMemset(e->skip_ctr, 0, 4));
    }
    if (on && !e->skip_on) {
        PF_HIP(c, hipStreamSynchronize(c->stream));
        PF_HIP(c, hipMemset(e->skip_cache, 0, (size_t)e->nseq * d.n_layers * d.n_embd * 4));
    }
    e->skip_on = on;
    e->skip_thr = threshold;
    e->skip_interval = interval;
    e->graphs_valid = false;   // thresholds and launches are baked into captured rounds
    return PF_OK;
}

// FFN blocks skipped (rows that count) since the engine was created or reset.
extern "C" pf_status pf_engine_layer_skip_count(pf_engine* e, uint64_t* count) {
    if (!e || !count) return PF_ERR_ARG;
    uint32_t v = 0;
    if (e->skip_ctr) {
        PF_HIP(e->c, hipStreamSynchronize(e->c->stream));
        PF_HIP(e->c, hipMemcpy(&v, e->skip_ctr, 4, hipMemcpyDeviceToHost));
    }
    *count = v;
    return PF_OK;
}

extern "C" uint32_t pf_engine_position(const pf_engine* e) { return e ? e->pos : 0; }

// State snapshot of one (sequence, layer, head) plane at the sequence's
// position P: the rows of KVCache's attention order (sink, pooled, window
// oldest first; src/kv_cache.cpp:137-155) followed by the evicted window
// rows the next pooled row will fold (src/kv_cache.cpp:77-109 keeps their
// running sum).  The pooled rows P's view needs are folded first (the next
// pass would write the same values).
extern "C" pf_status pf_engine_kv_export(pf_engine* e, uint32_t seq, uint32_t layer, uint32_t head, int8_t* k,
                                         float* ks, int8_t* v, float* vs, uint32_t cap, uint32_t* counts) {
    if (!e || !k || !ks || !v || !vs || !counts) return PF_ERR_ARG;
    pf_ctx* c = e->c;
    const KvGeom& g = e->g;
    if (seq >= e->nseq || layer >= g.n_layers || head >= g.n_heads) return fail(c, PF_ERR_ARG, "plane out of range");
    const uint32_t P = seq == 0 ? e->pos : e->spos[seq];
    const KvView vw = kv_view(g, P);
    const uint32_t n_win = vw.win_hi - vw.win_lo, n_pend = vw.win_lo - vw.pool * g.pool_block;
    const uint32_t total = vw.sink + vw.pool + n_win + n_pend;
    if (total > cap) return fail(c, PF_ERR_ARG, "export capacity below the plane's row count");
    const size_t plane = ((size_t)seq * g.n_layers + layer) * g.n_heads + head;
    const uint32_t r_lo = kv_view(g, P > 0 ? P - 1 : 0).pool;
    for (uint32_t r = r_lo; r < vw.pool && r < g.pool_cap; r++)
        hipLaunchKernelGGL(k_pool_row_one, dim3(1), dim3(g.head_dim <= 64 ? 64 : 128), 0, c->stream, g, e->kv,
                           (uint32_t)plane, r);
    PF_LAUNCHED(c);
    PF_HIP(c, hipStreamSynchronize(c->stream));
    const uint32_t hd = g.head_dim;
    std::vector<int8_t> hk((size_t)g.rows * hd), hv((size_t)g.rows * hd);
    std::vector<float> hks(g.rows), hvs(g.rows);
    PF_HIP(c, hipMemcpy(hk.data(), e->kv.k + plane * g.rows * hd, hk.size(), hipMemcpyDeviceToHost));
    PF_HIP(c, hipMemcpy(hv.data(), e->kv.v + plane * g.rows * hd, hv.size(), hipMemcpyDeviceToHost));
    PF_HIP(c, hipMemcpy(hks.data(), e->kv.ks + plane * g.rows, g.rows * 4, hipMemcpyDeviceToHost));
    PF_HIP(c, hipMemcpy(hvs.data(), e->kv.vs + plane * g.rows, g.rows * 4, hipMemcpyDeviceToHost));
    uint32_t o = 0;
    auto put = [&](uint32_t row) {
        std::memcpy(k + (size_t)o * hd, hk.data() + (size_t)row * hd, hd);
        std::memcpy(v + (size_t)o * hd, hv.data() + (size_t)row * hd, hd);
        ks[o] = hks[row];
        vs[o] = hvs[row];
        o++;
    };
    for (uint32_t j = 0; j < vw.sink; j++) put(j);
    for (uint32_t j = 0; j < vw.pool; j++) put(KV_SINK_ROWS + g.ring + j);
    for (uint32_t w = vw.win_lo; w < vw.win_hi; w++) put(KV_SINK_ROWS + w % g.ring);
    for (uint32_t w = vw.pool * g.pool_block; w < vw.win_lo; w++) put(KV_SINK_ROWS + w % g.ring);
    counts[0] = vw.sink;
    counts[1] = vw.pool;
    counts[2] = n_win;
    counts[3] = n_pend;
    return PF_OK;
}

extern "C" pf_status pf_engine_set_verify_full(pf_engine* e, int32_t full) {
    if (!e) return PF_ERR_ARG;
    e->verify_full = full != 0;
    return PF_OK;
}

extern "C" pf_status pf_engine_set_mtp_enabled(pf_engine* e, int32_t enabled) {
    if (!e) return PF_ERR_ARG;
    e->mtp_enabled = enabled != 0;
    return PF_OK;
}

extern "C" pf_status pf_engine_set_max_memory(pf_engine* e, size_t bytes) {
    if (!e) return PF_ERR_ARG;
    e->max_memory = bytes;
    return PF_OK;
}

static pf_status timed_begin(pf_engine* e, bool verify, TimedPass** tp) {
    *tp = nullptr;
    if (e->capturing) return PF_OK;   // events inside captured graphs cannot be timed
    if (e->timed_used == e->timed.size()) {
        TimedPass t{};
        PF_HIP(e->c, hipEventCreate(&t.a));
        PF_HIP(e->c, hipEventCreate(&t.b));
        e->timed.push_back(t);
    }
    TimedPass* t = &e->timed[e->timed_used++];
    t->verify = verify;
    PF_HIP(e->c, hipEventRecord(t->a, e->c->stream));
    *tp = t;
    return PF_OK;
}

// Accumulates the pass event pairs [t_lo, t_hi) and GEMV event pairs
// [k_lo, k_hi) (a replayed graph's events hold that replay's times).
static pf_status harvest_events(pf_engine* e, size_t t_lo, size_t t_hi, size_t k_lo, size_t k_hi) {
    for (size_t i = 0; i < e->aev_used; i++) {
        float ms = 0;
        PF_HIP(e->c, hipEventElapsedTime(&ms, e->aev[i].a, e->aev[i].b));
        e->aev_us += ms * 1000.0;
        e->aev_n++;
    }
    e->aev_used = 0;
    for (size_t i = t_lo; i < t_hi; i++) {
        float ms = 0;
        PF_HIP(e->c, hipEventElapsedTime(&ms, e->timed[i].a, e->timed[i].b));
        if (e->timed[i].verify) { e->verify_us += ms * 1000.0; e->verify_n++; }
        else { e->base_us += ms * 1000.0; e->base_n++; }
    }
    for (size_t i = k_lo; i < k_hi; i++) {
        float ms = 0;
        PF_HIP(e->c, hipEventElapsedTime(&ms, e->kev[i].a, e->kev[i].b));
        e->kev_us += ms * 1000.0;
        e->kev_bytes_sum += e->kev_bytes[i];
        e->kev_n++;
        auto& bucket = e->kev_by_size[e->kev_bytes[i]];
        bucket.first += ms * 1000.0;
        bucket.second++;
    }
    return PF_OK;
}

// One int8-activation product of a pass: the GEMV (M <= 8; it quantizes
// its own input, x / xs / nw / a8 of `a`) or, for taller passes, the GEMM
// over act / as.  In profiling mode the dispatches of verify passes carry
// HIP start/stop events (kernel execution time, as rocprofv3 reports it).
static pf_status pass_mm(pf_engine* e, const pf_matrix* W, MmKind kind, uint32_t M, GemvArgs a, const float* as_in) {
    hipStream_t st = e->c->stream;
    a.W = W->data;
    a.N = W->rows;
    a.K = W->cols;
    a.M = M;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    if (e->profile == 1 && e->in_verify && !e->capturing) {
        if (e->kev_used == e->kev.size()) {
            TimedPass n{};
            PF_HIP(e->c, hipEventCreate(&n.a));
            PF_HIP(e->c, hipEventCreate(&n.b));
            e->kev.push_back(n);
            e->kev_bytes.push_back(0.0);
        }
        // weights, fp32 (or int8) input rows and fp32 outputs
        const double in_b = kind == MM_O ? 1.0 : 4.0;
        e->kev_bytes[e->kev_used] = (double)W->bytes + in_b * M * W->cols + 4.0 * M * W->rows;
        TimedPass* t = &e->kev[e->kev_used++];
        ev0 = t->a;
        ev1 = t->b;
    }
    if (M <= GEMV_MAX_M) {
        launch_gemv(st, W, kind, a, ev0, ev1);
    } else {
        GemmArgs g{};
        g.W = a.W; g.N = a.N; g.K = a.K; g.M = M;
        g.act = e->act; g.act_stride = e->kmax; g.as = as_in; g.gate = a.gate; g.e = a.e;
        launch_gemm(st, W, kind, g, ev0, ev1);
    }
    return PF_OK;
}

// The tiled matrix W as the next kernel's weights, loaded into the L2 of
// the XCD whose workgroups read each group by `blocks` prefetch blocks of
// the current kernel (none when blocks is 0 or W is not tiled).
static bool prefetchable(const pf_matrix* W) {
    const uint32_t groups = W ? W->rows / 32 : 0u;
    return W && !W->rowmajor && groups && W->bytes % groups == 0 && (W->bytes / groups) % 16 == 0;
}
static Prefetch prefetch_of(const pf_engine* e, const pf_matrix* W, uint32_t blocks, uint32_t xoff = 0) {
    if (!blocks || !prefetchable(W)) return Prefetch{nullptr, 0, 0, 0, e->sink, 0};
    const uint32_t groups = W->rows / 32;
    return Prefetch{W->data, (uint32_t)(W->bytes / groups), groups, blocks, e->sink, xoff};
}

// LayerSkipController's threshold for layer l (src/layer_skip.cpp:43-55):
// doubled for mid/2 < l < mid + mid/2 (mid = layers / 2), never skipping
// (-1) for the first and last two layers.  An anchor interval of 0 anchors
// every token (tokens_since_anchor_ stays 0, src/layer_skip.cpp:29-35: no
// skip, cache updated), which the threshold -1 reproduces.
static float skip_threshold(const pf_engine* e, uint32_t l) {
    const uint32_t L = e->m->d.n_layers, mid = L / 2;
    float thr = e->skip_thr;
    if (l > mid / 2 && l < mid + mid / 2) thr *= 2.0f;
    if (l < 2 || l >= L - 2 || e->skip_interval == 0) thr = -1.0f;
    return thr;
}

// Cache update for the rows j0 <= j < j1 of each sequence of a pass, or,
// with verify, for the rows the round's acceptance keeps.
static void launch_skip_commit(pf_engine* e, const PassDesc* pd, uint32_t M, uint32_t j0, uint32_t j1,
                               bool verify) {
    const pf_model_desc& d = e->m->d;
    if (!d.n_layers) return;
    hipLaunchKernelGGL(k_skip_commit, dim3(d.n_layers, e->nseq), dim3(256), 0, e->c->stream, pd, M,
                       (const float*)e->skip_stage, (const uint32_t*)e->skip_flags, e->rows, e->skip_cache,
                       d.n_layers, d.n_embd, j0, j1, verify ? (const DecodeState*)e->st : nullptr, d.n_mtp,
                       e->skip_ctr);
}

// A wait of k_qkv_attn's attention blocks that ran out of rounds (its
// results are invalid): reported by the call that ran the passes, and
// cleared.  Waits end within microseconds in practice; the bound only keeps a
// launch from running forever.
static pf_status ll_check(pf_engine* e) {
    uint32_t v = 0;
    PF_HIP(e->c, hipMemcpyAsync(&v, e->ll_err, 4, hipMemcpyDeviceToHost, e->c->stream));
    PF_HIP(e->c, hipStreamSynchronize(e->c->stream));
    if (!v) return PF_OK;
    PF_HIP(e->c, hipMemsetAsync(e->ll_err, 0, 4, e->c->stream));
    PF_HIP(e->c, hipStreamSynchronize(e->c->stream));
    return fail(e->c, PF_ERR_DEVICE, "a wait for the QKV product's rows timed out inside k_qkv_attn");
}

// Chunk capacity of the merge prologue's loads: the chunks of the largest
// list the engine's buffers hold, if heads * chunks fits its LDS tables.
static uint32_t merge_ncap(const pf_engine* e) {
    const uint32_t n = e->cstride - 1;
    return e->m->d.n_heads * n <= 2048 ? n : 0u;
}

// k_o_ffn serves layer l of a decode pass of at most 8 rows: three Q4
// matrices, F a multiple of 256 up to 6144 (at most three 256-column chunks
// per wave of the down product), D <= 2048 (one 256-column chunk per wave
// of the O and gate|up products), no layer skip.
static bool o_ffn_ok(const pf_engine* e, uint32_t l) {
    const pf_model* m = e->m;
    const uint32_t F = m->d.n_ff;
    return e->o_ffn && !e->skip_on && m->o[l]->fmt == FMT_Q4 && m->gu[l]->fmt == FMT_Q4 &&
           m->down[l]->fmt == FMT_Q4 && F % 256 == 0 && F <= 6144 && m->d.n_embd <= 2048;
}

template <int CPWD, int MR>
static void o_ffn_one(hipStream_t st, const GemvArgs& ao, const GemvArgs& ag, const GemvArgs& ad, hipEvent_t ev0,
                      hipEvent_t ev1) {
    const uint32_t n_mg = ao.M * ((ao.K + 511) / 512), n_o = ao.N / 32, n_gu = ag.N / 32;
    const uint32_t n_dn = MR == 1 ? ad.N / 32 : 0u;
    static bool attr = false;   // LDS beyond 64 KiB is granted per kernel
    if (!attr) {
        (void)hipFuncSetAttribute((const void*)k_o_ffn<FMT_Q4, CPWD, MR>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  o_ffn_smem(MR, 2048, 6144));
        attr = true;
    }
    const uint32_t smem = o_ffn_smem(ao.M, ao.K, ad.K);
    const dim3 grid(n_mg + n_o + n_gu + n_dn);
    // the merge workgroups' inputs lead the argument list (preloaded into SGPRs)
    if (ev0)
        hipExtLaunchKernelGGL((k_o_ffn<FMT_Q4, CPWD, MR>), grid, dim3(512), smem, st, ev0, ev1, 0, n_mg, n_o, n_gu,
                              ao.S, ao.Up, ao.s_stride, ao.cstride, ao.K, ao.e.hd, ao.ncap, ao.lli.ep, ao.e.pd, ao, ag,
                              ad);
    else
        hipLaunchKernelGGL((k_o_ffn<FMT_Q4, CPWD, MR>), grid, dim3(512), smem, st, n_mg, n_o, n_gu, ao.S, ao.Up,
                           ao.s_stride, ao.cstride, ao.K, ao.e.hd, ao.ncap, ao.lli.ep, ao.e.pd, ao, ag, ad);
}

template <int MR>
static void o_ffn_rows(hipStream_t st, const GemvArgs& ao, const GemvArgs& ag, const GemvArgs& ad, hipEvent_t ev0,
                       hipEvent_t ev1) {
    switch ((ad.K / 256 + GEMV_WAVES - 1) / GEMV_WAVES) {
        case 1: o_ffn_one<1, MR>(st, ao, ag, ad, ev0, ev1); break;
        case 2: o_ffn_one<2, MR>(st, ao, ag, ad, ev0, ev1); break;
        default: o_ffn_one<3, MR>(st, ao, ag, ad, ev0, ev1); break;
    }
}

// Rows held in registers: 1, 5 (verify passes of four heads), else 8.  With
// more than one row the launch ends with gate|up (no down role).
static void launch_o_ffn(hipStream_t st, const GemvArgs& ao, const GemvArgs& ag, const GemvArgs& ad, hipEvent_t ev0,
                         hipEvent_t ev1) {
    if (ao.M == 1) o_ffn_rows<1>(st, ao, ag, ad, ev0, ev1);
    else if (ao.M <= 5) o_ffn_one<1, 5>(st, ao, ag, ad, ev0, ev1);
    else o_ffn_one<1, 8>(st, ao, ag, ad, ev0, ev1);
}

template <int P, int CPWD>
static void layer_one(hipStream_t st, const GemvArgs& a, const AttnGroupArgs& b, const GemvArgs& ao,
                      const GemvArgs& ag, const GemvArgs& ad, uint32_t tasks, hipEvent_t ev0, hipEvent_t ev1) {
    static bool attr = false;   // LDS beyond 64 KiB is granted per kernel
    if (!attr) {
        (void)hipFuncSetAttribute((const void*)k_layer<FMT_Q4, P, CPWD>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  layer_smem(2048, 6144));
        attr = true;
    }
    const uint32_t nq = a.N / 32, n_mg = (ao.K + 511) / 512, n_o = ao.N / 32, n_gu = ag.N / 32, n_dn = ad.N / 32;
    const uint32_t smem = layer_smem(ao.K, ad.K);
    const dim3 grid(nq + tasks + n_mg + n_o + n_gu + n_dn);
    if (ev0)
        hipExtLaunchKernelGGL((k_layer<FMT_Q4, P, CPWD>), grid, dim3(512), smem, st, ev0, ev1, 0, nq, tasks, n_mg, n_o,
                              n_gu, b.pd, a.W, a.x, a.nw, a, b, ao, ag, ad);
    else
        hipLaunchKernelGGL((k_layer<FMT_Q4, P, CPWD>), grid, dim3(512), smem, st, nq, tasks, n_mg, n_o, n_gu, b.pd,
                           a.W, a.x, a.nw, a, b, ao, ag, ad);
}

template <int P>
static void layer_cpw(hipStream_t st, const GemvArgs& a, const AttnGroupArgs& b, const GemvArgs& ao,
                      const GemvArgs& ag, const GemvArgs& ad, uint32_t tasks, hipEvent_t ev0, hipEvent_t ev1) {
    switch ((ad.K / 256 + GEMV_WAVES - 1) / GEMV_WAVES) {
        case 1: layer_one<P, 1>(st, a, b, ao, ag, ad, tasks, ev0, ev1); break;
        case 2: layer_one<P, 2>(st, a, b, ao, ag, ad, tasks, ev0, ev1); break;
        default: layer_one<P, 3>(st, a, b, ao, ag, ad, tasks, ev0, ev1); break;
    }
}

static void launch_layer(hipStream_t st, uint32_t hd, const GemvArgs& a, const AttnGroupArgs& b, const GemvArgs& ao,
                         const GemvArgs& ag, const GemvArgs& ad, uint32_t tasks, hipEvent_t ev0, hipEvent_t ev1) {
    if (hd == 64) layer_cpw<4>(st, a, b, ao, ag, ad, tasks, ev0, ev1);
    else layer_cpw<8>(st, a, b, ao, ag, ad, tasks, ev0, ev1);
}

template <int FG, int FD, int P, int CPWD>
static void stack_one(hipStream_t st, uint32_t nl, const StackLayer* lw, const GemvArgs& a, const AttnGroupArgs& b,
                      const GemvArgs& ao, const GemvArgs& ag, const GemvArgs& ad, uint32_t tasks, hipEvent_t ev0,
                      hipEvent_t ev1) {
    static bool attr = false;   // LDS beyond 64 KiB is granted per kernel
    if (!attr) {
        (void)hipFuncSetAttribute((const void*)k_stack<FMT_Q4, FG, FD, P, CPWD>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, layer_smem(2048, 6144));
        attr = true;
    }
    const uint32_t nq = a.N / 32, n_mg = (ao.K + 511) / 512, n_o = ao.N / 32, n_gu = ag.N / 32, n_dn = ad.N / 32;
    const uint32_t G = nq + tasks + n_mg + n_o + n_gu + n_dn;
    const uint32_t smem = layer_smem(ao.K, ad.K);
    const dim3 grid(G * nl);
    if (ev0)
        hipExtLaunchKernelGGL((k_stack<FMT_Q4, FG, FD, P, CPWD>), grid, dim3(512), smem, st, ev0, ev1, 0, nq, tasks,
                              n_mg, n_o, n_gu, G, b.pd, lw, a, b, ao, ag, ad);
    else
        hipLaunchKernelGGL((k_stack<FMT_Q4, FG, FD, P, CPWD>), grid, dim3(512), smem, st, nq, tasks, n_mg, n_o, n_gu,
                           G, b.pd, lw, a, b, ao, ag, ad);
}

template <int FG, int FD>
static void stack_fmt(hipStream_t st, uint32_t hd, uint32_t nl, const StackLayer* lw, const GemvArgs& a,
                      const AttnGroupArgs& b, const GemvArgs& ao, const GemvArgs& ag, const GemvArgs& ad,
                      uint32_t tasks, hipEvent_t ev0, hipEvent_t ev1) {
    const uint32_t cpw = (ad.K / 256 + GEMV_WAVES - 1) / GEMV_WAVES;
    if (hd == 64) {
        if (cpw == 1) stack_one<FG, FD, 4, 1>(st, nl, lw, a, b, ao, ag, ad, tasks, ev0, ev1);
        else if (cpw == 2) stack_one<FG, FD, 4, 2>(st, nl, lw, a, b, ao, ag, ad, tasks, ev0, ev1);
        else stack_one<FG, FD, 4, 3>(st, nl, lw, a, b, ao, ag, ad, tasks, ev0, ev1);
    } else {
        if (cpw == 1) stack_one<FG, FD, 8, 1>(st, nl, lw, a, b, ao, ag, ad, tasks, ev0, ev1);
        else if (cpw == 2) stack_one<FG, FD, 8, 2>(st, nl, lw, a, b, ao, ag, ad, tasks, ev0, ev1);
        else stack_one<FG, FD, 8, 3>(st, nl, lw, a, b, ao, ag, ad, tasks, ev0, ev1);
    }
}

static void launch_stack(hipStream_t st, int32_t fg, uint32_t hd, uint32_t nl, const StackLayer* lw,
                         const GemvArgs& a, const AttnGroupArgs& b, const GemvArgs& ao, const GemvArgs& ag,
                         const GemvArgs& ad, uint32_t tasks, hipEvent_t ev0, hipEvent_t ev1) {
    if (fg == FMT_Q4) stack_fmt<FMT_Q4, FMT_Q4>(st, hd, nl, lw, a, b, ao, ag, ad, tasks, ev0, ev1);
    else stack_fmt<FMT_Q2, FMT_Q15>(st, hd, nl, lw, a, b, ao, ag, ad, tasks, ev0, ev1);
}

// One forward pass of M rows (the PassDesc at `pd` holds positions and
// tokens; pos0 is the host's copy of the first position).  hidden/logits
// outputs are device [M][D] / [M][V]; either may be null.  A batched pass
// (the descriptor gives every row its sequence and position) passes
// batch = true and the highest position of its rows as pos_last.
//
// Per layer, for M <= 8 rows: QKV product (RMSNorm + quantize prologue,
// RoPE epilogue), KV store, attention chunks, chunk merge + quantize, O
// product (residual epilogue), gate|up product (RMSNorm + quantize
// prologue, SwiGLU epilogue), down product (quantize prologue, residual
// epilogue): seven kernels.  Taller passes quantize their rows in row
// kernels and run the GEMM with the same epilogues.
static pf_status run_pass(pf_engine* e, PassDesc* pd, uint32_t M, uint32_t pos0, float* logits, float* hidden,
                          bool batch = false, uint32_t pos_last = 0) {
    pf_ctx* c = e->c;
    const pf_model* m = e->m;
    const pf_model_desc& d = m->d;
    const KvGeom& g = e->g;
    hipStream_t st = c->stream;
    const uint32_t D = d.n_embd, F = d.n_ff, H = d.n_heads, hd = d.head_dim;
    if (!batch) pos_last = pos0 + M - 1;
    if (M == 0 || M > e->rows) return fail(c, PF_ERR_ARG, "pass height beyond the engine's pass buffers");
    if (!e->capturing && pos_last + 1 > e->rope_pos)
        return fail(c, PF_ERR_CAPACITY, "position beyond the engine's max_context");
    // captured passes replay at any position: grids sized for the largest view
    const uint32_t cmax = e->capturing ? e->cmax : kv_view(g, pos_last).count();
    // attention tasks: (head, 256-entry chunk)
    const uint32_t attn_tasks = H * ((cmax + 1 + 255) / 256);
    const uint32_t ks = e->kmax;
    const bool tall = M > GEMV_MAX_M;
    const bool merge_in_o = M == 1 && D <= 2048;
    // activation scales [4][rows] of the tall passes' row kernels
    float* as0 = e->as;                   // attention-norm act
    float* as1 = e->as + e->rows;         // attention output act
    float* as2 = e->as + 2 * e->rows;     // ffn-norm act
    float* as3 = e->as + 3 * e->rows;     // swiglu act

    // pooled rows the pass can see (folded from window entries still in the ring)
    // and the embedded rows, in one launch (k_pass_prep)
    {
        const uint32_t n_pool = g.n_layers * g.n_heads * (batch ? M : e->pool_rows_max);
        hipLaunchKernelGGL(k_pass_prep, dim3(n_pool + (D + 127) / 128 * M), dim3(128), 0, st, g, e->kv, pd, n_pool,
                           m->emb->data, m->emb->scales, d.n_vocab, D, e->x, e->ep, (int32_t)m->emb->fmt);
    }
    // one-row passes: every layer in one launch (k_stack); LL words of the
    // residual rows between layers after the three of k_layer in llt
    const bool stack = M == 1 && e->stack && e->stack_ok && e->qkv_attn && e->o_ffn && !e->skip_on;
    if (stack) {
        const uint32_t nl = d.n_layers;
        unsigned long long* const lx = e->llt;
        unsigned long long* const lsg = e->llt + D;
        unsigned long long* const lmg = lsg + F;
        unsigned long long* const lxo = lmg + D;
        const LLIn li{nullptr, e->ep, nl, 0u, e->ll_err};
        GemvArgs a{};
        a.e.rc = e->rope_c; a.e.rs = e->rope_s; a.e.pd = pd; a.e.D = D; a.e.hd = hd;
        a.e.ll = e->ll; a.e.ep = e->ep; a.e.fmul = nl; a.e.fadd = 0;
        a.x = e->x; a.xs = D;
        a.N = m->qkv[0]->rows; a.K = D; a.M = 1;
        a.lli = li;
        a.lli.ll = lxo;
        a.lli.sent = D - 1;
        // layers after the first: the QKV weight loads wait for the layer
        // before's O product, the attention's cached K/V loads for its down
        // product, so that neither competes with that layer's hand-offs
        a.lli.gate = lx;
        a.lli.gate_off = D - 1;
        a.lli.gate_back = 1;
        AttnGroupArgs b{pd, g, e->kv, 0u, 1, e->S, e->s_stride, e->Wp, e->cstride, prefetch_of(e, nullptr, 0),
                        LLIn{e->ll, e->ep, nl, 0u, e->ll_err}};
        b.lli.out = e->lla;
        b.lli.sreg = H * e->s_stride;
        b.lli.gate = lxo;
        b.lli.gate_off = D - 1;
        GemvArgs ao{}, ag{}, ad{};
        ao.N = D; ao.K = D; ao.M = 1; ao.xs = D; ao.g = g;
        ao.e.pd = pd; ao.e.hd = hd; ao.e.D = D;
        ao.e.y = e->x; ao.e.y_stride = D; ao.e.ll = lx; ao.e.llold = lxo;
        ao.lli = li;
        ao.lli.ll = lmg;
        ag.N = m->gu[0]->rows; ag.K = D; ag.M = 1; ag.xs = D;
        ag.e.y_stride = F; ag.e.ll = lsg;
        ag.lli = li;
        ag.lli.ll = lx;
        ad.N = D; ad.K = F; ad.M = 1; ad.xs = F;
        ad.e.y = e->x; ad.e.y_stride = D; ad.e.llold = lx; ad.e.ll = lxo;
        if (hidden) ad.e.y2 = hidden;
        ad.lli = li;
        ad.lli.ll = lsg;
        for (GemvArgs* x : {&ao, &ag, &ad}) {   // weight loads after the layer's QKV product
            x->lli.gate = e->ll;
            x->lli.gate_off = 3 * D - 1;
        }
        hipEvent_t ev0 = nullptr, ev1 = nullptr;
        if (e->profile == 1 && e->in_verify && !e->capturing) {
            if (e->kev_used == e->kev.size()) {
                TimedPass n{};
                PF_HIP(c, hipEventCreate(&n.a));
                PF_HIP(c, hipEventCreate(&n.b));
                e->kev.push_back(n);
                e->kev_bytes.push_back(0.0);
            }
            // every layer's four matrices with their fp32 input and output
            // rows, and the visible K/V rows with their scales
            double bytes = 0.0;
            for (uint32_t l = 0; l < nl; l++)
                for (const pf_matrix* W : {m->qkv[l], m->o[l], m->gu[l], m->down[l]})
                    bytes += (double)W->bytes + 4.0 * W->cols + 4.0 * W->rows;
            bytes += 2.0 * nl * H * (hd + 4.0) * kv_view(g, pos_last).count();
            e->kev_bytes[e->kev_used] = bytes;
            ev0 = e->kev[e->kev_used].a;
            ev1 = e->kev[e->kev_used].b;
            e->kev_used++;
        }
        launch_stack(st, m->gu[0]->fmt, hd, nl, e->lw, a, b, ao, ag, ad, attn_tasks, ev0, ev1);
    }
    for (uint32_t l = 0; l < (stack ? 0u : d.n_layers); l++) {
        const float* an = m->attn_norm + (size_t)l * D;
        const float* fn = m->ffn_norm + (size_t)l * D;
        // Q/K/V with RoPE (src/engine.cpp:515-523, 693-749)
        GemvArgs a{};
        a.e.q = e->q; a.e.k = e->k; a.e.v = e->v;
        a.e.rc = e->rope_c; a.e.rs = e->rope_s; a.e.pd = pd; a.e.D = D; a.e.hd = hd;
        a.x = e->x; a.xs = D; a.nw = an;
        if (tall)
            PF_PER1024_SWITCH(D, hipLaunchKernelGGL(k_norm_quant<PER>, dim3(M), dim3(1024), 0, st, (const float*)e->x,
                                                    D, an, e->act, ks, as0));
        // passes of at most 8 rows: the QKV product and the attention in one
        // launch (its attention blocks load the cached K/V rows while the
        // product runs)
        const bool qa = e->qkv_attn && !tall && attn_fused(M) && m->qkv[l]->fmt == FMT_Q4 && (hd == 64 || hd == 128);
        // one-row passes: the whole layer in one launch (k_layer)
        if (M == 1 && qa && e->layer_fuse && D <= 2048 && o_ffn_ok(e, l) && e->cstride - 1 <= 64) {
            const LLIn li{nullptr, e->ep, d.n_layers, l, e->ll_err};
            a.W = m->qkv[l]->data;
            a.N = m->qkv[l]->rows;
            a.K = m->qkv[l]->cols;
            a.M = 1;
            a.e.ll = e->ll;
            a.e.ep = e->ep;
            a.e.fmul = d.n_layers;
            a.e.fadd = l;
            AttnGroupArgs b{pd, g, e->kv, l, 1, e->S, e->s_stride, e->Wp, e->cstride, prefetch_of(e, nullptr, 0),
                            LLIn{e->ll, e->ep, d.n_layers, l, e->ll_err}};
            b.lli.out = e->lla;
            b.lli.sreg = H * e->s_stride;
            unsigned long long* const lx = e->llt;
            unsigned long long* const lsg = e->llt + D;
            unsigned long long* const lmg = lsg + F;
            GemvArgs ao{}, ag{}, ad{};
            ao.W = m->o[l]->data; ao.N = D; ao.K = D; ao.M = 1; ao.xs = D; ao.g = g;
            ao.e.pd = pd; ao.e.hd = hd; ao.e.D = D;
            ao.e.y = e->x; ao.e.y_stride = D; ao.e.ll = lx;
            ao.nx = prefetch_of(e, l + 1 < d.n_layers ? m->qkv[l + 1] : nullptr, e->l2_blocks ? D / 32 : 0u);
            ao.lli = li;
            ao.lli.ll = lmg;
            ag.W = m->gu[l]->data; ag.N = m->gu[l]->rows; ag.K = D; ag.M = 1; ag.xs = D; ag.nw = fn;
            ag.e.y_stride = F; ag.e.ll = lsg;
            ag.lli = li;
            ag.lli.ll = lx;
            ad.W = m->down[l]->data; ad.N = D; ad.K = F; ad.M = 1; ad.xs = F;
            ad.e.y = e->x; ad.e.y_stride = D; ad.e.llold = lx;
            if (l + 1 == d.n_layers && hidden) ad.e.y2 = hidden;
            ad.lli = li;
            ad.lli.ll = lsg;
            for (GemvArgs* x : {&ao, &ag, &ad}) {   // weight loads after the QKV product's last word
                x->lli.gate = e->ll;
                x->lli.gate_off = 3 * D - 1;
            }
            hipEvent_t ev0 = nullptr, ev1 = nullptr;
            if (e->profile == 1 && e->in_verify && !e->capturing) {
                if (e->kev_used == e->kev.size()) {
                    TimedPass n{};
                    PF_HIP(c, hipEventCreate(&n.a));
                    PF_HIP(c, hipEventCreate(&n.b));
                    e->kev.push_back(n);
                    e->kev_bytes.push_back(0.0);
                }
                // the four matrices with their fp32 input and output rows, and
                // the visible K/V rows with their scales
                double bytes = 0.0;
                for (const pf_matrix* W : {m->qkv[l], m->o[l], m->gu[l], m->down[l]})
                    bytes += (double)W->bytes + 4.0 * W->cols + 4.0 * W->rows;
                bytes += 2.0 * H * (hd + 4.0) * kv_view(g, pos_last).count();
                e->kev_bytes[e->kev_used] = bytes;
                ev0 = e->kev[e->kev_used].a;
                ev1 = e->kev[e->kev_used].b;
                e->kev_used++;
            }
            launch_layer(st, hd, a, b, ao, ag, ad, attn_tasks, ev0, ev1);
            continue;
        }
        if (!qa)
            if (pf_status s = pass_mm(e, m->qkv[l], MM_QKV, M, a, as0)) return s;
        if (!attn_fused(M))
            hipLaunchKernelGGL(k_kv_store_pass, dim3(M, H), dim3(64), 0, st, (const PassDesc*)pd, g, e->kv, l,
                               (const float*)e->k, (const float*)e->v);
        hipEvent_t aev0 = nullptr, aev1 = nullptr;
        if (e->profile == 1 && e->in_verify && !e->capturing) {
            if (e->aev_used == e->aev.size()) {
                TimedPass n{};
                PF_HIP(c, hipEventCreate(&n.a));
                PF_HIP(c, hipEventCreate(&n.b));
                e->aev.push_back(n);
            }
            aev0 = e->aev[e->aev_used].a;
            aev1 = e->aev[e->aev_used].b;
            e->aev_used++;
        }
        // one-row passes merge the chunks in the O product's prologue, and the
        // attention's extra blocks load the O weights into the L2 of the XCDs
        // whose O workgroups read them; other passes run the merge kernel,
        // whose extra blocks do.  Each decode GEMV's extra blocks do the same
        // for the next product (O -> gate|up -> down -> next layer's QKV).
        // with k_o_ffn the O, gate|up and down workgroups follow the merge
        // workgroups in its grid, so their XCDs are offset by those before them
        const bool tail = !tall && D <= 2048 && o_ffn_ok(e, l);
        const uint32_t n_mg = M * ((D + 511) / 512), n_gu = m->gu[l]->rows / 32;
        const Prefetch opf = tail ? prefetch_of(e, m->o[l], e->pf_blocks, n_mg)
                                  : (merge_in_o ? prefetch_of(e, m->o[l], e->pf_blocks) : prefetch_of(e, nullptr, 0));
        if (qa) {
            a.W = m->qkv[l]->data;
            a.N = m->qkv[l]->rows;
            a.K = m->qkv[l]->cols;
            a.M = M;
            a.e.ll = e->ll;
            a.e.ep = e->ep;
            a.e.fmul = d.n_layers;
            a.e.fadd = l;
            AttnGroupArgs b{pd, g, e->kv, l, M, e->S, e->s_stride, e->Wp, e->cstride, opf,
                            LLIn{e->ll, e->ep, d.n_layers, l, e->ll_err}};
            // one-row passes: the gate|up and down weights too (with more rows
            // the heavier attention is slowed more by those loads than
            // k_o_ffn gains: 5 rows 18.9 -> 21.5 us against 24.3 -> 20.7 us)
            if (tail && M == 1) {
                b.pf2 = prefetch_of(e, m->gu[l], e->pf_blocks, n_mg + D / 32);
                b.pf3 = prefetch_of(e, m->down[l], e->pf_blocks, n_mg + D / 32 + n_gu);
            }
            if (hd == 64) qkv_attn_rows<4>(st, a, b, attn_tasks, aev0, aev1);
            else qkv_attn_rows<8>(st, a, b, attn_tasks, aev0, aev1);
        } else {
            launch_attn(st, hd, M, attn_tasks, pd, g, e->kv, l, e->q, e->k, e->v, e->S, e->s_stride, e->Wp,
                        e->cstride, opf, batch, batch ? e->batch_group : 0u, aev0, aev1);
        }
        if (!merge_in_o && !tail)
            PF_PER1024_SWITCH(D, hipLaunchKernelGGL(k_attn_merge_quant<PER>, dim3(M + e->pf_blocks), dim3(1024), 0, st,
                                                    pd, g, (const float*)e->S, e->s_stride, (const float*)e->Wp,
                                                    e->cstride, e->act, ks, as1, (int32_t*)nullptr, 0u, M,
                                                    prefetch_of(e, m->o[l], e->pf_blocks)));
        // decode passes without layer skip: the merge, O, gate|up and down in
        // one launch; LL words in llt: residual rows [M][D], SwiGLU rows
        // [M][F], merged attention rows [M][D]
        if (tail) {
            const LLIn li{nullptr, e->ep, d.n_layers, l, e->ll_err};
            unsigned long long* const lx = e->llt;
            unsigned long long* const lsg = e->llt + (size_t)M * D;
            unsigned long long* const lmg = lsg + (size_t)M * F;
            GemvArgs ao{}, ag{}, ad{};
            ao.W = m->o[l]->data; ao.N = D; ao.K = D; ao.M = M;
            ao.xs = D;
            ao.S = e->S; ao.s_stride = e->s_stride; ao.Up = e->Wp; ao.cstride = e->cstride; ao.g = g;
            ao.ncap = e->cstride - 1;
            ao.e.pd = pd; ao.e.hd = hd; ao.e.D = D;
            ao.e.y = e->x; ao.e.y_stride = D; ao.e.ll = lx;
            ao.nx = prefetch_of(e, l + 1 < d.n_layers ? m->qkv[l + 1] : nullptr, e->l2_blocks ? D / 32 : 0u);
            ao.lli = li;
            ao.lli.ll = lmg;
            ag.W = m->gu[l]->data; ag.N = m->gu[l]->rows; ag.K = D; ag.M = M;
            ag.xs = D; ag.nw = fn;
            ag.e.y_stride = F; ag.e.ll = lsg;
            if (M > 1) {   // rows and maxima for the separate down launch
                ag.e.y = e->sg;
                ag.e.pmax = e->pmax;
                ao.e.y2 = e->x;   // and the residual rows after O, which it adds to
                // the O workgroups then load that launch's weights into L2
                ao.nx = prefetch_of(e, m->down[l], e->l2_blocks ? D / 32 : 0u);
            }
            ag.lli = li;
            ag.lli.ll = lx;
            ad.W = m->down[l]->data; ad.N = D; ad.K = F; ad.M = M;
            ad.xs = F;
            ad.e.y = e->x; ad.e.y_stride = D; ad.e.llold = lx;
            if (l + 1 == d.n_layers && hidden) ad.e.y2 = hidden;
            ad.lli = li;
            ad.lli.ll = lsg;
            hipEvent_t ev0 = nullptr, ev1 = nullptr;
            if (e->profile == 1 && e->in_verify && !e->capturing) {
                if (e->kev_used == e->kev.size()) {
                    TimedPass n{};
                    PF_HIP(c, hipEventCreate(&n.a));
                    PF_HIP(c, hipEventCreate(&n.b));
                    e->kev.push_back(n);
                    e->kev_bytes.push_back(0.0);
                }
                // the three matrices, their fp32 input rows and outputs
                double b = 0.0;
                for (const pf_matrix* W : {m->o[l], m->gu[l], m->down[l]})
                    if (M == 1 || W != m->down[l]) b += (double)W->bytes + 4.0 * M * W->cols + 4.0 * M * W->rows;
                e->kev_bytes[e->kev_used] = b;
                ev0 = e->kev[e->kev_used].a;
                ev1 = e->kev[e->kev_used].b;
                e->kev_used++;
            }
            launch_o_ffn(st, ao, ag, ad, ev0, ev1);
            if (M == 1) continue;
        } else {
            // O projection + residual (src/engine.cpp:789-800)
            a = GemvArgs{};
            a.a8 = e->act; a.a8s = as1; a.xs = ks;
            a.e.y = e->x; a.e.y_stride = D;
            a.nx = prefetch_of(e, m->gu[l], e->l2_blocks);
            if (merge_in_o) {
                a.S = e->S; a.s_stride = e->s_stride; a.Up = e->Wp; a.cstride = e->cstride; a.g = g;
                a.ncap = merge_ncap(e);
                a.e.pd = pd; a.e.hd = hd; a.e.D = D;
            }
            if (pf_status s = pass_mm(e, m->o[l], merge_in_o ? MM_O_MERGE : MM_O, M, a, as1)) return s;
            // FFN (src/engine.cpp:526-541, 805-854); with layer skip on, the
            // normed rows are staged for the skip decisions and the products run
            // only if some row needs them (gate word)
            a = GemvArgs{};
            a.e.y = e->sg; a.e.y_stride = F;
            a.e.pmax = tall ? nullptr : e->pmax;
            a.nx = prefetch_of(e, m->down[l], e->l2_blocks);
            if (e->skip_on) {
                float* nout = e->skip_stage + (size_t)l * e->rows * D;
                PF_PER1024_SWITCH(D, hipLaunchKernelGGL(k_norm_rows<PER>, dim3(M), dim3(1024), 0, st,
                                                        (const float*)e->x, D, fn, nout, e->skip_nrun + l));
                hipLaunchKernelGGL(k_layer_skip, dim3(e->nseq), dim3(1024), 0, st, (const PassDesc*)pd, M,
                                   (const float*)nout, (const float*)e->skip_cache + (size_t)l * D,
                                   (size_t)d.n_layers * D, D, skip_threshold(e, l), e->skip_flags + (size_t)l * e->rows,
                                   e->skip_nrun + l);
                a.x = nout; a.xs = D; a.gate = e->skip_nrun + l;
                if (tall)
                    PF_PER1024_SWITCH(D, hipLaunchKernelGGL(k_quant_rows_wide<PER>, dim3(M), dim3(1024), 0, st,
                                                            (const float*)nout, D, e->act, ks, as2,
                                                            (int32_t*)nullptr, 0u));
                if (pf_status s = pass_mm(e, m->gu[l], MM_GU_SKIP, M, a, as2)) return s;
            } else {
                a.x = e->x; a.xs = D; a.nw = fn;
                if (tall)
                    PF_PER1024_SWITCH(D, hipLaunchKernelGGL(k_norm_quant<PER>, dim3(M), dim3(1024), 0, st,
                                                            (const float*)e->x, D, fn, e->act, ks, as2));
                if (pf_status s = pass_mm(e, m->gu[l], MM_GU, M, a, as2)) return s;
            }
        }
        // down + residual; rows whose FFN was skipped take no residual
        a = GemvArgs{};
        a.x = e->sg; a.xs = F; a.pin = e->pmax; a.np = 2 * F / 32;
        a.e.y = e->x; a.e.y_stride = D;
        a.nx = prefetch_of(e, l + 1 < d.n_layers ? m->qkv[l + 1] : nullptr, e->l2_blocks);
        // the last down product also writes the pass's hidden output (a
        // gated launch may write nothing, so layer skip keeps the copy)
        if (l + 1 == d.n_layers && hidden && !e->skip_on) a.e.y2 = hidden;
        if (e->skip_on) {
            a.gate = e->skip_nrun + l;
            a.e.skipm = e->skip_flags + (size_t)l * e->rows;
        }
        if (tall)
            PF_PER1024_SWITCH(F, hipLaunchKernelGGL(k_quant_rows_wide<PER>, dim3(M), dim3(1024), 0, st,
                                                    (const float*)e->sg, F, e->act, ks, as3, (int32_t*)nullptr, 0u));
        if (pf_status s = pass_mm(e, m->down[l], e->skip_on ? MM_DOWN_SKIP : MM_DOWN, M, a, as3)) return s;
    }
    // every row of a pass counts for the skip caches except in verify passes,
    // whose caller commits the rows the acceptance keeps
    if (e->skip_on && !e->in_verify) launch_skip_commit(e, pd, M, 0, 0xFFFFFFFFu, false);
    if (hidden && (e->skip_on || d.n_layers == 0))
        hipLaunchKernelGGL(k_copy_f32, dim3((M * D + 255) / 256), dim3(256), 0, st, (const float*)e->x, hidden, M * D);
    if (logits) launch_gemv_f32(st, m->emb, M, e->x, D, logits, d.n_vocab, nullptr);
    PF_LAUNCHED(c);
    if (!e->capturing) e->hidden_valid = true;   // capture must not change host state
    return PF_OK;
}

extern "C" pf_status pf_forward(pf_engine* e, const int32_t* tokens, uint32_t n, float* logits, float* hidden) {
    if (!e || !tokens || n == 0) return PF_ERR_ARG;
    if (e->nseq != 1) return fail(e->c, PF_ERR_STATE, "multi-sequence engine: use pf_batch_forward");
    if (n > ((logits || hidden) ? MAX_PASS_ROWS : e->prefill_rows))
        return fail(e->c, PF_ERR_ARG, "pass too tall: 8 rows with outputs, else one window up to 256 rows");
    if (e->pos + n > e->rope_pos) return fail(e->c, PF_ERR_CAPACITY, "position beyond the engine's max_context");
    pf_ctx* c = e->c;
    const pf_model_desc& d = e->m->d;
    PassDesc pd{};
    pd.pos0 = e->pos;
    pd.m = n;
    for (uint32_t i = 0; i < n; i++) {
        if (tokens[i] < 0 || (uint32_t)tokens[i] >= d.n_vocab) return fail(c, PF_ERR_ARG, "token id out of range");
        pd.tok[i] = tokens[i];
    }
    PF_HIP(c, hipMemcpyAsync(e->pdP, &pd, sizeof(pd), hipMemcpyHostToDevice, c->stream));
    pf_status s = run_pass(e, e->pdP, n, e->pos, logits ? e->logitsA : nullptr, hidden ? e->hiddenA : nullptr);
    if (s) return s;
    e->pos += n;
    if (logits)
        PF_HIP(c, hipMemcpyAsync(logits, e->logitsA, (size_t)n * d.n_vocab * 4, hipMemcpyDeviceToHost, c->stream));
    if (hidden) PF_HIP(c, hipMemcpyAsync(hidden, e->hiddenA, (size_t)n * d.n_embd * 4, hipMemcpyDeviceToHost, c->stream));
    PF_HIP(c, hipStreamSynchronize(c->stream));
    return ll_check(e);
}

// MTPHeads::forward chain on the device hidden state h0 (src/mtp.cpp:63-127):
// gate, up, silu(gate) * up, down + residual per head, head k's state in row
// k of mcur (head 0 reads h0 itself, head k > 0 row k - 1), then the tied
// unembedding of all the heads' rows in one product (each row's logits are
// those of its own product), the logits of head k in row k of mlogits.
// waves: at most this many waves per launch (few when the chain runs beside
// a verify pass, whose launch it should leave the CUs to)
static pf_status mtp_chain(pf_engine* e, const float* h0, hipStream_t st, uint32_t waves = 4096) {
    pf_ctx* c = e->c;
    const pf_model* m = e->m;
    const pf_model_desc& d = m->d;
    const uint32_t D = d.n_embd, V = d.n_vocab;
    for (uint32_t k = 0; k < d.n_mtp; k++) {
        const float* hin = k == 0 ? h0 : e->mcur + (size_t)(k - 1) * D;
        launch_gemv_f32_glu(st, m->mtp[k * 3 + 0], m->mtp[k * 3 + 1], 1, hin, D, e->ma, D, std::min(waves, 2048u));
        launch_gemv_f32(st, m->mtp[k * 3 + 2], 1, e->ma, D, e->mcur + (size_t)k * D, D, hin, waves);
    }
    if (d.n_mtp) launch_gemv_f32(st, m->emb, d.n_mtp, e->mcur, D, e->mlogits, V, nullptr, waves);
    PF_LAUNCHED(c);
    return PF_OK;
}

extern "C" pf_status pf_mtp_forward(pf_engine* e, const float* hidden, float* logits) {
    if (!e || !hidden || !logits) return PF_ERR_ARG;
    pf_ctx* c = e->c;
    const pf_model_desc& d = e->m->d;
    PF_HIP(c, hipMemcpyAsync(e->hiddenA, hidden, d.n_embd * 4, hipMemcpyHostToDevice, c->stream));
    pf_status s = mtp_chain(e, e->hiddenA, c->stream);
    if (s) return s;
    PF_HIP(c, hipMemcpyAsync(logits, e->mlogits, (size_t)d.n_mtp * d.n_vocab * 4, hipMemcpyDeviceToHost, c->stream));
    PF_HIP(c, hipStreamSynchronize(c->stream));
    return PF_OK;
}

static SamplingCfg to_cfg(const pf_sampling* s) {
    SamplingCfg c{0.8f, 0.95f, 40u, 0};   // SamplingConfig defaults, include/forge/types.hpp:36-41
    if (s) { c.temperature = s->temperature; c.top_p = s->top_p; c.top_k = s->top_k; c.greedy = s->greedy; }
    return c;
}

// Engine::step_mtp (src/engine.cpp:402-448) on the device: the head chain,
// the drafts (k_step_drafts writes them into the pass descriptor), one pass
// of n_mtp rows, and the greedy check (k_step_accept); 4 bytes and the draw
// counter come back, and the rejecting row's logits when a draft fails.
extern "C" pf_status pf_step_mtp(pf_engine* e, int32_t current_token, const float* hidden, const pf_sampling* cfg,
                                 uint64_t seed, uint64_t* draw_index, int32_t* accepted_out, int32_t* acc_out,
                                 int32_t* rej_out, float* logits_out, int32_t* has_logits) {
    if (!e || !hidden || !accepted_out || !acc_out || !rej_out || !has_logits) return PF_ERR_ARG;
    pf_ctx* c = e->c;
    const pf_model_desc& d = e->m->d;
    const uint32_t NH = d.n_mtp, V = d.n_vocab;
    if (NH == 0 || NH > MAX_PASS_ROWS) return fail(c, PF_ERR_STATE, "step_mtp needs MTP heads (at most 8)");
    if (e->nseq != 1) return fail(c, PF_ERR_STATE, "multi-sequence engine: step_mtp serves one sequence");
    if (current_token < 0 || (uint32_t)current_token >= V) return fail(c, PF_ERR_ARG, "token id out of range");
    if (e->pos + NH > e->rope_pos) return fail(c, PF_ERR_CAPACITY, "position beyond the engine's max_context");
    hipStream_t st = c->stream;
    DecodeState ds{};
    ds.draw = draw_index ? *draw_index : 0;
    PassDesc pd{};
    pd.pos0 = e->pos;
    pd.m = NH;
    pd.tok[0] = current_token;
    PF_HIP(c, hipMemcpyAsync(e->st, &ds, sizeof(ds), hipMemcpyHostToDevice, st));
    PF_HIP(c, hipMemcpyAsync(e->pdP, &pd, sizeof(pd), hipMemcpyHostToDevice, st));
    PF_HIP(c, hipMemcpyAsync(e->hiddenA, hidden, (size_t)d.n_embd * 4, hipMemcpyHostToDevice, st));
    if (pf_status s = mtp_chain(e, e->hiddenA, st)) return s;
    hipLaunchKernelGGL(k_step_drafts, dim3(NH), dim3(1024), 0, st, (const float*)e->mlogits, V, to_cfg(cfg), seed,
                       e->st, e->pdP);
    if (pf_status s = run_pass(e, e->pdP, NH, e->pos, e->logitsB, nullptr)) return s;
    hipLaunchKernelGGL(k_step_accept, dim3(NH), dim3(1024), 0, st, (const float*)e->logitsB, V, e->st);
    PF_LAUNCHED(c);
    PF_HIP(c, hipMemcpyAsync(&ds, e->st, sizeof(ds), hipMemcpyDeviceToHost, st));
    PF_HIP(c, hipStreamSynchronize(st));
    if (pf_status s = ll_check(e)) return s;
    const uint32_t a = ds.round_word;
    *accepted_out = (int32_t)a;
    if (draw_index) *draw_index = ds.draw;
    if (a < NH) {   // rows 0 .. a were forwarded; row a rejected draft a
        e->pos += a + 1;
        *acc_out = 0;
        *rej_out = (int32_t)(NH - a);
        *has_logits = 1;
        if (logits_out)
            PF_HIP(c, hipMemcpy(logits_out, e->logitsB + (size_t)a * V, (size_t)V * 4, hipMemcpyDeviceToHost));
    } else {
        e->pos += NH;
        *acc_out = (int32_t)a;
        *rej_out = 0;
        *has_logits = 0;
    }
    e->hidden_valid = false;
    return PF_OK;
}

extern "C" pf_status pf_sample(pf_engine* e, const float* logits, const pf_sampling* cfg, uint64_t seed,
                               uint64_t* draw_index, int32_t* token) {
    if (!e || !logits || !token) return PF_ERR_ARG;
    pf_ctx* c = e->c;
    const uint32_t V = e->m->d.n_vocab;
    DecodeState st{};
    st.draw = draw_index ? *draw_index : 0;
    PF_HIP(c, hipMemcpyAsync(e->st, &st, sizeof(st), hipMemcpyHostToDevice, c->stream));
    PF_HIP(c, hipMemcpyAsync(e->logitsA, logits, (size_t)V * 4, hipMemcpyHostToDevice, c->stream));
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(1024), 0, c->stream, e->logitsA, V, 0, V, to_cfg(cfg), seed, e->st,
                       (int32_t*)nullptr, 0u, (int32_t)ROLE_PLAIN, (int32_t*)&e->st->round_word);
    PF_LAUNCHED(c);
    PF_HIP(c, hipMemcpyAsync(&st, e->st, sizeof(st), hipMemcpyDeviceToHost, c->stream));
    PF_HIP(c, hipStreamSynchronize(c->stream));
    *token = (int32_t)st.round_word;
    if (draw_index) *draw_index = st.draw;
    return PF_OK;
}

// One decode round, all on the engine's stream (capturable): the base pass
// (or reuse of the last verify row), then either the MTP round
// (src/engine.cpp:308-365: T1, drafts, the first verify segment of h rows,
// acceptance, corrective) or the single-token step (src/engine.cpp:377-386).
// Verify row j sits at row j of logitsB / hiddenB in every segment.
static pf_status round_body(pf_engine* e, bool reuse, bool mtp, const SamplingCfg& cfg, uint64_t seed,
                            uint32_t h) {
    const bool greedy = cfg.greedy || cfg.temperature <= 0.0f;   // Engine::sample's greedy branch
    pf_ctx* c = e->c;
    hipStream_t st = c->stream;
    const pf_model_desc& d = e->m->d;
    const uint32_t V = d.n_vocab, D = d.n_embd, NM = d.n_mtp;
    pf_status s;
    TimedPass* tp = nullptr;
    const float* base_logits;
    const float* base_hidden;
    if (reuse) {
        hipLaunchKernelGGL(k_ctl_reuse_row, dim3(1), dim3(1), 0, st, e->st);
        // the reused row (F(cur), the last verify row) is this round's base pass
        if (e->skip_on) launch_skip_commit(e, e->pdB, NM + 1, NM, NM + 1, false);
        base_logits = e->logitsB + (size_t)NM * V;
        base_hidden = e->hiddenB + (size_t)NM * D;
    } else {
        hipLaunchKernelGGL(k_ctl_pass_a, dim3(1), dim3(1), 0, st, e->st, e->pdA);
        if ((s = timed_begin(e, false, &tp))) return s;
        if ((s = run_pass(e, e->pdA, 1, e->pos, e->logitsA, e->hiddenA))) return s;
        if (tp) PF_HIP(c, hipEventRecord(tp->b, st));
        base_logits = e->logitsA;
        base_hidden = e->hiddenA;
    }
    if (mtp) {
        // the heads run from the base row's hidden state; T1 and the drafts
        // are sampled together, one block each.  A one-row verify segment
        // needs only T1: T1 is sampled first, and the heads and the drafts
        // run on the second stream beside the verify pass, joined before the
        // acceptance (the same draws either way)
        const bool ovl = e->mtp_overlap && h == 1 && !e->skip_on;
        if (ovl) {
            hipLaunchKernelGGL(k_sample_round, dim3(1), dim3(1024), 0, st, base_logits, (const float*)e->mlogits, V,
                               cfg, seed, e->st, e->tokens, e->tok_cap, e->pdB, (int32_t)h, 0u, 0);
            PF_HIP(c, hipEventRecord(e->evf, st));
            PF_HIP(c, hipStreamWaitEvent(e->st2, e->evf, 0));
            if ((s = mtp_chain(e, base_hidden, e->st2, e->mtp_side_waves))) return s;
            hipLaunchKernelGGL(k_sample_round, dim3(NM), dim3(1024), 0, e->st2, base_logits,
                               (const float*)e->mlogits, V, cfg, seed, e->st, e->tokens, e->tok_cap, e->pdB,
                               (int32_t)h, 1u, 1);
            PF_HIP(c, hipEventRecord(e->evj, e->st2));
        } else {
            if ((s = mtp_chain(e, base_hidden, st))) return s;
            hipLaunchKernelGGL(k_sample_round, dim3(1 + NM), dim3(1024), 0, st, base_logits,
                               (const float*)e->mlogits, V, cfg, seed, e->st, e->tokens, e->tok_cap, e->pdB,
                               (int32_t)h, 0u, 1);
        }
        if ((s = timed_begin(e, true, &tp))) return s;
        e->in_verify = true;
        s = run_pass(e, e->pdB, h, e->pos + 1, e->logitsB, e->hiddenB);
        e->in_verify = false;
        if (s) return s;
        if (tp) PF_HIP(c, hipEventRecord(tp->b, st));
        if (ovl) PF_HIP(c, hipStreamWaitEvent(st, e->evj, 0));
        hipLaunchKernelGGL(k_verify_accept, dim3(h), dim3(1024), 0, st, (const float*)e->logitsB, V, V, e->st,
                           (const PassDesc*)e->pdB, e->tokens, e->tok_cap, greedy ? 1 : 0);
        if (e->skip_on) launch_skip_commit(e, e->pdB, NM + 1, 0, 0, true);
        if (!greedy)
            hipLaunchKernelGGL(k_sample, dim3(1), dim3(1024), 0, st, e->logitsB, V, -1, V, cfg, seed, e->st,
                               e->tokens, e->tok_cap, (int32_t)ROLE_CORRECTIVE, (int32_t*)nullptr);
        hipLaunchKernelGGL(k_word_out, dim3(1), dim3(64), 0, st, (const DecodeState*)e->st, e->word_dev);
    } else {
        hipLaunchKernelGGL(k_sample, dim3(1), dim3(1024), 0, st, base_logits, V, 0, V, cfg, seed, e->st, e->tokens,
                           e->tok_cap, (int32_t)ROLE_FALLBACK, (int32_t*)nullptr);
    }
    PF_LAUNCHED(c);
    return PF_OK;
}

// The verify segment that continues a round whose first segment (one row)
// accepted its draft: rows 1 .. n_mtp (inputs d0 .. d{n-1}) at verify rows
// 1 .. n_mtp of logitsB, acceptance and corrective.
static pf_status segment_body(pf_engine* e, const SamplingCfg& cfg, uint64_t seed) {
    pf_ctx* c = e->c;
    hipStream_t st = c->stream;
    const pf_model_desc& d = e->m->d;
    const uint32_t V = d.n_vocab, D = d.n_embd, NM = d.n_mtp;
    pf_status s;
    TimedPass* tp = nullptr;
    hipLaunchKernelGGL(k_ctl_segment, dim3(1), dim3(1), 0, st, e->st, e->pdB);
    if ((s = timed_begin(e, true, &tp))) return s;
    e->in_verify = true;
    s = run_pass(e, e->pdB, NM, e->pos, e->logitsB + V, e->hiddenB + D);
    e->in_verify = false;
    if (s) return s;
    if (tp) PF_HIP(c, hipEventRecord(tp->b, st));
    const bool greedy = cfg.greedy || cfg.temperature <= 0.0f;   // Engine::sample's greedy branch
    hipLaunchKernelGGL(k_verify_accept, dim3(NM), dim3(1024), 0, st, (const float*)(e->logitsB + V), V, V, e->st,
                       (const PassDesc*)e->pdB, e->tokens, e->tok_cap, greedy ? 1 : 0);
    if (!greedy)
        hipLaunchKernelGGL(k_sample, dim3(1), dim3(1024), 0, st, e->logitsB, V, -1, V, cfg, seed, e->st, e->tokens,
                           e->tok_cap, (int32_t)ROLE_CORRECTIVE, (int32_t*)nullptr);
    hipLaunchKernelGGL(k_word_out, dim3(1), dim3(64), 0, st, (const DecodeState*)e->st, e->word_dev);
    PF_LAUNCHED(c);
    return PF_OK;
}

// Captures the round variants (reuse x MTP x first-segment height) and the
// continuation segment as graphs for this sampling configuration and seed
// (kernel arguments are baked into the graphs; the positions and tokens
// live in device memory).
static pf_status capture(pf_engine* e, hipGraphExec_t* out, int which, bool reuse, bool mtp, uint32_t h,
                         const SamplingCfg& cfg, uint64_t seed) {
    pf_ctx* c = e->c;
    hipGraph_t graph = nullptr;
    PF_HIP(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    e->capturing = true;
    pf_status s = which == 0 ? round_body(e, reuse, mtp, cfg, seed, h) : segment_body(e, cfg, seed);
    e->capturing = false;
    hipError_t ee = hipStreamEndCapture(c->stream, &graph);
    if (s) { if (graph) (void)hipGraphDestroy(graph); return s; }
    if (ee != hipSuccess) return fail(c, PF_ERR_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(ee));
    ee = hipGraphInstantiate(out, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ee != hipSuccess) return fail(c, PF_ERR_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(ee));
    return PF_OK;
}

static pf_status ensure_round_graphs(pf_engine* e, const SamplingCfg& cfg, uint64_t seed) {
    if (e->graphs_valid && e->graph_seed == seed && e->graph_profile == e->profile &&
        std::memcmp(&e->graph_cfg, &cfg, sizeof(cfg)) == 0)
        return PF_OK;
    for (auto& row : e->round_exec)
        for (auto& col : row)
            for (auto& g : col)
                if (g) { (void)hipGraphExecDestroy(g); g = nullptr; }
    if (e->cont_exec) { (void)hipGraphExecDestroy(e->cont_exec); e->cont_exec = nullptr; }
    e->graphs_valid = false;
    e->timed_used = 0;
    e->kev_used = 0;
    const uint32_t NM = e->m->d.n_mtp;
    for (int reuse = 0; reuse < 2; reuse++)
        for (int mtp = 0; mtp < 2; mtp++)
            for (int full = 0; full < (mtp ? 2 : 1); full++)
                if (pf_status s = capture(e, &e->round_exec[reuse][mtp][full], 0, reuse != 0, mtp != 0,
                                          full ? NM + 1 : 1u, cfg, seed))
                    return s;
    if (NM > 1)
        if (pf_status s = capture(e, &e->cont_exec, 1, false, true, NM, cfg, seed)) return s;
    e->graph_cfg = cfg;
    e->graph_seed = seed;
    e->graph_profile = e->profile;
    e->graphs_valid = true;
    return PF_OK;
}

// Token buffers of every sequence with `cap` entries each (tokens + s * cap).
static pf_status ensure_tokens(pf_engine* e, uint32_t cap) {
    if (e->tokens) dfree(e->c, e->tokens, e->tok_alloc * 4);
    e->tokens = nullptr;
    e->tok_cap = 0;
    e->tok_alloc = 0;
    const size_t n = (size_t)e->nseq * cap;
    if (pf_status s = dalloc_t(e->c, &e->tokens, n)) return s;
    e->tok_cap = cap;
    e->tok_alloc = n;
    e->graphs_valid = false;   // the captured rounds hold the old buffer
    return PF_OK;
}

// Engine::generate, src/engine.cpp:276-396.  Prompt prefilled in passes
// of up to 8 tokens; then MTP rounds (src/engine.cpp:304-373) as one base
// pass (skipped when the previous round accepted every draft: its last
// verify row already is F(cur)), the draft chain, one verify pass over
// [T1, drafts], acceptance and the corrective on the device; the host reads
// one word per round.
extern "C" pf_status pf_generate(pf_engine* e, const int32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                                 const pf_sampling* scfg, uint64_t seed, int32_t* tokens_out, uint32_t tokens_cap,
                                 pf_gen_result* res) {
    if (!e || (!prompt && n_prompt) || !tokens_out || !res) return PF_ERR_ARG;
    if (e->nseq != 1) return fail(e->c, PF_ERR_STATE, "multi-sequence engine: use pf_batch_generate");
    pf_ctx* c = e->c;
    const pf_model_desc& d = e->m->d;
    hipStream_t st = c->stream;
    const uint32_t V = d.n_vocab, D = d.n_embd, NM = d.n_mtp;
    std::memset(res, 0, sizeof(*res));
    if ((uint64_t)n_prompt + max_new + 1 > tokens_cap) return fail(c, PF_ERR_CAPACITY, "tokens_cap < prompt + max_new + 1");
    if ((uint64_t)e->pos + n_prompt + max_new + MAX_PASS_ROWS > e->rope_pos)
        return fail(c, PF_ERR_CAPACITY, "prompt + max_new_tokens exceed the engine's max_context");
    for (uint32_t i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || (uint32_t)prompt[i] >= V) return fail(c, PF_ERR_ARG, "prompt token id out of range");
    const SamplingCfg cfg = to_cfg(scfg);
    if (e->tok_cap < tokens_cap) {
        if (pf_status s = ensure_tokens(e, tokens_cap)) return s;
    }
    if (n_prompt) PF_HIP(c, hipMemcpyAsync(e->tokens, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice, st));
    auto t0 = std::chrono::steady_clock::now();
    // prefill (src/engine.cpp:286-290): every prompt token forwarded in order,
    // in passes of up to one window (256 rows), whose GEMMs run on MFMA
    for (uint32_t i = 0; i < n_prompt; i += e->prefill_rows) {
        const uint32_t n = std::min(e->prefill_rows, n_prompt - i);
        e->pd_host.pos0 = e->pos;
        e->pd_host.m = n;
        for (uint32_t r = 0; r < n; r++) e->pd_host.tok[r] = prompt[i + r];
        PF_HIP(c, hipMemcpyAsync(e->pdP, &e->pd_host, sizeof(PassDesc), hipMemcpyHostToDevice, st));
        // the copy reads e->pd_host before the host overwrites it for the next pass
        PF_HIP(c, hipStreamSynchronize(st));
        pf_status s = run_pass(e, e->pdP, n, e->pos, nullptr, nullptr);
        if (s) return s;
        e->pos += n;
    }
    DecodeState s0{};
    s0.pos = e->pos;
    s0.cur = n_prompt ? prompt[n_prompt - 1] : 0;
    s0.n_tokens = n_prompt;
    s0.n_mtp = NM;
    PF_HIP(c, hipMemcpyAsync(e->st, &s0, sizeof(s0), hipMemcpyHostToDevice, st));
    PF_HIP(c, hipStreamSynchronize(st));
    auto t1 = std::chrono::steady_clock::now();

    e->verify_us = e->base_us = 0;
    e->verify_n = e->base_n = 0;
    e->kev_us = e->kev_bytes_sum = 0;
    e->kev_n = 0;
    e->kev_by_size.clear();
    e->aev_us = 0;
    e->aev_n = 0;
    e->aev_used = 0;
    e->round_us = 0;
    e->round_n = 0;
    const bool graphs = e->use_graphs && !e->profile;   // profiling times dispatches one by one
    if (graphs) {
        pf_status s = ensure_round_graphs(e, cfg, seed);
        if (s) return s;
    }
    uint32_t n_gen = 0;
    bool have_row = false;
    uint32_t last_acc = 0;   // drafts the previous MTP round accepted
    // MTP rounds that followed a round with no accepted draft, and those of
    // them that accepted d0 (observed under either segment height)
    uint32_t z_rounds = 0, z_d0 = 0;
    // One segment (a graph or, in profiling mode, its kernels one by one)
    // timed with the round events and its dispatch events harvested.
    auto segment = [&](hipGraphExec_t g, bool cont, bool reuse, bool mtp, uint32_t h) -> pf_status {
        size_t ev[4] = {0, 0, 0, 0};
        if (e->round_timing) PF_HIP(c, hipEventRecord(e->rev0, st));
        if (graphs) {
            PF_HIP(c, hipGraphLaunch(g, st));
        } else {
            e->timed_used = 0;
            e->kev_used = 0;
            pf_status s = cont ? segment_body(e, cfg, seed) : round_body(e, reuse, mtp, cfg, seed, h);
            if (s) return s;
            ev[1] = e->timed_used;
            ev[3] = e->kev_used;
        }
        if (e->round_timing) PF_HIP(c, hipEventRecord(e->rev1, st));
        PF_HIP(c, hipStreamSynchronize(st));
        if (pf_status s = harvest_events(e, ev[0], ev[1], ev[2], ev[3])) return s;
        if (mtp && e->round_timing) {
            float rms = 0;
            PF_HIP(c, hipEventElapsedTime(&rms, e->rev0, e->rev1));
            e->round_us += rms * 1000.0;
        }
        return PF_OK;
    };
    while (n_gen < max_new) {
        if (e->max_memory && c->bytes > e->max_memory) {   // src/engine.cpp:297-301
            res->oom_protected = 1;
            break;
        }
        const bool mtp_round = e->mtp_enabled && NM > 0 && e->hidden_valid && n_gen + 4 <= max_new;   // src/engine.cpp:304-305
        if (e->pos + NM + 2 > e->rope_pos)
            return fail(c, PF_ERR_CAPACITY, "position beyond the engine's max_context");
        // first verify segment: every row after a round that accepted a draft
        // (or when asked for); one row, the reference's first verify forward,
        // after a round whose first draft was rejected, unless d0 was accepted
        // in more than 3 of 10 such rounds so far.  A one-row segment saves the
        // other rows' work only when d0 is rejected (accepted, it needs a second
        // segment), and a one-row pass costs about 0.7 of a five-row pass.
        const bool d0_likely = z_rounds >= 2 && 10u * z_d0 > 3u * z_rounds;
        const bool full = e->verify_full || e->skip_on || last_acc > 0 || NM < 2 || d0_likely;
        const uint32_t h = full ? NM + 1 : 1u;
        if (pf_status s = segment(graphs ? e->round_exec[have_row][mtp_round][mtp_round && full] : nullptr, false,
                                  have_row, mtp_round, h))
            return s;
        e->hidden_valid = true;
        res->passes += (have_row ? 0 : 1) + (mtp_round ? 1 : 0);
        e->pos += 1;   // the base position (pass A, or the reused verify row)
        if (mtp_round) {
            uint32_t w = e->word[0], a = w & 0xFFu, pushed = (w >> 8) & 1u, more = (w >> 9) & 1u;
            uint32_t k0 = 0, m = h;
            if (more) {   // the one-row segment accepted d0: rows for d1 .. d{n-1} and F(d{n-1})
                if (a != 1 || h != 1) return fail(c, PF_ERR_STATE, "verify continuation from an unexpected draft");
                e->pos += m;
                if (pf_status s = segment(e->cont_exec, true, false, true, NM)) return s;
                res->passes += 1;
                res->continued += 1;
                w = e->word[0];
                a = w & 0xFFu;
                pushed = (w >> 8) & 1u;
                if ((w >> 9) & 1u) return fail(c, PF_ERR_STATE, "verify segment left drafts unchecked");
                k0 = 1;
                m = NM;
            }
            e->round_n++;
            n_gen += 1 + a + pushed;
            res->rounds++;
            const uint32_t r = a - k0;   // rows of the last segment whose drafts were accepted
            if (a < NM) {
                e->pos += r + 1;
                have_row = false;
            } else if (r < m) {
                e->pos += r;
                have_row = true;         // that segment's last row holds F(cur)
            } else {
                e->pos += m;
                have_row = false;
            }
            if (last_acc == 0) {
                z_rounds++;
                z_d0 += a > 0 ? 1u : 0u;
            }
            last_acc = a;
        } else {
            n_gen += 1;
            have_row = false;
        }
    }
    DecodeState sf{};
    PF_HIP(c, hipMemcpyAsync(&sf, e->st, sizeof(sf), hipMemcpyDeviceToHost, st));
    PF_HIP(c, hipStreamSynchronize(st));
    auto t2 = std::chrono::steady_clock::now();
    if (pf_status s = ll_check(e)) return s;
    if (sf.pos != e->pos) return fail(c, PF_ERR_STATE, "device and host positions diverged");
    const uint32_t nt = std::min(sf.n_tokens, tokens_cap);
    PF_HIP(c, hipMemcpy(tokens_out, e->tokens, (size_t)nt * 4, hipMemcpyDeviceToHost));
    res->n_tokens = nt;
    res->mtp_accepted = (int32_t)sf.accepted;
    res->mtp_rejected = (int32_t)sf.rejected;
    res->prefill_seconds = std::chrono::duration<double>(t1 - t0).count();
    res->decode_seconds = std::chrono::duration<double>(t2 - t1).count();
    return PF_OK;
}

extern "C" pf_status pf_engine_profile(pf_engine* e, int32_t enable) {
    if (!e) return PF_ERR_ARG;
    if (enable < 0 || enable > 2) return PF_ERR_ARG;
    e->profile = enable;
    return PF_OK;
}

extern "C" pf_status pf_engine_gemv_stats(pf_engine* e, uint32_t* launches, double* avg_us, double* avg_bytes) {
    if (!e) return PF_ERR_ARG;
    const double n = (double)e->kev_n;
    if (launches) *launches = e->kev_n;
    if (avg_us) *avg_us = n ? e->kev_us / n : 0.0;
    if (avg_bytes) *avg_bytes = n ? e->kev_bytes_sum / n : 0.0;
    return PF_OK;
}

extern "C" pf_status pf_engine_gemv_by_size(const pf_engine* e, uint32_t cap, double* bytes, uint32_t* launches,
                                             double* avg_us, uint32_t* n) {
    if (!e || !n || (cap && (!bytes || !launches || !avg_us))) return PF_ERR_ARG;
    uint32_t i = 0;
    for (const auto& kv : e->kev_by_size) {
        if (i < cap) {
            bytes[i] = kv.first;
            launches[i] = kv.second.second;
            avg_us[i] = kv.second.first / kv.second.second;
        }
        i++;
    }
    *n = i;
    return PF_OK;
}

extern "C" pf_status pf_engine_attn_stats(const pf_engine* e, uint32_t* launches, double* avg_us) {
    if (!e) return PF_ERR_ARG;
    if (launches) *launches = e->aev_n;
    if (avg_us) *avg_us = e->aev_n ? e->aev_us / e->aev_n : 0.0;
    return PF_OK;
}

extern "C" pf_status pf_engine_set_round_timing(pf_engine* e, int32_t on) {
    if (!e) return PF_ERR_ARG;
    e->round_timing = on != 0;
    return PF_OK;
}

extern "C" pf_status pf_engine_round_time(const pf_engine* e, double* round_us, uint32_t* rounds) {
    if (!e) return PF_ERR_ARG;
    if (round_us) *round_us = e->round_n ? e->round_us / e->round_n : 0.0;
    if (rounds) *rounds = e->round_n;
    return PF_OK;
}

extern "C" pf_status pf_engine_pass_times(const pf_engine* e, double* verify_us, double* base_us, uint32_t* vn,
                                          uint32_t* bn) {
    if (!e) return PF_ERR_ARG;
    if (verify_us) *verify_us = e->verify_n ? e->verify_us / e->verify_n : 0.0;
    if (base_us) *base_us = e->base_n ? e->base_us / e->base_n : 0.0;
    if (vn) *vn = e->verify_n;
    if (bn) *bn = e->base_n;
    return PF_OK;
}

#include "pf_batch.hip"
