// .squeeze files (include/forge/quant_format.hpp:13-48, src/quant_format.cpp)
// read on the host and uploaded in the device layout.
//
// File: a 256-byte header (magic "FORGE", version, block count, the model
// configuration, index offset and size), the zstd-compressed matrices, and at
// index_offset an array of WeightBlock records as the struct lies in memory
// (include/forge/types.hpp:205-214, not packed: six uint32 -- layer, matrix,
// rows, cols, compressed size, original size -- the quant type byte, three
// padding bytes and the uint32 data offset; 32 bytes), read field by field.
// A matrix is stored row-major and cut into blocks
// of 32 elements of the flattened array:
//   type 0 (Q8)   f32 inverse scale s = 127/amax, 32 bytes round(x s + 0.5)
//   type 1 (Q4)   f32 s = 7/amax, 16 bytes of nibbles (code + 8, low first)
//   type 2 (Q2)   f32 s = 1/amax, 8 bytes of 2-bit fields (code + 2, low first)
//   type 3 (Q1.5) 16 bytes of 2-bit fields in bits 0-1 and 2-3 of each byte
//                 (0 -> -1, 1 -> 0, 2 -> +1), no scale
// (src/quant_format.cpp:41-154).  An element's value is code / s (code for
// Q1.5); s = 0 marks an all-zero block.  The reference loader drops the
// scales of Q4 and Q2 blocks (src/quant_format.cpp:399-412); here they are
// parsed, and a layer matrix is repacked to the device's block layout with
// the multiplicative fp16 scale d = 1/s (1 for Q1.5).
//
// zstd is the system's libzstd.so.1, loaded on first use.
#include <dlfcn.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/pf_gpu.h"

namespace pf_host {
uint16_t half_rne(float f);
}

namespace {

std::string g_sq_error;

struct Block {
    uint32_t layer, matrix, rows, cols, csize, osize;
    uint8_t qtype;
    uint32_t offset;
};

constexpr size_t HEADER_BYTES = 256;
constexpr size_t RECORD_STRIDE = 32;   // sizeof(forge::WeightBlock) on LP64

typedef size_t (*zstd_decompress_t)(void*, size_t, const void*, size_t);
typedef unsigned (*zstd_iserror_t)(size_t);

struct Zstd {
    zstd_decompress_t decompress = nullptr;
    zstd_iserror_t is_error = nullptr;
    bool tried = false;
};

Zstd& zstd() {
    static Zstd z;
    if (!z.tried) {
        z.tried = true;
        void* h = dlopen("libzstd.so.1", RTLD_NOW | RTLD_LOCAL);
        if (h) {
            z.decompress = (zstd_decompress_t)dlsym(h, "ZSTD_decompress");
            z.is_error = (zstd_iserror_t)dlsym(h, "ZSTD_isError");
        }
    }
    return z;
}

uint32_t rd32(const uint8_t* p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}

uint64_t rd64(const uint8_t* p) {
    uint64_t v;
    std::memcpy(&v, p, 8);
    return v;
}

float rdf(const uint8_t* p) {
    float v;
    std::memcpy(&v, p, 4);
    return v;
}

}  // namespace

struct pf_squeeze {
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
    pf_squeeze_info info{};
    std::vector<Block> index;
    std::string err;
};

static pf_status sq_fail(pf_squeeze* s, pf_status code, const std::string& msg) {
    if (s) s->err = msg;
    g_sq_error = msg;
    return code;
}

extern "C" const char* pf_squeeze_last_error(const pf_squeeze* s) {
    return s ? s->err.c_str() : g_sq_error.c_str();
}

extern "C" void pf_squeeze_close(pf_squeeze* s) {
    if (!s) return;
    if (s->map) munmap((void*)s->map, s->size);
    if (s->fd >= 0) ::close(s->fd);
    delete s;
}

// WeightLoader::open (src/quant_format.cpp:231-283): map the file, check the
// magic, read the configuration and the block index.  Index records and
// block data are checked against the file size.
extern "C" pf_status pf_squeeze_open(const char* path, pf_squeeze** out) {
    if (!path || !out) return sq_fail(nullptr, PF_ERR_ARG, "null argument");
    *out = nullptr;
    pf_squeeze* s = new pf_squeeze();
    s->fd = ::open(path, O_RDONLY);
    if (s->fd < 0) {
        pf_squeeze_close(s);
        return sq_fail(nullptr, PF_ERR_ARG, std::string("cannot open ") + path);
    }
    struct stat st;
    if (fstat(s->fd, &st) < 0 || (size_t)st.st_size < HEADER_BYTES) {
        pf_squeeze_close(s);
        return sq_fail(nullptr, PF_ERR_FORMAT, "file shorter than the 256-byte header");
    }
    s->size = (size_t)st.st_size;
    void* m = mmap(nullptr, s->size, PROT_READ, MAP_SHARED, s->fd, 0);
    if (m == MAP_FAILED) {
        s->map = nullptr;
        pf_squeeze_close(s);
        return sq_fail(nullptr, PF_ERR_ARG, "mmap failed");
    }
    s->map = (const uint8_t*)m;
    const uint8_t* h = s->map;
    if (std::memcmp(h, "FORGE", 5) != 0) {
        pf_squeeze_close(s);
        return sq_fail(nullptr, PF_ERR_FORMAT, "bad magic (not a .squeeze file)");
    }
    pf_squeeze_info& I = s->info;
    I.version = rd32(h + 8);
    I.n_blocks = rd32(h + 12);
    I.n_layers = rd32(h + 16);
    I.n_embd = rd32(h + 20);
    I.n_heads = rd32(h + 24);
    I.n_kv_heads = rd32(h + 28);
    I.n_ff = rd32(h + 32);
    I.n_vocab = rd32(h + 36);
    I.max_seq_len = rd32(h + 40);
    I.mtp_heads = rd32(h + 44);
    const uint64_t ioff = rd64(h + 48);
    if (ioff > s->size || (uint64_t)I.n_blocks * RECORD_STRIDE > s->size - ioff) {
        pf_squeeze_close(s);
        return sq_fail(nullptr, PF_ERR_FORMAT, "block index outside the file");
    }
    s->index.resize(I.n_blocks);
    for (uint32_t i = 0; i < I.n_blocks; i++) {
        const uint8_t* r = s->map + ioff + (size_t)i * RECORD_STRIDE;
        Block& b = s->index[i];
        b.layer = rd32(r);
        b.matrix = rd32(r + 4);
        b.rows = rd32(r + 8);
        b.cols = rd32(r + 12);
        b.csize = rd32(r + 16);
        b.osize = rd32(r + 20);
        b.qtype = r[24];
        b.offset = rd32(r + 28);
        if ((uint64_t)b.offset + b.csize > s->size) {
            pf_squeeze_close(s);
            return sq_fail(nullptr, PF_ERR_FORMAT, "block data outside the file");
        }
    }
    *out = s;
    return PF_OK;
}

extern "C" pf_status pf_squeeze_get_info(const pf_squeeze* s, pf_squeeze_info* out) {
    if (!s || !out) return PF_ERR_ARG;
    *out = s->info;
    return PF_OK;
}

static const Block* find_block(const pf_squeeze* s, uint32_t layer, uint32_t matrix) {
    for (const Block& b : s->index)
        if (b.layer == layer && b.matrix == matrix) return &b;
    return nullptr;
}

extern "C" pf_status pf_squeeze_block_shape(const pf_squeeze* s, uint32_t layer, uint32_t matrix, uint32_t* rows,
                                            uint32_t* cols, uint32_t* quant_type) {
    if (!s || !rows || !cols || !quant_type) return PF_ERR_ARG;
    const Block* b = find_block(s, layer, matrix);
    if (!b) return PF_ERR_ARG;
    *rows = b->rows;
    *cols = b->cols;
    *quant_type = b->qtype;
    return PF_OK;
}

// WeightLoader::load_block_with_scales (src/quant_format.cpp:321-425) with
// the block scales parsed: codes [rows * cols] as signed integers, and per
// 32-element block of the flattened matrix the multiplier of its codes
// (1 / s, 0 for s = 0, 1 for Q1.5).
extern "C" pf_status pf_squeeze_load_block(pf_squeeze* s, uint32_t layer, uint32_t matrix, int8_t* codes,
                                           float* block_scales) {
    if (!s || !codes || !block_scales) return PF_ERR_ARG;
    const Block* b = find_block(s, layer, matrix);
    if (!b) return sq_fail(s, PF_ERR_ARG, "no block for this layer and matrix");
    const uint64_t n = (uint64_t)b->rows * b->cols;
    const uint64_t nb = (n + 31) / 32;
    static const uint32_t bytes_per_block[4] = {36, 20, 12, 16};
    if (b->qtype > 3) return sq_fail(s, PF_ERR_FORMAT, "unknown quant type");
    if ((uint64_t)b->osize != nb * bytes_per_block[b->qtype])
        return sq_fail(s, PF_ERR_FORMAT, "block size does not match its shape and quant type");
    Zstd& z = zstd();
    if (!z.decompress || !z.is_error) return sq_fail(s, PF_ERR_UNSUPPORTED, "libzstd.so.1 not available");
    std::vector<uint8_t> raw(b->osize);
    const size_t got = z.decompress(raw.data(), raw.size(), s->map + b->offset, b->csize);
    if (z.is_error(got) || got != raw.size()) return sq_fail(s, PF_ERR_FORMAT, "zstd decompression failed");
    const uint8_t* p = raw.data();
    for (uint64_t k = 0; k < nb; k++) {
        const uint64_t e0 = 32 * k, e1 = std::min<uint64_t>(e0 + 32, n);
        if (b->qtype == 3) {
            block_scales[k] = 1.0f;
            for (uint64_t i = e0; i < e1; i++) {
                const uint32_t j = (uint32_t)(i - e0);
                const int c = (p[j / 2] >> (2 * (j & 1))) & 3;
                codes[i] = (int8_t)(c == 0 ? -1 : (c == 1 ? 0 : (c == 2 ? 1 : 0)));
            }
            p += 16;
            continue;
        }
        const float inv = rdf(p);
        p += 4;
        block_scales[k] = inv == 0.0f ? 0.0f : 1.0f / inv;
        for (uint64_t i = e0; i < e1; i++) {
            const uint32_t j = (uint32_t)(i - e0);
            if (b->qtype == 0) codes[i] = (int8_t)p[j];
            else if (b->qtype == 1) codes[i] = (int8_t)((int)((p[j / 2] >> (4 * (j & 1))) & 15) - 8);
            else codes[i] = (int8_t)((int)((p[j / 4] >> (2 * (j & 3))) & 3) - 2);
        }
        p += bytes_per_block[b->qtype] - 4;
    }
    return PF_OK;
}

// Device interchange layout of one matrix from decoded codes and block
// multipliers: fmt PF_FMT_Q8 (quant type 0, codes kept as stored, the
// reference's round(x s + 0.5) rule included), PF_FMT_Q4 (1), PF_FMT_Q2 (2)
// or PF_FMT_Q15 (3); codes [rows][cols/32][32 | 16 | 8], fp16 scales
// [rows][cols/32].
static pf_status repack(pf_squeeze* s, uint32_t layer, uint32_t matrix, uint32_t want_rows, uint32_t want_cols,
                        int32_t* fmt, std::vector<uint8_t>& codes, std::vector<uint16_t>& scales) {
    uint32_t rows, cols, qt;
    if (pf_squeeze_block_shape(s, layer, matrix, &rows, &cols, &qt))
        return sq_fail(s, PF_ERR_STATE, "matrix " + std::to_string(matrix) + " of layer " + std::to_string(layer) +
                                            " is missing");
    if (rows != want_rows || cols != want_cols || cols % 32)
        return sq_fail(s, PF_ERR_FORMAT, "matrix " + std::to_string(matrix) + " of layer " + std::to_string(layer) +
                                             " has the wrong shape");
    std::vector<int8_t> c((size_t)rows * cols);
    std::vector<float> d((size_t)rows * cols / 32);
    if (pf_status st = pf_squeeze_load_block(s, layer, matrix, c.data(), d.data())) return st;
    *fmt = qt == 0 ? PF_FMT_Q8 : (qt == 1 ? PF_FMT_Q4 : (qt == 2 ? PF_FMT_Q2 : PF_FMT_Q15));
    const uint32_t bb = qt == 0 ? 32 : (qt == 1 ? 16 : 8);
    codes.assign(d.size() * bb, 0);
    scales.resize(d.size());
    for (size_t k = 0; k < d.size(); k++) {
        scales[k] = pf_host::half_rne(d[k]);
        uint8_t* o = codes.data() + k * bb;
        for (uint32_t j = 0; j < 32; j++) {
            const int v = c[32 * k + j];
            if (qt == 0) o[j] = (uint8_t)(int8_t)v;
            else if (qt == 1) o[j / 2] |= (uint8_t)((v + 8) << (4 * (j & 1)));
            else if (qt == 2) o[j / 4] |= (uint8_t)((v + 2) << (2 * (j & 3)));
            else o[j / 4] |= (uint8_t)((v + 1) << (2 * (j & 3)));
        }
    }
    return PF_OK;
}

// Norm weights of one layer (matrices 7 and 8): code * multiplier per element,
// any quant type; absent blocks leave the default 1.0.
static pf_status load_norm(pf_squeeze* s, pf_model* m, uint32_t layer, uint32_t matrix, uint32_t D) {
    uint32_t rows, cols, qt;
    if (pf_squeeze_block_shape(s, layer, matrix, &rows, &cols, &qt)) return PF_OK;
    const uint64_t n = (uint64_t)rows * cols;
    if (n < D) return sq_fail(s, PF_ERR_FORMAT, "norm block shorter than n_embd");
    std::vector<int8_t> c(n);
    std::vector<float> d((n + 31) / 32);
    if (pf_status st = pf_squeeze_load_block(s, layer, matrix, c.data(), d.data())) return st;
    std::vector<float> w(D);
    for (uint32_t i = 0; i < D; i++) w[i] = (float)c[i] * d[i / 32];
    return pf_model_set_norm(m, layer, (int32_t)matrix, w.data());
}

// Engine::load_model + load_layer_weights (src/engine.cpp:48-201, 606-640)
// with every layer resident in HBM: layer matrices 0-6 (Q K V O gate up
// down), norms 7 and 8, the tied embedding (layer 0, matrix 10, Q4 or Q8).  MTP
// heads are not in the file format; set them with pf_model_set_mtp (n_mtp of
// the model is the header's mtp_heads).
extern "C" pf_status pf_squeeze_load_model(pf_ctx* ctx, pf_squeeze* s, pf_model** out) {
    if (!ctx || !s || !out) return PF_ERR_ARG;
    *out = nullptr;
    const pf_squeeze_info& I = s->info;
    if (I.n_heads == 0 || I.n_embd % I.n_heads) return sq_fail(s, PF_ERR_FORMAT, "n_embd not a multiple of n_heads");
    if (I.n_kv_heads != 0 && I.n_kv_heads != I.n_heads)
        return sq_fail(s, PF_ERR_UNSUPPORTED, "grouped KV heads (n_kv_heads != n_heads)");
    pf_model_desc d{I.n_layers, I.n_embd, I.n_heads, I.n_embd / I.n_heads, I.n_ff, I.n_vocab, I.mtp_heads};
    pf_model* m = nullptr;
    if (pf_status st = pf_model_create(ctx, &d, &m)) return sq_fail(s, st, pf_last_error(ctx));
    const uint32_t D = I.n_embd, F = I.n_ff;
    const uint32_t shape[7][2] = {{D, D}, {D, D}, {D, D}, {D, D}, {F, D}, {F, D}, {D, F}};
    std::vector<uint8_t> codes;
    std::vector<uint16_t> scales;
    pf_status st = PF_OK;
    for (uint32_t l = 0; l < I.n_layers && !st; l++) {
        for (uint32_t id = 0; id < 7 && !st; id++) {
            int32_t fmt = 0;
            st = repack(s, l, id, shape[id][0], shape[id][1], &fmt, codes, scales);
            if (!st && (st = pf_model_set_matrix(m, l, (int32_t)id, fmt, codes.data(), scales.data())))
                sq_fail(s, st, pf_last_error(ctx));
        }
        if (!st) st = load_norm(s, m, l, 7, D);
        if (!st) st = load_norm(s, m, l, 8, D);
    }
    if (!st) {
        int32_t fmt = 0;
        st = repack(s, 0, 10, I.n_vocab, D, &fmt, codes, scales);
        if (!st && fmt != PF_FMT_Q4 && fmt != PF_FMT_Q8)
            st = sq_fail(s, PF_ERR_UNSUPPORTED, "the embedding table must be Q4 or Q8");
        if (!st && (st = pf_model_set_embedding_fmt(m, fmt, codes.data(), scales.data())))
            sq_fail(s, st, pf_last_error(ctx));
    }
    if (st) {
        pf_model_destroy(m);
        return st;
    }
    *out = m;
    return PF_OK;
}
