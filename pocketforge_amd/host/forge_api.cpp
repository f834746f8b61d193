// forge:: classes and functions (include/forge/*.hpp) over the C ABI of
// libpocketforge_amd.so.  Nothing here computes on the host except
// load-time unpacking and bookkeeping: every kernel-level function and every
// engine method runs on the GPU.  A missing GPU or library error raises
// std::runtime_error with the library's message (the reference's functions
// have no error return).
#include <algorithm>
#include <chrono>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "forge/batch_engine.hpp"
#include "forge/engine.hpp"
#include "forge/kv_cache.hpp"
#include "forge/matmul_neon.hpp"
#include "forge/mtp.hpp"
#include "pf_gpu.h"

namespace forge {
namespace {

void check(const pf_ctx* c, pf_status s, const char* what) {
    if (s == PF_OK) return;
    const char* msg = pf_last_error(c);
    throw std::runtime_error(std::string(what) + ": " + (msg ? msg : "error") + " (status " + std::to_string(s) + ")");
}

// One device context per host thread, shared by the objects created on it
// (each keeps a reference, so the context outlives them).
std::shared_ptr<pf_ctx> shared_ctx() {
    thread_local std::weak_ptr<pf_ctx> cached;
    if (auto p = cached.lock()) return p;
    pf_ctx* c = nullptr;
    check(nullptr, pf_init(0, &c), "pf_init");
    std::shared_ptr<pf_ctx> p(c, [](pf_ctx* x) { pf_destroy(x); });
    cached = p;
    return p;
}

// Growable device buffers of the kernel-level functions.
struct Scratch {
    std::shared_ptr<pf_ctx> ctx = shared_ctx();
    void* buf[4] = {nullptr, nullptr, nullptr, nullptr};
    size_t cap[4] = {0, 0, 0, 0};
    void* get(int slot, size_t bytes) {
        if (bytes == 0) bytes = 4;
        if (bytes > cap[slot]) {
            if (buf[slot]) pf_free(ctx.get(), buf[slot], cap[slot]);
            buf[slot] = nullptr;
            check(ctx.get(), pf_malloc(ctx.get(), bytes, &buf[slot]), "pf_malloc");
            cap[slot] = bytes;
        }
        return buf[slot];
    }
    void up(void* dst, const void* src, size_t n) { check(ctx.get(), pf_memcpy(ctx.get(), dst, src, n, 0), "pf_memcpy"); }
    void down(void* dst, const void* src, size_t n) { check(ctx.get(), pf_memcpy(ctx.get(), dst, src, n, 1), "pf_memcpy"); }
};

// Held until the process ends (not torn down at exit, after the HIP runtime).
Scratch& scratch() {
    thread_local Scratch* s = new Scratch();
    return *s;
}

// Seeded N(0, 0.02) block-quantized matrix (pf_gen_matrix, host).
struct HostMatrix {
    std::vector<uint8_t> codes;
    std::vector<uint16_t> scales;
};

HostMatrix gen_matrix(uint64_t seed, uint32_t stream, uint32_t rows, uint32_t cols, int32_t fmt) {
    HostMatrix m;
    m.codes.resize((size_t)rows * (cols / 32) * (fmt == PF_FMT_Q4 ? 16 : 8));
    m.scales.resize((size_t)rows * (cols / 32));
    check(nullptr, pf_gen_matrix(seed, stream, 0.02f, rows, cols, fmt, m.codes.data(), m.scales.data()),
          "pf_gen_matrix");
    return m;
}

// A device model of the seeded synthetic weights: layer l, matrix j from
// stream 16 l + j, the tied embedding from 0x10000, MTP head k matrix j from
// 0x20000 + 3 k + j (the benchmark's streams).  MHA only.
bool make_random_model(pf_ctx* ctx, const ModelConfig& cfg, uint64_t seed, const WeightFormats& formats,
                       pf_model** out, size_t* weight_bytes, size_t* mtp_bytes) {
    *out = nullptr;
    const uint32_t D = cfg.n_embd, F = cfg.n_ff, V = cfg.n_vocab;
    if (cfg.n_kv_heads != cfg.n_heads) return false;
    pf_model_desc d{cfg.n_layers, D, cfg.n_heads, cfg.head_dim(), F, V, cfg.mtp_heads};
    pf_model* m = nullptr;
    if (pf_model_create(ctx, &d, &m) != PF_OK) return false;
    std::unique_ptr<pf_model, void (*)(pf_model*)> guard(m, pf_model_destroy);
    const int32_t fa = (int32_t)formats.attention, fg = (int32_t)formats.ffn_gate_up, fd = (int32_t)formats.ffn_down;
    const struct { uint32_t rows, cols; int32_t fmt; } shape[7] = {
        {D, D, fa}, {D, D, fa}, {D, D, fa}, {D, D, fa}, {F, D, fg}, {F, D, fg}, {D, F, fd}};
    *weight_bytes = 0;
    for (uint32_t l = 0; l < cfg.n_layers; l++)
        for (int32_t j = 0; j < 7; j++) {
            HostMatrix h = gen_matrix(seed, l * 16u + (uint32_t)j, shape[j].rows, shape[j].cols, shape[j].fmt);
            if (pf_model_set_matrix(m, l, j, shape[j].fmt, h.codes.data(), h.scales.data()) != PF_OK) return false;
            *weight_bytes += h.codes.size() + h.scales.size() * 2;
        }
    {
        HostMatrix h = gen_matrix(seed, 0x10000u, V, D, PF_FMT_Q4);
        if (pf_model_set_embedding(m, h.codes.data(), h.scales.data()) != PF_OK) return false;
        *weight_bytes += h.codes.size() + h.scales.size() * 2;
    }
    *mtp_bytes = 0;
    for (uint32_t k = 0; k < cfg.mtp_heads; k++)
        for (int32_t j = 0; j < 3; j++) {
            HostMatrix h = gen_matrix(seed, 0x20000u + 3u * k + (uint32_t)j, D, D, PF_FMT_Q4);
            if (pf_model_set_mtp(m, k, j, h.codes.data(), h.scales.data()) != PF_OK) return false;
            *mtp_bytes += h.codes.size() + h.scales.size() * 2;
        }
    *out = guard.release();
    return true;
}

// A device model of a .squeeze file (src/engine.cpp:48-201), every layer
// resident; cfg takes the file's configuration.  The format holds no MTP
// heads; the reference draws them at load time (MTPHeads::init_weights),
// here they are the seeded heads of make_random_model with seed 0.
bool make_squeeze_model(pf_ctx* ctx, const std::string& path, ModelConfig& cfg, pf_model** out,
                        size_t* mtp_bytes) {
    *out = nullptr;
    pf_squeeze* sq = nullptr;
    if (pf_squeeze_open(path.c_str(), &sq) != PF_OK) return false;
    pf_squeeze_info info{};
    pf_squeeze_get_info(sq, &info);
    pf_model* m = nullptr;
    const pf_status st = pf_squeeze_load_model(ctx, sq, &m);
    pf_squeeze_close(sq);
    if (st != PF_OK) return false;
    std::unique_ptr<pf_model, void (*)(pf_model*)> guard(m, pf_model_destroy);
    cfg.n_layers = info.n_layers;
    cfg.n_embd = info.n_embd;
    cfg.n_heads = info.n_heads;
    cfg.n_kv_heads = info.n_kv_heads ? info.n_kv_heads : info.n_heads;
    cfg.n_ff = info.n_ff;
    cfg.n_vocab = info.n_vocab;
    cfg.max_seq_len = info.max_seq_len;
    cfg.mtp_heads = info.mtp_heads;
    const uint32_t D = cfg.n_embd;
    *mtp_bytes = 0;
    for (uint32_t k = 0; k < cfg.mtp_heads; k++)
        for (int32_t j = 0; j < 3; j++) {
            HostMatrix h = gen_matrix(0, 0x20000u + 3u * k + (uint32_t)j, D, D, PF_FMT_Q4);
            if (pf_model_set_mtp(m, k, j, h.codes.data(), h.scales.data()) != PF_OK) return false;
            *mtp_bytes += h.codes.size() + h.scales.size() * 2;
        }
    *out = guard.release();
    return true;
}

// The reference's KVCacheConfig from ModelConfig (src/engine.cpp:58-67).
pf_cache_desc cache_of(const ModelConfig& cfg) {
    return pf_cache_desc{4u, std::min(cfg.kv_cache_size, (uint32_t)8192), 64u, cfg.max_seq_len};
}

}  // namespace

// ======================================================== matmul_neon.hpp

void quantize_activation_row(const float* src, int8_t* dst, float* scale_out, uint32_t n) {
    Scratch& s = scratch();
    void* x = s.get(0, (size_t)n * 4);
    void* q = s.get(1, n);
    void* sc = s.get(2, 4);
    s.up(x, src, (size_t)n * 4);
    check(s.ctx.get(), pf_quantize_activation_rows(s.ctx.get(), (const float*)x, (int8_t*)q, (float*)sc, 1, n),
          "pf_quantize_activation_rows");
    s.down(dst, q, n);
    s.down(scale_out, sc, 4);
}

void dequant_q4_to_int8(const uint8_t* q4, int8_t* out, float, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) {
        const uint8_t b = q4[i >> 1];
        out[i] = (int8_t)(((i & 1u) ? (b >> 4) : (b & 15u)) - 8);
    }
}

void dequant_q2_to_int8(const uint8_t* q2, int8_t* out, float, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) out[i] = (int8_t)(((q2[i >> 2] >> (2 * (i & 3u))) & 3u) - 2);
}

void dequant_ternary_to_int8(const uint8_t* t, int8_t* out, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) {
        const uint32_t c = (t[i >> 1] >> (2 * (i & 1u))) & 3u;   // codes 0, 1, 2 -> -1, 0, +1; 3 -> 0
        out[i] = (int8_t)(c == 3u ? 0 : (int)c - 1);
    }
}

void matmul_int8(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N, uint32_t K) {
    Scratch& s = scratch();
    void* a = s.get(0, (size_t)M * K);
    void* b = s.get(1, (size_t)N * K);
    void* c = s.get(2, (size_t)M * N * 4);
    s.up(a, A, (size_t)M * K);
    s.up(b, B, (size_t)N * K);
    check(s.ctx.get(), pf_matmul_int8(s.ctx.get(), (const int8_t*)a, (const int8_t*)b, (int32_t*)c, M, N, K),
          "pf_matmul_int8");
    s.down(C, c, (size_t)M * N * 4);
}

void matmul_quantized(const float* A, const int8_t* B, float* C, uint32_t M, uint32_t N, uint32_t K,
                      const float* weight_scales, const float* act_scales) {
    Scratch& s = scratch();
    const size_t a_bytes = ((size_t)M * K * 4 + 255) & ~(size_t)255;
    const size_t w_bytes = ((size_t)N * 4 + 255) & ~(size_t)255;
    char* p = (char*)s.get(0, a_bytes + w_bytes + (size_t)M * 4);
    void* b = s.get(1, (size_t)N * K);
    void* c = s.get(2, (size_t)M * N * 4);
    s.up(p, A, (size_t)M * K * 4);
    s.up(p + a_bytes, weight_scales, (size_t)N * 4);
    if (act_scales) s.up(p + a_bytes + w_bytes, act_scales, (size_t)M * 4);
    s.up(b, B, (size_t)N * K);
    check(s.ctx.get(),
          pf_matmul_quantized(s.ctx.get(), (const float*)p, (const int8_t*)b, (float*)c, M, N, K,
                              (const float*)(p + a_bytes), act_scales ? (const float*)(p + a_bytes + w_bytes) : nullptr),
          "pf_matmul_quantized");
    s.down(C, c, (size_t)M * N * 4);
}

float dot_product(const float* a, const float* b, uint32_t n) {
    Scratch& s = scratch();
    void* x = s.get(0, (size_t)n * 4);
    void* y = s.get(1, (size_t)n * 4);
    void* o = s.get(2, 4);
    s.up(x, a, (size_t)n * 4);
    s.up(y, b, (size_t)n * 4);
    check(s.ctx.get(), pf_dot_product(s.ctx.get(), (const float*)x, (const float*)y, n, (float*)o), "pf_dot_product");
    float r = 0.0f;
    s.down(&r, o, 4);
    return r;
}

void softmax(float* vals, uint32_t n) {
    if (n == 0) return;
    Scratch& s = scratch();
    void* x = s.get(0, (size_t)n * 4);
    s.up(x, vals, (size_t)n * 4);
    check(s.ctx.get(), pf_softmax(s.ctx.get(), (float*)x, n), "pf_softmax");
    s.down(vals, x, (size_t)n * 4);
}

void rmsnorm(float* out, const float* x, const float* weight, uint32_t n) {
    if (n == 0) return;
    Scratch& s = scratch();
    void* dx = s.get(0, (size_t)n * 4);
    void* dw = s.get(1, (size_t)n * 4);
    void* dy = s.get(2, (size_t)n * 4);
    s.up(dx, x, (size_t)n * 4);
    s.up(dw, weight, (size_t)n * 4);
    check(s.ctx.get(), pf_rmsnorm(s.ctx.get(), (float*)dy, (const float*)dx, (const float*)dw, n), "pf_rmsnorm");
    s.down(out, dy, (size_t)n * 4);
}

// =========================================================== kv_cache.hpp

struct KVCache::Device {
    std::shared_ptr<pf_ctx> ctx;
    pf_kv* kv = nullptr;
    ~Device() { pf_kv_destroy(kv); }
};

KVCache::KVCache(const KVCacheConfig& cfg) : cfg_(cfg), dev_(new Device) {
    dev_->ctx = shared_ctx();
    pf_kv_config c{cfg.n_layers, cfg.n_kv_heads, cfg.head_dim, cfg.sink_size, cfg.window_size, cfg.pool_block,
                   cfg.max_context};
    check(dev_->ctx.get(), pf_kv_create(dev_->ctx.get(), &c, &dev_->kv), "pf_kv_create");
}

KVCache::~KVCache() = default;

void KVCache::store(uint32_t layer, uint32_t head, uint32_t pos, const float* key, const float* value) {
    check(dev_->ctx.get(), pf_kv_store(dev_->kv, layer, head, pos, key, value), "pf_kv_store");
}

uint32_t KVCache::attention_scores(uint32_t layer, uint32_t head, const float* query, float* scores_out) {
    uint32_t n = 0;
    check(dev_->ctx.get(), pf_kv_attention_scores(dev_->kv, layer, head, query, scores_out, &n),
          "pf_kv_attention_scores");
    return n;
}

void KVCache::attention_weighted_sum(uint32_t layer, uint32_t head, const float* scores, float* output,
                                     uint32_t count) {
    check(dev_->ctx.get(), pf_kv_attention_weighted_sum(dev_->kv, layer, head, scores, output, count),
          "pf_kv_attention_weighted_sum");
}

uint32_t KVCache::size() const { return pf_kv_size(dev_->kv); }

void KVCache::clear() { check(dev_->ctx.get(), pf_kv_clear(dev_->kv), "pf_kv_clear"); }

size_t KVCache::memory_usage() const { return pf_kv_memory_usage(dev_->kv); }

// ================================================================ mtp.hpp

struct MTPHeads::Device {
    std::shared_ptr<pf_ctx> ctx;
    pf_mtp* mtp = nullptr;
    ~Device() { pf_mtp_destroy(mtp); }
};

MTPHeads::MTPHeads(const MTPConfig& cfg) : cfg_(cfg), dev_(new Device) {
    if (cfg.mtp_ff_dim != cfg.n_embd)
        throw std::runtime_error("MTPHeads: mtp_ff_dim must equal n_embd (the engine's heads, src/engine.cpp:79)");
    dev_->ctx = shared_ctx();
    check(dev_->ctx.get(), pf_mtp_create(dev_->ctx.get(), cfg.n_mtp_heads, cfg.n_embd, cfg.n_vocab, &dev_->mtp),
          "pf_mtp_create");
    init_weights();   // the reference's constructor draws weights too (src/mtp.cpp:11)
}

MTPHeads::~MTPHeads() = default;

void MTPHeads::init_weights() {
    const uint64_t seed = 0x4D545048454144ULL;   // one fixed seed; each call takes the next streams
    for (uint32_t k = 0; k < cfg_.n_mtp_heads; k++)
        for (int32_t w = 0; w < 3; w++) {
            HostMatrix m = gen_matrix(seed, 0x30000u + 0x1000u * draws_ + 3u * k + (uint32_t)w, cfg_.n_embd,
                                      cfg_.n_embd, PF_FMT_Q4);
            check(dev_->ctx.get(), pf_mtp_set_head(dev_->mtp, k, w, m.codes.data(), m.scales.data()),
                  "pf_mtp_set_head");
        }
    draws_++;
}

void MTPHeads::set_head_weights(uint32_t head, int which, const uint8_t* codes, const uint16_t* scales) {
    check(dev_->ctx.get(), pf_mtp_set_head(dev_->mtp, head, which, codes, scales), "pf_mtp_set_head");
}

std::vector<std::vector<float>> MTPHeads::forward(const float* hidden, const std::vector<float>& table) const {
    const size_t V = cfg_.n_vocab, D = cfg_.n_embd;
    const bool tied = table.size() >= V * D;        // src/mtp.cpp:53
    check(dev_->ctx.get(), pf_mtp_set_table(dev_->mtp, tied ? table.data() : nullptr), "pf_mtp_set_table");
    std::vector<float> flat(cfg_.n_mtp_heads * V);
    check(dev_->ctx.get(), pf_mtp_heads_forward(dev_->mtp, hidden, flat.data()), "pf_mtp_heads_forward");
    std::vector<std::vector<float>> out(cfg_.n_mtp_heads);
    for (uint32_t h = 0; h < cfg_.n_mtp_heads; h++) out[h].assign(flat.begin() + h * V, flat.begin() + (h + 1) * V);
    return out;
}

// src/mtp.cpp:131-143: heads 1.. in order while their argmax equals token;
// the count starts at 1.
int MTPHeads::speculative_accept(int32_t token, const std::vector<std::vector<float>>& mtp_logits) const {
    int accepted = 1;
    const size_t n = std::min<size_t>(mtp_logits.size(), cfg_.n_mtp_heads);
    for (size_t h = 1; h < n; h++) {
        if (argmax(mtp_logits[h].data(), cfg_.n_vocab) != token) break;
        accepted++;
    }
    return accepted;
}

int32_t MTPHeads::argmax(const float* logits, uint32_t n) {
    if (n == 0) return 0;
    Scratch& s = scratch();
    void* x = s.get(0, (size_t)n * 4);
    void* o = s.get(1, 4);
    s.up(x, logits, (size_t)n * 4);
    check(s.ctx.get(), pf_argmax(s.ctx.get(), (const float*)x, n, (int32_t*)o), "pf_argmax");
    int32_t r = 0;
    s.down(&r, o, 4);
    return r;
}

size_t MTPHeads::memory_usage() const { return pf_mtp_memory(dev_->mtp); }

// ============================================================= engine.hpp

bool ModelConfig::check_memory_budget() const {   // src/engine.cpp:17-27
    const size_t hd = head_dim();
    const size_t window = std::min(kv_cache_size, (uint32_t)8192);
    const size_t pool = max_seq_len > window ? (max_seq_len - window) / 64 : 0;
    const size_t kv = (size_t)n_layers * n_kv_heads * (window + pool) * hd * 2;
    const size_t mtp = (size_t)mtp_heads * n_embd * n_embd * 3 / 2;
    const size_t act = (size_t)n_embd * 20 * 4;
    return kv + mtp + act < max_memory;
}

struct Engine::Device {
    std::shared_ptr<pf_ctx> ctx;
    pf_model* model = nullptr;
    pf_engine* eng = nullptr;
    bool mtp_enabled = true;
    size_t max_memory = 0;           // 0: no device-memory guard
    float skip_threshold = 0.0f;     // layer skip off until set_layer_skip_threshold
    uint64_t draw = 0;               // stochastic draws of sample()
    size_t weight_bytes = 0, mtp_bytes = 0;
    ~Device() {
        pf_engine_destroy(eng);
        pf_model_destroy(model);
    }
};

Engine::Engine() : dev_(new Device) {}
Engine::~Engine() = default;

size_t Engine::MemoryStats::total() const {
    return weights_mmap + weights_decompressed + kv_cache + activations + prefetch_buffer + mtp_heads + other;
}

// src/engine.cpp:48-201: the .squeeze file's configuration and weights
// (every layer resident in HBM), MTP heads as make_squeeze_model says.
bool Engine::load_model(const std::string& path) {
    if (!dev_->ctx) dev_->ctx = shared_ctx();
    pf_engine_destroy(dev_->eng);
    dev_->eng = nullptr;
    pf_model_destroy(dev_->model);
    dev_->model = nullptr;
    ModelConfig cfg = config_;
    dev_->weight_bytes = 0;   // not tracked for loaded files
    if (!make_squeeze_model(dev_->ctx.get(), path, cfg, &dev_->model, &dev_->mtp_bytes)) return false;
    config_ = cfg;
    dev_->mtp_enabled = cfg.mtp_enabled;
    return rebuild_engine();
}
bool Engine::load_norm_weights_from_gguf(const std::string&) { return false; }

bool Engine::rebuild_engine() {
    pf_engine_destroy(dev_->eng);
    dev_->eng = nullptr;
    if (!dev_->model) return false;
    pf_cache_desc kc = cache_of(config_);
    if (pf_engine_create(dev_->model, &kc, &dev_->eng) != PF_OK) return false;
    pf_engine_set_mtp_enabled(dev_->eng, dev_->mtp_enabled ? 1 : 0);
    pf_engine_set_max_memory(dev_->eng, dev_->max_memory);
    pf_engine_set_layer_skip(dev_->eng, dev_->skip_threshold, config_.skip_interval);
    return true;
}

bool Engine::load_random_model(const ModelConfig& cfg, uint64_t seed, const WeightFormats& formats) {
    if (!dev_->ctx) dev_->ctx = shared_ctx();
    pf_engine_destroy(dev_->eng);
    dev_->eng = nullptr;
    pf_model_destroy(dev_->model);
    dev_->model = nullptr;
    config_ = cfg;
    if (!make_random_model(dev_->ctx.get(), cfg, seed, formats, &dev_->model, &dev_->weight_bytes, &dev_->mtp_bytes))
        return false;
    dev_->mtp_enabled = cfg.mtp_enabled;
    return rebuild_engine();
}

void Engine::set_max_context(uint32_t tokens) {   // src/engine.cpp:232-237
    config_.max_seq_len = std::min(tokens, (uint32_t)131072);
    config_.kv_cache_size = std::min(tokens, (uint32_t)8192);
    if (dev_->eng) rebuild_engine();
}

void Engine::set_mtp_enabled(bool enabled) {
    config_.mtp_enabled = enabled;
    dev_->mtp_enabled = enabled;
    if (dev_->eng) pf_engine_set_mtp_enabled(dev_->eng, enabled ? 1 : 0);
}

// src/engine.cpp:266-269.  The reference creates its controller at load time
// with ModelConfig::skip_threshold (0.01); here the controller stays off
// until this call, since skipping changes the outputs.
// GenerationResult::layers_skipped stays 0 as in the reference, whose
// controller never increments its counter; pf_engine_layer_skip_count has
// the real count.
void Engine::set_layer_skip_threshold(float threshold) {
    config_.skip_threshold = threshold;
    dev_->skip_threshold = threshold;
    if (dev_->eng) pf_engine_set_layer_skip(dev_->eng, threshold, config_.skip_interval);
}

void Engine::set_max_memory(size_t bytes) {
    config_.max_memory = bytes;
    dev_->max_memory = bytes;
    if (dev_->eng) pf_engine_set_max_memory(dev_->eng, bytes);
}

GenerationResult Engine::generate(const std::vector<int32_t>& prompt, uint32_t max_new, TokenCallback callback,
                                  ProgressCallback progress) {
    return generate(prompt, max_new, SamplingConfig(), 42, std::move(callback), std::move(progress));
}

GenerationResult Engine::generate(const std::vector<int32_t>& prompt, uint32_t max_new,
                                  const SamplingConfig& sc, uint64_t seed, TokenCallback callback,
                                  ProgressCallback progress) {
    GenerationResult r;
    if (!dev_->eng) return r;
    const auto t0 = std::chrono::steady_clock::now();
    pf_sampling s{sc.temperature, sc.top_p, sc.top_k, sc.greedy ? 1 : 0};
    std::vector<int32_t> out(prompt.size() + max_new + 8);
    pf_gen_result g{};
    check(dev_->ctx.get(),
          pf_generate(dev_->eng, prompt.data(), (uint32_t)prompt.size(), max_new, &s, seed, out.data(),
                      (uint32_t)out.size(), &g),
          "pf_generate");
    out.resize(g.n_tokens);
    const float secs = std::chrono::duration<float>(std::chrono::steady_clock::now() - t0).count();
    r.tokens = std::move(out);
    r.tokens_per_second = secs > 0.0f ? (float)r.tokens.size() / secs : 0.0f;   // prompt included, as the reference
    r.mtp_accepted = g.mtp_accepted;
    r.mtp_rejected = g.mtp_rejected;
    r.oom_protected = g.oom_protected != 0;
    r.peak_memory_bytes = get_memory_stats().total();
    // the decode runs on the device as one call; the callbacks see its tokens afterwards
    if (callback)
        for (size_t i = prompt.size(); i < r.tokens.size(); i++) callback(r.tokens[i], 1.0f);
    if (progress) progress(1.0f);
    return r;
}

std::vector<float> Engine::forward_with_hidden(const std::vector<int32_t>& tokens, std::vector<float>& hidden_out) {
    std::vector<float> logits;
    if (!dev_->eng || tokens.empty()) return logits;
    const uint32_t V = config_.n_vocab, D = config_.n_embd;
    std::vector<float> lg, hd;
    for (size_t i = 0; i < tokens.size(); i += 8) {
        const uint32_t n = (uint32_t)std::min<size_t>(8, tokens.size() - i);
        const bool last = i + n == tokens.size();    // only the last pass's rows are copied back
        lg.resize(last ? (size_t)n * V : 0);
        hd.resize(last ? (size_t)n * D : 0);
        check(dev_->ctx.get(),
              pf_forward(dev_->eng, tokens.data() + i, n, last ? lg.data() : nullptr, last ? hd.data() : nullptr),
              "pf_forward");
    }
    logits.assign(lg.end() - V, lg.end());
    hidden_out.assign(hd.end() - D, hd.end());
    return logits;
}

std::vector<float> Engine::forward(const std::vector<int32_t>& tokens) {
    std::vector<float> hidden;
    return forward_with_hidden(tokens, hidden);
}

std::pair<int, std::vector<float>> Engine::step_mtp(int32_t current_token, const std::vector<float>& hidden_state,
                                                    const std::vector<float>& embedding_table, int& acc_out,
                                                    int& rej_out) {
    acc_out = 0;
    rej_out = 0;
    // src/engine.cpp:413-416: no heads, or no table, is one plain forward.  As
    // in the reference, ModelConfig::mtp_enabled is not consulted here.
    if (!dev_->eng || config_.mtp_heads == 0 || embedding_table.empty()) return {0, forward({current_token})};
    if (hidden_state.size() < config_.n_embd)
        throw std::invalid_argument("Engine::step_mtp: hidden_state shorter than n_embd");
    // The heads run on the engine's device-resident tied table; the caller's
    // fp32 table is only checked for emptiness.  Engine::generate passes the
    // dequantized tied table itself (src/engine.cpp:318-319), so the two agree
    // for the reference's own caller.  The drafts are sampled with
    // Engine::sample's defaults (seed 42, the engine's draw counter) and
    // verified in one pass on the device (pf_step_mtp).
    const SamplingConfig dflt;
    const pf_sampling s{dflt.temperature, dflt.top_p, dflt.top_k, dflt.greedy ? 1 : 0};
    std::vector<float> logits(config_.n_vocab);
    int32_t accepted = 0, has = 0;
    check(dev_->ctx.get(),
          pf_step_mtp(dev_->eng, current_token, hidden_state.data(), &s, 42, &dev_->draw, &accepted, &acc_out,
                      &rej_out, logits.data(), &has),
          "pf_step_mtp");
    if (!has) logits.clear();
    return {accepted, logits};
}

int32_t Engine::sample(const float* logits, uint32_t n_vocab, const SamplingConfig& cfg) {
    if (!dev_->eng || n_vocab != config_.n_vocab) throw std::runtime_error("Engine::sample: no model of that vocabulary");
    pf_sampling s{cfg.temperature, cfg.top_p, cfg.top_k, cfg.greedy ? 1 : 0};
    int32_t t = 0;
    check(dev_->ctx.get(), pf_sample(dev_->eng, logits, &s, 42, &dev_->draw, &t), "pf_sample");
    return t;
}

int32_t Engine::sample_greedy(const float* logits, uint32_t n_vocab) {
    SamplingConfig c;
    c.greedy = true;
    return sample(logits, n_vocab, c);
}

int32_t Engine::sample_top_k(const float* logits, uint32_t n_vocab, uint32_t k, float temp) {
    SamplingConfig c;
    c.temperature = temp;
    c.top_p = 1.0f;   // outside (0, 1): the dispatch reaches top-k (src/engine.cpp:887-893)
    c.top_k = k;
    return sample(logits, n_vocab, c);
}

int32_t Engine::sample_top_p(const float* logits, uint32_t n_vocab, float p, float temp) {
    SamplingConfig c;
    c.temperature = temp;
    c.top_p = p;
    c.top_k = 0;
    return sample(logits, n_vocab, c);
}

Engine::MemoryStats Engine::get_memory_stats() const {
    MemoryStats m;
    if (!dev_->ctx) return m;
    const size_t total = pf_device_bytes(dev_->ctx.get());
    m.weights_decompressed = dev_->weight_bytes;
    m.mtp_heads = dev_->mtp_bytes;
    const uint32_t hd = config_.head_dim();
    const size_t window = std::min(config_.kv_cache_size, (uint32_t)8192);
    const size_t rows = 8 + window + 64 + 8 + (config_.max_seq_len > window ? (config_.max_seq_len - window) / 64 + 1 : 1);
    m.kv_cache = dev_->eng ? (size_t)config_.n_layers * config_.n_heads * rows * (2 * hd + 8) : 0;
    const size_t known = m.weights_decompressed + m.mtp_heads + m.kv_cache;
    m.activations = total > known ? total - known : 0;
    return m;
}

// ======================================================== batch_engine.hpp

struct BatchEngine::Device {
    std::shared_ptr<pf_ctx> ctx;
    pf_model* model = nullptr;
    pf_engine* eng = nullptr;
    bool mtp_enabled = true;
    size_t weight_bytes = 0, mtp_bytes = 0;
    ~Device() {
        pf_engine_destroy(eng);
        pf_model_destroy(model);
    }
};

BatchEngine::BatchEngine(uint32_t n_sequences) : n_seq_(n_sequences), dev_(new Device) {}
BatchEngine::~BatchEngine() = default;

bool BatchEngine::rebuild_engine() {
    pf_engine_destroy(dev_->eng);
    dev_->eng = nullptr;
    if (!dev_->model || n_seq_ == 0) return false;
    pf_cache_desc kc = cache_of(config_);
    if (pf_batch_create(dev_->model, &kc, n_seq_, &dev_->eng) != PF_OK) return false;
    pf_engine_set_mtp_enabled(dev_->eng, dev_->mtp_enabled ? 1 : 0);
    return true;
}

bool BatchEngine::load_model(const std::string& path) {
    if (!dev_->ctx) dev_->ctx = shared_ctx();
    pf_engine_destroy(dev_->eng);
    dev_->eng = nullptr;
    pf_model_destroy(dev_->model);
    dev_->model = nullptr;
    ModelConfig cfg = config_;
    if (!make_squeeze_model(dev_->ctx.get(), path, cfg, &dev_->model, &dev_->mtp_bytes)) return false;
    config_ = cfg;
    dev_->mtp_enabled = cfg.mtp_enabled;
    return rebuild_engine();
}

bool BatchEngine::load_random_model(const ModelConfig& cfg, uint64_t seed, const WeightFormats& formats) {
    if (!dev_->ctx) dev_->ctx = shared_ctx();
    pf_engine_destroy(dev_->eng);
    dev_->eng = nullptr;
    pf_model_destroy(dev_->model);
    dev_->model = nullptr;
    config_ = cfg;
    if (!make_random_model(dev_->ctx.get(), cfg, seed, formats, &dev_->model, &dev_->weight_bytes, &dev_->mtp_bytes))
        return false;
    dev_->mtp_enabled = cfg.mtp_enabled;
    return rebuild_engine();
}

void BatchEngine::set_max_context(uint32_t tokens) {   // as Engine::set_max_context (src/engine.cpp:232-237)
    config_.max_seq_len = std::min(tokens, (uint32_t)131072);
    config_.kv_cache_size = std::min(tokens, (uint32_t)8192);
    if (dev_->eng) rebuild_engine();
}

void BatchEngine::set_mtp_enabled(bool enabled) {
    config_.mtp_enabled = enabled;
    dev_->mtp_enabled = enabled;
    if (dev_->eng) pf_engine_set_mtp_enabled(dev_->eng, enabled ? 1 : 0);
}

uint32_t BatchEngine::position(uint32_t seq) const { return dev_->eng ? pf_batch_position(dev_->eng, seq) : 0; }

void BatchEngine::reset() {
    if (dev_->eng) check(dev_->ctx.get(), pf_engine_reset(dev_->eng), "pf_engine_reset");
}

std::vector<GenerationResult> BatchEngine::generate(const std::vector<std::vector<int32_t>>& prompts,
                                                    uint32_t max_new, const SamplingConfig& sc,
                                                    const std::vector<uint64_t>& seeds,
                                                    BatchTokenCallback callback) {
    if (!dev_->eng) throw std::runtime_error("BatchEngine::generate: no model loaded");
    if (prompts.size() != n_seq_) throw std::invalid_argument("BatchEngine::generate: one prompt per sequence");
    if (!seeds.empty() && seeds.size() != n_seq_)
        throw std::invalid_argument("BatchEngine::generate: one seed per sequence");
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<uint32_t> lens(n_seq_);
    std::vector<int32_t> flat;
    size_t longest = 0;
    for (uint32_t i = 0; i < n_seq_; i++) {
        lens[i] = (uint32_t)prompts[i].size();
        flat.insert(flat.end(), prompts[i].begin(), prompts[i].end());
        longest = std::max(longest, prompts[i].size());
    }
    if (flat.empty()) flat.push_back(0);
    std::vector<uint64_t> sd = seeds.empty() ? std::vector<uint64_t>(n_seq_, 42) : seeds;
    const uint32_t cap = (uint32_t)longest + max_new + 8;
    std::vector<int32_t> out((size_t)n_seq_ * cap);
    std::vector<pf_gen_result> g(n_seq_);
    pf_sampling s{sc.temperature, sc.top_p, sc.top_k, sc.greedy ? 1 : 0};
    check(dev_->ctx.get(),
          pf_batch_generate(dev_->eng, flat.data(), lens.data(), max_new, &s, sd.data(), out.data(), cap, g.data()),
          "pf_batch_generate");
    const float secs = std::chrono::duration<float>(std::chrono::steady_clock::now() - t0).count();
    std::vector<GenerationResult> r(n_seq_);
    for (uint32_t i = 0; i < n_seq_; i++) {
        r[i].tokens.assign(out.begin() + (size_t)i * cap, out.begin() + (size_t)i * cap + g[i].n_tokens);
        r[i].tokens_per_second = secs > 0.0f ? (float)r[i].tokens.size() / secs : 0.0f;
        r[i].mtp_accepted = g[i].mtp_accepted;
        r[i].mtp_rejected = g[i].mtp_rejected;
        r[i].oom_protected = g[i].oom_protected != 0;
        r[i].peak_memory_bytes = pf_device_bytes(dev_->ctx.get());
        if (callback)
            for (size_t k = prompts[i].size(); k < r[i].tokens.size(); k++) callback(i, r[i].tokens[k]);
    }
    return r;
}

}  // namespace forge
