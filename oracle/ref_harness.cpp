// C entry points over the reference's own translation units
// (src/matmul_neon.cpp, src/kv_cache.cpp, src/mtp.cpp), so the Python golden
// generator can call them through ctypes.  Test infrastructure only.
#include <vector>
#include <cstdint>
#include <cstring>
#include <cstdlib>
#include <string>
#include <memory>
#include <functional>
#include "forge/matmul_neon.hpp"
#include "forge/kv_cache.hpp"
#include "forge/layer_skip.hpp"
// MTPHeads keeps its weights private; the harness reads and writes them to
// run the reference forward on chosen weights.
#define private public
#include "forge/mtp.hpp"
#undef private

extern "C" {

void ref_quantize_activation_row(const float* s, int8_t* d, float* sc, uint32_t n) {
    forge::quantize_activation_row(s, d, sc, n);
}
void ref_dequant_q4_to_int8(const uint8_t* q, int8_t* o, uint32_t n) { forge::dequant_q4_to_int8(q, o, 1.0f, n); }
void ref_dequant_q2_to_int8(const uint8_t* q, int8_t* o, uint32_t n) { forge::dequant_q2_to_int8(q, o, 1.0f, n); }
void ref_dequant_ternary_to_int8(const uint8_t* q, int8_t* o, uint32_t n) { forge::dequant_ternary_to_int8(q, o, n); }
void ref_matmul_int8(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N, uint32_t K) {
    forge::matmul_int8(A, B, C, M, N, K);
}
void ref_matmul_quantized(const float* A, const int8_t* B, float* C, uint32_t M, uint32_t N, uint32_t K,
                          const float* ws, const float* as) {
    forge::matmul_quantized(A, B, C, M, N, K, ws, as);
}
float ref_dot_product(const float* a, const float* b, uint32_t n) { return forge::dot_product(a, b, n); }
void ref_softmax(float* v, uint32_t n) { forge::softmax(v, n); }
void ref_rmsnorm(float* o, const float* x, const float* w, uint32_t n) { forge::rmsnorm(o, x, w, n); }

void* ref_kv_create(uint32_t L, uint32_t H, uint32_t hd, uint32_t sink, uint32_t win, uint32_t pool, uint32_t maxc) {
    forge::KVCacheConfig c;
    c.n_layers = L; c.n_kv_heads = H; c.head_dim = hd; c.sink_size = sink;
    c.window_size = win; c.pool_block = pool; c.max_context = maxc;
    return new forge::KVCache(c);
}
void ref_kv_destroy(void* k) { delete (forge::KVCache*)k; }
void ref_kv_store(void* k, uint32_t l, uint32_t h, uint32_t pos, const float* key, const float* val) {
    ((forge::KVCache*)k)->store(l, h, pos, key, val);
}
uint32_t ref_kv_attention_scores(void* k, uint32_t l, uint32_t h, const float* q, float* out) {
    return ((forge::KVCache*)k)->attention_scores(l, h, q, out);
}
void ref_kv_attention_weighted_sum(void* k, uint32_t l, uint32_t h, const float* s, float* out, uint32_t n) {
    ((forge::KVCache*)k)->attention_weighted_sum(l, h, s, out, n);
}
uint32_t ref_kv_size(void* k) { return ((forge::KVCache*)k)->size(); }
void ref_kv_clear(void* k) { ((forge::KVCache*)k)->clear(); }
uint64_t ref_kv_memory_usage(void* k) { return ((forge::KVCache*)k)->memory_usage(); }

void* ref_mtp_create(uint32_t heads, uint32_t d, uint32_t vocab) {
    forge::MTPConfig c;
    c.n_mtp_heads = heads; c.n_embd = d; c.n_vocab = vocab; c.mtp_ff_dim = d;
    return new forge::MTPHeads(c);
}
void ref_mtp_destroy(void* m) { delete (forge::MTPHeads*)m; }
// which: 0 gate, 1 up, 2 down.  q4: rows * d/2 bytes, scales: rows floats.
void ref_mtp_set(void* m, uint32_t head, uint32_t which, const uint8_t* q4, const float* scales, uint32_t rows, uint32_t d) {
    auto& hw = ((forge::MTPHeads*)m)->heads_[head];
    std::vector<uint8_t>& q = which == 0 ? hw.gate_q4 : (which == 1 ? hw.up_q4 : hw.down_q4);
    std::vector<float>& s = which == 0 ? hw.gate_scale : (which == 1 ? hw.up_scale : hw.down_scale);
    q.assign(q4, q4 + (size_t)rows * (d / 2));
    s.assign(scales, scales + rows);
}
void ref_mtp_forward(void* m, const float* hidden, const float* emb, uint32_t emb_len, float* out) {
    std::vector<float> e(emb, emb + emb_len);
    auto r = ((forge::MTPHeads*)m)->forward(hidden, e);
    size_t off = 0;
    for (auto& v : r) { std::memcpy(out + off, v.data(), v.size() * sizeof(float)); off += v.size(); }
}
int32_t ref_mtp_argmax(const float* x, uint32_t n) { return forge::MTPHeads::argmax(x, n); }
int32_t ref_mtp_speculative_accept(void* m, int32_t tok, const float* logits, uint32_t heads, uint32_t vocab) {
    std::vector<std::vector<float>> l(heads);
    for (uint32_t h = 0; h < heads; h++) l[h].assign(logits + (size_t)h * vocab, logits + (size_t)(h + 1) * vocab);
    return ((forge::MTPHeads*)m)->speculative_accept(tok, l);
}

// LayerSkipController (src/layer_skip.cpp) with a ModelConfig holding the
// given layer count, width, threshold and anchor interval.
void* ref_skip_create(uint32_t n_layers, uint32_t n_embd, float threshold, uint32_t interval) {
    forge::ModelConfig c;
    c.n_layers = n_layers; c.n_embd = n_embd; c.skip_threshold = threshold; c.skip_interval = interval;
    return new forge::LayerSkipController(c);
}
void ref_skip_destroy(void* s) { delete (forge::LayerSkipController*)s; }
int ref_skip_should_skip_ffn(void* s, uint32_t layer, const float* normed, uint32_t n) {
    return ((forge::LayerSkipController*)s)->should_skip_ffn(layer, normed, n) ? 1 : 0;
}

}  // extern "C"
