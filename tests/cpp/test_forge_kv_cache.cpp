// forge::KVCache on the GPU: the reference's checks (tests/test_kv_cache.cpp)
// plus bit-exact parity with the oracle's cache on the same stores.
#include <vector>

#include "forge/kv_cache.hpp"
#include "forge_test.hpp"
#include "pf_oracle.h"

int run() {
    std::cout << "forge KVCache on the GPU\n";
    forge::KVCacheConfig cfg;
    cfg.n_layers = 2;
    cfg.n_kv_heads = 2;
    cfg.head_dim = 4;
    cfg.sink_size = 2;
    cfg.window_size = 16;
    cfg.pool_block = 4;
    cfg.max_context = 128;
    forge::KVCache cache(cfg);
    orc_kv* ref = orc_kv_create(2, 2, 4, 2, 16, 4, 128);
    CHECK("initial size 0", cache.size() == 0);
    CHECK("memory usage > 0", cache.memory_usage() > 0);
    auto both = [&](uint32_t l, uint32_t h, uint32_t pos, const float* k, const float* v) {
        cache.store(l, h, pos, k, v);
        orc_kv_store(ref, l, h, pos, k, v);
    };
    float k[4] = {1, 2, 3, 4}, v[4] = {5, 6, 7, 8};
    both(0, 0, 0, k, v);
    both(0, 0, 1, k, v);
    CHECK("sink stored", cache.size() >= 1);
    for (uint32_t i = 2; i < 18; i++) {
        float kv[4] = {(float)i, (float)i, (float)i, (float)i};
        both(0, 0, i, kv, kv);
    }
    CHECK("window filled", cache.size() >= 17);
    for (uint32_t i = 18; i < 30; i++) {
        float kv[4] = {(float)i, (float)i * 0.5f, -(float)i, 1.0f};
        both(0, 0, i, kv, kv);
    }
    CHECK("pooling triggered", cache.size() >= 29 && cache.size() == orc_kv_size(ref));
    float q[4] = {1, 1, 1, 1};
    float scores[256] = {0}, rs[256] = {0};
    uint32_t count = cache.attention_scores(0, 0, q, scores);
    uint32_t rcount = orc_kv_attention_scores(ref, 0, 0, q, rs);
    CHECK("scores returned", count > 0);
    CHECK("scores finite", std::isfinite(scores[0]));
    CHECK("scores include sink + pool + window", count >= 2 + 16);
    bool same = count == rcount;
    for (uint32_t i = 0; same && i < count; i++) same = scores[i] == rs[i];
    CHECK("scores equal the oracle", same);
    std::vector<float> p(count);
    for (uint32_t i = 0; i < count; i++) p[i] = 1.0f / (float)count;
    float out[4] = {0}, ro[4] = {0};
    cache.attention_weighted_sum(0, 0, p.data(), out, count);
    orc_kv_attention_weighted_sum(ref, 0, 0, p.data(), ro, count);
    CHECK("weighted sum finite", std::isfinite(out[0]) && std::isfinite(out[1]));
    CHECK("weighted sum equals the oracle", out[0] == ro[0] && out[1] == ro[1] && out[2] == ro[2] && out[3] == ro[3]);
    both(1, 1, 0, k, v);
    CHECK("other layer and head", cache.attention_scores(1, 1, q, scores) >= 1);
    cache.clear();
    CHECK("size after clear", cache.size() == 0);
    orc_kv_destroy(ref);
    forge::KVCacheConfig big;
    big.n_layers = 24;
    big.n_kv_heads = 4;
    big.head_dim = 64;
    big.window_size = 8192;
    big.max_context = 131072;
    big.pool_block = 64;
    forge::KVCache big_cache(big);
    std::cout << "  131K-context cache: " << big_cache.memory_usage() / (1024 * 1024) << " MiB of HBM\n";
    CHECK("131K context under 150 MB", big_cache.memory_usage() < 150u * 1024 * 1024);
    return finish("test_forge_kv_cache");
}
