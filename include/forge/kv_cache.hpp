// 3-tier int8 KV cache (include/forge/kv_cache.hpp:23-56), HBM-resident.
#ifndef FORGE_KV_CACHE_HPP
#define FORGE_KV_CACHE_HPP

#include <cstddef>
#include <cstdint>
#include <memory>

#include "types.hpp"

namespace forge {

struct KVCacheConfig {
    uint32_t n_layers = 24;
    uint32_t n_kv_heads = 4;
    uint32_t head_dim = 64;
    uint32_t sink_size = 4;
    uint32_t window_size = 8192;
    uint32_t pool_block = 64;
    uint32_t max_context = 131072;
};

class KVCache {
public:
    explicit KVCache(const KVCacheConfig& cfg);
    ~KVCache();
    KVCache(const KVCache&) = delete;
    KVCache& operator=(const KVCache&) = delete;

    void store(uint32_t layer, uint32_t head, uint32_t pos, const float* key, const float* value);
    // Returns the number of scores written.
    uint32_t attention_scores(uint32_t layer, uint32_t head, const float* query, float* scores_out);
    void attention_weighted_sum(uint32_t layer, uint32_t head, const float* scores, float* output, uint32_t count);

    uint32_t size() const;
    void clear();
    size_t memory_usage() const;

private:
    struct Device;
    KVCacheConfig cfg_;
    std::unique_ptr<Device> dev_;
};

}  // namespace forge
#endif
