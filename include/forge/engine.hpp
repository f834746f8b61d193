// The decode engine (include/forge/engine.hpp:15-74) on one MI355X: model
// weights, KV cache, MTP heads and the decode rounds live in HBM; the
// methods below keep the reference's signatures.
#ifndef FORGE_ENGINE_HPP
#define FORGE_ENGINE_HPP

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "kv_cache.hpp"
#include "mtp.hpp"
#include "types.hpp"

namespace forge {

class Engine {
public:
    Engine();
    ~Engine();
    Engine(const Engine&) = delete;
    Engine& operator=(const Engine&) = delete;

    // Reads a .squeeze file (src/quant_format.cpp:231-425 format): Q4, Q2 and
    // Q1.5 layer matrices, norms and the Q4 tied embedding go to the device;
    // the MTP heads (absent from the format) are the seeded synthetic ones.
    // Returns false when the file is missing, malformed or holds a matrix type
    // without a device format (Q8 layer matrices).
    bool load_model(const std::string& squeezef_path);
    // This build's loader: seeded N(0, 0.02) weights (Philox4x32-10 +
    // Box-Muller, stream = matrix id), block-quantized, RMSNorm weights 1,
    // a Q4 tied embedding and cfg.mtp_heads Q4 heads.  MHA only
    // (n_kv_heads = n_heads), head_dim 64 or 128.
    bool load_random_model(const ModelConfig& cfg, uint64_t seed = 1234, const WeightFormats& formats = {});

    void set_max_context(uint32_t tokens);
    void set_mtp_enabled(bool enabled);
    void set_layer_skip_threshold(float threshold);
    void set_max_memory(size_t bytes);

    // With the reference's default SamplingConfig.
    GenerationResult generate(const std::vector<int32_t>& prompt_tokens, uint32_t max_new_tokens,
                              TokenCallback callback = nullptr, ProgressCallback progress = nullptr);
    // The same with an explicit sampling configuration and seed.
    GenerationResult generate(const std::vector<int32_t>& prompt_tokens, uint32_t max_new_tokens,
                              const SamplingConfig& sampling, uint64_t seed = 42, TokenCallback callback = nullptr,
                              ProgressCallback progress = nullptr);

    std::vector<float> forward(const std::vector<int32_t>& tokens);
    std::vector<float> forward_with_hidden(const std::vector<int32_t>& tokens, std::vector<float>& hidden_out);

    // src/engine.cpp:402-448: drafts from the MTP heads on hidden_state,
    // verified one token at a time with greedy argmax.  Returns (accepted,
    // logits of the rejecting forward, or empty when all were accepted).  As
    // in the reference, mtp_accepted_out stays 0 on a rejection and
    // mtp_rejected_out = heads - accepted.  The heads use the engine's tied
    // table (embedding_table is only tested for emptiness: empty means one
    // plain forward, like a model without heads); a hidden_state shorter than
    // n_embd throws std::invalid_argument.
    std::pair<int, std::vector<float>> step_mtp(int32_t current_token, const std::vector<float>& hidden_state,
                                                const std::vector<float>& embedding_table, int& mtp_accepted_out,
                                                int& mtp_rejected_out);

    int32_t sample(const float* logits, uint32_t n_vocab, const SamplingConfig& cfg = SamplingConfig());
    int32_t sample_greedy(const float* logits, uint32_t n_vocab);
    int32_t sample_top_k(const float* logits, uint32_t n_vocab, uint32_t k, float temp);
    int32_t sample_top_p(const float* logits, uint32_t n_vocab, float p, float temp);

    struct MemoryStats {
        size_t weights_mmap = 0;
        size_t weights_decompressed = 0;
        size_t kv_cache = 0;
        size_t activations = 0;
        size_t prefetch_buffer = 0;
        size_t mtp_heads = 0;
        size_t other = 0;
        size_t total() const;
    };
    MemoryStats get_memory_stats() const;

    const ModelConfig& config() const { return config_; }

    // GGUF reading is not part of this build: returns false.
    bool load_norm_weights_from_gguf(const std::string& gguf_path);

private:
    struct Device;
    ModelConfig config_;
    std::unique_ptr<Device> dev_;
    bool rebuild_engine();
};

}  // namespace forge
#endif
