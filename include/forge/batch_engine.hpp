// Many independent sequences decoded together on one MI355X over one
// model.  No counterpart in the reference, which serves every request with
// its own Engine::generate call (src/forge_server.cpp:280, 398 call
// include/forge/engine.hpp:27-32 once per request).  A caller switches by
// handing the prompts of concurrent requests to one generate call: each
// sequence's result is exactly the result Engine::generate gives for that
// prompt and seed, while every forward pass covers all the sequences.
#ifndef FORGE_BATCH_ENGINE_HPP
#define FORGE_BATCH_ENGINE_HPP

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "types.hpp"

namespace forge {

// Called after generate with each generated token of each sequence, in order.
using BatchTokenCallback = std::function<void(uint32_t sequence, int32_t token)>;

class BatchEngine {
public:
    // n_sequences * (mtp_heads + 1) <= 512 (one verify pass holds every
    // sequence's rows).
    explicit BatchEngine(uint32_t n_sequences);
    ~BatchEngine();
    BatchEngine(const BatchEngine&) = delete;
    BatchEngine& operator=(const BatchEngine&) = delete;

    // The loaders of forge::Engine: a .squeeze file, or the seeded synthetic
    // weights (the same streams as Engine::load_random_model).
    bool load_model(const std::string& squeezef_path);
    bool load_random_model(const ModelConfig& cfg, uint64_t seed = 1234, const WeightFormats& formats = {});

    // As Engine::set_max_context / set_mtp_enabled, for every sequence.
    void set_max_context(uint32_t tokens);
    void set_mtp_enabled(bool enabled);

    uint32_t sequences() const { return n_seq_; }
    // Tokens sequence `seq` has forwarded (its next position).
    uint32_t position(uint32_t seq) const;
    // Clears every sequence's KV cache and position.
    void reset();

    // Engine::generate (src/engine.cpp:276-396) for every sequence at once:
    // prompts.size() == sequences(), seeds[i] the seed of sequence i (empty:
    // 42 for all, Engine::generate's default).  Like Engine::generate, each
    // sequence continues from its current state (its cache is not cleared).
    // Result i holds sequence i's prompt and generated tokens.
    std::vector<GenerationResult> generate(const std::vector<std::vector<int32_t>>& prompts,
                                           uint32_t max_new_tokens, const SamplingConfig& sampling = SamplingConfig(),
                                           const std::vector<uint64_t>& seeds = {},
                                           BatchTokenCallback callback = nullptr);

    const ModelConfig& config() const { return config_; }

private:
    struct Device;
    ModelConfig config_;
    uint32_t n_seq_;
    std::unique_ptr<Device> dev_;
    bool rebuild_engine();
};

}  // namespace forge
#endif
