// Multi-token-prediction heads (include/forge/mtp.hpp:23-53) on the GPU:
// n_mtp_heads chained heads of n_embd x n_embd Q4 gate/up/down (mtp_ff_dim
// must equal n_embd, as the engine builds them, src/engine.cpp:79), tied
// fp32 unembedding.
#ifndef FORGE_MTP_HPP
#define FORGE_MTP_HPP

#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

#include "types.hpp"

namespace forge {

struct MTPConfig {
    uint32_t n_mtp_heads = 4;
    uint32_t n_embd = 2048;
    uint32_t n_vocab = 32000;
    uint32_t mtp_ff_dim = 2048;
};

class MTPHeads {
public:
    explicit MTPHeads(const MTPConfig& cfg);
    ~MTPHeads();
    MTPHeads(const MTPHeads&) = delete;
    MTPHeads& operator=(const MTPHeads&) = delete;

    // N(0, 0.02) weights in Q4 blocks, a new draw per call.
    void init_weights();
    // This build's extension: load head `head`'s matrix which (0 gate, 1 up,
    // 2 down) from interchange Q4 codes [n_embd][n_embd/32][16] and fp16
    // block scales [n_embd][n_embd/32].
    void set_head_weights(uint32_t head, int which, const uint8_t* codes, const uint16_t* scales);

    // Per head: logits [n_vocab] from the chained hidden state; with an
    // embedding_table smaller than n_vocab * n_embd, the reference's
    // placeholder logits.
    std::vector<std::vector<float>> forward(const float* hidden, const std::vector<float>& embedding_table) const;

    int speculative_accept(int32_t token, const std::vector<std::vector<float>>& mtp_logits) const;
    static int32_t argmax(const float* logits, uint32_t n);
    size_t memory_usage() const;

private:
    struct Device;
    MTPConfig cfg_;
    uint32_t draws_ = 0;
    std::unique_ptr<Device> dev_;
};

}  // namespace forge
#endif
