// forge::MTPHeads on the GPU: the reference's checks (tests/test_mtp.cpp)
// at a width the device heads support (n_embd a multiple of 256), plus
// bit-exact parity with the oracle for given head weights and table.
#include <random>
#include <vector>

#include "forge/mtp.hpp"
#include "forge_test.hpp"
#include "pf_gpu.h"
#include "pf_oracle.h"

int run() {
    std::cout << "forge MTPHeads on the GPU\n";
    forge::MTPConfig cfg;
    cfg.n_mtp_heads = 4;
    cfg.n_embd = 256;
    cfg.n_vocab = 128;
    cfg.mtp_ff_dim = 256;
    forge::MTPHeads mtp(cfg);
    CHECK("heads initialized", mtp.memory_usage() > 0);
    std::mt19937 g(1);
    std::uniform_real_distribution<float> u(-1.0f, 1.0f);
    std::vector<float> hidden(cfg.n_embd);
    for (auto& x : hidden) x = u(g);
    auto logits = mtp.forward(hidden.data(), {});
    CHECK("one logits row per head", logits.size() == cfg.n_mtp_heads);
    CHECK("head 0 logits cover the vocabulary", logits[0].size() == cfg.n_vocab);
    bool fin = true;
    for (auto& r : logits)
        for (float x : r) fin = fin && std::isfinite(x);
    CHECK("logits finite", fin);
    CHECK("placeholder logits (src/mtp.cpp:117-121)",
          logits[1][5] == (float)((5ull * 2654435761ull + 1ull) % 128) / 128.0f);
    float tl[5] = {-1.0f, 3.0f, 0.5f, -0.2f, 2.0f};
    CHECK("argmax at index 1", forge::MTPHeads::argmax(tl, 5) == 1);
    {
        std::vector<std::vector<float>> t(4, std::vector<float>(cfg.n_vocab, -1.0f));
        t[0][5] = 10.0f;
        t[1][5] = 10.0f;
        t[2][7] = 10.0f;
        t[3][5] = 10.0f;
        CHECK("speculative accept stops at mismatch", mtp.speculative_accept(5, t) == 2);
    }
    std::vector<float> tied((size_t)cfg.n_vocab * cfg.n_embd);
    for (auto& x : tied) x = u(g) * 0.005f;
    auto l1 = mtp.forward(hidden.data(), tied);
    std::vector<float> hidden2(cfg.n_embd, 0.0f);
    auto l2 = mtp.forward(hidden2.data(), tied);
    CHECK("tied embeddings give logits", !l1[0].empty());
    bool diff = false;
    for (uint32_t v = 0; v < cfg.n_vocab; v++) diff = diff || std::fabs(l1[0][v] - l2[0][v]) > 1e-6f;
    CHECK("different hidden gives different logits", diff);
    // given weights: GPU == oracle, bit for bit
    const uint32_t D = cfg.n_embd, nb = D / 32;
    std::vector<std::vector<uint8_t>> codes(12, std::vector<uint8_t>((size_t)D * nb * 16));
    std::vector<std::vector<uint16_t>> scales(12, std::vector<uint16_t>((size_t)D * nb));
    std::vector<orc_qmat> qm(12);
    for (uint32_t i = 0; i < 12; i++) {
        pf_gen_matrix(77, 500 + i, 0.02f, D, D, PF_FMT_Q4, codes[i].data(), scales[i].data());
        mtp.set_head_weights(i / 3, (int)(i % 3), codes[i].data(), scales[i].data());
        qm[i] = orc_qmat{ORC_Q4, D, D, codes[i].data(), scales[i].data()};
    }
    auto got = mtp.forward(hidden.data(), tied);
    std::vector<float> want((size_t)4 * cfg.n_vocab);
    orc_mtp_heads_forward(qm.data(), 4, D, cfg.n_vocab, tied.data(), hidden.data(), want.data());
    bool same = true;
    for (uint32_t h = 0; h < 4; h++)
        for (uint32_t v = 0; v < cfg.n_vocab; v++) same = same && got[h][v] == want[(size_t)h * cfg.n_vocab + v];
    CHECK("forward with given heads equals the oracle", same);
    return finish("test_forge_mtp");
}
