// forge::Engine on the GPU: the reference's checks (tests/test_engine.cpp,
// with this build's synthetic loader in place of the .squeeze file) plus
// parity with the oracle engine on the same weights: forward logits bit for
// bit, greedy and top-p token streams, MTP counters, step_mtp and the
// MTP-disabled loop.
#include <cstdlib>
#include <cstring>
#include <vector>

#include "forge/engine.hpp"
#include "forge_test.hpp"
#include "pf_gpu.h"
#include "pf_oracle.h"

// The synthetic weights of Engine::load_random_model, regenerated for the
// oracle: layer l matrix j -> stream 16 l + j, embedding 0x10000, MTP head k
// matrix j -> 0x20000 + 3 k + j.
struct OracleModel {
    std::vector<std::vector<uint8_t>> codes;
    std::vector<std::vector<uint16_t>> scales;
    std::vector<orc_qmat> layers, mtp;
    orc_qmat emb{};
    std::vector<float> ones;
    orc_model_desc desc{};

    orc_qmat gen(uint64_t seed, uint32_t stream, uint32_t rows, uint32_t cols) {
        codes.emplace_back((size_t)rows * (cols / 32) * 16);
        scales.emplace_back((size_t)rows * (cols / 32));
        pf_gen_matrix(seed, stream, 0.02f, rows, cols, PF_FMT_Q4, codes.back().data(), scales.back().data());
        return orc_qmat{ORC_Q4, rows, cols, codes.back().data(), scales.back().data()};
    }

    OracleModel(const forge::ModelConfig& c, uint64_t seed, uint32_t n_mtp) {
        codes.reserve(1024);
        scales.reserve(1024);
        const uint32_t D = c.n_embd, F = c.n_ff;
        const uint32_t rows[7] = {D, D, D, D, F, F, D}, cols[7] = {D, D, D, D, D, D, F};
        for (uint32_t l = 0; l < c.n_layers; l++)
            for (uint32_t j = 0; j < 7; j++) layers.push_back(gen(seed, l * 16 + j, rows[j], cols[j]));
        emb = gen(seed, 0x10000, c.n_vocab, D);
        for (uint32_t k = 0; k < c.mtp_heads; k++)
            for (uint32_t j = 0; j < 3; j++) mtp.push_back(gen(seed, 0x20000 + 3 * k + j, D, D));
        ones.assign((size_t)c.n_layers * D, 1.0f);
        desc = orc_model_desc{c.n_layers, D, c.n_heads, c.head_dim(), F, c.n_vocab, n_mtp, 4,
                              std::min(c.kv_cache_size, 8192u), 64, c.max_seq_len,
                              layers.data(), &emb, mtp.data(), ones.data(), ones.data()};
    }
};

int run() {
    std::cout << "forge Engine on the GPU\n";
    forge::ModelConfig cfg;
    cfg.n_layers = 2;
    cfg.n_embd = 256;
    cfg.n_heads = 4;
    cfg.n_kv_heads = 4;
    cfg.head_dim_ = 64;
    cfg.n_ff = 512;
    cfg.n_vocab = 1024;
    cfg.max_seq_len = 512;
    cfg.kv_cache_size = 64;
    cfg.mtp_heads = 4;
    forge::Engine engine;
    CHECK("a missing .squeeze file does not load", !engine.load_model("/nonexistent.squeeze"));
    if (const char* sq = std::getenv("PF_TEST_SQUEEZE")) {
        // a file in the reference's .squeeze format (written by the test driver)
        forge::Engine fe;
        CHECK(".squeeze model loads", fe.load_model(sq));
        CHECK(".squeeze config layers", fe.config().n_layers == 2 && fe.config().n_embd == 256);
        CHECK(".squeeze config vocab and heads", fe.config().n_vocab == 1024 && fe.config().mtp_heads == 4);
        std::vector<int32_t> prompt = {5, 6, 7};
        auto r = fe.generate(prompt, 12, nullptr, nullptr);
        CHECK(".squeeze model generates", r.tokens.size() == prompt.size() + 12);
    }
    CHECK("engine loads a synthetic model", engine.load_random_model(cfg, 1234));
    CHECK("config matches layers", engine.config().n_layers == cfg.n_layers);
    CHECK("config matches embd", engine.config().n_embd == cfg.n_embd);
    {
        std::vector<int32_t> prompt = {101, 102, 103};
        int calls = 0;
        auto r = engine.generate(prompt, 10, [&](int32_t, float) { calls++; }, nullptr);
        CHECK("generated tokens returned", !r.tokens.empty());
        CHECK("generation tps > 0", r.tokens_per_second > 0);
        CHECK("peak memory tracked", r.peak_memory_bytes > 0);
        CHECK("includes prompt tokens", r.tokens.size() >= prompt.size() &&
                                            std::equal(prompt.begin(), prompt.end(), r.tokens.begin()));
        CHECK("callback sees every generated token", calls == (int)(r.tokens.size() - prompt.size()));
    }
    {
        auto logits = engine.forward({42});
        CHECK("forward returns logits", logits.size() == cfg.n_vocab);
        bool fin = true;
        for (float x : logits) fin = fin && std::isfinite(x);
        CHECK("logits finite", fin);
    }
    {
        auto stats = engine.get_memory_stats();
        CHECK("memory stats total > 0", stats.total() > 0);
        CHECK("KV cache tracked", stats.kv_cache > 0);
        CHECK("activations tracked", stats.activations > 0);
    }
    // parity with the oracle on fresh engines
    OracleModel om(cfg, 1234, cfg.mtp_heads);
    {
        forge::Engine e;
        e.load_random_model(cfg, 1234);
        orc_engine* o = orc_engine_create(&om.desc);
        std::vector<float> lo(cfg.n_vocab), ho(cfg.n_embd), hid;
        bool same = true;
        const int32_t toks[12] = {5, 900, 17, 3, 1023, 44, 8, 8, 600, 71, 2, 250};
        for (int i = 0; i < 12; i++) {
            auto lg = e.forward_with_hidden({toks[i]}, hid);
            orc_forward(o, toks[i], lo.data(), ho.data());
            same = same && lg == lo && hid == ho;
        }
        CHECK("forward logits and hidden equal the oracle (12 tokens)", same);
        // step_mtp (src/engine.cpp:402-448) on the last hidden state, against
        // the oracle's restatement on the same state: default sampling
        // (top-p), seed 42, the engine's draw counter (0: only forwards ran)
        const forge::SamplingConfig dflt;
        const orc_sampling os{dflt.temperature, dflt.top_p, dflt.top_k, 0};
        uint64_t draw = 0;
        for (int round = 0; round < 3; round++) {
            int acc = -1, rej = -1;
            std::vector<float> table(1, 0.0f);
            const int32_t tok = 7 + 100 * round;
            auto st = e.step_mtp(tok, hid, table, acc, rej);
            std::vector<float> ol(cfg.n_vocab);
            uint32_t nl = 0;
            int32_t oacc = -1, orej = -1;
            const int32_t ok = orc_step_mtp(o, tok, hid.data(), 1, &os, 42, &draw, ol.data(), &nl, &oacc, &orej);
            ol.resize(nl);
            CHECK("step_mtp (accepted, counters, logits) equal the oracle",
                  st.first == ok && acc == oacc && rej == orej && st.second == ol);
            e.forward_with_hidden({tok}, hid);
            orc_forward(o, tok, lo.data(), ho.data());
            CHECK("forward after step_mtp equals the oracle", hid == ho);
        }
        int acc2 = -1, rej2 = -1;
        auto st2 = e.step_mtp(7, hid, {}, acc2, rej2);
        uint32_t nl = 0;
        int32_t oacc = -1, orej = -1;
        std::vector<float> ol(cfg.n_vocab);
        orc_step_mtp(o, 7, hid.data(), 0, &os, 42, &draw, ol.data(), &nl, &oacc, &orej);
        CHECK("step_mtp without a table forwards the token",
              st2.first == 0 && acc2 == 0 && rej2 == 0 && nl == cfg.n_vocab && st2.second == ol);
        orc_engine_destroy(o);
    }
    for (int greedy = 1; greedy >= 0; greedy--) {
        forge::Engine e;
        e.load_random_model(cfg, 1234);
        orc_engine* o = orc_engine_create(&om.desc);
        forge::SamplingConfig sc;
        sc.greedy = greedy != 0;
        std::vector<int32_t> prompt = {3, 14, 15, 92, 65, 35, 89, 79, 32, 38};
        auto r = e.generate(prompt, 60, sc, 7);
        std::vector<int32_t> ot(prompt.size() + 80);
        uint32_t n = 0;
        int32_t oa = 0, orj = 0;
        orc_sampling os{sc.temperature, sc.top_p, sc.top_k, sc.greedy ? 1 : 0};
        orc_generate(o, prompt.data(), (uint32_t)prompt.size(), 60, &os, 7, ot.data(), (uint32_t)ot.size(), &n, &oa,
                     &orj);
        ot.resize(n);
        CHECK(greedy ? "greedy stream equals the oracle" : "top-p stream equals the oracle", r.tokens == ot);
        CHECK("MTP counters equal the oracle", r.mtp_accepted == oa && r.mtp_rejected == orj);
        orc_engine_destroy(o);
    }
    {
        forge::Engine e;
        e.load_random_model(cfg, 1234);
        e.set_mtp_enabled(false);
        OracleModel plain(cfg, 1234, 0);
        orc_engine* o = orc_engine_create(&plain.desc);
        forge::SamplingConfig sc;
        sc.greedy = true;
        std::vector<int32_t> prompt = {1, 2, 3};
        auto r = e.generate(prompt, 20, sc, 7);
        std::vector<int32_t> ot(64);
        uint32_t n = 0;
        int32_t oa = 0, orj = 0;
        orc_sampling os{sc.temperature, sc.top_p, sc.top_k, 1};
        orc_generate(o, prompt.data(), 3, 20, &os, 7, ot.data(), 64, &n, &oa, &orj);
        ot.resize(n);
        CHECK("MTP disabled: single-token loop equals the oracle", r.tokens == ot && r.mtp_accepted == 0);
        e.set_layer_skip_threshold(0.5f);
        CHECK("layer-skip threshold kept", e.config().skip_threshold == 0.5f);
        orc_engine_destroy(o);
    }
    return finish("test_forge_engine");
}
