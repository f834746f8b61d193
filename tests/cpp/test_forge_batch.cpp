// forge::BatchEngine on the GPU: every sequence's result equals what
// forge::Engine::generate gives for the same prompt and seed (tokens and
// MTP counters), for greedy and top-p sampling, across two generate calls
// that continue each sequence's state, and for a single sequence.
#include <vector>

#include "forge/batch_engine.hpp"
#include "forge/engine.hpp"
#include "forge_test.hpp"

static std::vector<int32_t> prompt_of(uint32_t n, uint32_t salt, uint32_t vocab) {
    std::vector<int32_t> p(n);
    for (uint32_t i = 0; i < n; i++) p[i] = (int32_t)((i * 2654435761u + salt * 40503u + 11u) % vocab);
    return p;
}

static bool same(const forge::GenerationResult& a, const forge::GenerationResult& b) {
    return a.tokens == b.tokens && a.mtp_accepted == b.mtp_accepted && a.mtp_rejected == b.mtp_rejected;
}

int run() {
    std::cout << "forge BatchEngine on the GPU\n";
    forge::ModelConfig cfg;
    cfg.n_layers = 2;
    cfg.n_embd = 256;
    cfg.n_heads = 4;
    cfg.n_kv_heads = 4;
    cfg.head_dim_ = 64;
    cfg.n_ff = 512;
    cfg.n_vocab = 1024;
    cfg.max_seq_len = 512;
    cfg.kv_cache_size = 64;           // a short window: the long prompt evicts and pools
    const uint32_t S = 5;
    const std::vector<uint32_t> lens = {17, 150, 1, 40, 9};
    const std::vector<uint64_t> seeds = {3, 1, 4, 1, 5};

    forge::BatchEngine b(S);
    CHECK("load_random_model", b.load_random_model(cfg, 7));
    CHECK("sequences", b.sequences() == S);

    forge::SamplingConfig greedy;
    greedy.greedy = true;
    forge::SamplingConfig top_p;   // the reference's defaults: temperature 0.8, top-p 0.95

    std::vector<std::vector<int32_t>> prompts(S), more(S);
    for (uint32_t i = 0; i < S; i++) {
        prompts[i] = prompt_of(lens[i], i, cfg.n_vocab);
        more[i] = prompt_of(3 + i, 100 + i, cfg.n_vocab);
    }
    std::vector<std::vector<int32_t>> cb(S);
    auto r1 = b.generate(prompts, 24, greedy, seeds,
                         [&](uint32_t s, int32_t t) { cb[s].push_back(t); });
    auto r2 = b.generate(more, 16, top_p, seeds);
    CHECK("one result per sequence", r1.size() == S && r2.size() == S);
    for (uint32_t i = 0; i < S; i++) {
        forge::Engine e;
        e.load_random_model(cfg, 7);
        const auto w1 = e.generate(prompts[i], 24, greedy, seeds[i]);
        const auto w2 = e.generate(more[i], 16, top_p, seeds[i]);
        CHECK("greedy sequence " + std::to_string(i) + " equals Engine::generate", same(r1[i], w1));
        CHECK("top-p continuation " + std::to_string(i) + " equals Engine::generate", same(r2[i], w2));
        CHECK("callback tokens " + std::to_string(i),
              cb[i] == std::vector<int32_t>(r1[i].tokens.begin() + lens[i], r1[i].tokens.end()));
        CHECK("position " + std::to_string(i),
              b.position(i) > lens[i] + 3 + i && b.position(i) <= lens[i] + 3 + i + 24 + 16 + 8);
    }
    b.reset();
    CHECK("reset clears positions", b.position(0) == 0 && b.position(S - 1) == 0);

    forge::BatchEngine one(1);
    one.load_random_model(cfg, 7);
    forge::Engine e;
    e.load_random_model(cfg, 7);
    CHECK("one sequence equals Engine::generate (default seed)",
          same(one.generate({prompts[1]}, 20, top_p)[0], e.generate(prompts[1], 20, top_p, 42)));
    bool threw = false;
    try {
        one.generate({prompts[0], prompts[1]}, 4);
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    CHECK("prompt count must match", threw);
    return finish("test_forge_batch");
}
