"""Engine-level parity of the gfx950 path against the oracle: forward
passes (token by token and batched, across window eviction and pooling),
MTP heads, and whole generate() token streams, bit-exact."""
import numpy as np
import pytest

import oracle as O
import pocketforge_amd as pf
from pocketforge_amd import weights as W

pytestmark = pytest.mark.gpu

KV = dict(sink_size=4, window_size=64, pool_block=6, max_context=512)


def _oracle(cfg, w, kv=KV):
    c = dict(cfg)
    c.update(kv)
    return O.Model(c, w)


def test_forward_token_by_token(tiny_weights, tiny_engine):
    cfg, w = tiny_weights
    om = _oracle(cfg, w)
    toks = W.prompt_ids(12, cfg["n_vocab"], seed=3)
    for t in toks:
        lg, hg = tiny_engine.forward([t])
        lo, ho = om.forward(t)
        np.testing.assert_array_equal(hg[0], ho)
        np.testing.assert_array_equal(lg[0], lo)
    om.close()


@pytest.mark.parametrize("chunks", [[8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8],
                                    [5, 1, 5, 1, 5, 1, 7, 3, 8, 2, 5, 5, 5, 5, 5, 5, 5, 5, 5, 5, 5, 5]])
def test_batched_passes_across_eviction_and_pooling(tiny_weights, tiny_engine, chunks):
    """Rows of a pass equal sequential forwards, past the window (64) with
    pooled blocks of 6 and 4 sink rows."""
    cfg, w = tiny_weights
    om = _oracle(cfg, w)
    n = sum(chunks)
    toks = W.prompt_ids(n, cfg["n_vocab"], seed=11)
    i = 0
    for c in chunks:
        lg, hg = tiny_engine.forward(toks[i:i + c])
        for j in range(c):
            lo, ho = om.forward(toks[i + j])
            np.testing.assert_array_equal(hg[j], ho, err_msg=f"row {i + j}")
            np.testing.assert_array_equal(lg[j], lo, err_msg=f"row {i + j}")
        i += c
    assert tiny_engine.pos == n
    om.close()


def test_mtp_forward(tiny_weights, tiny_engine):
    cfg, w = tiny_weights
    om = _oracle(cfg, w)
    rng = np.random.default_rng(4)
    h = rng.standard_normal(cfg["n_embd"]).astype(np.float32)
    np.testing.assert_array_equal(tiny_engine.mtp_forward(h), om.mtp_forward(h))
    om.close()


def _zero_mats(w, layers=True, mtp=True, scale=0.0, seed=0):
    """Copy of a weight set with zeroed (or tiny random) matrices."""
    import copy
    w2 = copy.deepcopy(w)
    rng = np.random.default_rng(seed)
    if layers:
        for lw in w2["layers"]:
            for n in W.NAMES:
                fmt, codes, scales = lw[n]
                if scale == 0.0:
                    codes = np.full_like(codes, 0x88 if fmt == pf.FMT_Q4 else (0xAA if fmt == pf.FMT_Q2 else 0x55))
                    scales = np.zeros_like(scales)
                else:
                    r, nb, _ = codes.shape
                    x = (rng.standard_normal((r, nb * 32)) * scale).astype(np.float32)
                    codes, scales = pf.quantize_matrix(x, fmt)
                lw[n] = (fmt, codes, scales)
    if mtp:
        for hw in w2["mtp"]:
            for n in ("gate", "up", "down"):
                fmt, codes, scales = hw[n]
                hw[n] = (fmt, np.full_like(codes, 0x88), np.zeros_like(scales))
    return w2


GREEDY = pf.Sampling(0.8, 0.95, 40, 1)
TOP_P = pf.Sampling(0.8, 0.95, 40, 0)
TEMP = pf.Sampling(1.1, 1.0, 0, 0)
TOP_K = pf.Sampling(0.9, 1.0, 12, 0)


def _gen_both(gpu, cfg, w, prompt, max_new, samp, kv=KV, seed=7):
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **kv)
    toks, res = e.generate(prompt, max_new, samp, seed)
    om = _oracle(cfg, w, kv)
    ot, oa, orj = om.generate(prompt, max_new, O.Sampling(samp.temperature, samp.top_p, samp.top_k, samp.greedy),
                              seed)
    om.close()
    e.close()
    m.close()
    return toks, res, ot, oa, orj


@pytest.mark.parametrize("case", ["random", "full_accept", "mixed"])
def test_generate_greedy_matches_oracle(gpu, tiny_weights, case):
    cfg, w = tiny_weights
    if case == "full_accept":
        w = _zero_mats(w)                         # the model repeats its input: every draft is accepted
    elif case == "mixed":
        w = _zero_mats(w, scale=0.004, seed=5)    # mostly repeats: accept/reject mix
    prompt = W.prompt_ids(20, cfg["n_vocab"], seed=9)
    toks, res, ot, oa, orj = _gen_both(gpu, cfg, w, prompt, 70, GREEDY)
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)
    if case == "full_accept":
        assert oa > 40
    if case == "mixed":
        print("mixed: accepted", oa, "rejected", orj)


@pytest.mark.parametrize("case", ["full_accept", "mixed", "random"])
@pytest.mark.parametrize("full", [0, 1])
def test_generate_verify_segments(gpu, tiny_weights, case, full):
    """Both verify policies give the oracle's stream: every draft in one
    pass, or a one-row first segment after a round with no accepted draft,
    continued by a second segment when that draft is accepted (the full
    acceptance case starts that way: its first round accepts everything
    through the continuation and hands F(cur) to the next round)."""
    cfg, w = tiny_weights
    if case == "full_accept":
        w = _zero_mats(w)
    elif case == "mixed":
        w = _zero_mats(w, scale=0.004, seed=5)
    prompt = W.prompt_ids(20, cfg["n_vocab"], seed=9)
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **KV)
    e.set_verify_full(full)
    toks, res = e.generate(prompt, 70, GREEDY, 7)
    om = _oracle(cfg, w, KV)
    ot, oa, orj = om.generate(prompt, 70, O.Sampling(0.8, 0.95, 40, 1), 7)
    om.close()
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)
    # passes: one base pass per round without a reused row, one verify
    # segment per round, one more for every continued round, and the
    # single-token steps of the last tokens (n + 4 > N)
    assert res.passes >= res.rounds
    if full:
        assert res.passes <= 2 * res.rounds + 4
    e.close()
    m.close()


@pytest.mark.parametrize("samp,std", [(TOP_P, 0.15), (TEMP, 0.18)], ids=["top_p", "temperature"])
@pytest.mark.parametrize("full", [0, 1])
def test_generate_verify_segments_stochastic(gpu, tiny_weights, samp, std, full):
    """Stochastic sampling through both verify policies, on weights whose
    drafts are accepted often but not always: every layer and head matrix
    zero and an embedding of std 0.15 / 0.18, so that a token's logits peak
    at the token itself (the oracle accepts 23 and rejects 17 drafts with
    top-p, 28 and 13 with temperature sampling).  Under the default policy a
    round after one with no accepted draft verifies d0 alone; when d0 is
    accepted the round continues with a second segment, and a draft
    rejected there takes its corrective from that segment's row
    (k_sample reads row round_acc of the verify logits)."""
    cfg, _ = tiny_weights
    w = _zero_mats(W.make_weights(cfg, seed=31, std=std))
    prompt = W.prompt_ids(12, cfg["n_vocab"], seed=4)
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **KV)
    e.set_verify_full(full)
    toks, res = e.generate(prompt, 60, samp, 99)
    om = _oracle(cfg, w, KV)
    ot, oa, orj = om.generate(prompt, 60, O.Sampling(samp.temperature, samp.top_p, samp.top_k, samp.greedy), 99)
    om.close()
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)
    assert oa > 10 and orj > 10
    if full:
        assert res.continued == 0
    else:
        assert res.continued > 0            # second segments ran
        assert res.passes > res.rounds + res.continued
    e.close()
    m.close()


@pytest.mark.parametrize("samp", [TOP_P, TEMP, TOP_K], ids=["top_p", "temperature", "top_k"])
def test_generate_stochastic_matches_oracle(gpu, tiny_weights, samp):
    cfg, w = tiny_weights
    w = _zero_mats(w, scale=0.004, seed=6)
    prompt = W.prompt_ids(10, cfg["n_vocab"], seed=2)
    toks, res, ot, oa, orj = _gen_both(gpu, cfg, w, prompt, 50, samp, seed=123)
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)


@pytest.mark.parametrize("n_prompt,max_new", [(0, 9), (1, 3), (5, 4), (3, 5), (17, 1)])
def test_generate_edges(gpu, tiny_weights, n_prompt, max_new):
    """Empty prompt (fallback first token), max_new < 4 (fallback only), the
    n+4 <= N gate with its one-token overshoot."""
    cfg, w = tiny_weights
    w = _zero_mats(w, scale=0.004, seed=8)
    prompt = W.prompt_ids(n_prompt, cfg["n_vocab"], seed=1)
    toks, res, ot, oa, orj = _gen_both(gpu, cfg, w, prompt, max_new, GREEDY)
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)


def test_generate_long_context_pooling(gpu, tiny_weights):
    """Window 16 / pool 3 / sink 2 with a 60-token prompt: decode rounds see
    eviction and pooled rows created inside verify passes."""
    cfg, w = tiny_weights
    w = _zero_mats(w, scale=0.004, seed=10)
    kv = dict(sink_size=2, window_size=16, pool_block=3, max_context=256)
    prompt = W.prompt_ids(60, cfg["n_vocab"], seed=5)
    toks, res, ot, oa, orj = _gen_both(gpu, cfg, w, prompt, 60, GREEDY, kv=kv)
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)


def test_oom_guard_stops_generation(gpu, tiny_weights, tiny_engine):
    cfg, _ = tiny_weights
    tiny_engine.set_max_memory(1)
    toks, res = tiny_engine.generate(W.prompt_ids(4, cfg["n_vocab"]), 10, GREEDY)
    assert res.oom_protected == 1 and len(toks) == 4


def test_generate_without_graphs_matches(gpu, tiny_weights, monkeypatch):
    """The kernels issued one by one (profiling path) give the same stream
    as the captured round graphs."""
    cfg, w = tiny_weights
    w = _zero_mats(w, scale=0.004, seed=12)
    prompt = W.prompt_ids(9, cfg["n_vocab"], seed=4)
    monkeypatch.setenv("PF_NO_GRAPHS", "1")
    toks, res, ot, oa, orj = _gen_both(gpu, cfg, w, prompt, 33, GREEDY)
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)


@pytest.mark.parametrize("overlap", ["1", "0"])
@pytest.mark.parametrize("graphs", ["1", "0"])
def test_generate_mtp_overlap(gpu, tiny_weights, monkeypatch, overlap, graphs):
    """The MTP head chain and the drafts' sampling on a second stream beside
    a one-row verify segment (PF_MTP_OVERLAP=1, the default) or after it
    (0), replayed from graphs or issued one by one: with top-p sampling and
    drafts both accepted and rejected, the draws, tokens and counters equal
    the oracle's."""
    cfg, _ = tiny_weights
    w = _zero_mats(W.make_weights(cfg, seed=31, std=0.15))
    monkeypatch.setenv("PF_MTP_OVERLAP", overlap)
    if graphs == "0":
        monkeypatch.setenv("PF_NO_GRAPHS", "1")
    prompt = W.prompt_ids(12, cfg["n_vocab"], seed=4)
    toks, res, ot, oa, orj = _gen_both(gpu, cfg, w, prompt, 60, TOP_P, seed=99)
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)
    assert oa > 10 and orj > 10


def test_profiled_generate_matches(gpu, tiny_weights):
    cfg, w = tiny_weights
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **KV)
    prompt = W.prompt_ids(12, cfg["n_vocab"], seed=8)
    t1, _ = e.generate(prompt, 20, GREEDY)
    e.reset()
    e.profile(True)
    t2, _ = e.generate(prompt, 20, GREEDY)
    n, us, by = e.gemv_stats()
    np.testing.assert_array_equal(t1, t2)
    assert n > 0 and us > 0 and by > 0
    e.close()
    m.close()


def test_multi_chunk_attention_with_pooling(gpu, tiny_weights):
    """Lists longer than one 256-entry attention chunk (window 600, pool 8,
    sink 4): prefill of 900 tokens in passes of 8, then single-row and
    5-row passes whose lists hold 3 chunks with pooled rows; every row's
    logits and hidden state bit-exact."""
    cfg, w = tiny_weights
    kv = dict(sink_size=4, window_size=600, pool_block=8, max_context=2048)
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **kv)
    om = _oracle(cfg, w, kv)
    toks = W.prompt_ids(920, cfg["n_vocab"], seed=21)
    i = 0
    for c in [8] * 112 + [1, 5, 3, 1]:
        lg, hg = e.forward(toks[i:i + c])
        for j in range(c):
            lo, ho = om.forward(toks[i + j])
            if i + j >= 250 and (i + j) % 37 == 0 or i + c > 890:
                np.testing.assert_array_equal(hg[j], ho, err_msg=f"row {i + j}")
                np.testing.assert_array_equal(lg[j], lo, err_msg=f"row {i + j}")
        i += c
    om.close()
    e.close()
    m.close()


def test_generate_multi_chunk_matches_oracle(gpu, tiny_weights):
    """generate() with a 700-token prompt under window 600 / pool 8: MTP
    rounds over 3-chunk attention lists, token streams identical."""
    cfg, w = tiny_weights
    kv = dict(sink_size=4, window_size=600, pool_block=8, max_context=2048)
    prompt = W.prompt_ids(700, cfg["n_vocab"], seed=13)
    toks, res, ot, oa, orj = _gen_both(gpu, cfg, w, prompt, 40, GREEDY, kv=kv)
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)


@pytest.mark.parametrize("samp", [GREEDY, TOP_P], ids=["greedy", "top_p"])
def test_generate_mtp_disabled(gpu, tiny_weights, samp):
    """Engine::set_mtp_enabled(false): the single-token loop only
    (src/engine.cpp:304, 367-386), equal to an oracle engine without heads."""
    cfg, w = tiny_weights
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **KV)
    e.set_mtp_enabled(False)
    prompt = W.prompt_ids(11, cfg["n_vocab"], seed=6)
    toks, res = e.generate(prompt, 30, samp, 9)
    c = dict(cfg)
    c["n_mtp"] = 0
    om = _oracle(c, w)
    ot, oa, orj = om.generate(prompt, 30, O.Sampling(samp.temperature, samp.top_p, samp.top_k, samp.greedy), 9)
    np.testing.assert_array_equal(toks, ot)
    assert res.rounds == 0 and res.mtp_accepted == 0 and (oa, orj) == (0, 0)
    e.set_mtp_enabled(True)
    toks2, res2 = e.generate(prompt, 30, samp, 9)
    assert res2.rounds > 0
    om.close()
    e.close()
    m.close()


@pytest.mark.parametrize("kv,n,chunk", [(dict(sink_size=4, window_size=64, pool_block=6, max_context=512), 200, 64),
                                        (dict(sink_size=4, window_size=600, pool_block=8, max_context=2048), 700, 256),
                                        (dict(sink_size=4, window_size=600, pool_block=8, max_context=2048), 300, 37)])
def test_batched_prefill_equals_token_by_token(gpu, tiny_weights, kv, n, chunk):
    """Prompt passes of up to 256 rows (int8 MFMA GEMMs, one window at
    most) leave the cache and state exactly as n single-token forwards: the
    next forward's logits and hidden state are bit-identical to the oracle's."""
    cfg, w = tiny_weights
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **kv)
    om = _oracle(cfg, w, kv)
    toks = W.prompt_ids(n + 1, cfg["n_vocab"], seed=31)
    for i in range(0, n, chunk):
        e.prefill(toks[i:min(i + chunk, n)])
    for t in toks[:n]:
        om.forward(t)
    assert e.pos == n
    lg, hg = e.forward(toks[n:n + 1])
    lo, ho = om.forward(toks[n])
    np.testing.assert_array_equal(hg[0], ho)
    np.testing.assert_array_equal(lg[0], lo)
    om.close()
    e.close()
    m.close()
