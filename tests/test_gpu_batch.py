"""Multi-sequence engine: every sequence of a batched engine produces
exactly what a single-sequence engine (itself pinned to the oracle) produces
for the same prompt and seed -- forward rows, logits, hidden states, token
streams and acceptance counters, bit-exact -- with passes that mix
sequences at different positions, across window eviction and pooling, on
the GEMV (<= 8 rows) and the MFMA GEMM (> 8 rows) paths."""
import numpy as np
import pytest

import oracle as O
import pocketforge_amd as pf
from pocketforge_amd import weights as W

pytestmark = pytest.mark.gpu

KV = dict(sink_size=4, window_size=64, pool_block=6, max_context=512)
GREEDY = pf.Sampling(0.8, 0.95, 40, 1)
TOP_P = pf.Sampling(0.8, 0.95, 40, 0)
TEMP = pf.Sampling(1.1, 1.0, 0, 0)


def _mix(w, scale, seed):
    """Weights whose model mostly repeats its input (drafts accepted and
    rejected), MTP heads zeroed."""
    import copy
    w2 = copy.deepcopy(w)
    rng = np.random.default_rng(seed)
    for lw in w2["layers"]:
        for n in W.NAMES:
            fmt, codes, scales = lw[n]
            r, nb, _ = codes.shape
            x = (rng.standard_normal((r, nb * 32)) * scale).astype(np.float32)
            codes, scales = pf.quantize_matrix(x, fmt)
            lw[n] = (fmt, codes, scales)
    for hw in w2["mtp"]:
        for n in ("gate", "up", "down"):
            fmt, codes, scales = hw[n]
            hw[n] = (fmt, np.full_like(codes, 0x88), np.zeros_like(scales))
    return w2


def _prefill_all(b, singles, prompts):
    for s, (e, p) in enumerate(zip(singles, prompts)):
        b.prefill_seq(s, p)
        i = 0
        while i < len(p):
            e.prefill(p[i:i + 8])
            i += 8


@pytest.mark.parametrize("n_seq,rows", [(4, 1), (4, 5), (3, 3), (2, 5), (20, 5)])
def test_batch_forward_matches_single_engines(gpu, tiny_weights, n_seq, rows):
    """Sequences at different positions (prompts of 1 to 75 tokens: some
    past the 64-entry window with pooled rows), several batched passes,
    compared row by row with one single-sequence engine per sequence."""
    cfg, w = tiny_weights
    m = pf.Model(gpu, cfg, w)
    b = pf.BatchEngine(m, n_seq, **KV)
    singles = [pf.Engine(m, **KV) for _ in range(n_seq)]
    lens = [(7 + 17 * s) % 76 + 1 for s in range(n_seq)]
    prompts = [W.prompt_ids(n, cfg["n_vocab"], seed=100 + s) for s, n in enumerate(lens)]
    _prefill_all(b, singles, prompts)
    for s in range(n_seq):
        assert b.position(s) == lens[s]
    rng = np.random.default_rng(5)
    for step in range(4):
        # a pass over a subset of the sequences in a scrambled order
        seqs = rng.permutation(n_seq)[: max(1, n_seq - step)]
        toks = rng.integers(0, cfg["n_vocab"], (len(seqs), rows)).astype(np.int32)
        print(f"step {step}: {len(seqs)} sequences x {rows} rows", flush=True)
        lb, hb = b.forward_batch(seqs, toks)
        for i, s in enumerate(seqs):
            ls, hs = singles[s].forward(toks[i])
            np.testing.assert_array_equal(hb[i], hs, err_msg=f"hidden, step {step}, sequence {s}")
            np.testing.assert_array_equal(lb[i], ls, err_msg=f"logits, step {step}, sequence {s}")
    for s in range(n_seq):
        assert b.position(s) == singles[s].pos
    for e in singles:
        e.close()
    b.close()
    m.close()


@pytest.mark.parametrize("which,samp", [("mixed", GREEDY), ("random", GREEDY), ("mixed", TOP_P),
                                        ("mixed", TEMP)], ids=["greedy_mixed", "greedy_random", "top_p", "temp"])
def test_batch_generate_matches_single_engines(gpu, tiny_weights, which, samp):
    """Prompts of 0 to 70 tokens, a seed per sequence; max_new 23 leaves
    sequences at different n_gen, so rounds mix MTP rounds and single-token
    steps (the n + 4 <= N gate) until every sequence is done."""
    cfg, w = tiny_weights
    if which == "mixed":
        w = _mix(w, 0.004, seed=21)
    n_seq = 6
    m = pf.Model(gpu, cfg, w)
    lens = [0, 1, 5, 20, 64, 70]
    prompts = [W.prompt_ids(n, cfg["n_vocab"], seed=200 + s) for s, n in enumerate(lens)]
    seeds = np.arange(n_seq, dtype=np.uint64) * 977 + 3
    b = pf.BatchEngine(m, n_seq, **KV)
    toks_b, res_b = b.generate_batch(prompts, 23, samp, seeds)
    b.close()
    accepted = 0
    for s in range(n_seq):
        print(f"sequence {s}: prompt {lens[s]}", flush=True)
        e = pf.Engine(m, **KV)
        e.set_verify_full(1)      # the batched rounds verify every draft in one pass
        t, r = e.generate(prompts[s], 23, samp, int(seeds[s]))
        e.close()
        np.testing.assert_array_equal(toks_b[s], t, err_msg=f"sequence {s}")
        assert (res_b[s].mtp_accepted, res_b[s].mtp_rejected) == (r.mtp_accepted, r.mtp_rejected)
        assert (res_b[s].rounds, res_b[s].passes, res_b[s].n_tokens) == (r.rounds, r.passes, r.n_tokens)
        accepted += r.mtp_accepted
    if which == "mixed" and samp is GREEDY:
        assert accepted > 0
    m.close()


def test_batch_generate_matches_oracle_wide_mixed(gpu):
    """head_dim 128, Q4 attention / Q2 gate-up / Q1.5 down, 12 sequences
    (verify passes of 60 rows on the MFMA GEMM), two sequences checked
    against the oracle directly, all against single-sequence engines."""
    cfg = dict(n_layers=2, n_embd=512, n_heads=4, head_dim=128, n_ff=1024, n_vocab=1024, n_mtp=4)
    w = _mix(W.make_weights(cfg, seed=77, fmts=W.MIXED), 0.003, seed=4)
    kv = dict(sink_size=4, window_size=32, pool_block=4, max_context=256)
    n_seq = 12
    m = pf.Model(gpu, cfg, w)
    prompts = [W.prompt_ids(10 + 3 * s, cfg["n_vocab"], seed=300 + s) for s in range(n_seq)]
    seeds = np.full(n_seq, 11, np.uint64)
    b = pf.BatchEngine(m, n_seq, **kv)
    toks_b, res_b = b.generate_batch(prompts, 30, GREEDY, seeds)
    b.close()
    c = dict(cfg)
    c.update(kv)
    for s in (0, n_seq - 1):
        om = O.Model(c, w)
        ot, oa, orj = om.generate(prompts[s], 30, O.Sampling(0.8, 0.95, 40, 1), 11)
        om.close()
        np.testing.assert_array_equal(toks_b[s], ot, err_msg=f"sequence {s} vs oracle")
        assert (res_b[s].mtp_accepted, res_b[s].mtp_rejected) == (oa, orj)
    for s in range(n_seq):
        e = pf.Engine(m, **kv)
        t, r = e.generate(prompts[s], 30, GREEDY, 11)
        e.close()
        np.testing.assert_array_equal(toks_b[s], t, err_msg=f"sequence {s}")
    m.close()


def test_batch_rejects_single_sequence_calls(gpu, tiny_weights):
    cfg, w = tiny_weights
    m = pf.Model(gpu, cfg, w)
    b = pf.BatchEngine(m, 2, **KV)
    with pytest.raises(pf.PFError):
        b.forward([1, 2])
    with pytest.raises(pf.PFError):
        b.forward_batch([0, 0], np.zeros((2, 1), np.int32))
    b.close()
    with pytest.raises(pf.PFError):
        pf.BatchEngine(m, 200, **KV)
    m.close()
