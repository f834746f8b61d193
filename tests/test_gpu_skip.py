"""Layer skip (LayerSkipController, src/layer_skip.cpp) on the gfx950 path
against the oracle's restatement: forward passes of several heights and
whole generate() streams, single- and multi-sequence, bit-exact, with the
same number of skipped FFN blocks.  The 8-layer model has four layers
(2..5) that may skip; thresholds 0.05 and 0.1 skip some of their FFN blocks
and not others."""
import numpy as np
import pytest

import oracle as O
import pocketforge_amd as pf
from pocketforge_amd import weights as W

from test_gpu_engine import GREEDY, TOP_P, KV, _zero_mats

pytestmark = pytest.mark.gpu

CFG = dict(W.TINY, n_layers=8)


@pytest.fixture(scope="module")
def w8():
    return W.make_weights(CFG, seed=1234)


def _oracle(w, thr, interval, kv=KV):
    c = dict(CFG)
    c.update(kv)
    om = O.Model(c, w)
    om.set_layer_skip(thr, interval)
    return om


@pytest.mark.parametrize("thr", [0.05, 0.1])
def test_skip_forward_matches_oracle(gpu, w8, thr):
    """Passes of 8, 5, 1 and 7 rows, then single tokens: within a pass each
    row's decision follows the rows before it.  Runs of a repeated token
    bring FFN inputs close to the cached ones."""
    m = pf.Model(gpu, CFG, w8)
    e = pf.Engine(m, **KV)
    e.set_layer_skip(thr, 4)
    om = _oracle(w8, thr, 4)
    base = W.prompt_ids(12, CFG["n_vocab"], seed=3)
    toks = np.repeat(base, [3, 1, 2, 4, 1, 3, 2, 1, 5, 2, 3, 3])[:30]
    i = 0
    for n in (8, 5, 1, 7, 1, 1, 1, 1, 1, 1, 1, 1, 1):
        print(f"thr {thr}: rows {i}..{i + n}", flush=True)
        lg, hg = e.forward(toks[i:i + n])
        for r in range(n):
            lo, ho = om.forward(toks[i + r])
            np.testing.assert_array_equal(hg[r], ho, err_msg=f"row {i + r}")
            np.testing.assert_array_equal(lg[r], lo, err_msg=f"row {i + r}")
        i += n
    assert 0 < om.skip_count < 4 * i
    assert e.layer_skip_count() == om.skip_count
    e.close()
    om.close()
    m.close()


CASES = [("random", 0.05, 4, GREEDY), ("random", 0.1, 4, TOP_P), ("mixed", 0.05, 4, GREEDY),
         ("full", 0.05, 4, GREEDY), ("random", 0.1, 0, GREEDY)]


@pytest.mark.parametrize("case,thr,interval,samp", CASES,
                         ids=["random-0.05", "random-0.1-top_p", "mixed-0.05", "full-0.05", "anchor"])
@pytest.mark.parametrize("graphs", [True, False], ids=["graphs", "no_graphs"])
def test_skip_generate_matches_oracle(gpu, w8, case, thr, interval, samp, graphs, monkeypatch):
    """Verify passes run every draft row, but only the rows the acceptance
    keeps (and the reused last row) count for the caches and the skip count."""
    if not graphs:
        monkeypatch.setenv("PF_NO_GRAPHS", "1")
    w = w8 if case == "random" else (_zero_mats(w8, scale=0.004, seed=5) if case == "mixed" else _zero_mats(w8))
    prompt = W.prompt_ids(20, CFG["n_vocab"], seed=9)
    m = pf.Model(gpu, CFG, w)
    e = pf.Engine(m, **KV)
    e.set_layer_skip(thr, interval)
    toks, res = e.generate(prompt, 70, samp, 7)
    om = _oracle(w, thr, interval)
    ot, oa, orj = om.generate(prompt, 70, O.Sampling(samp.temperature, samp.top_p, samp.top_k, samp.greedy), 7)
    print(case, thr, interval, "skips", om.skip_count, "accepted", oa, "rejected", orj, flush=True)
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)
    assert e.layer_skip_count() == om.skip_count
    if interval == 0:
        assert om.skip_count == 0
    else:
        assert om.skip_count > 0
    e.close()
    om.close()
    m.close()


def test_skip_off_leaves_outputs(gpu, w8):
    """Threshold 0 is off: the stream equals the oracle's without skipping;
    switched on it still matches the oracle's controller."""
    prompt = W.prompt_ids(12, CFG["n_vocab"], seed=21)
    m = pf.Model(gpu, CFG, w8)
    for thr in (0.0, 0.1):
        e = pf.Engine(m, **KV)
        e.set_layer_skip(thr, 4)
        toks, res = e.generate(prompt, 40, GREEDY, 5)
        om = _oracle(w8, thr, 4)
        ot, oa, orj = om.generate(prompt, 40, O.Sampling(0.8, 0.95, 40, 1), 5)
        np.testing.assert_array_equal(toks, ot, err_msg=f"threshold {thr}")
        assert e.layer_skip_count() == om.skip_count
        e.close()
        om.close()
    m.close()


def test_skip_profiled_generate_matches(gpu, w8):
    """Profiling mode times every verify-pass dispatch with its own events,
    the gated FFN products included."""
    prompt = W.prompt_ids(16, CFG["n_vocab"], seed=31)
    m = pf.Model(gpu, CFG, w8)
    e = pf.Engine(m, **KV)
    e.set_layer_skip(0.1, 4)
    e.profile(True)
    toks, res = e.generate(prompt, 40, GREEDY, 7)
    n, avg_us, _ = e.gemv_stats()
    assert n > 0 and avg_us > 0
    om = _oracle(w8, 0.1, 4)
    ot, oa, orj = om.generate(prompt, 40, O.Sampling(0.8, 0.95, 40, 1), 7)
    np.testing.assert_array_equal(toks, ot)
    assert e.layer_skip_count() == om.skip_count
    e.close()
    om.close()
    m.close()


def test_skip_reset_and_rejections(gpu, w8):
    m = pf.Model(gpu, CFG, w8)
    e = pf.Engine(m, **KV)
    with pytest.raises(pf.PFError):
        e.set_layer_skip(float("nan"), 4)
    e.set_layer_skip(0.1, 4)
    toks = np.repeat(W.prompt_ids(3, CFG["n_vocab"], seed=8), [3, 2, 3])
    e.forward(toks[:8])
    assert e.layer_skip_count() > 0
    e.reset()
    assert e.layer_skip_count() == 0
    # after reset the caches are zero again: the same passes repeat exactly
    om = _oracle(w8, 0.1, 4)
    lg, _ = e.forward(toks[:8])
    for r in range(8):
        lo, _ = om.forward(toks[r])
        np.testing.assert_array_equal(lg[r], lo)
    assert e.layer_skip_count() == om.skip_count
    e.close()
    om.close()
    m.close()


@pytest.mark.parametrize("thr", [0.05, 0.1])
def test_skip_batch_generate_matches_oracle(gpu, w8, thr):
    """Each sequence keeps its own caches: four sequences decoded together
    give each one's oracle stream and, summed, the oracle skip counts."""
    n_seq = 4
    m = pf.Model(gpu, CFG, w8)
    prompts = [W.prompt_ids(n, CFG["n_vocab"], seed=400 + s) for s, n in enumerate((5, 12, 20, 9))]
    seeds = np.array([3, 5, 7, 9], np.uint64)
    b = pf.BatchEngine(m, n_seq, **KV)
    b.set_layer_skip(thr, 4)
    toks_b, res_b = b.generate_batch(prompts, 30, GREEDY, seeds)
    total = 0
    for s in range(n_seq):
        om = _oracle(w8, thr, 4)
        ot, oa, orj = om.generate(prompts[s], 30, O.Sampling(0.8, 0.95, 40, 1), int(seeds[s]))
        print(f"sequence {s}: skips {om.skip_count} accepted {oa}", flush=True)
        np.testing.assert_array_equal(toks_b[s], ot, err_msg=f"sequence {s}")
        assert (res_b[s].mtp_accepted, res_b[s].mtp_rejected) == (oa, orj)
        total += om.skip_count
        om.close()
    assert b.layer_skip_count() == total and total > 0
    b.close()
    m.close()
