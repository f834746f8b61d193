"""The persistent decode pass (PF_PERSISTENT=1: one kernel per pass of up to
8 rows) against the kernel-per-step pass and against the oracle: logits,
hidden states and token streams bit-exact, for every pass height, both
head widths (64 and 128), mixed weight formats, window eviction, pooling
and multi-chunk attention lists."""
import numpy as np
import pytest

import oracle as O
import pocketforge_amd as pf
from pocketforge_amd import weights as W

pytestmark = pytest.mark.gpu

KV = dict(sink_size=4, window_size=64, pool_block=6, max_context=512)
WIDE = dict(n_layers=2, n_embd=512, n_heads=4, head_dim=128, n_ff=1024, n_vocab=1024, n_mtp=4)
GREEDY = pf.Sampling(0.8, 0.95, 40, 1)
TOP_P = pf.Sampling(0.8, 0.95, 40, 0)


def _engines(gpu, cfg, w, kv, monkeypatch):
    m = pf.Model(gpu, cfg, w)
    monkeypatch.setenv("PF_PERSISTENT", "0")
    ref = pf.Engine(m, **kv)
    monkeypatch.setenv("PF_PERSISTENT", "1")
    per = pf.Engine(m, **kv)
    return m, ref, per


@pytest.fixture(scope="module")
def wide_weights():
    return WIDE, W.make_weights(WIDE, seed=77, fmts=W.MIXED)


@pytest.mark.parametrize("which", ["tiny", "wide"])
def test_forward_all_heights_match_step_kernels(gpu, tiny_weights, wide_weights, which, monkeypatch):
    """Passes of 1..8 rows across window eviction (64) and pooling (6)."""
    cfg, w = tiny_weights if which == "tiny" else wide_weights
    m, ref, per = _engines(gpu, cfg, w, KV, monkeypatch)
    heights = [1, 2, 3, 4, 5, 6, 7, 8, 5, 1, 8, 8, 8, 8, 8, 8, 3, 5, 5, 5, 1, 7, 8, 8, 8, 8, 8, 8, 8]
    toks = W.prompt_ids(sum(heights), cfg["n_vocab"], seed=21)
    i = 0
    for n in heights:
        print(f"pass rows {n} at position {i}", flush=True)
        lr, hr = ref.forward(toks[i:i + n])
        lp, hp = per.forward(toks[i:i + n])
        np.testing.assert_array_equal(hp, hr, err_msg=f"hidden, pass at {i} of {n} rows")
        np.testing.assert_array_equal(lp, lr, err_msg=f"logits, pass at {i} of {n} rows")
        i += n
    ref.close()
    per.close()
    m.close()


def test_forward_matches_oracle_wide(gpu, wide_weights, monkeypatch):
    """head_dim 128 with Q4 attention, Q2 gate/up and Q1.5 down weights."""
    cfg, w = wide_weights
    monkeypatch.setenv("PF_PERSISTENT", "1")
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **KV)
    c = dict(cfg)
    c.update(KV)
    om = O.Model(c, w)
    toks = W.prompt_ids(30, cfg["n_vocab"], seed=5)
    i = 0
    for n in [5, 1, 8, 3, 5, 8]:
        lg, hg = e.forward(toks[i:i + n])
        for j in range(n):
            lo, ho = om.forward(toks[i + j])
            np.testing.assert_array_equal(hg[j], ho, err_msg=f"row {i + j}")
            np.testing.assert_array_equal(lg[j], lo, err_msg=f"row {i + j}")
        i += n
    om.close()
    e.close()
    m.close()


@pytest.mark.parametrize("samp", [GREEDY, TOP_P], ids=["greedy", "top_p"])
@pytest.mark.parametrize("which", ["tiny", "wide"])
def test_generate_matches_step_kernels(gpu, tiny_weights, wide_weights, which, samp, monkeypatch):
    cfg, w = tiny_weights if which == "tiny" else wide_weights
    m, ref, per = _engines(gpu, cfg, w, KV, monkeypatch)
    prompt = W.prompt_ids(20, cfg["n_vocab"], seed=9)
    t1, r1 = ref.generate(prompt, 60, samp, seed=3)
    t2, r2 = per.generate(prompt, 60, samp, seed=3)
    np.testing.assert_array_equal(t2, t1)
    assert (r2.mtp_accepted, r2.mtp_rejected) == (r1.mtp_accepted, r1.mtp_rejected)
    ref.close()
    per.close()
    m.close()


def test_multi_chunk_lists_match_step_kernels(gpu, tiny_weights, monkeypatch):
    """Attention lists of up to 3 chunks of 256 entries (window 600, pooled
    rows): prefill 700 tokens, then decode passes of 1 and 5 rows."""
    cfg, w = tiny_weights
    kv = dict(sink_size=4, window_size=600, pool_block=8, max_context=2048)
    m, ref, per = _engines(gpu, cfg, w, kv, monkeypatch)
    toks = W.prompt_ids(760, cfg["n_vocab"], seed=31)
    for e in (ref, per):
        e.prefill(toks[:256])
        e.prefill(toks[256:512])
        e.prefill(toks[512:700])
    i = 700
    for n in [1, 5, 5, 1, 8, 5, 5, 5, 5, 5, 5, 5, 5]:
        lr, hr = ref.forward(toks[i:i + n])
        lp, hp = per.forward(toks[i:i + n])
        np.testing.assert_array_equal(hp, hr, err_msg=f"hidden at {i}")
        np.testing.assert_array_equal(lp, lr, err_msg=f"logits at {i}")
        i += n
    ref.close()
    per.close()
    m.close()
