"""Parity at the benchmark configurations' shapes: the GPU engine against
the oracle on the same seeded weights and prompts.

* S (150M: 12 layers, d 768, 12 x 64 heads, ff 2048, vocab 16384): the full
  256-token greedy stream after a 64-token prompt.
* B-mix (1B with Q4 attention, Q2 gate/up, Q1.5 down; temperature 0.8,
  top-k 40, top-p 0.95, which the reference's dispatch runs as top-p): the
  first 32 tokens after a 32-token prompt.
* B-long cache geometry (sink 4, window 4096, pool 16) on a small model: a
  5000-token prompt, so that every verify pass slides the window and sees
  pooled rows, then 40 greedy tokens.
"""
import numpy as np
import pytest

import oracle as O
import pocketforge_amd as pf
from pocketforge_amd import weights as W

pytestmark = pytest.mark.gpu


def _both(gpu, cfg, w, kv, prompt, max_new, samp, seed):
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **kv)
    toks, res = e.generate(prompt, max_new, samp, seed)
    c = dict(cfg)
    c.update(kv)
    om = O.Model(c, w)
    ot, oa, orj = om.generate(prompt, max_new, O.Sampling(samp.temperature, samp.top_p, samp.top_k, samp.greedy),
                              seed)
    om.close()
    e.close()
    m.close()
    return toks, res, ot, oa, orj


def test_config_s_full_greedy_stream(gpu):
    cfg = W.SMALL
    w = W.make_weights(cfg, seed=1234)
    prompt = W.prompt_ids(64, cfg["n_vocab"], seed=42)
    kv = dict(sink_size=4, window_size=8192, pool_block=64, max_context=64 + 256 + 64)
    toks, res, ot, oa, orj = _both(gpu, cfg, w, kv, prompt, 256, pf.Sampling(0.8, 0.95, 40, 1), 7)
    assert len(toks) == 64 + 256
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)


def _repeating_1b():
    """The 1B shapes with layer matrices N(0, 0.016^2), the Q4 tied embedding
    N(0, 0.02^2) and zero MTP heads: the residual stream stays close to the
    token's embedding, so the model mostly repeats its input and most greedy
    drafts are accepted (the oracle accepts 29 and rejects 3 over 40 tokens
    after a 16-token prompt).  Random N(0, 0.02^2) weights accept none."""
    cfg = W.ONE_B
    w = W.make_weights(cfg, seed=1234, std=0.016)
    codes, scales = pf.gen_matrix(1234, 0x10000, 0.02, cfg["n_vocab"], cfg["n_embd"], pf.FMT_Q4)
    w["emb"] = (pf.FMT_Q4, codes, scales)
    for hw in w["mtp"]:
        for n in ("gate", "up", "down"):
            fmt, c, sc = hw[n]
            hw[n] = (fmt, np.full_like(c, 0x88), np.zeros_like(sc))
    return cfg, w


def test_config_b_accepted_drafts_stream(gpu):
    """Acceptance at the 1B shape: the rounds that commit every row of a
    verify pass, reuse its last row as the next base pass, and continue a
    one-row first segment with a second one, under both verify policies,
    against the oracle's stream and counters."""
    cfg, w = _repeating_1b()
    prompt = W.prompt_ids(16, cfg["n_vocab"], seed=42)
    kv = dict(sink_size=4, window_size=8192, pool_block=64, max_context=256)
    samp = pf.Sampling(0.8, 0.95, 40, 1)
    c = dict(cfg)
    c.update(kv)
    om = O.Model(c, w)
    ot, oa, orj = om.generate(prompt, 40, O.Sampling(0.8, 0.95, 40, 1), 7)
    om.close()
    assert oa > 20 and orj > 0
    m = pf.Model(gpu, cfg, w)
    for full in (0, 1):
        e = pf.Engine(m, **kv)
        e.set_verify_full(full)
        toks, res = e.generate(prompt, 40, samp, 7)
        np.testing.assert_array_equal(toks, ot, err_msg=f"verify_full={full}")
        assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)
        if not full:
            assert res.continued > 0
        e.close()
    m.close()


def test_config_bmix_top_p_prefix(gpu):
    cfg = W.ONE_B
    w = W.make_weights(cfg, seed=1234, fmts=W.MIXED)
    prompt = W.prompt_ids(32, cfg["n_vocab"], seed=42)
    kv = dict(sink_size=4, window_size=8192, pool_block=64, max_context=256)
    toks, res, ot, oa, orj = _both(gpu, cfg, w, kv, prompt, 32, pf.Sampling(0.8, 0.95, 40, 0), 7)
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)


def test_config_blong_cache_geometry(gpu, tiny_weights):
    cfg, w = tiny_weights
    prompt = W.prompt_ids(5000, cfg["n_vocab"], seed=42)
    kv = dict(sink_size=4, window_size=4096, pool_block=16, max_context=8192)
    toks, res, ot, oa, orj = _both(gpu, cfg, w, kv, prompt, 40, pf.Sampling(0.8, 0.95, 40, 1), 7)
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)


# ------------------------------------------------ full-size token streams
#
# The oracle's streams at the benchmark configurations' full sizes are
# fixtures (tests/golden/stream_*.npz, written by
# tests/golden/make_config_streams.py on the host): B (2048-token prompt,
# 64 greedy tokens), B-mix (1024-token prompt, 64 top-p tokens), one
# sequence of configuration E (8192-token prompt, 32 greedy tokens) and
# B-long's cache geometry (sink 4 / window 4096 / pool 16) on the 1B model
# with a 5000-token prompt (full window, 56 pooled rows), 32 greedy tokens.

import importlib.util  # noqa: E402
import os  # noqa: E402

_GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_spec = importlib.util.spec_from_file_location("config_streams", os.path.join(_GOLDEN, "make_config_streams.py"))
_streams = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(_streams)
_WEIGHTS = {}


def _weights(model, fmts):
    if (model, fmts) not in _WEIGHTS:
        _WEIGHTS.clear()                      # one 1B weight set in host memory at a time
        _WEIGHTS[(model, fmts)] = W.make_weights(getattr(W, model), seed=1234, fmts=getattr(W, fmts))
    return _WEIGHTS[(model, fmts)]


@pytest.mark.parametrize("name", ["B", "E0", "B-long-5k", "B-mix"])
def test_config_full_size_stream_matches_oracle_fixture(gpu, name):
    path = os.path.join(_GOLDEN, f"stream_{name}.npz")
    if not os.path.exists(path):
        pytest.skip(f"fixture {path} not generated")
    ref = np.load(path)
    spec = _streams.STREAMS[name]
    cfg = getattr(W, spec[0])
    w = _weights(spec[0], spec[1])
    prompt = W.prompt_ids(spec[3], cfg["n_vocab"], seed=spec[4])
    print(f"{name}: prompt {spec[3]}, {spec[5]} tokens", flush=True)
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **_streams.kv_of(spec))
    toks, res = e.generate(prompt, spec[5], pf.Sampling(*spec[6]), _streams.SEED)
    e.close()
    m.close()
    assert int(ref["n_prompt"]) == spec[3]
    np.testing.assert_array_equal(toks, ref["tokens"])
    assert (res.mtp_accepted, res.mtp_rejected) == (int(ref["accepted"]), int(ref["rejected"]))
