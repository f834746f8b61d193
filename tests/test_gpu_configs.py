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
