"""One-row passes through each of the fused launch layouts, bit-exact
against the oracle: every layer in one launch (the default), one launch per
layer (PF_STACK=0) and the QKV + attention and O + FFN launches
(PF_STACK=0 PF_LAYER=0).  Models of 1, 2 and 12 layers, hidden sizes 256 and 768, all
Q4 or with Q2 gate|up and Q1.5 down, and attention lists of one and three 256-entry
chunks."""
import numpy as np
import pytest

import oracle as O
import pocketforge_amd as pf
from pocketforge_amd import weights as W

pytestmark = pytest.mark.gpu

MODES = {"stack": {}, "layer": {"PF_STACK": "0"}, "two": {"PF_STACK": "0", "PF_LAYER": "0"}}
GREEDY = pf.Sampling(0.8, 0.95, 40, 1)
TOP_P = pf.Sampling(0.8, 0.95, 40, 0)


def _setenv(monkeypatch, mode):
    monkeypatch.delenv("PF_STACK", raising=False)
    monkeypatch.delenv("PF_LAYER", raising=False)
    for k, v in MODES[mode].items():
        monkeypatch.setenv(k, v)


def _oracle(cfg, w, kv):
    c = dict(cfg)
    c.update(kv)
    return O.Model(c, w)


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("layers,kv,n", [
    (2, dict(sink_size=4, window_size=64, pool_block=6, max_context=512), 90),
    (1, dict(sink_size=4, window_size=64, pool_block=6, max_context=512), 40),
    (2, dict(sink_size=4, window_size=600, pool_block=8, max_context=2048), 620),
])
def test_one_row_forwards(gpu, monkeypatch, mode, layers, kv, n):
    """Token-by-token forwards (every pass one row) past the window, with
    pooled blocks; the hidden state and logits of every checked row equal
    the oracle's."""
    _setenv(monkeypatch, mode)
    cfg = dict(W.TINY, n_layers=layers)
    w = W.make_weights(cfg, seed=1234)
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **kv)
    om = _oracle(cfg, w, kv)
    toks = W.prompt_ids(n, cfg["n_vocab"], seed=17)
    for i, t in enumerate(toks):
        lg, hg = e.forward([t])
        lo, ho = om.forward(t)
        if i < 8 or i % 23 == 0 or i >= n - 4:
            np.testing.assert_array_equal(hg[0], ho, err_msg=f"{mode} row {i}")
            np.testing.assert_array_equal(lg[0], lo, err_msg=f"{mode} row {i}")
    om.close()
    e.close()
    m.close()


@pytest.mark.parametrize("mode", list(MODES))
def test_one_row_forwards_mixed_formats(gpu, monkeypatch, mode):
    """Q4 attention matrices with Q2 gate|up and Q1.5 down (the layer stack's
    second format set; the other layouts run these as separate products)."""
    _setenv(monkeypatch, mode)
    cfg = W.TINY
    kv = dict(sink_size=4, window_size=64, pool_block=6, max_context=512)
    w = W.make_weights(cfg, seed=321, fmts=W.MIXED)
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **kv)
    om = _oracle(cfg, w, kv)
    toks = W.prompt_ids(80, cfg["n_vocab"], seed=8)
    for i, t in enumerate(toks):
        lg, hg = e.forward([t])
        lo, ho = om.forward(t)
        if i < 8 or i % 13 == 0 or i >= 76:
            np.testing.assert_array_equal(hg[0], ho, err_msg=f"{mode} row {i}")
            np.testing.assert_array_equal(lg[0], lo, err_msg=f"{mode} row {i}")
    om.close()
    e.close()
    m.close()


@pytest.mark.parametrize("mode", list(MODES))
def test_one_row_forwards_twelve_layers(gpu, monkeypatch, mode):
    """A 12-layer model of hidden size 768 (12 heads of 64): the residual
    row passes through every layer hand-off of the one-launch stack."""
    _setenv(monkeypatch, mode)
    cfg = dict(W.SMALL, n_vocab=2048)
    kv = dict(sink_size=4, window_size=64, pool_block=6, max_context=512)
    w = W.make_weights(cfg, seed=99)
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **kv)
    om = _oracle(cfg, w, kv)
    toks = W.prompt_ids(24, cfg["n_vocab"], seed=5)
    for i, t in enumerate(toks):
        lg, hg = e.forward([t])
        lo, ho = om.forward(t)
        np.testing.assert_array_equal(hg[0], ho, err_msg=f"{mode} row {i}")
        np.testing.assert_array_equal(lg[0], lo, err_msg=f"{mode} row {i}")
    om.close()
    e.close()
    m.close()


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("samp", [GREEDY, TOP_P], ids=["greedy", "top_p"])
def test_single_token_generate(gpu, monkeypatch, mode, samp):
    """generate() with the MTP heads off: every pass is one row, replayed
    from captured graphs; the stream equals the oracle's."""
    _setenv(monkeypatch, mode)
    cfg = W.TINY
    kv = dict(sink_size=4, window_size=64, pool_block=6, max_context=512)
    w = W.make_weights(cfg, seed=1234)
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **kv)
    e.set_mtp_enabled(False)
    prompt = W.prompt_ids(13, cfg["n_vocab"], seed=6)
    toks, res = e.generate(prompt, 60, samp, 9)
    c = dict(cfg)
    c["n_mtp"] = 0
    om = _oracle(c, w, kv)
    ot, _, _ = om.generate(prompt, 60, O.Sampling(samp.temperature, samp.top_p, samp.top_k, samp.greedy), 9)
    np.testing.assert_array_equal(toks, ot)
    om.close()
    e.close()
    m.close()
