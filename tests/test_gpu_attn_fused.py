"""Attention with the chunk merge in the same kernel (PF_ATTN_FUSED=1,
k_attn_chunk_mq: the last (head, chunk) block of a row merges and quantizes
it) against the two-kernel path (k_attn_chunk + k_attn_merge_quant) and the
oracle: logits, hidden states and token streams bit-exact for passes of 1-8
rows, both head widths (64 and 128), multi-chunk attention lists, window
eviction and pooled rows."""
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
    monkeypatch.setenv("PF_ATTN_FUSED", "0")
    ref = pf.Engine(m, **kv)
    monkeypatch.setenv("PF_ATTN_FUSED", "1")
    fus = pf.Engine(m, **kv)
    monkeypatch.delenv("PF_ATTN_FUSED")
    return m, ref, fus


@pytest.fixture(scope="module")
def wide_weights():
    return WIDE, W.make_weights(WIDE, seed=77, fmts=W.MIXED)


@pytest.mark.parametrize("which", ["tiny", "wide"])
def test_forward_all_heights_match_two_kernel_path(gpu, tiny_weights, wide_weights, which, monkeypatch):
    cfg, w = tiny_weights if which == "tiny" else wide_weights
    m, ref, fus = _engines(gpu, cfg, w, KV, monkeypatch)
    toks = W.prompt_ids(120, cfg["n_vocab"], seed=5)
    i = 0
    for n in [8, 1, 2, 3, 4, 5, 6, 7, 8, 5, 1, 5, 5, 5, 5, 5, 5, 5, 5, 5, 5]:
        lr, hr = ref.forward(toks[i:i + n])
        lf, hf = fus.forward(toks[i:i + n])
        np.testing.assert_array_equal(hf, hr, err_msg=f"hidden, rows {i}..{i + n}")
        np.testing.assert_array_equal(lf, lr, err_msg=f"logits, rows {i}..{i + n}")
        i += n
    ref.close()
    fus.close()
    m.close()


def test_forward_matches_oracle_wide(gpu, wide_weights, monkeypatch):
    cfg, w = wide_weights
    m = pf.Model(gpu, cfg, w)
    monkeypatch.setenv("PF_ATTN_FUSED", "1")
    e = pf.Engine(m, **KV)
    monkeypatch.delenv("PF_ATTN_FUSED")
    c = dict(cfg)
    c.update(KV)
    om = O.Model(c, w)
    toks = W.prompt_ids(40, cfg["n_vocab"], seed=8)
    i = 0
    for n in [5, 1, 5, 5, 8, 5, 1, 5]:
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
def test_generate_matches_two_kernel_path(gpu, wide_weights, samp, monkeypatch):
    cfg, w = wide_weights
    m, ref, fus = _engines(gpu, cfg, w, KV, monkeypatch)
    prompt = W.prompt_ids(20, cfg["n_vocab"], seed=9)
    t1, r1 = ref.generate(prompt, 60, samp, seed=3)
    t2, r2 = fus.generate(prompt, 60, samp, seed=3)
    np.testing.assert_array_equal(t2, t1)
    assert (r2.mtp_accepted, r2.mtp_rejected) == (r1.mtp_accepted, r1.mtp_rejected)
    ref.close()
    fus.close()
    m.close()


def test_multi_chunk_lists_match_two_kernel_path(gpu, tiny_weights, monkeypatch):
    """Attention lists of up to 3 chunks of 256 entries (window 600, pooled
    rows): prefill 700 tokens, then decode passes of 1, 5 and 8 rows."""
    cfg, w = tiny_weights
    kv = dict(sink_size=4, window_size=600, pool_block=8, max_context=2048)
    m, ref, fus = _engines(gpu, cfg, w, kv, monkeypatch)
    toks = W.prompt_ids(760, cfg["n_vocab"], seed=31)
    for e in (ref, fus):
        e.prefill(toks[:256])
        e.prefill(toks[256:512])
        e.prefill(toks[512:700])
    i = 700
    for n in [1, 5, 5, 1, 8, 5, 5, 5, 5, 5, 5, 5, 5]:
        lr, hr = ref.forward(toks[i:i + n])
        lf, hf = fus.forward(toks[i:i + n])
        np.testing.assert_array_equal(hf, hr, err_msg=f"hidden at {i}")
        np.testing.assert_array_equal(lf, lr, err_msg=f"logits at {i}")
        i += n
    ref.close()
    fus.close()
    m.close()
