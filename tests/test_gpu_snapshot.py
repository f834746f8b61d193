"""State-snapshot parity at the long configurations' full sizes.

The oracle cannot replay a 32768-token prompt (B-long) or 64 prompts of
8192 tokens (E) in a test's time, so the GPU runs the prompts, every KV
plane is exported (pf_engine_kv_export: sink, pooled and window rows plus
the evicted rows of the pooled row being built) and imported into the
oracle (orc_kv_import), and from that common state both sides run the
passes of one verify round: the base pass (one row) and the verify pass
(five rows), compared bit for bit, logits and hidden states.

* B-long: the 1B model (Q4) with sink 4, window 4096, pool 16 after a
  32768-token prompt: 1791 pooled rows and 12 pending evicted rows per
  plane, and the verify pass slides the window and completes a pooled row.
* E: 64 sequences of the 1B model, each after an 8192-token prompt, one
  batched verify pass of 64 x 5 = 320 rows (the int8 MFMA GEMM and the
  attention of passes taller than 8 rows); two sequences are checked.
"""
import numpy as np
import pytest

import oracle as O
import pocketforge_amd as pf
from pocketforge_amd import weights as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def one_b(gpu):
    cfg = W.ONE_B
    w = W.make_weights(cfg, seed=1234)
    m = pf.Model(gpu, cfg, w)
    yield cfg, w, m
    m.close()


def _import_state(e, seq, om, cfg, kv):
    """Every KV plane of sequence seq from the GPU engine into the oracle."""
    P = e.position(seq) if isinstance(e, pf.BatchEngine) else e.pos
    cap = 8 + kv["window_size"] + kv["pool_block"] + P // kv["pool_block"] + 8
    for l in range(cfg["n_layers"]):
        for h in range(cfg["n_heads"]):
            k, ks, v, vs, counts = e.kv_export(seq, l, h, cap)
            win_pos0 = kv["sink_size"] + counts[1] * kv["pool_block"] + counts[3]
            om.kv_import(l, h, counts, win_pos0, k, ks, v, vs)
    om.set_state(P)
    return P


def _oracle_rows(om, tokens):
    logits, hidden = [], []
    for t in tokens:
        lg, hd = om.forward(int(t))
        logits.append(lg)
        hidden.append(hd)
    return np.stack(logits), np.stack(hidden)


def test_blong_32k_snapshot_round(one_b):
    cfg, w, m = one_b
    L = 32768
    kv = dict(sink_size=4, window_size=4096, pool_block=16, max_context=L + 64)
    prompt = W.prompt_ids(L, cfg["n_vocab"], seed=42)
    e = pf.Engine(m, **kv)
    toks, _ = e.generate(prompt, 0)
    assert e.pos == L and len(toks) == L
    c = dict(cfg)
    c.update(kv)
    om = O.Model(c, w)
    print(f"B-long snapshot: prompt {L}, importing {cfg['n_layers'] * cfg['n_heads']} planes", flush=True)
    _import_state(e, 0, om, cfg, kv)
    k0, ks0, v0, vs0, counts = e.kv_export(0, 0, 0, 8192)
    assert counts == (4, 1791, 4096, 12)
    base = [int(prompt[-1])]
    verify = [int(x) for x in W.prompt_ids(5, cfg["n_vocab"], seed=77)]
    for rows in (base, verify):
        gl, gh = e.forward(rows)
        ol, oh = _oracle_rows(om, rows)
        np.testing.assert_array_equal(gh, oh, err_msg=f"hidden, rows {rows}")
        np.testing.assert_array_equal(gl, ol, err_msg=f"logits, rows {rows}")
    # the plane after the verify pass: one more pooled row, same rows as the oracle's
    k1, ks1, v1, vs1, counts1 = e.kv_export(0, 5, 3, 8192)
    assert counts1[1] == 1792
    ok, oks, ov, ovs = (np.zeros((8192, 128), np.int8), np.zeros(8192, np.float32),
                        np.zeros((8192, 128), np.int8), np.zeros(8192, np.float32))
    n = O.lib().orc_kv_export(O.lib().orc_engine_kv(om.h), 5, 3, O.ptr(ok, O.i8p), O.ptr(oks, O.f32p),
                              O.ptr(ov, O.i8p), O.ptr(ovs, O.f32p))
    vis = counts1[0] + counts1[1] + counts1[2]
    assert n == vis
    np.testing.assert_array_equal(k1[:vis], ok[:n])
    np.testing.assert_array_equal(v1[:vis], ov[:n])
    np.testing.assert_array_equal(ks1[:vis], oks[:n])
    np.testing.assert_array_equal(vs1[:vis], ovs[:n])
    om.close()
    e.close()


def test_e_64x8k_snapshot_batched_verify(one_b):
    cfg, w, m = one_b
    S, L = 64, 8192
    kv = dict(sink_size=4, window_size=8192, pool_block=64, max_context=L + 64)
    e = pf.BatchEngine(m, S, **kv)
    for s in range(S):
        e.prefill_seq(s, W.prompt_ids(L, cfg["n_vocab"], seed=100 + s))
    assert all(e.position(s) == L for s in range(S))
    c = dict(cfg)
    c.update(kv)
    checked = (0, 37)
    oms = {}
    for s in checked:
        print(f"E snapshot: importing sequence {s}", flush=True)
        oms[s] = O.Model(c, w)
        _import_state(e, s, oms[s], cfg, kv)
    rows = np.stack([W.prompt_ids(5, cfg["n_vocab"], seed=500 + s) for s in range(S)]).astype(np.int32)
    gl, gh = e.forward_batch(np.arange(S, dtype=np.uint32), rows)
    for s in checked:
        ol, oh = _oracle_rows(oms[s], rows[s])
        np.testing.assert_array_equal(gh[s], oh, err_msg=f"hidden, sequence {s}")
        np.testing.assert_array_equal(gl[s], ol, err_msg=f"logits, sequence {s}")
        oms[s].close()
    e.close()


def test_e_sliding_window_snapshot_batched_verify(one_b):
    """E's shape once decoding has slid the window: 8 sequences of the 1B
    model after 8318 + s tokens (window 8192, pool 64: one pooled row and
    a window sliding by one entry per verify row), one batched pass of 5
    rows per sequence.  The attention of that pass serves each sequence's
    rows together although their lists differ by one entry per row; for
    sequences 2-5 a pooled row completes between two of the rows."""
    cfg, w, m = one_b
    S, L = 8, 8318
    kv = dict(sink_size=4, window_size=8192, pool_block=64, max_context=L + S + 64)
    e = pf.BatchEngine(m, S, **kv)
    for s in range(S):
        e.prefill_seq(s, W.prompt_ids(L + s, cfg["n_vocab"], seed=700 + s))
    c = dict(cfg)
    c.update(kv)
    checked = (0, 3, 7)
    oms = {}
    for s in checked:
        print(f"E sliding snapshot: importing sequence {s}", flush=True)
        oms[s] = O.Model(c, w)
        _import_state(e, s, oms[s], cfg, kv)
    rows = np.stack([W.prompt_ids(5, cfg["n_vocab"], seed=900 + s) for s in range(S)]).astype(np.int32)
    gl, gh = e.forward_batch(np.arange(S, dtype=np.uint32), rows)
    for s in checked:
        ol, oh = _oracle_rows(oms[s], rows[s])
        np.testing.assert_array_equal(gh[s], oh, err_msg=f"hidden, sequence {s}")
        np.testing.assert_array_equal(gl[s], ol, err_msg=f"logits, sequence {s}")
        oms[s].close()
    e.close()
