"""Continuous batching (pf_batch_open / admit / step / take): requests join
and leave a running batch between rounds; every request's tokens and MTP
counters equal a single-sequence Engine.generate for its prompt and seed
(the reference serves each request with its own Engine::generate,
src/forge_server.cpp:280, 398)."""
import numpy as np
import pytest

import pocketforge_amd as pf
from pocketforge_amd import weights as W

pytestmark = pytest.mark.gpu

KV = dict(sink_size=4, window_size=64, pool_block=6, max_context=512)
GREEDY = pf.Sampling(0.8, 0.95, 40, 1)
TOP_P = pf.Sampling(0.8, 0.95, 40, 0)


def _single(gpu, cfg, w, prompt, max_new, samp, seed):
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **KV)
    toks, res = e.generate(prompt, max_new, samp, seed)
    out = (toks.copy(), res.mtp_accepted, res.mtp_rejected)
    e.close()
    m.close()
    return out


@pytest.mark.parametrize("samp", [GREEDY, TOP_P], ids=["greedy", "top_p"])
def test_requests_join_and_leave(gpu, tiny_weights, samp):
    cfg, w = tiny_weights
    reqs = [  # (prompt, budget, seed, round it arrives at)
        (W.prompt_ids(9, cfg["n_vocab"], seed=1), 20, 11, 0),
        (W.prompt_ids(30, cfg["n_vocab"], seed=2), 6, 12, 0),
        (W.prompt_ids(5, cfg["n_vocab"], seed=3), 14, 13, 2),
        (W.prompt_ids(17, cfg["n_vocab"], seed=4), 9, 14, 3),
        (W.prompt_ids(12, cfg["n_vocab"], seed=5), 25, 15, 4),
    ]
    m = pf.Model(gpu, cfg, w)
    b = pf.BatchEngine(m, 3, **KV)
    b.open(samp, tokens_cap=128)
    free = [0, 1, 2]
    slot_of, waiting, done = {}, list(range(len(reqs))), {}
    rnd = 0
    while len(done) < len(reqs):
        for i in list(waiting):
            if reqs[i][3] <= rnd and free:
                s = free.pop(0)
                b.admit(s, reqs[i][0], reqs[i][1], reqs[i][2])
                slot_of[s] = i
                waiting.remove(i)
        for s in b.step():
            toks, r = b.take(s)
            done[slot_of.pop(s)] = (toks, r.mtp_accepted, r.mtp_rejected)
            free.append(s)
        rnd += 1
        assert rnd < 200
    b.close()
    m.close()
    for i, (prompt, budget, seed, _) in enumerate(reqs):
        toks, acc, rej = done[i]
        st, sacc, srej = _single(gpu, cfg, w, prompt, budget, samp, seed)
        np.testing.assert_array_equal(toks, st, err_msg=f"request {i}")
        assert (acc, rej) == (sacc, srej), f"request {i}"


def test_leaving_early_and_slot_reuse(gpu, tiny_weights):
    """A request taken before its budget is spent leaves the batch; its slot
    takes a new request from an empty cache, whose tokens equal a fresh
    single engine's."""
    cfg, w = tiny_weights
    m = pf.Model(gpu, cfg, w)
    b = pf.BatchEngine(m, 2, **KV)
    b.open(GREEDY, tokens_cap=128)
    p0, p1, p2 = (W.prompt_ids(n, cfg["n_vocab"], seed=s) for n, s in ((10, 21), (14, 22), (7, 23)))
    b.admit(0, p0, 40, 5)
    b.admit(1, p1, 12, 6)
    for _ in range(3):
        b.step()
    toks0, _ = b.take(0)   # leaves with part of its budget
    assert len(toks0) > len(p0)
    b.admit(0, p2, 16, 8)
    fin = {}
    while len(fin) < 2:
        for s in b.step():
            fin[s] = b.take(s)
    b.close()
    m.close()
    for s, (p, n, seed) in {0: (p2, 16, 8), 1: (p1, 12, 6)}.items():
        st, sacc, srej = _single(gpu, cfg, w, p, n, GREEDY, seed)
        np.testing.assert_array_equal(fin[s][0], st, err_msg=f"slot {s}")
        assert (fin[s][1].mtp_accepted, fin[s][1].mtp_rejected) == (sacc, srej)
    st, _, _ = _single(gpu, cfg, w, p0, 40, GREEDY, 5)
    np.testing.assert_array_equal(toks0, st[: len(toks0)])
