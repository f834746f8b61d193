"""The oracle's state import (orc_kv_import, orc_engine_set_state) and the
decode loop from a state (orc_generate_continue), which the GPU snapshot
parity tests and the bench's CPU baseline use to start the oracle at a long
context without re-running the prompt.

Pins: an imported KV plane must behave exactly like the plane that stored
the same rows, through further stores that evict window rows and complete
pooled rows (src/kv_cache.cpp:59-127), and the decode continuation must
reproduce orc_generate's stream."""
import numpy as np
import pytest

import oracle as O
from pocketforge_amd import weights as W


def P(a, t):
    return a.ctypes.data_as(t)


def _export(L, kv, l, h, cap, hd):
    K8 = np.zeros((cap, hd), np.int8)
    Ks = np.zeros(cap, np.float32)
    V8 = np.zeros((cap, hd), np.int8)
    Vs = np.zeros(cap, np.float32)
    n = L.orc_kv_export(kv, l, h, P(K8, O.i8p), P(Ks, O.f32p), P(V8, O.i8p), P(Vs, O.f32p))
    return K8[:n], Ks[:n], V8[:n], Vs[:n]


def _view(p, sink, window, pool):
    """Counts of the state after positions 0..p-1: sink, pooled, window,
    pending (evicted, not yet pooled) rows, and the first window position."""
    n_sink = min(p, sink, 8)
    nw = max(p - sink, 0)
    win_lo = max(nw - window, 0)
    n_pool = win_lo // pool
    return n_sink, n_pool, nw - win_lo, win_lo - n_pool * pool, sink + win_lo


# (sink, window, pool, positions before the snapshot, positions after)
CASES = [(4, 16, 4, 37, 23), (2, 8, 3, 8, 20), (4, 32, 16, 77, 41), (8, 16, 1, 30, 5), (4, 16, 4, 3, 40)]


@pytest.mark.parametrize("case", CASES)
def test_kv_import_continues_like_the_stored_plane(case):
    sink, window, pool, p0, extra = case
    L = O.lib()
    Ln, H, hd, maxc = 2, 2, 8, 512
    rng = np.random.default_rng(sink * 100 + window + p0)
    n = p0 + extra
    keys = (rng.standard_normal((n, Ln, H, hd)) * 2).astype(np.float32)
    vals = (rng.standard_normal((n, Ln, H, hd)) * 2).astype(np.float32)
    keys[5 % n, 0, 1] = 0.0                                # an all-zero row (scale 1)
    a = L.orc_kv_create(Ln, H, hd, sink, window, pool, maxc)
    # every position's quantized row, from a cache whose window never evicts
    rows = L.orc_kv_create(Ln, H, hd, sink, maxc, pool, maxc)
    for p in range(n):
        for l in range(Ln):
            for h in range(H):
                if p < p0:
                    L.orc_kv_store(a, l, h, p, P(keys[p, l, h], O.f32p), P(vals[p, l, h], O.f32p))
                L.orc_kv_store(rows, l, h, p, P(keys[p, l, h], O.f32p), P(vals[p, l, h], O.f32p))
    b = L.orc_kv_create(Ln, H, hd, sink, window, pool, maxc)
    n_sink, n_pool, n_win, n_pend, wpos0 = _view(p0, sink, window, pool)
    for l in range(Ln):
        for h in range(H):
            ka, ksa, va, vsa = _export(L, a, l, h, 1024, hd)
            assert len(ka) == n_sink + n_pool + n_win
            assert L.orc_kv_pool_count(a, l, h) == n_pool
            kr, ksr, vr, vsr = _export(L, rows, l, h, 1024, hd)
            # row of position q in the never-evicting cache: sink slot q, or
            # window entry (q - sink) after its sink rows
            def at(q):
                return q if q < sink else min(sink, 8) + (q - sink)
            pend = [at(q) for q in range(wpos0 - n_pend, wpos0)]
            k = np.concatenate([ka, kr[pend]]) if pend else ka
            ks = np.concatenate([ksa, ksr[pend]]) if pend else ksa
            v = np.concatenate([va, vr[pend]]) if pend else va
            vs = np.concatenate([vsa, vsr[pend]]) if pend else vsa
            O.kv_import(b, l, h, (n_sink, n_pool, n_win, n_pend), wpos0, k, ks, v, vs)
    q = rng.standard_normal(hd).astype(np.float32)
    ks_self = rng.standard_normal(hd).astype(np.float32)
    vs_self = rng.standard_normal(hd).astype(np.float32)
    for p in range(p0, n + 1):
        for l in range(Ln):
            for h in range(H):
                ea, eb = _export(L, a, l, h, 1024, hd), _export(L, b, l, h, 1024, hd)
                for x, y in zip(ea, eb):
                    np.testing.assert_array_equal(x, y, err_msg=f"{case} position {p} plane {l},{h}")
                assert L.orc_kv_pool_count(a, l, h) == L.orc_kv_pool_count(b, l, h)
                oa, ob = np.zeros(hd, np.float32), np.zeros(hd, np.float32)
                L.orc_attn_head(a, l, h, P(q, O.f32p), P(ks_self, O.f32p), P(vs_self, O.f32p), P(oa, O.f32p))
                L.orc_attn_head(b, l, h, P(q, O.f32p), P(ks_self, O.f32p), P(vs_self, O.f32p), P(ob, O.f32p))
                np.testing.assert_array_equal(oa, ob)
        if p == n:
            break
        for l in range(Ln):
            for h in range(H):
                for kv in (a, b):
                    L.orc_kv_store(kv, l, h, p, P(keys[p, l, h], O.f32p), P(vals[p, l, h], O.f32p))
    for kv in (a, b, rows):
        L.orc_kv_destroy(kv)


def test_kv_import_rebuilds_the_pooling_sum():
    """A plane imported with pending rows folds them, with the rows evicted
    after the import, into the same pooled row as the plane that stored
    them; without them the block is still incomplete after those stores."""
    L = O.lib()
    hd, sink, window, pool = 4, 2, 8, 4
    a = L.orc_kv_create(1, 1, hd, sink, window, pool, 256)
    rows = L.orc_kv_create(1, 1, hd, sink, 256, pool, 256)
    vals = [np.full(hd, float(i + 1) * (1 + 0.25 * (i % 3)), np.float32) for i in range(16)]
    p0 = 12                                   # positions 2, 3 evicted from the window, pending
    for p in range(16):
        if p < p0:
            L.orc_kv_store(a, 0, 0, p, P(vals[p], O.f32p), P(vals[p], O.f32p))
        L.orc_kv_store(rows, 0, 0, p, P(vals[p], O.f32p), P(vals[p], O.f32p))
    n_sink, n_pool, n_win, n_pend, wpos0 = _view(p0, sink, window, pool)
    assert (n_sink, n_pool, n_win, n_pend, wpos0) == (2, 0, 8, 2, 4)
    ka, ksa, va, vsa = _export(L, a, 0, 0, 64, hd)
    kr, ksr, vr, vsr = _export(L, rows, 0, 0, 64, hd)
    results = []
    for with_pending in (True, False):
        b = L.orc_kv_create(1, 1, hd, sink, window, pool, 256)
        if with_pending:
            k, ks = np.concatenate([ka, kr[2:4]]), np.concatenate([ksa, ksr[2:4]])
            v, vs = np.concatenate([va, vr[2:4]]), np.concatenate([vsa, vsr[2:4]])
            O.kv_import(b, 0, 0, (2, 0, 8, 2), wpos0, k, ks, v, vs)
        else:
            O.kv_import(b, 0, 0, (2, 0, 8, 0), wpos0, ka, ksa, va, vsa)
        for p in (12, 13):                    # evicts positions 4, 5: the block 2..5 completes
            L.orc_kv_store(b, 0, 0, p, P(vals[p], O.f32p), P(vals[p], O.f32p))
        assert L.orc_kv_pool_count(b, 0, 0) == (1 if with_pending else 0)
        results.append(_export(L, b, 0, 0, 64, hd))
        L.orc_kv_destroy(b)
    for p in (12, 13):
        L.orc_kv_store(a, 0, 0, p, P(vals[p], O.f32p), P(vals[p], O.f32p))
    want = _export(L, a, 0, 0, 64, hd)
    # the pooled row (index 2, after the sink) is the mean of positions 2..5
    np.testing.assert_allclose(want[0][2] * want[1][2], np.mean([vals[i] for i in range(2, 6)], axis=0),
                               rtol=0.02)
    for x, y in zip(want, results[0]):
        np.testing.assert_array_equal(x, y)
    assert len(results[1][0]) == len(want[0]) - 1
    L.orc_kv_destroy(a)
    L.orc_kv_destroy(rows)


@pytest.mark.parametrize("greedy", [1, 0])
def test_generate_continue_matches_generate(greedy):
    cfg = dict(W.TINY)
    cfg.update(sink_size=4, window_size=64, pool_block=6, max_context=512)
    w = W.make_weights(W.TINY, seed=1234)
    prompt = W.prompt_ids(40, cfg["n_vocab"], seed=3)
    s = O.Sampling(0.8, 0.95, 40, greedy)
    a = O.Model(cfg, w)
    toks, acc, rej = a.generate(prompt, 24, s, 9)
    b = O.Model(cfg, w)
    b.generate(prompt, 0, s, 9)                   # the prompt only
    assert b.pos == len(prompt)
    gen, acc2, rej2 = b.generate_continue(prompt[-1], 24, s, 9)
    np.testing.assert_array_equal(gen, toks[len(prompt):])
    assert (acc2, rej2) == (acc, rej)
    a.close()
    b.close()
