"""Engine::step_mtp (src/engine.cpp:402-448) on the device (pf_step_mtp):
the heads from a hidden state, one sampled draft per head, one pass over
[current, d0 .. d2] and the greedy check, against the oracle's restatement
(orc_step_mtp, which forwards the rows one at a time and stops at the first
mismatch).  Accepted count, counters, the rejecting row's logits and the
draw counter must be equal, and a forward after each step must give the
oracle's hidden state (the engine's positions follow the rows the reference
forwarded)."""
import copy

import numpy as np
import pytest

import oracle as O
import pocketforge_amd as pf
from pocketforge_amd import weights as W

pytestmark = pytest.mark.gpu

KV = dict(sink_size=4, window_size=64, pool_block=6, max_context=512)
SAMPLERS = {"greedy": (0.8, 0.95, 40, 1), "top_p": (0.8, 0.95, 40, 0)}


def _weights(cfg, w, case):
    """random: drafts rejected; repeat: zero layer and head matrices, so the
    model repeats its input and every greedy draft is accepted; mostly: tiny
    random layer matrices (accept/reject mix)."""
    if case == "random":
        return w
    w2 = copy.deepcopy(w)
    rng = np.random.default_rng(5)
    for lw in w2["layers"]:
        for n in W.NAMES:
            fmt, codes, scales = lw[n]
            if case == "repeat":
                codes, scales = np.full_like(codes, 0x88), np.zeros_like(scales)
            else:
                r, nb, _ = codes.shape
                codes, scales = pf.quantize_matrix((rng.standard_normal((r, nb * 32)) * 0.004).astype(np.float32), fmt)
            lw[n] = (fmt, codes, scales)
    for hw in w2["mtp"]:
        for n in ("gate", "up", "down"):
            fmt, codes, scales = hw[n]
            hw[n] = (fmt, np.full_like(codes, 0x88), np.zeros_like(scales))
    return w2


@pytest.mark.parametrize("samp", list(SAMPLERS))
@pytest.mark.parametrize("case", ["random", "repeat", "mostly"])
def test_step_mtp_matches_oracle(gpu, tiny_weights, case, samp):
    cfg, w = tiny_weights
    w = _weights(cfg, w, case)
    m = pf.Model(gpu, cfg, w)
    e = pf.Engine(m, **KV)
    c = dict(cfg)
    c.update(KV)
    om = O.Model(c, w)
    s_gpu = pf.Sampling(*SAMPLERS[samp])
    s_orc = O.Sampling(*SAMPLERS[samp])
    toks = W.prompt_ids(10, cfg["n_vocab"], seed=19)
    hidden, last = None, None
    for t in toks:
        _, hg = e.forward([t])
        _, ho = om.forward(t)
        hidden, last = hg[0], int(t)
    np.testing.assert_array_equal(hidden, ho)
    draw_g = draw_o = 3
    accepted = []
    for r in range(6):
        # the token whose forward gave `hidden` (a repeating model then
        # accepts every greedy draft), or an unrelated one
        tok = last if case != "random" else 11 + 97 * r
        a, lg, acc, rej, draw_g = e.step_mtp(tok, hidden, s_gpu, 42, draw_g)
        k, olg, oacc, orej, draw_o = om.step_mtp(tok, hidden, 1, s_orc, 42, draw_o)
        assert (a, acc, rej, draw_g) == (k, oacc, orej, draw_o), f"round {r}"
        assert (lg is None) == (olg is None), f"round {r}"
        if lg is not None:
            np.testing.assert_array_equal(lg, olg, err_msg=f"round {r}")
        accepted.append(a)
        nxt = int(toks[(r + 3) % len(toks)])
        _, hg = e.forward([nxt])
        _, ho = om.forward(nxt)
        np.testing.assert_array_equal(hg[0], ho, err_msg=f"forward after round {r}")
        hidden, last = hg[0], nxt
    if case == "repeat" and samp == "greedy":
        assert max(accepted) == cfg["n_mtp"]
    if case == "random":
        assert max(accepted) < cfg["n_mtp"]
    om.close()
    e.close()
    m.close()
