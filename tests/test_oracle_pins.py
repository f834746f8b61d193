"""Pins for the oracle functions that no reference-built golden covers: each
is checked against something other than itself -- published known-answer
vectors, a float64 brute force, hand-derived control-flow cases, or a
closed form.  CPU only."""
import ctypes as C
import math

import numpy as np
import pytest

import oracle as O

P = O.ptr


# ------------------------------------------------------------ Philox4x32-10

# Known-answer vectors of Philox4x32-10 published with Random123 (Salmon,
# Moraes, Dror, Shaw, SC'11): (counter, key) -> output.
PHILOX_KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff, 0xffffffff, 0xffffffff, 0xffffffff), (0xffffffff, 0xffffffff),
     (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX_KAT)
def test_philox_known_answer_vectors(ctr, key, want):
    assert tuple(int(x) for x in O.philox4x32_10(ctr, key)) == want


def test_uniform_is_the_top_24_bits_of_word_zero():
    # draw idx of a run seeded `seed`: counter (idx lo, idx hi, 'SAMP', 0),
    # key (seed lo, seed hi); u = (word0 >> 8) * 2^-24, so u in [0, 1) on a
    # 2^-24 grid
    L = O.lib()
    us = []
    for seed in (0, 7, 42, 0x1234567890AB):
        for idx in (0, 1, 2, 5, 1 << 33):
            ctr = (idx & 0xFFFFFFFF, idx >> 32, 0x53414D50, 0)
            w0 = int(O.philox4x32_10(ctr, (seed & 0xFFFFFFFF, seed >> 32))[0])
            u = L.orc_uniform(seed, idx)
            assert u == (w0 >> 8) * 2.0 ** -24
            us.append(u)
    assert all(0.0 <= u < 1.0 for u in us)
    many = np.array([L.orc_uniform(3, i) for i in range(4000)])
    assert abs(many.mean() - 0.5) < 0.02 and many.min() >= 0.0 and many.max() < 1.0


# ------------------------------------------------------ block-quantized GEMV

def decode_interchange(fmt, codes):
    """Signed weight codes [rows][cols] from the interchange bytes, written
    from the reference decoders (src/matmul_neon.cpp:34-75): Q4 byte j holds
    elements 2j (low nibble) and 2j + 1 (high), value nibble - 8; Q2 byte j
    holds elements 4j..4j+3 at bits 0, 2, 4, 6, value code - 2; Q1.5 the same
    positions with value code - 1."""
    rows, nb, _ = codes.shape
    if fmt == O.Q8:     # Q8_0 (include/forge/types.hpp:17-20): one signed byte per element
        return codes.view(np.int8).astype(np.int64).reshape(rows, nb * 32)
    if fmt == O.Q4:
        lo = (codes & 15).astype(np.int64) - 8
        hi = (codes >> 4).astype(np.int64) - 8
        w = np.stack([lo, hi], axis=-1)
    else:
        off = 2 if fmt == O.Q2 else 1
        w = np.stack([((codes >> (2 * t)) & 3).astype(np.int64) - off for t in range(4)], axis=-1)
    return w.reshape(rows, nb * 32)


def f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


@pytest.mark.parametrize("fmt", [O.Q4, O.Q2, O.Q15, O.Q8])
@pytest.mark.parametrize("rows,cols,seed", [(7, 256, 1), (33, 1024, 2), (5, 5632, 3)])
def test_gemv_i8_against_float64_brute_force(fmt, rows, cols, seed):
    # y[n] = (float)(S_n * (double)a_s) with S_n the exact sum over k of
    # a_k * w_nk * d_n,b(k): every product is exact in float64 and the sum is
    # taken exactly (math.fsum), elementwise, with no per-block grouping
    rng = np.random.default_rng(seed)
    w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    w[0, :64] *= 40.0                       # scales of one row over a wider range
    codes, scales = O.quantize_matrix(w, fmt)
    a = rng.integers(-127, 128, cols).astype(np.int8)
    a_s = np.float32(rng.uniform(0.001, 0.05))
    y = O.gemv_i8(fmt, codes, scales, a, a_s)
    wc = decode_interchange(fmt, codes)
    d = np.repeat(f16(scales), 32, axis=1)
    for n in range(rows):
        S = math.fsum((a.astype(np.float64) * wc[n].astype(np.float64) * d[n]).tolist())
        want = np.float32(np.float64(S) * np.float64(a_s))
        assert y[n] == want, (n, y[n], want)


def test_gemv_i8_decoder_agrees_with_reference_dequantizers():
    # the brute force's decoder against the oracle's block decoder, which is
    # itself pinned to the reference dequantizer goldens
    rng = np.random.default_rng(9)
    for fmt in (O.Q4, O.Q2, O.Q15, O.Q8):
        w = rng.normal(0, 0.02, (3, 96)).astype(np.float32)
        codes, scales = O.quantize_matrix(w, fmt)
        q = O.qmat(fmt, codes, scales)
        wc = decode_interchange(fmt, codes)
        for r in range(3):
            for c in (0, 1, 17, 31, 32, 63, 95):
                assert O.lib().orc_block_code(C.byref(q), r, c) == wc[r, c]


# ------------------------------------------------------------------ sampling

def samp(temp=0.8, top_p=0.95, top_k=40, greedy=0):
    return O.Sampling(temp, top_p, top_k, greedy)


def ref_sample64(logits, cfg, r):
    """Engine::sample (src/engine.cpp:881-1003) in float64, written from the
    reference text: greedy (first maximum) when greedy or temperature <= 0;
    top-p when 0 < p < 1 (full descending sort, probabilities over the whole
    vocabulary, cutoff = first cumulative >= p, then the first of the nucleus
    whose cumulative reaches r, else scored[cutoff - 1], no renormalisation);
    top-k when 0 < k < V (softmax over the k best, inverse CDF, else the
    last); else full-vocabulary temperature sampling in index order.  Equal
    logits sort by ascending index.  Returns (token, margin): margin is the
    distance of r from the nearest cumulative edge that decided it."""
    x = np.asarray(logits, np.float64)
    V = x.size
    if cfg.greedy or cfg.temperature <= 0:
        return int(np.argmax(x)), 1.0
    T = max(cfg.temperature, 0.001)
    order = sorted(range(V), key=lambda i: (-x[i], i))
    if 0 < cfg.top_p < 1:
        p = np.exp((x[order] - x[order[0]]) / T)
        p /= p.sum()
        cum = np.cumsum(p)
        cutoff = next((i + 1 for i in range(V) if cum[i] >= cfg.top_p), V)
        margin = min(abs(cum[:cutoff] - r).min(), abs(cum[cutoff - 1] - cfg.top_p) + 1.0)
        for i in range(cutoff):
            if r <= cum[i]:
                return order[i], margin
        return order[cutoff - 1], margin
    if 0 < cfg.top_k < V:
        k = cfg.top_k
        p = np.exp((x[order[:k]] - x[order[0]]) / T)
        cum = np.cumsum(p / p.sum())
        margin = abs(cum - r).min()
        for i in range(k):
            if r <= cum[i]:
                return order[i], margin
        return order[k - 1], margin
    p = np.exp((x - x.max()) / T)
    cum = np.cumsum(p / p.sum())
    margin = abs(cum - r).min()
    for i in range(V):
        if r <= cum[i]:
            return i, margin
    return V - 1, margin


CFGS = {
    "greedy": samp(greedy=1),
    "temp0": samp(temp=0.0),
    "top_p": samp(0.8, 0.95, 40),
    "top_p_narrow": samp(1.3, 0.3, 40),
    "top_k": samp(0.7, 1.0, 5),
    "temperature": samp(1.1, 1.0, 0),
    "top_k_ge_V": samp(0.9, 0.0, 64),
}


@pytest.mark.parametrize("name", sorted(CFGS))
@pytest.mark.parametrize("V", [7, 32, 64])
def test_sample_dispatch_against_float64_restatement(name, V):
    cfg = CFGS[name]
    rng = np.random.default_rng(V * 31 + len(name))
    checked = 0
    draw = 0
    for trial in range(60):
        logits = rng.normal(0, 2.0, V).astype(np.float32)
        if trial % 5 == 0:
            logits[rng.integers(0, V, 3)] = logits.max()          # tied maxima
        r = O.lib().orc_uniform(11, draw)
        want, margin = ref_sample64(logits, cfg, r)
        got, nd = O.sample(logits, cfg, 11, draw)
        stochastic = not (cfg.greedy or cfg.temperature <= 0)
        assert nd == draw + (1 if stochastic else 0)
        draw = nd if stochastic else draw + 1
        if margin < 1e-5:
            continue                         # r on a cumulative edge: float32 may go either way
        assert got == want, (name, V, trial, got, want)
        checked += 1
    assert checked >= 50


def test_top_p_falls_back_to_the_last_of_the_nucleus():
    # flat logits: p = 0.3 keeps the first ceil(0.3 V) tokens, whose mass is
    # about 0.3; a draw r above it returns scored[cutoff - 1] (no
    # renormalisation of the nucleus, src/engine.cpp:998-1002)
    V = 10
    logits = np.zeros(V, np.float32)
    cfg = samp(1.0, 0.3, 0)
    idx = next(i for i in range(100) if O.lib().orc_uniform(5, i) > 0.5)
    got, _ = O.sample(logits, cfg, 5, idx)
    assert got == 2          # cutoff = 3 (cumulative 0.1, 0.2, 0.3 >= 0.3), equal logits in index order
    idx = next(i for i in range(100) if O.lib().orc_uniform(5, i) < 0.05)
    got, _ = O.sample(logits, cfg, 5, idx)
    assert got == 0


def test_sampling_ties_go_to_the_lowest_index():
    logits = np.array([0.0, 3.0, 1.0, 3.0, 3.0], np.float32)
    assert O.sample(logits, samp(greedy=1), 0, 0)[0] == 1
    # top-k of 1 with three tied maxima keeps index 1
    assert O.sample(logits, samp(0.5, 1.0, 1), 0, 0)[0] == 1


# ------------------------------------------------------ generate control flow

V16 = 16


def one_hot(t, V=V16, hot=50.0):
    x = np.zeros(V, np.float32)
    x[t % V] = hot
    return x


def chain_model(n_mtp, wrong_at=None):
    """Main model: the greedy next token of t is t + 1 (mod 16).  Heads on
    the hidden state of F(c) propose c + 2, c + 3, ... (the tokens after T1 =
    c + 1); head `wrong_at` proposes a token the main model will not pick."""
    m = None

    def fwd(tok):
        return one_hot(tok + 1)

    def heads(hidden):
        c = m.calls[-1]
        out = np.stack([one_hot(c + 2 + k) for k in range(n_mtp)]) if n_mtp else np.zeros((0, V16))
        if wrong_at is not None:
            out[wrong_at] = one_hot(c + 2 + wrong_at + 7)
        return out

    m = O.ScriptedModel(V16, n_mtp, fwd, heads)
    return m


GREEDY = samp(greedy=1)


def test_generate_full_accept_then_single_token_steps():
    m = chain_model(4)
    rc, toks, acc, rej = m.generate([3], 7, GREEDY)
    assert rc == 0
    # round 1 (0 + 4 <= 7): F(3) -> T1 4; drafts 5 6 7 8 all accepted;
    # then 5 + 4 > 7: single-token steps F(8) -> 9, F(9) -> 10
    assert toks.tolist() == [3, 4, 5, 6, 7, 8, 9, 10]
    assert (acc, rej) == (4, 0)
    # the prompt token is forwarded twice: once in the prompt loop, once as
    # the current token of the first round
    assert m.calls == [3, 3, 4, 5, 6, 7, 8, 9]
    assert m.mtp_calls == 1


@pytest.mark.parametrize("h", [0, 1, 2, 3])
def test_generate_reject_at_head(h):
    m = chain_model(4, wrong_at=h)
    rc, toks, acc, rej = m.generate([3], 4 + h + 1, GREEDY)
    assert rc == 0
    # round 1: T1 = 4, drafts 5 .. accepted up to head h, head h rejected
    # (F(3 + h + 1) gives 5 + h), the greedy corrective 5 + h differs from the
    # draft and is pushed.  Greedy MTP emits exactly the plain greedy chain.
    n1 = 1 + h + 1
    want_calls = [3, 3] + list(range(4, 4 + h + 1))
    assert toks[: 1 + n1].tolist() == list(range(3, 3 + n1 + 1))
    assert m.calls[: len(want_calls)] == want_calls
    # the rest: one more round when it fits (n + 4 <= N), else single steps
    assert toks.tolist() == list(range(3, 3 + 4 + h + 1 + 1))
    rounds_after = 1 if n1 + 4 <= 4 + h + 1 else 0
    assert acc == h + (h if rounds_after else 0)
    assert rej == 1 + rounds_after


def test_generate_overshoots_by_one_when_every_draft_is_accepted():
    # n + 4 <= N gates the round, and a full round commits 5 tokens
    m = chain_model(4)
    rc, toks, acc, rej = m.generate([3], 4, GREEDY)
    assert rc == 0 and toks.tolist() == [3, 4, 5, 6, 7, 8] and (acc, rej) == (4, 0)


def test_generate_empty_prompt_starts_with_a_single_token_step():
    # no prompt: current token 0 and no hidden state yet, so the first step is
    # the single-token path; the next one is an MTP round
    m = chain_model(4)
    rc, toks, acc, rej = m.generate([], 6, GREEDY)
    assert rc == 0
    assert toks.tolist() == [1, 2, 3, 4, 5, 6]
    assert m.calls == [0, 1, 2, 3, 4, 5]
    assert (acc, rej) == (4, 0) and m.mtp_calls == 1


def test_generate_without_heads_is_plain_decoding():
    m = chain_model(0)
    rc, toks, acc, rej = m.generate([9, 2], 5, GREEDY)
    assert rc == 0 and toks.tolist() == [9, 2, 3, 4, 5, 6, 7]
    assert m.calls == [9, 2, 2, 3, 4, 5, 6] and (acc, rej) == (0, 0) and m.mtp_calls == 0


def test_generate_reports_a_too_small_token_buffer():
    m = chain_model(4)
    rc, toks, _, _ = m.generate([3], 7, GREEDY, cap=4)
    assert rc == -1 and toks.tolist() == [3, 4, 5, 6]


def _corrective_script(p_draft_wins):
    """Temperature sampling (top-p 1, top-k 0, T = 1).  Call 0 (prompt), 1
    (F(3), T1 = 4) and the head logits are one-hot; call 2 (verify F(4))
    puts logit 0.1 on token 9 and 0 on the draft 5, the rest at -30, so the
    argmax 9 rejects the draft and the stochastic corrective is 5 with
    probability 1 / (1 + e^0.1) = 0.475 (index order reaches 5 first).
    Later calls are one-hot chains."""
    state = {"n": 0}
    m = None

    def fwd(tok):
        n = state["n"]
        state["n"] += 1
        if n == 2:
            x = np.full(V16, -30.0, np.float32)
            x[9] = 0.1
            x[5] = 0.0
            return x
        return one_hot(tok + 7 if n == 3 else tok + 1)

    def heads(hidden):
        c = m.calls[-1]
        return np.stack([one_hot(c + 2 + k) for k in range(4)])

    m = O.ScriptedModel(V16, 4, fwd, heads)
    return m


def test_generate_drops_a_stochastic_corrective_equal_to_the_draft():
    cfg = samp(1.0, 1.0, 0)
    p5 = 1.0 / (1.0 + math.exp(0.1))
    # draws: T1 (0), drafts (1..4), corrective (5); one-hot draws need r > 0
    def ok(seed, want_drop):
        us = [O.lib().orc_uniform(seed, i) for i in range(9)]
        if min(us) < 1e-3:
            return False
        return (us[5] < p5 - 0.05) if want_drop else (us[5] > p5 + 0.05)

    seed = next(s for s in range(500) if ok(s, True))
    m = _corrective_script(True)
    rc, toks, acc, rej = m.generate([3], 4, cfg, seed=seed)
    # round 1: T1 = 4 pushed; verify F(4) rejects draft 5; the corrective is
    # 5 again, so it is dropped and not counted (src/engine.cpp:357-363);
    # current token = tokens.back() = 4, re-forwarded by the single steps
    # (1 + 4 > 4): F(4) -> 11 (call 3 maps t to t + 7), F(11) -> 12, F(12) -> 13
    assert rc == 0 and (acc, rej) == (0, 0)
    assert toks.tolist() == [3, 4, 11, 12, 13]
    assert m.calls == [3, 3, 4, 4, 11, 12]

    seed = next(s for s in range(500) if ok(s, False))
    m = _corrective_script(False)
    rc, toks, acc, rej = m.generate([3], 4, cfg, seed=seed)
    # the corrective 9 differs from the draft: pushed and counted
    assert rc == 0 and (acc, rej) == (0, 1)
    assert toks.tolist() == [3, 4, 9, 16 % 16, 1]
    assert m.calls == [3, 3, 4, 9, 0]


# ------------------------------------------------------------------ step_mtp

def test_step_mtp_every_draft_accepted():
    m = chain_model(4)
    hidden = np.zeros(8, np.float32)
    m.calls.append(3)                       # heads read the last forwarded token
    k, logits, a, r, _ = m.step_mtp(4, hidden, 1, GREEDY)
    # drafts 5 6 7 8; verify inputs current_token, 5, 6, 7 (src/engine.cpp:425-427)
    assert (k, a, r) == (4, 4, 0) and logits is None
    assert m.calls[1:] == [4, 5, 6, 7]


@pytest.mark.parametrize("h", [0, 1, 3])
def test_step_mtp_rejection_returns_its_logits(h):
    m = chain_model(4, wrong_at=h)
    m.calls.append(3)
    k, logits, a, r, _ = m.step_mtp(4, np.zeros(8, np.float32), 1, GREEDY)
    # the rejecting forward is of the input 4 + h; mtp_accepted_out stays 0
    # and mtp_rejected_out = heads - accepted (src/engine.cpp:437-440)
    assert (k, a, r) == (h, 0, 4 - h)
    assert np.array_equal(logits, one_hot(4 + h + 1))
    assert m.calls[1:] == list(range(4, 4 + h + 1))


def test_step_mtp_without_table_or_heads_is_one_forward():
    for m, has_table in ((chain_model(4), 0), (chain_model(0), 1)):
        k, logits, a, r, d = m.step_mtp(6, np.zeros(8, np.float32), has_table, samp())
        assert (k, a, r, d) == (0, 0, 0, 0) and np.array_equal(logits, one_hot(7))
        assert m.calls == [6] and m.mtp_calls == 0


def test_step_mtp_draws_one_uniform_per_head():
    m = chain_model(4)
    m.calls.append(3)
    k, logits, a, r, d = m.step_mtp(4, np.zeros(8, np.float32), 1, samp(0.8, 0.95, 40), seed=42, draw=10)
    assert d == 14 and (k, a, r) == (4, 4, 0)


# ---------------------------------------------------------------------- RoPE

@pytest.mark.parametrize("hd", [64, 128])
def test_rope_table_closed_form(hd):
    # angle of pair t at position p: p * theta^(-2t / hd), theta = 5e6
    # (src/engine.cpp:656-682); float rounding of the frequency and of the
    # product bounds the angle error by |angle| * 2^-22
    L = O.lib()
    half = hd // 2
    c = np.zeros(half, np.float32)
    s = np.zeros(half, np.float32)
    for p in (0, 1, 7, 300, 2049, 32767):
        L.orc_rope_table(hd, p, P(c, O.f32p), P(s, O.f32p))
        ang = p * np.power(5e6, -2.0 * np.arange(half) / hd)
        tol = np.abs(ang) * 2.0 ** -22 + 2e-7
        assert np.all(np.abs(c - np.cos(ang)) <= tol), p
        assert np.all(np.abs(s - np.sin(ang)) <= tol), p
    L.orc_rope_table(hd, 0, P(c, O.f32p), P(s, O.f32p))
    assert np.all(c == 1.0) and np.all(s == 0.0)


def test_rope_rotation_closed_form():
    # (x0 + i x1) * e^{i angle}: a rotation of each pair, norm preserved
    L = O.lib()
    rng = np.random.default_rng(4)
    hd = 128
    c = np.zeros(hd // 2, np.float32)
    s = np.zeros(hd // 2, np.float32)
    for p in (1, 100, 5000):
        L.orc_rope_table(hd, p, P(c, O.f32p), P(s, O.f32p))
        x = rng.normal(0, 1, hd).astype(np.float32)
        y = x.copy()
        L.orc_rope_rotate(P(y, O.f32p), hd, P(c, O.f32p), P(s, O.f32p))
        z = (x[0::2].astype(np.float64) + 1j * x[1::2]) * (c.astype(np.float64) + 1j * s)
        np.testing.assert_allclose(y[0::2], z.real, rtol=0, atol=2e-6)
        np.testing.assert_allclose(y[1::2], z.imag, rtol=0, atol=2e-6)
        np.testing.assert_allclose(np.hypot(y[0::2], y[1::2]), np.hypot(x[0::2], x[1::2]), rtol=1e-5)
