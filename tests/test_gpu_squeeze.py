"""A model loaded from a .squeeze file (pf_squeeze_load_model: host decode,
repack to the device layout, upload) runs bit-exact with the oracle over the
same decoded weights, and with the same weights uploaded from Python."""
import numpy as np
import pytest

import oracle as O
import pocketforge_amd as pf
from pocketforge_amd import weights as W
import squeeze_writer as SW

from test_gpu_engine import GREEDY, KV

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=2, n_embd=256, n_heads=4, head_dim=64, n_ff=512, n_vocab=1024, n_mtp=4)
NAMES = ["wq", "wk", "wv", "wo", "wgate", "wup", "wdown"]
QT = [SW.Q4, SW.Q4, SW.Q4, SW.Q4, SW.Q2, SW.Q2, SW.Q15]
QT8 = [SW.Q8] * 7
FMT = {SW.Q4: pf.FMT_Q4, SW.Q2: pf.FMT_Q2, SW.Q15: pf.FMT_Q15, SW.Q8: pf.FMT_Q8}


def _write(path, seed=5, qt=QT, emb_qt=SW.Q4):
    rng = np.random.default_rng(seed)
    D, F, V = CFG["n_embd"], CFG["n_ff"], CFG["n_vocab"]
    shapes = [(D, D)] * 4 + [(F, D), (F, D), (D, F)]
    blocks = []
    for l in range(CFG["n_layers"]):
        for m, (r, c) in enumerate(shapes):
            std = 0.3 if qt[m] == SW.Q15 else 0.02
            blocks.append((l, m, (std * rng.standard_normal((r, c))).astype(np.float32), qt[m]))
        blocks.append((l, 7, (1 + 0.1 * rng.standard_normal((1, D))).astype(np.float32), SW.Q8))
        blocks.append((l, 8, (1 + 0.1 * rng.standard_normal((1, D))).astype(np.float32), SW.Q8))
    blocks.append((0, 10, (0.02 * rng.standard_normal((V, D))).astype(np.float32), emb_qt))
    hdr = dict(n_layers=CFG["n_layers"], n_embd=D, n_heads=CFG["n_heads"], n_kv_heads=CFG["n_heads"], n_ff=F,
               n_vocab=V, max_seq_len=512, mtp_heads=CFG["n_mtp"])
    SW.write_squeeze(str(path), hdr, blocks)


def _pack(codes, mult, qt):
    """Interchange layout ([rows][cols/32][16|8] codes, fp16 scales) of decoded
    codes, written independently of the library's repack."""
    rows, cols = codes.shape
    c = codes.reshape(rows, cols // 32, 32).astype(np.int64)
    if qt == SW.Q8:
        packed = c.astype(np.int8).view(np.uint8)
    elif qt == SW.Q4:
        u = (c + 8).astype(np.uint8)
        packed = (u[..., 0::2] | (u[..., 1::2] << 4)).astype(np.uint8)
    else:
        u = (c + (2 if qt == SW.Q2 else 1)).astype(np.uint8)
        packed = (u[..., 0::4] | (u[..., 1::4] << 2) | (u[..., 2::4] << 4) | (u[..., 3::4] << 6)).astype(np.uint8)
    scales = mult.astype(np.float16).view(np.uint16).reshape(rows, cols // 32)
    return FMT[qt], np.ascontiguousarray(packed), np.ascontiguousarray(scales)


def _decoded_weights(path, mtp):
    s = pf.Squeeze(path)
    layers = []
    an, fn = [], []
    for l in range(CFG["n_layers"]):
        lw = {}
        for m, n in enumerate(NAMES):
            codes, mult, qt = s.load_block(l, m)
            lw[n] = _pack(codes, mult, qt)
        layers.append(lw)
        for m, dst in ((7, an), (8, fn)):
            codes, mult, _ = s.load_block(l, m)
            dst.append(codes.reshape(-1).astype(np.float32) * np.repeat(mult, 32)[:codes.size])
    codes, mult, qt = s.load_block(0, 10)
    emb = _pack(codes, mult, qt)
    s.close()
    return dict(layers=layers, emb=emb, mtp=mtp, attn_norm=np.stack(an), ffn_norm=np.stack(fn))


@pytest.fixture(scope="module")
def squeezed(tmp_path_factory):
    p = tmp_path_factory.mktemp("sq") / "tiny.squeeze"
    _write(p)
    mtp = W.make_weights(dict(CFG), seed=9)["mtp"]
    return p, mtp, _decoded_weights(p, mtp)


@pytest.fixture(scope="module")
def squeezed_q8(tmp_path_factory):
    """Every layer matrix and the embedding table in Q8_0.  The file's Q8 rule
    round(x s + 0.5) turns each block's positive maximum (x s = 127) into 128,
    stored as the byte 0x80 = -128, so every block holds a -128 code."""
    p = tmp_path_factory.mktemp("sq8") / "tiny_q8.squeeze"
    _write(p, seed=6, qt=QT8, emb_qt=SW.Q8)
    mtp = W.make_weights(dict(CFG), seed=10)["mtp"]
    w = _decoded_weights(p, mtp)
    return p, mtp, w


def test_squeeze_model_forward_matches_oracle(gpu, squeezed):
    p, mtp, w = squeezed
    m = pf.Model.from_squeeze(gpu, p, mtp=mtp)
    assert m.cfg == CFG
    e = pf.Engine(m, **KV)
    c = dict(CFG)
    c.update(KV)
    om = O.Model(c, w)
    m2 = pf.Model(gpu, CFG, w)
    e2 = pf.Engine(m2, **KV)
    toks = W.prompt_ids(12, CFG["n_vocab"], seed=3)
    for t in toks:
        lg, hg = e.forward([t])
        lo, ho = om.forward(t)
        lg2, hg2 = e2.forward([t])
        np.testing.assert_array_equal(hg[0], ho)
        np.testing.assert_array_equal(lg[0], lo)
        np.testing.assert_array_equal(lg2[0], lg[0])
    for x in (e, e2, om, m, m2):
        x.close()


def test_squeeze_model_generate_matches_oracle(gpu, squeezed):
    p, mtp, w = squeezed
    m = pf.Model.from_squeeze(gpu, p, mtp=mtp)
    e = pf.Engine(m, **KV)
    prompt = W.prompt_ids(10, CFG["n_vocab"], seed=8)
    toks, res = e.generate(prompt, 30, GREEDY, 7)
    c = dict(CFG)
    c.update(KV)
    om = O.Model(c, w)
    ot, oa, orj = om.generate(prompt, 30, O.Sampling(0.8, 0.95, 40, 1), 7)
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)
    for x in (e, om, m):
        x.close()


def test_squeeze_q8_model_matches_oracle(gpu, squeezed_q8):
    """Q8_0 layer matrices and embedding table run on the device as signed
    bytes (the -128 codes included), bit-exact with the oracle's forward and
    MTP generation over the same decoded weights."""
    p, mtp, w = squeezed_q8
    assert all(w["layers"][l][n][0] == pf.FMT_Q8 for l in range(CFG["n_layers"]) for n in NAMES)
    assert w["emb"][0] == pf.FMT_Q8
    assert (w["layers"][0]["wq"][1] == 0x80).any()
    m = pf.Model.from_squeeze(gpu, p, mtp=mtp)
    e = pf.Engine(m, **KV)
    c = dict(CFG)
    c.update(KV)
    om = O.Model(c, w)
    for t in W.prompt_ids(10, CFG["n_vocab"], seed=4):
        lg, hg = e.forward([t])
        lo, ho = om.forward(t)
        np.testing.assert_array_equal(hg[0], ho)
        np.testing.assert_array_equal(lg[0], lo)
    om.close()
    e.close()
    e = pf.Engine(m, **KV)
    om = O.Model(c, w)
    prompt = W.prompt_ids(9, CFG["n_vocab"], seed=11)
    toks, res = e.generate(prompt, 24, GREEDY, 5)
    ot, oa, orj = om.generate(prompt, 24, O.Sampling(0.8, 0.95, 40, 1), 5)
    np.testing.assert_array_equal(toks, ot)
    assert (res.mtp_accepted, res.mtp_rejected) == (oa, orj)
    for x in (e, om, m):
        x.close()


def test_squeeze_model_rejects_unsupported(gpu, tmp_path):
    """Grouped KV heads have no device path; a missing matrix is an error."""
    D = 256
    hdr = dict(n_layers=1, n_embd=D, n_heads=4, n_kv_heads=4, n_ff=D, n_vocab=64, mtp_heads=0)
    ws = [(0, m, np.ones((D, D), np.float32) * 0.01, SW.Q4) for m in range(7)]
    p = tmp_path / "gqa.squeeze"
    SW.write_squeeze(str(p), dict(hdr, n_kv_heads=2), ws)
    with pytest.raises(pf.PFError, match="grouped"):
        pf.Model.from_squeeze(gpu, p)
    p2 = tmp_path / "short.squeeze"
    SW.write_squeeze(str(p2), hdr, ws[1:3])
    with pytest.raises(pf.PFError, match="missing"):
        pf.Model.from_squeeze(gpu, p2)
