""".squeeze files read by the library's host loader (pf_squeeze_*, no GPU
use) against files written by tests/squeeze_writer.py, a restatement of the
reference's writer (src/quant_format.cpp:41-217), and the checks of the
reference's own tests/test_quant_format.cpp: the configuration round trip,
block count and shape, a missing block, the code rules of each quant type."""
import numpy as np
import pytest

import pocketforge_amd as pf
import squeeze_writer as SW

CFG = dict(n_layers=2, n_embd=64, n_heads=2, n_kv_heads=2, n_ff=128, n_vocab=96, max_seq_len=512, mtp_heads=4)


def _blocks(seed=42):
    rng = np.random.default_rng(seed)
    D, F = CFG["n_embd"], CFG["n_ff"]
    shapes = [(D, D)] * 4 + [(F, D), (F, D), (D, F)]
    out = []
    for l in range(CFG["n_layers"]):
        for m, (r, c) in enumerate(shapes):
            w = rng.uniform(-1, 1, (r, c)).astype(np.float32)
            out.append((l, m, w, [SW.Q4, SW.Q2, SW.Q15][(l * 7 + m) % 3]))
        out.append((l, 7, (1 + 0.1 * rng.standard_normal((1, D))).astype(np.float32), SW.Q8))
        out.append((l, 8, (1 + 0.1 * rng.standard_normal((1, D))).astype(np.float32), SW.Q8))
    out.append((0, 10, (0.02 * rng.standard_normal((CFG["n_vocab"], D))).astype(np.float32), SW.Q4))
    return out


def _decode(w, qt):
    """Codes and block multipliers the writer's rule gives for w (a second,
    float64 restatement used to check the library's decode)."""
    x = w.astype(np.float64).reshape(-1)
    nb = (x.size + 31) // 32
    codes = np.zeros(x.size, np.int64)
    mult = np.zeros(nb, np.float32)
    for b in range(nb):
        v = x[32 * b:32 * b + 32]
        if qt == SW.Q15:
            codes[32 * b:32 * b + len(v)] = np.where(v > np.float32(0.35), 1, np.where(v < np.float32(-0.35), -1, 0))
            mult[b] = 1.0
            continue
        amax = np.float32(np.abs(v).max())
        num = {SW.Q8: 127, SW.Q4: 7, SW.Q2: 1}[qt]
        s = np.float32(0) if amax == 0 else np.float32(np.float32(num) / amax)
        y = (v.astype(np.float32) * s).astype(np.float32)
        if qt == SW.Q8:
            y = (y + np.float32(0.5)).astype(np.float32)
        r = np.where(y >= 0, np.floor(y.astype(np.float64) + 0.5), -np.floor(-y.astype(np.float64) + 0.5))
        if qt == SW.Q4:
            r = np.clip(r, -8, 7)
        elif qt == SW.Q2:
            r = np.clip(r, -2, 1)
        else:
            r = (r.astype(np.int64) + 128) % 256 - 128
        codes[32 * b:32 * b + len(v)] = r
        mult[b] = 0 if s == 0 else np.float32(1) / s
    return codes.reshape(w.shape), mult


@pytest.fixture(scope="module")
def sqfile(tmp_path_factory):
    p = tmp_path_factory.mktemp("sq") / "tiny.squeeze"
    blocks = _blocks()
    SW.write_squeeze(str(p), CFG, blocks)
    return p, blocks


def test_config_and_index_round_trip(sqfile):
    p, blocks = sqfile
    s = pf.Squeeze(p)
    i = s.info()
    for k in ("n_layers", "n_embd", "n_heads", "n_kv_heads", "n_ff", "n_vocab", "max_seq_len", "mtp_heads"):
        assert i[k] == CFG[k], k
    assert i["n_blocks"] == len(blocks) and i["version"] == 1
    for l, m, w, qt in blocks:
        assert s.block_shape(l, m) == (w.shape[0], w.shape[1], qt)
    with pytest.raises(pf.PFError):
        s.load_block(99, 99)          # a missing block (test_quant_format.cpp:139-140)
    s.close()


def test_blocks_decode_to_the_writer_codes_and_scales(sqfile):
    p, blocks = sqfile
    s = pf.Squeeze(p)
    for l, m, w, qt in blocks:
        codes, mult, q = s.load_block(l, m)
        ec, em = _decode(w, qt)
        np.testing.assert_array_equal(codes.astype(np.int64), ec, err_msg=f"codes {l},{m}")
        np.testing.assert_array_equal(mult, em, err_msg=f"scales {l},{m}")
        if qt in (SW.Q4, SW.Q2):
            # round trip inside half a step (Q2 also clips at +1 step)
            val = codes.reshape(-1, 32).astype(np.float64) * mult[:, None]
            step = mult[:, None].astype(np.float64)
            err = np.abs(val - w.reshape(-1, 32))
            lim = 0.5 * step * (1 + 1e-5) if qt == SW.Q4 else 1.0 * step * (1 + 1e-5)
            assert np.all(err <= lim), (l, m)
    s.close()


def test_code_rules_known_answers(tmp_path):
    """One block per type with hand-checked codes: amax maps to the top code,
    Q4 nibbles and Q2 fields sit low-first, Q1.5 thresholds at +-0.35."""
    x = np.zeros((1, 32), np.float32)
    x[0, :6] = [2.0, -2.0, 1.0, 0.5, -0.36, 0.34]
    p = tmp_path / "ka.squeeze"
    SW.write_squeeze(str(p), dict(CFG, n_layers=1), [(0, 0, x, SW.Q4), (0, 1, x, SW.Q2), (0, 2, x, SW.Q15),
                                                    (0, 3, x, SW.Q8)])
    s = pf.Squeeze(p)
    c4, m4, _ = s.load_block(0, 0)
    assert list(c4[0, :6]) == [7, -7, 4, 2, -1, 1] and m4[0] == np.float32(1) / np.float32(7.0 / 2.0)
    c2, m2, _ = s.load_block(0, 1)
    assert list(c2[0, :6]) == [1, -1, 1, 0, 0, 0] and m2[0] == np.float32(2.0)
    c15, m15, _ = s.load_block(0, 2)
    assert list(c15[0, :6]) == [1, -1, 1, 1, -1, 0] and m15[0] == 1.0
    c8, m8, _ = s.load_block(0, 3)
    # round(x * 63.5 + 0.5): 127.5 + 0.5 -> 128 wraps to -128 as an int8
    assert list(c8[0, :4]) == [-128, -127, 64, 32]
    s.close()


def test_malformed_files_are_rejected(tmp_path):
    p = tmp_path / "bad.squeeze"
    p.write_bytes(b"NOTFORGE" + bytes(300))
    with pytest.raises(pf.PFError, match="magic"):
        pf.Squeeze(p)
    p.write_bytes(b"FORGE" + bytes(10))
    with pytest.raises(pf.PFError):
        pf.Squeeze(p)
    good = tmp_path / "t.squeeze"
    SW.write_squeeze(str(good), dict(CFG, n_layers=1), [(0, 0, np.ones((64, 64), np.float32), SW.Q4)])
    raw = bytearray(good.read_bytes())
    raw[12:16] = (1000).to_bytes(4, "little")    # index longer than the file
    p.write_bytes(bytes(raw))
    with pytest.raises(pf.PFError, match="index"):
        pf.Squeeze(p)
    with pytest.raises(pf.PFError):
        pf.Squeeze(tmp_path / "missing.squeeze")
