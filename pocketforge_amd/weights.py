"""Model shapes of the benchmark configurations and synthetic weights.

Weights are N(0, 0.02^2) from Philox4x32-10 + Box-Muller (seed 1234, one
stream per matrix), quantized to 32-element blocks with an fp16 scale on the
host (pf_gen_matrix).  RMSNorm weights are 1.0, the reference's fallback
(src/engine.cpp:171-173).  The tied embedding table is Q4; MTP heads are
n_embd x n_embd Q4 matrices (src/engine.cpp:79: ff = n_embd).
"""
import numpy as np

from . import FMT_Q2, FMT_Q4, FMT_Q15, gen_matrix

# 150M: 12 layers, hidden 768, 12 heads x 64, SwiGLU 2048, vocab 16384
SMALL = dict(n_layers=12, n_embd=768, n_heads=12, head_dim=64, n_ff=2048, n_vocab=16384, n_mtp=4)
# 1B-class: 24 layers, hidden 2048, 16 heads x 128, SwiGLU 5632, vocab 16384
ONE_B = dict(n_layers=24, n_embd=2048, n_heads=16, head_dim=128, n_ff=5632, n_vocab=16384, n_mtp=4)
# A few-layer model for parity tests
TINY = dict(n_layers=2, n_embd=256, n_heads=4, head_dim=64, n_ff=512, n_vocab=1024, n_mtp=4)

ALL_Q4 = dict(attn=FMT_Q4, gate_up=FMT_Q4, down=FMT_Q4)
# attention Q4, FFN up/gate Q2, FFN down Q1.5
MIXED = dict(attn=FMT_Q4, gate_up=FMT_Q2, down=FMT_Q15)

NAMES = ["wq", "wk", "wv", "wo", "wgate", "wup", "wdown"]


def make_weights(cfg, seed=1234, std=0.02, fmts=ALL_Q4):
    D, F, V = cfg["n_embd"], cfg["n_ff"], cfg["n_vocab"]
    shapes = {"wq": (D, D), "wk": (D, D), "wv": (D, D), "wo": (D, D), "wgate": (F, D), "wup": (F, D),
              "wdown": (D, F)}
    kinds = {"wq": "attn", "wk": "attn", "wv": "attn", "wo": "attn", "wgate": "gate_up", "wup": "gate_up",
             "wdown": "down"}
    layers = []
    for l in range(cfg["n_layers"]):
        lw = {}
        for j, n in enumerate(NAMES):
            fmt = fmts[kinds[n]]
            r, c = shapes[n]
            codes, scales = gen_matrix(seed, l * 16 + j, std, r, c, fmt)
            lw[n] = (fmt, codes, scales)
        layers.append(lw)
    codes, scales = gen_matrix(seed, 0x10000, std, V, D, FMT_Q4)
    emb = (FMT_Q4, codes, scales)
    mtp = []
    for k in range(cfg["n_mtp"]):
        hw = {}
        for j, n in enumerate(["gate", "up", "down"]):
            codes, scales = gen_matrix(seed, 0x20000 + 3 * k + j, std, D, D, FMT_Q4)
            hw[n] = (FMT_Q4, codes, scales)
        mtp.append(hw)
    ones = np.ones((max(1, cfg["n_layers"]), D), np.float32)
    return dict(layers=layers, emb=emb, mtp=mtp, attn_norm=ones, ffn_norm=ones.copy())


def packed_bytes(w):
    """Bytes of every weight matrix as the GPU stores them (codes + fp16 scales)."""
    tot = 0
    for lw in w["layers"]:
        for n in NAMES:
            _, codes, scales = lw[n]
            tot += codes.nbytes + scales.nbytes
    return tot


def prompt_ids(n, vocab, seed=42):
    """Uniform random prompt ids in [0, vocab)."""
    rng = np.random.default_rng(seed)
    return rng.integers(0, vocab, n, dtype=np.int32)
