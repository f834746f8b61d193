"""Writes the oracle's token streams at the benchmark configurations' full
sizes, for the GPU parity tests of tests/test_gpu_configs.py: the same
seeded weights (pocketforge_amd.weights, seed 1234), prompts (prompt_ids)
and sampling as bench.py, run through the C restatement (oracle/) on the
host.  The 1B runs take minutes (B: 13 minutes on 6 host cores),
up to an hour (one sequence of configuration E, 8192-token prompt; B-long's
geometry with a 5000-token prompt), so their outputs are kept
here as fixtures: stream_<name>.npz with the prompt length, the generated
tokens (prompt included) and the acceptance counters.

Run:  python tests/golden/make_config_streams.py [B B-mix E0 B-long-5k]
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as O  # noqa: E402
from pocketforge_amd import weights as W  # noqa: E402

# name: (model, formats, (sink, window, pool), prompt length, prompt seed, generated, sampling)
STREAMS = {
    "B": ("ONE_B", "ALL_Q4", (4, 8192, 64), 2048, 42, 64, (0.8, 0.95, 40, 1)),
    "B-mix": ("ONE_B", "MIXED", (4, 8192, 64), 1024, 42, 64, (0.8, 0.95, 40, 0)),
    "E0": ("ONE_B", "ALL_Q4", (4, 8192, 64), 8192, 42, 32, (0.8, 0.95, 40, 1)),
    # B-long's cache geometry on the 1B model with a 5000-token prompt: the
    # window is full and 56 pooled rows exist before decoding starts (the
    # 32768-token prompt itself would take hours in the oracle)
    "B-long-5k": ("ONE_B", "ALL_Q4", (4, 4096, 16), 5000, 42, 32, (0.8, 0.95, 40, 1)),
}
SEED = 7


def kv_of(spec):
    sink, window, pool = spec[2]
    return dict(sink_size=sink, window_size=window, pool_block=pool, max_context=spec[3] + spec[5] + 64)


def run(name):
    spec = STREAMS[name]
    cfg = getattr(W, spec[0])
    w = W.make_weights(cfg, seed=1234, fmts=getattr(W, spec[1]))
    prompt = W.prompt_ids(spec[3], cfg["n_vocab"], seed=spec[4])
    c = dict(cfg)
    c.update(kv_of(spec))
    om = O.Model(c, w)
    t = time.time()
    toks, acc, rej = om.generate(prompt, spec[5], O.Sampling(*spec[6]), SEED)
    om.close()
    out = os.path.join(HERE, f"stream_{name}.npz")
    np.savez(out, n_prompt=np.int64(spec[3]), tokens=np.asarray(toks, np.int32), accepted=np.int64(acc),
             rejected=np.int64(rej))
    print(f"{name}: {len(toks) - spec[3]} tokens, accepted {acc}, rejected {rej}, {time.time() - t:.0f}s -> {out}",
          flush=True)


if __name__ == "__main__":
    for n in sys.argv[1:] or list(STREAMS):
        run(n)
