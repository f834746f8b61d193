"""Summary of the persistent decode pass's phase timeline.

With PF_PERSISTENT=1 and PF_DECODE_TRACE=<file>, a profiled verify pass
(Engine.profile(True)) records, per layer and workgroup, the wall-clock
time (100 MHz) at which each phase point was reached, and pf_generate
writes them to <file>: three uint64 header words (layers, workgroups, words
per workgroup), then [layers][workgroups][words] timestamps (0 = not
reached).  This prints, per layer, the minimum / median / maximum time of
each point in microseconds from the first timestamp of the pass.

Usage: python -m pocketforge_amd.decode_trace <file> [layer,layer,...]
"""
import sys

import numpy as np

# Phase points in the order of their slots (pf_decode.hip, TR_*).
POINTS = ["Q_WAIT", "Q_NORM", "Q_DONE", "A_WAIT", "A_QKV", "A_DONE", "MERGE", "O_WAIT", "O_DONE", "O_FIN",
          "G_WAIT", "G_DONE", "G_FIN", "D_WAIT", "D_DONE", "D_FIN", "A_KVQ", "A_SELF", "A_SCORE", "A_EXP",
          "A_WSUM", "G_NORM", "O_AMAX", "D_AMAX", "SA_BEG", "SA_END", "SF_BEG", "SF_END", "Q_STATS", "G_STATS",
          "M_T", "M_END"]


def load(path):
    b = np.fromfile(path, dtype=np.uint64)
    L, G, T = (int(v) for v in b[:3])
    t = b[3:3 + L * G * T].reshape(L, G, T).astype(np.int64)
    t0 = t[t > 0].min()
    return np.where(t > 0, (t - t0) * 0.01, np.nan)   # microseconds


def summary(us, layers):
    L, G, T = us.shape
    lines = [f"workgroups {G}, layers {L}"]
    for l in layers:
        lines.append(f"layer {l}")
        order = sorted(range(T), key=lambda k: np.nanmedian(us[l, :, k]) if np.isfinite(us[l, :, k]).any() else 1e18)
        for k in order:
            v = us[l, :, k]
            v = v[np.isfinite(v)]
            if v.size == 0:
                continue
            name = POINTS[k] if k < len(POINTS) else f"slot{k}"
            lines.append(f"  {name:8s} n={v.size:4d} min {v.min():9.2f} med {np.median(v):9.2f} max {v.max():9.2f}")
    ends = [np.nanmax(us[l]) for l in range(L)]
    lines.append("per-layer span (us): " + " ".join(f"{d:.1f}" for d in np.diff([0.0] + ends)))
    return "\n".join(lines)


def main(argv):
    if len(argv) < 2:
        print(__doc__)
        return 2
    us = load(argv[1])
    layers = [int(x) for x in argv[2].split(",")] if len(argv) > 2 else [0, 1, us.shape[0] // 2]
    print(summary(us, layers))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
