"""Writes the golden fixtures in this directory by running the reference's own
translation units (src/matmul_neon.cpp, src/kv_cache.cpp, src/mtp.cpp),
compiled from /root/reference by oracle/Makefile (`make -C oracle ref`).

Two builds are recorded: the reference's CMake x86 flags (-O3 -march=native,
which contract `a += b * c` into FMA) and -O2 -ffp-contract=off.  Integer
outputs must agree between them; float outputs may differ in the last bits.

Run:  python tests/golden/make_golden.py
Outputs: ref_kernels.npz, ref_kv.npz, ref_mtp.npz (inputs and outputs).
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as O  # noqa: E402

f32p, i8p, u8p, i32p = O.f32p, O.i8p, O.u8p, O.i32p


def P(a, t):
    return a.ctypes.data_as(t)


def kernels(R, tag, out):
    rng = np.random.default_rng(1234)
    # quantize_activation_row (src/matmul_neon.cpp:16-29)
    xs = [rng.standard_normal(96).astype(np.float32) * 0.7,
          np.zeros(64, np.float32),
          (np.arange(-20, 20, dtype=np.float32) / 4.0),     # many .5 ties
          np.array([0.5, -1.0, 0.0, 0.75, -0.25, 1.0, -0.5, 0.1], np.float32)]
    for i, x in enumerate(xs):
        q = np.zeros(x.size, np.int8)
        s = np.zeros(1, np.float32)
        R.ref_quantize_activation_row(P(x, f32p), P(q, i8p), P(s, f32p), x.size)
        out[f"qa{i}_x"] = x
        out[f"qa{i}_q_{tag}"] = q
        out[f"qa{i}_s_{tag}"] = s
    # dequantizers (src/matmul_neon.cpp:34-75)
    b = rng.integers(0, 256, 64, dtype=np.uint8)
    out["dq_bytes"] = b
    for name, n in (("q4", 128), ("q2", 256), ("ternary", 128)):
        o = np.zeros(n, np.int8)
        getattr(R, f"ref_dequant_{name}_to_int8")(P(b, u8p), P(o, i8p), n)
        out[f"dq_{name}_{tag}"] = o
    # matmul_int8 / matmul_quantized (src/matmul_neon.cpp:80-181)
    M, N, K = 5, 7, 96
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    B = rng.integers(-8, 8, (N, K), dtype=np.int8)
    Ci = np.zeros((M, N), np.int32)
    R.ref_matmul_int8(P(A, i8p), P(B, i8p), P(Ci, i32p), M, N, K)
    out["mm_A"], out["mm_B"], out[f"mm_C_{tag}"] = A, B, Ci
    Af = (rng.standard_normal((M, K)) * 0.5).astype(np.float32)
    ws = (rng.random(N) * 0.02 + 0.001).astype(np.float32)
    asc = (rng.random(M) * 0.01 + 0.001).astype(np.float32)
    Cf = np.zeros((M, N), np.float32)
    R.ref_matmul_quantized(P(Af, f32p), P(B, i8p), P(Cf, f32p), M, N, K, P(ws, f32p), None)
    Cf2 = np.zeros((M, N), np.float32)
    R.ref_matmul_quantized(P(Af, f32p), P(B, i8p), P(Cf2, f32p), M, N, K, P(ws, f32p), P(asc, f32p))
    out["mq_A"], out["mq_ws"], out["mq_as"] = Af, ws, asc
    out[f"mq_C_{tag}"], out[f"mq_Cas_{tag}"] = Cf, Cf2
    # dot / softmax / rmsnorm (src/matmul_neon.cpp:186-239)
    a = rng.standard_normal(300).astype(np.float32)
    b2 = rng.standard_normal(300).astype(np.float32)
    R.ref_dot_product.argtypes = [f32p, f32p, C.c_uint32]
    out["dot_a"], out["dot_b"] = a, b2
    out[f"dot_{tag}"] = np.float32(R.ref_dot_product(P(a, f32p), P(b2, f32p), 300))
    for i, n in enumerate((5, 257, 3000)):
        v = (rng.standard_normal(n) * 3).astype(np.float32)
        out[f"sm{i}_x"] = v.copy()
        R.ref_softmax(P(v, f32p), n)
        out[f"sm{i}_{tag}"] = v
        x = (rng.standard_normal(n) * 2).astype(np.float32)
        w = (rng.random(n) + 0.5).astype(np.float32)
        o = np.zeros(n, np.float32)
        R.ref_rmsnorm(P(o, f32p), P(x, f32p), P(w, f32p), n)
        out[f"rn{i}_x"], out[f"rn{i}_w"], out[f"rn{i}_{tag}"] = x, w, o


KV_CFGS = {
    # (layers, heads, hd, sink, window, pool, max_ctx, n_stores)
    "t": (2, 2, 4, 2, 16, 4, 128, 40),      # tests/test_kv_cache.cpp:22-29 shape
    "p": (1, 2, 32, 4, 24, 5, 400, 150),    # pooled blocks of 5
    "s": (1, 1, 16, 10, 12, 3, 60, 70),     # sink_size > 8 (rows 8, 9 dropped), pos >= max_context
}


def kv(R, tag, out):
    for key, (L, H, hd, sink, win, pool, maxc, n) in KV_CFGS.items():
        rng = np.random.default_rng(99)
        k = R.ref_kv_create(L, H, hd, sink, win, pool, maxc)
        keys = (rng.standard_normal((n, L, H, hd)) * 1.5).astype(np.float32)
        vals = (rng.standard_normal((n, L, H, hd)) * 1.5).astype(np.float32)
        qs = rng.standard_normal((8, hd)).astype(np.float32)
        out[f"{key}_keys"], out[f"{key}_vals"], out[f"{key}_qs"] = keys, vals, qs
        checkpoints = sorted(set([1, 3, sink + 1, sink + win, sink + win + pool, n // 2, n]))
        out[f"{key}_ckpt"] = np.array(checkpoints, np.int32)
        stored = 0
        for c in checkpoints:
            while stored < c:
                for l in range(L):
                    for h in range(H):
                        R.ref_kv_store(k, l, h, stored, P(keys[stored, l, h], f32p),
                                       P(vals[stored, l, h], f32p))
                stored += 1
            sc = np.zeros((L, H, 8, win + 64 + maxc), np.float32)
            cnt = np.zeros((L, H), np.int32)
            ws = np.zeros((L, H, 8, hd), np.float32)
            for l in range(L):
                for h in range(H):
                    for qi in range(8):
                        nn = R.ref_kv_attention_scores(k, l, h, P(qs[qi], f32p), P(sc[l, h, qi], f32p))
                        cnt[l, h] = nn
                        p = sc[l, h, qi, :nn].copy()
                        p = np.exp(p - p.max()).astype(np.float32)
                        p = (p / p.sum()).astype(np.float32)
                        R.ref_kv_attention_weighted_sum(k, l, h, P(p, f32p), P(ws[l, h, qi], f32p), nn)
            m = int(cnt.max())
            out[f"{key}_c{c}_count"] = cnt
            out[f"{key}_c{c}_scores_{tag}"] = sc[..., :m]
            out[f"{key}_c{c}_wsum_{tag}"] = ws
            out[f"{key}_c{c}_size"] = np.int32(R.ref_kv_size(k))
        R.ref_kv_clear(k)
        out[f"{key}_size_after_clear"] = np.int32(R.ref_kv_size(k))
        R.ref_kv_destroy(k)
    # the 131K-context memory bound (tests/test_kv_cache.cpp:82-94)
    k = R.ref_kv_create(24, 4, 64, 4, 8192, 64, 131072)
    out["kv_big_memory"] = np.uint64(R.ref_kv_memory_usage(k))
    R.ref_kv_destroy(k)


def mtp(R, tag, out):
    """MTPHeads::forward (src/mtp.cpp:47-129) on chosen weights: per-row
    scales that are exact fp16 values, so the same matrices are expressible
    as 32-block fp16 matrices with all blocks of a row sharing d."""
    rng = np.random.default_rng(7)
    H, d, V = 4, 64, 128
    m = R.ref_mtp_create(H, d, V)
    for h in range(H):
        for which in range(3):
            q4 = rng.integers(0, 256, (d, d // 2), dtype=np.uint8)
            s16 = (rng.random(d) * 0.02 + 0.01).astype(np.float16)
            s = s16.astype(np.float32)
            R.ref_mtp_set(m, h, which, P(q4, u8p), P(s, f32p), d, d)
            out[f"mtp_h{h}_w{which}_q4"] = q4
            out[f"mtp_h{h}_w{which}_s16"] = s16.view(np.uint16)
    emb = ((rng.random((V, d)) - 0.5) * 0.02).astype(np.float32)
    hid = (rng.random(d) * 2 - 1).astype(np.float32)
    lo = np.zeros((H, V), np.float32)
    R.ref_mtp_forward(m, P(hid, f32p), P(emb, f32p), emb.size, P(lo, f32p))
    out["mtp_emb"], out["mtp_hidden"], out[f"mtp_logits_{tag}"] = emb, hid, lo
    # argmax / speculative_accept known answers (tests/test_mtp.cpp:55-69)
    tl = np.array([-1.0, 3.0, 0.5, -0.2, 2.0], np.float32)
    out["argmax_x"] = tl
    out[f"argmax_{tag}"] = np.int32(R.ref_mtp_argmax(P(tl, f32p), 5))
    ties = np.array([1.0, 5.0, 5.0, -2.0, 5.0], np.float32)
    out["argmax_ties_x"] = ties
    out[f"argmax_ties_{tag}"] = np.int32(R.ref_mtp_argmax(P(ties, f32p), 5))
    sa = np.full((4, V), -1.0, np.float32)
    sa[0, 5] = sa[1, 5] = sa[3, 5] = 10.0
    sa[2, 7] = 10.0
    out["spec_logits"] = sa
    out[f"spec_accept_{tag}"] = np.int32(R.ref_mtp_speculative_accept(m, 5, P(sa, f32p), 4, V))
    R.ref_mtp_destroy(m)


# LayerSkipController decisions (src/layer_skip.cpp:22-67): configurations
# (layers, threshold, anchor interval) over one stream of FFN inputs
# [token][layer][width]; each token's input is base + eps * noise with eps
# cycling through values below, near and above the thresholds.  A stream is
# kept only if every delta sits at least 5% away from its threshold, so the
# decisions do not depend on the order of the sum of squares.
SKIP_CONFIGS = [(8, 0.02, 4), (8, 0.02, 0), (8, 0.0, 4), (3, 0.02, 4), (16, 0.02, 4), (16, 0.05, 1)]


def skip(R, out):
    R.ref_skip_create.restype = C.c_void_p
    R.ref_skip_create.argtypes = [C.c_uint32, C.c_uint32, C.c_float, C.c_uint32]
    R.ref_skip_destroy.argtypes = [C.c_void_p]
    R.ref_skip_should_skip_ffn.restype = C.c_int
    R.ref_skip_should_skip_ffn.argtypes = [C.c_void_p, C.c_uint32, f32p, C.c_uint32]
    T, Lmax, D = 10, 16, 128
    epss = np.array([0.0, 0.002, 0.008, 0.03, 0.2, 0.005], np.float64)
    for seed in range(100):
        rng = np.random.default_rng(1000 + seed)
        base = rng.standard_normal((Lmax, D))
        eps = epss[rng.integers(0, len(epss), (T, Lmax))]
        x = (base[None] + eps[..., None] * rng.standard_normal((T, Lmax, D))).astype(np.float32)
        ok = True
        decisions = {}
        for (L, thr, interval) in SKIP_CONFIGS:
            h = R.ref_skip_create(L, D, thr, interval)
            dec = np.zeros((T, L), np.int32)
            cache = np.zeros((L, D), np.float64)
            mid = L // 2
            for t in range(T):
                for l in range(L):
                    v = np.ascontiguousarray(x[t, l])
                    dec[t, l] = R.ref_skip_should_skip_ffn(h, l, P(v, f32p), D)
                    a = thr * (2.0 if (l > mid // 2 and l < mid + mid // 2) else 1.0)
                    never = l < 2 or l >= L - 2 or interval == 0
                    delta = np.sqrt(np.mean((v.astype(np.float64) - cache[l]) ** 2))
                    if not never and a > 0 and abs(delta - a) < 0.05 * a:
                        ok = False
                    if not dec[t, l]:
                        cache[l] = v
            R.ref_skip_destroy(h)
            decisions[(L, thr, interval)] = dec
        if ok:
            break
    else:
        raise SystemExit("no skip stream with clear margins")
    out["skip_x"] = x
    for i, (cfg, dec) in enumerate(decisions.items()):
        out[f"skip_cfg{i}"] = np.array(cfg, np.float64)
        out[f"skip_dec{i}"] = dec
    print("skip stream seed", 1000 + seed, {k: int(v.sum()) for k, v in decisions.items()})


def main(groups):
    O.build(ref=True)
    if groups == ["skip"]:
        R = O.ref_lib()
        if R is None:
            raise SystemExit("reference TUs not built (needs /root/reference)")
        d = {}
        skip(R, d)
        np.savez_compressed(os.path.join(HERE, "ref_skip.npz"), **d)
        return
    outs = {"kernels": {}, "kv": {}, "mtp": {}}
    for tag, nofma in (("fma", False), ("nofma", True)):
        R = O.ref_lib(nofma=nofma)
        if R is None:
            raise SystemExit("reference TUs not built (needs /root/reference)")
        kernels(R, tag, outs["kernels"])
        kv(R, tag, outs["kv"])
        mtp(R, tag, outs["mtp"])
    for name, d in outs.items():
        np.savez_compressed(os.path.join(HERE, f"ref_{name}.npz"), **d)
        print(name, len(d), "arrays")


if __name__ == "__main__":
    main(sys.argv[1:])
