"""Kernel-level parity of the gfx950 path against the oracle (bit-exact)."""
import ctypes as C
import os

import numpy as np
import pytest

import oracle as O
import pocketforge_amd as pf
from golden_cfg import KV_CFGS

pytestmark = pytest.mark.gpu

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


_CTX = []


def _t(a):
    return pf.DeviceArray.from_numpy(_CTX[0], a)


@pytest.fixture(autouse=True)
def _ctx(gpu):
    _CTX[:] = [gpu]
    yield


def test_quantize_activation_rows(gpu):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((6, 2048)) * 0.9).astype(np.float32)
    x[1] = 0.0
    x[2, :] = np.arange(2048, dtype=np.float32) / 16.0 - 64.0    # exact .5 ties after scaling
    q, s = gpu.quantize_activation_rows(_t(x))
    q, s = q.numpy(), s.numpy()
    for m in range(6):
        q2, s2 = O.quantize_activation_row(x[m])
        np.testing.assert_array_equal(q[m], q2)
        assert s[m] == np.float32(s2)


def test_matmul_int8_and_quantized(gpu):
    rng = np.random.default_rng(1)
    M, N, K = 5, 77, 300
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    B = rng.integers(-8, 8, (N, K), dtype=np.int8)
    Cm = gpu.matmul_int8(_t(A), _t(B)).numpy()
    np.testing.assert_array_equal(Cm, A.astype(np.int32) @ B.astype(np.int32).T)
    Af = (rng.standard_normal((M, K)) * 0.5).astype(np.float32)
    ws = (rng.random(N) * 0.02 + 0.001).astype(np.float32)
    asc = (rng.random(M) * 0.01 + 0.001).astype(np.float32)
    L = O.lib()
    for act in (None, asc):
        ref = np.zeros((M, N), np.float32)
        L.orc_matmul_quantized(O.ptr(Af, O.f32p), O.ptr(B, O.i8p), O.ptr(ref, O.f32p), M, N, K,
                               O.ptr(ws, O.f32p), O.ptr(act, O.f32p) if act is not None else None)
        got = gpu.matmul_quantized(_t(Af), _t(B), _t(ws), _t(act) if act is not None else None).numpy()
        np.testing.assert_array_equal(got, ref)


def test_matmul_reference_golden(gpu):
    K = dict(np.load(os.path.join(G, "ref_kernels.npz")))
    got = gpu.matmul_int8(_t(K["mm_A"]), _t(K["mm_B"])).numpy()
    np.testing.assert_array_equal(got, K["mm_C_fma"])
    got = gpu.matmul_quantized(_t(K["mq_A"]), _t(K["mm_B"]), _t(K["mq_ws"])).numpy()
    np.testing.assert_array_equal(got, K["mq_C_fma"])
    got = gpu.matmul_quantized(_t(K["mq_A"]), _t(K["mm_B"]), _t(K["mq_ws"]), _t(K["mq_as"])).numpy()
    np.testing.assert_array_equal(got, K["mq_Cas_fma"])


@pytest.mark.parametrize("fmt", [pf.FMT_Q4, pf.FMT_Q2, pf.FMT_Q15, pf.FMT_Q8])
@pytest.mark.parametrize("shape", [(128, 512), (320, 2048), (64, 1792)])
def test_gemv_int8_block(gpu, fmt, shape):
    N, K = shape
    codes, scales = pf.gen_matrix(99, fmt * 7 + N, 0.02, N, K, fmt)
    W = gpu.upload_matrix(fmt, codes, scales)
    rng = np.random.default_rng(N + K)
    for M in (1, 5, 8):
        x = (rng.standard_normal((M, K)) * 0.5).astype(np.float32)
        y = gpu.gemv_q(W, _t(x)).numpy()
        for m in range(M):
            a8, s = O.quantize_activation_row(x[m])
            ref = O.gemv_i8(fmt, codes, scales, a8, s)
            np.testing.assert_array_equal(y[m], ref, err_msg=f"fmt {fmt} M {M} row {m}")
    W.close()


def test_gemv_rejects_out_of_range_scales(gpu):
    codes, scales = pf.gen_matrix(5, 1, 0.02, 64, 256, pf.FMT_Q4)
    scales = scales.copy()
    scales[3, 0] = np.float16(1e-7).view(np.uint16)     # 2^-23 next to ~2^-7 scales
    scales[3, 1] = np.float16(1000.0).view(np.uint16)
    with pytest.raises(pf.PFError, match="binades"):
        gpu.upload_matrix(pf.FMT_Q4, codes, scales)
    codes, scales = pf.gen_matrix(5, 1, 0.02, 64, 256, pf.FMT_Q15)
    codes = codes.copy()
    codes[0, 0, 0] |= 3
    with pytest.raises(pf.PFError, match="code 3"):
        gpu.upload_matrix(pf.FMT_Q15, codes, scales)


@pytest.mark.parametrize("fmt", [pf.FMT_Q4, pf.FMT_Q8])
@pytest.mark.parametrize("K", [256, 768, 2048])
def test_gemv_f32(gpu, K, fmt):
    N = 640
    codes, scales = pf.gen_matrix(7, K, 0.02, N, K, fmt)
    W = gpu.upload_matrix(fmt, codes, scales, rowmajor=True)
    rng = np.random.default_rng(K)
    for M in (1, 5):
        h = (rng.standard_normal((M, K))).astype(np.float32)
        y = gpu.gemv_f32(W, _t(h)).numpy()
        for m in range(M):
            np.testing.assert_array_equal(y[m], O.gemv_f32(fmt, codes, scales, h[m]))
    W.close()


@pytest.mark.parametrize("key", sorted(KV_CFGS))
def test_kv_cache_api(gpu, key):
    """KVCache store / attention_scores / attention_weighted_sum on the GPU
    against the oracle and the reference's own outputs."""
    KV = dict(np.load(os.path.join(G, "ref_kv.npz")))
    Ln, H, hd, sink, win, pool, maxc, n = KV_CFGS[key]
    kv = pf.KVCache(gpu, Ln, H, hd, sink, win, pool, maxc)
    L = O.lib()
    ok = L.orc_kv_create(Ln, H, hd, sink, win, pool, maxc)
    keys, vals, qs = KV[f"{key}_keys"], KV[f"{key}_vals"], KV[f"{key}_qs"]
    stored = 0
    for c in KV[f"{key}_ckpt"]:
        while stored < c:
            for l in range(Ln):
                for h in range(H):
                    kv.store(l, h, stored, keys[stored, l, h], vals[stored, l, h])
                    L.orc_kv_store(ok, l, h, stored, O.ptr(keys[stored, l, h], O.f32p),
                                   O.ptr(vals[stored, l, h], O.f32p))
            stored += 1
        assert kv.size() == KV[f"{key}_c{c}_size"]
        for l in range(Ln):
            for h in range(H):
                for qi in range(8):
                    sc = kv.attention_scores(l, h, qs[qi])
                    assert len(sc) == KV[f"{key}_c{c}_count"][l, h]
                    np.testing.assert_array_equal(sc, KV[f"{key}_c{c}_scores_fma"][l, h, qi, :len(sc)])
                    p = np.exp(sc - sc.max()).astype(np.float32)
                    p = (p / p.sum()).astype(np.float32)
                    ws = kv.attention_weighted_sum(l, h, p)
                    ref = np.zeros(hd, np.float32)
                    L.orc_kv_attention_weighted_sum(ok, l, h, O.ptr(p, O.f32p), O.ptr(ref, O.f32p), len(p))
                    np.testing.assert_array_equal(ws, ref)
                    np.testing.assert_allclose(ws, KV[f"{key}_c{c}_wsum_fma"][l, h, qi], rtol=1e-5, atol=1e-6)
    kv.clear()
    assert kv.size() == 0
    assert len(kv.attention_scores(0, 0, qs[0])) == 0
    L.orc_kv_destroy(ok)
    kv.close()


SAMPLERS = {
    "greedy": pf.Sampling(0.8, 0.95, 40, 1),
    "temp0": pf.Sampling(0.0, 0.95, 40, 0),
    "top_p": pf.Sampling(0.8, 0.95, 40, 0),
    "top_k": pf.Sampling(0.8, 1.0, 40, 0),
    "temperature": pf.Sampling(1.3, 1.0, 0, 0),
}


@pytest.fixture(scope="module")
def engine_v16k(gpu):
    """A one-layer model with the benchmark vocabulary (16384), for the
    sampler at the size where its radix sort holds 16 keys per thread."""
    from pocketforge_amd import weights as W
    cfg = dict(n_layers=1, n_embd=256, n_heads=4, head_dim=64, n_ff=512, n_vocab=16384, n_mtp=4)
    m = pf.Model(gpu, cfg, W.make_weights(cfg, seed=1234))
    e = pf.Engine(m, sink_size=4, window_size=64, pool_block=6, max_context=256)
    yield e
    e.close()
    m.close()


@pytest.mark.parametrize("name", sorted(SAMPLERS))
@pytest.mark.parametrize("V", [1024, 16384])
def test_sampler(gpu, tiny_engine, engine_v16k, name, V):
    eng = tiny_engine if V == 1024 else engine_v16k
    assert eng.cfg["n_vocab"] == V
    cfg = SAMPLERS[name]
    ocfg = O.Sampling(cfg.temperature, cfg.top_p, cfg.top_k, cfg.greedy)
    rng = np.random.default_rng(V)
    for trial in range(12):
        logits = (rng.standard_normal(V) * (0.5 + trial)).astype(np.float32)
        if trial == 3:
            logits[::7] = logits.max()           # ties at the maximum
        draw = trial * 3
        t, d = eng.sample(logits, cfg, 7, draw)
        t2, d2 = O.sample(logits, ocfg, 7, draw)
        assert (t, d) == (t2, d2), (name, trial)


def test_dot_softmax_rmsnorm_argmax(gpu):
    """matmul_neon.hpp helpers on the device against the oracle's canonical
    orders (bit-exact), the reference's known answers
    (tests/test_matmul.cpp:103-153) and closed forms."""
    L = O.lib()
    rng = np.random.default_rng(5)
    for n in (1, 6, 255, 256, 300, 2048, 5000):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        assert np.float32(gpu.dot_product(_t(a), _t(b))) == np.float32(L.orc_dot_canon(O.ptr(a, O.f32p),
                                                                                         O.ptr(b, O.f32p), n))
        v = (a * 3).astype(np.float32)
        dv = _t(v)
        gpu.softmax(dv)
        ref = v.copy()
        L.orc_softmax(O.ptr(ref, O.f32p), n)
        np.testing.assert_array_equal(dv.numpy(), ref)
        w = rng.standard_normal(n).astype(np.float32)
        got = gpu.rmsnorm(_t(a), _t(w)).numpy()
        ref = np.zeros(n, np.float32)
        L.orc_rmsnorm(O.ptr(ref, O.f32p), O.ptr(a, O.f32p), O.ptr(w, O.f32p), n)
        np.testing.assert_array_equal(got, ref)
        x = a.copy()
        x[n // 2] = x.max() + 1.0
        if n > 3:
            x[n // 3] = x[n // 2]                       # tie: the first index wins
        assert gpu.argmax(_t(x)) == int(np.argmax(x))
    # reference known answers
    assert gpu.dot_product(_t(np.arange(1, 7, dtype=np.float32)), _t(np.arange(6, 0, -1, dtype=np.float32))) == 56.0
    sm = _t(np.array([2.0, 1.0, 0.1, 0.5, 3.0], np.float32))
    gpu.softmax(sm)
    s = sm.numpy()
    assert abs(s.sum() - 1.0) < 1e-3 and s[4] > s[0] > s[1] > s[3] > s[2]
    rn = gpu.rmsnorm(_t(np.array([1, 2, 3, 4], np.float32)), _t(np.array([0.5, 1, 1.5, 2], np.float32))).numpy()
    assert abs(rn[0] - 0.5 / np.sqrt(7.5)) < 0.01 and abs(rn[3] - 8 / np.sqrt(7.5)) < 0.01
    assert gpu.argmax(_t(np.array([-1.0, 3.0, 0.5, -0.2, 2.0], np.float32))) == 1


@pytest.mark.parametrize("with_table", [True, False])
def test_mtp_heads_standalone(gpu, with_table):
    """MTPHeads::forward outside an engine: 4 chained heads, fp32 tied table
    or the placeholder logits, bit-exact against the oracle."""
    d, V, H = 256, 1024, 4
    heads = []
    m = pf.MTPHeads(gpu, H, d, V)
    for k in range(H):
        trip = []
        for w in range(3):
            codes, scales = pf.gen_matrix(77, 100 + 3 * k + w, 0.02, d, d, pf.FMT_Q4)
            m.set_head(k, w, codes, scales)
            trip.append((O.Q4, codes, scales))
        heads.append(trip)
    rng = np.random.default_rng(3)
    table = (rng.standard_normal((V, d)) * 0.02).astype(np.float32) if with_table else None
    m.set_table(table)
    hidden = rng.standard_normal(d).astype(np.float32)
    got = m.forward(hidden)
    ref = O.mtp_heads_forward(heads, d, V, table, hidden)
    np.testing.assert_array_equal(got, ref)
    if not with_table:
        v = np.arange(V, dtype=np.uint64)
        np.testing.assert_array_equal(got[2], ((v * np.uint64(2654435761) + np.uint64(2)) % np.uint64(V))
                                      .astype(np.float32) / np.float32(V))
    assert m.memory_usage() > 0
    m.close()


@pytest.mark.parametrize("fmt", [pf.FMT_Q4, pf.FMT_Q2, pf.FMT_Q15, pf.FMT_Q8])
@pytest.mark.parametrize("shape", [(128, 512), (320, 2048), (64, 1792)])
def test_gemm_int8_block(gpu, fmt, shape):
    """The int8 MFMA GEMM (M > 8 rows: many-sequence verify, batched prefill)
    equals the oracle's exact block GEMV row by row, bit for bit, including
    M not a multiple of 32 and the 10 tiles of 320 rows."""
    N, K = shape
    codes, scales = pf.gen_matrix(98, fmt * 11 + N, 0.02, N, K, fmt)
    W = gpu.upload_matrix(fmt, codes, scales)
    rng = np.random.default_rng(N * 3 + K)
    for M in (9, 32, 45, 320):
        x = (rng.standard_normal((M, K)) * 0.5).astype(np.float32)
        x[M // 2] = 0.0                                   # an all-zero row (scale 1, codes 0)
        y = gpu.gemv_q(W, _t(x)).numpy()
        for m in range(M):
            a8, s = O.quantize_activation_row(x[m])
            np.testing.assert_array_equal(y[m], O.gemv_i8(fmt, codes, scales, a8, s), err_msg=f"fmt {fmt} M {M} row {m}")
    W.close()
