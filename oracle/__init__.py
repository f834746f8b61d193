"""ctypes binding of the CPU checker (pf_oracle.c).

Test infrastructure only: imported by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg.  The product (pocketforge_amd) never imports
it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "_build", "liboracle.so")
_REF = os.path.join(_HERE, "_ref", "libforge_ref.so")
_REF_NOFMA = os.path.join(_HERE, "_ref", "libforge_ref_nofma.so")

Q4, Q2, Q15, Q8 = 0, 1, 2, 3

f32p = C.POINTER(C.c_float)
i8p = C.POINTER(C.c_int8)
u8p = C.POINTER(C.c_uint8)
u16p = C.POINTER(C.c_uint16)
i32p = C.POINTER(C.c_int32)
u32p = C.POINTER(C.c_uint32)


def build(ref=False):
    subprocess.check_call(["make", "-s", "-C", _HERE])
    if ref and os.path.isdir("/root/reference/src"):
        subprocess.check_call(["make", "-s", "-C", _HERE, "ref"])


def ptr(a, t):
    return a.ctypes.data_as(t)


class QMat(C.Structure):
    _fields_ = [("fmt", C.c_int32), ("rows", C.c_uint32), ("cols", C.c_uint32),
                ("codes", u8p), ("scales", u16p)]


class ModelDesc(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("n_embd", C.c_uint32), ("n_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("n_ff", C.c_uint32), ("n_vocab", C.c_uint32),
                ("n_mtp", C.c_uint32), ("sink_size", C.c_uint32), ("window_size", C.c_uint32),
                ("pool_block", C.c_uint32), ("max_context", C.c_uint32),
                ("layers", C.POINTER(QMat)), ("emb", C.POINTER(QMat)), ("mtp", C.POINTER(QMat)),
                ("attn_norm", f32p), ("ffn_norm", f32p)]


class Sampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_uint32),
                ("greedy", C.c_int32)]


FWD_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_int32, f32p)
VALID_FN = C.CFUNCTYPE(C.c_int32, C.c_void_p)
MTP_FN = C.CFUNCTYPE(None, C.c_void_p, f32p, f32p)


class GenOps(C.Structure):
    _fields_ = [("ctx", C.c_void_p), ("n_vocab", C.c_uint32), ("n_mtp", C.c_uint32),
                ("forward", FWD_FN), ("hidden_valid", VALID_FN), ("mtp", MTP_FN)]


def _load(path):
    lib = C.CDLL(path)
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        L = _load(_LIB)
        L.orc_uniform.restype = C.c_float
        L.orc_uniform.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_expf.restype = C.c_float
        L.orc_expf.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_dot_product.restype = C.c_float
        L.orc_dot_product.argtypes = [f32p, f32p, C.c_uint32]
        L.orc_dot_canon.restype = C.c_float
        L.orc_dot_canon.argtypes = [f32p, f32p, C.c_uint32]
        L.orc_softmax.argtypes = [f32p, C.c_uint32]
        L.orc_rmsnorm.argtypes = [f32p, f32p, f32p, C.c_uint32]
        L.orc_engine_rmsnorm.argtypes = [f32p, f32p, f32p, C.c_uint32]
        L.orc_gemv_f32_dense.argtypes = [f32p, C.c_uint32, C.c_uint32, f32p, f32p]
        L.orc_mtp_heads_forward.argtypes = [C.POINTER(QMat), C.c_uint32, C.c_uint32, C.c_uint32, f32p, f32p, f32p]
        L.orc_canon_sum.restype = C.c_float
        L.orc_canon_sumsq.restype = C.c_float
        L.orc_canon_sum.argtypes = [f32p, C.c_uint32, C.c_uint32]
        L.orc_canon_sumsq.argtypes = [f32p, C.c_uint32, C.c_uint32]
        L.orc_quantize_activation_row.argtypes = [f32p, i8p, f32p, C.c_uint32]
        L.orc_gemv_i8.argtypes = [C.POINTER(QMat), i8p, C.c_float, f32p]
        L.orc_gemv_f32.argtypes = [C.POINTER(QMat), f32p, f32p]
        L.orc_kv_create.restype = C.c_void_p
        L.orc_kv_create.argtypes = [C.c_uint32] * 7
        L.orc_kv_destroy.argtypes = [C.c_void_p]
        L.orc_kv_store.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, f32p, f32p]
        L.orc_kv_attention_scores.restype = C.c_uint32
        L.orc_kv_attention_scores.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, f32p, f32p]
        for n in ("orc_kv_attention_weighted_sum", "orc_kv_attention_weighted_sum_ref"):
            getattr(L, n).argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, f32p, f32p, C.c_uint32]
        for n in ("orc_attn_head", "orc_attn_head_ref"):
            getattr(L, n).argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, f32p, f32p, f32p, f32p]
        L.orc_kv_size.restype = C.c_uint32
        L.orc_kv_size.argtypes = [C.c_void_p]
        L.orc_kv_clear.argtypes = [C.c_void_p]
        L.orc_kv_pool_count.restype = C.c_uint32
        L.orc_kv_pool_count.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32]
        L.orc_kv_export.restype = C.c_uint32
        L.orc_kv_export.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, i8p, f32p, i8p, f32p]
        L.orc_kv_import.argtypes = [C.c_void_p] + [C.c_uint32] * 7 + [i8p, f32p, i8p, f32p]
        L.orc_engine_set_state.argtypes = [C.c_void_p, C.c_uint32, f32p]
        L.orc_generate_continue.restype = C.c_int32
        L.orc_generate_continue.argtypes = [C.c_void_p, C.c_int32, C.c_uint32, C.POINTER(Sampling), C.c_uint64,
                                            i32p, C.c_uint32, u32p, i32p, i32p]
        L.orc_engine_create.restype = C.c_void_p
        L.orc_engine_create.argtypes = [C.POINTER(ModelDesc)]
        L.orc_engine_destroy.argtypes = [C.c_void_p]
        L.orc_engine_reset.argtypes = [C.c_void_p]
        L.orc_engine_pos.restype = C.c_uint32
        L.orc_engine_pos.argtypes = [C.c_void_p]
        L.orc_engine_kv.restype = C.c_void_p
        L.orc_engine_kv.argtypes = [C.c_void_p]
        L.orc_forward.argtypes = [C.c_void_p, C.c_int32, f32p, f32p]
        L.orc_mtp_forward.argtypes = [C.c_void_p, f32p, f32p]
        L.orc_argmax.restype = C.c_int32
        L.orc_argmax.argtypes = [f32p, C.c_uint32]
        L.orc_sample.restype = C.c_int32
        L.orc_sample.argtypes = [f32p, C.c_uint32, C.POINTER(Sampling), C.c_uint64,
                                 C.POINTER(C.c_uint64)]
        L.orc_generate.restype = C.c_int32
        L.orc_generate.argtypes = [C.c_void_p, i32p, C.c_uint32, C.c_uint32, C.POINTER(Sampling),
                                   C.c_uint64, i32p, C.c_uint32, u32p, i32p, i32p]
        L.orc_rope_table.argtypes = [C.c_uint32, C.c_uint32, f32p, f32p]
        L.orc_philox4x32_10.argtypes = [u32p, u32p, u32p]
        L.orc_rope_rotate.argtypes = [f32p, C.c_uint32, f32p, f32p]
        L.orc_generate_ops.restype = C.c_int32
        L.orc_generate_ops.argtypes = [C.POINTER(GenOps), i32p, C.c_uint32, C.c_uint32, C.POINTER(Sampling),
                                       C.c_uint64, i32p, C.c_uint32, u32p, i32p, i32p]
        step_args = [C.POINTER(Sampling), C.c_uint64, C.POINTER(C.c_uint64), f32p, u32p, i32p, i32p]
        L.orc_step_mtp_ops.restype = C.c_int32
        L.orc_step_mtp_ops.argtypes = [C.POINTER(GenOps), C.c_int32, f32p, C.c_int32] + step_args
        L.orc_step_mtp.restype = C.c_int32
        L.orc_step_mtp.argtypes = [C.c_void_p, C.c_int32, f32p, C.c_int32] + step_args
        L.orc_engine_set_layer_skip.argtypes = [C.c_void_p, C.c_float, C.c_uint32]
        L.orc_engine_skip_count.restype = C.c_uint32
        L.orc_engine_skip_count.argtypes = [C.c_void_p]
        L.orc_skip_delta.restype = C.c_float
        L.orc_skip_delta.argtypes = [f32p, f32p, C.c_uint32]
        L.orc_skip_decide.restype = C.c_int
        L.orc_skip_decide.argtypes = [f32p, C.c_uint32, C.c_uint32, C.c_float, C.c_uint32, C.c_uint32, f32p]
        L.orc_quantize_matrix.argtypes = [f32p, C.c_uint32, C.c_uint32, C.c_int32, u8p, u16p]
        L.orc_num_threads.restype = C.c_int
        L.orc_set_num_threads.argtypes = [C.c_int]
        L.orc_last_decode_seconds.restype = C.c_double
        _lib = L
    return _lib


def ref_lib(nofma=False):
    """The reference's own TUs (built in this container from /root/reference)."""
    path = _REF_NOFMA if nofma else _REF
    if not os.path.exists(path):
        return None
    L = _load(path)
    L.ref_dot_product.restype = C.c_float
    L.ref_kv_create.restype = C.c_void_p
    L.ref_kv_create.argtypes = [C.c_uint32] * 7
    L.ref_kv_destroy.argtypes = [C.c_void_p]
    L.ref_kv_store.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, f32p, f32p]
    L.ref_kv_attention_scores.restype = C.c_uint32
    L.ref_kv_attention_scores.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, f32p, f32p]
    L.ref_kv_attention_weighted_sum.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, f32p, f32p,
                                               C.c_uint32]
    L.ref_kv_size.restype = C.c_uint32
    L.ref_kv_size.argtypes = [C.c_void_p]
    L.ref_kv_clear.argtypes = [C.c_void_p]
    L.ref_kv_memory_usage.restype = C.c_uint64
    L.ref_kv_memory_usage.argtypes = [C.c_void_p]
    L.ref_mtp_create.restype = C.c_void_p
    L.ref_mtp_create.argtypes = [C.c_uint32] * 3
    L.ref_mtp_destroy.argtypes = [C.c_void_p]
    L.ref_mtp_set.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, u8p, f32p, C.c_uint32, C.c_uint32]
    L.ref_mtp_forward.argtypes = [C.c_void_p, f32p, f32p, C.c_uint32, f32p]
    L.ref_mtp_argmax.restype = C.c_int32
    L.ref_mtp_argmax.argtypes = [f32p, C.c_uint32]
    L.ref_mtp_speculative_accept.restype = C.c_int32
    L.ref_mtp_speculative_accept.argtypes = [C.c_void_p, C.c_int32, f32p, C.c_uint32, C.c_uint32]
    return L


# ------------------------------------------------------------- helpers

def qmat(fmt, codes, scales):
    """QMat view over numpy arrays (kept alive by the caller)."""
    rows, nb = scales.shape
    return QMat(fmt, rows, nb * 32, ptr(codes, u8p), ptr(scales, u16p))


def quantize_matrix(w, fmt):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    bb = {Q4: 16, Q8: 32}.get(fmt, 8)
    codes = np.zeros((rows, cols // 32, bb), np.uint8)
    scales = np.zeros((rows, cols // 32), np.uint16)
    lib().orc_quantize_matrix(ptr(w, f32p), rows, cols, fmt, ptr(codes, u8p), ptr(scales, u16p))
    return codes, scales


def gemv_i8(fmt, codes, scales, a8, a_scale):
    q = qmat(fmt, codes, scales)
    y = np.zeros(scales.shape[0], np.float32)
    a8 = np.ascontiguousarray(a8, np.int8)
    lib().orc_gemv_i8(C.byref(q), ptr(a8, i8p), C.c_float(a_scale), ptr(y, f32p))
    return y


def gemv_f32(fmt, codes, scales, h):
    q = qmat(fmt, codes, scales)
    y = np.zeros(scales.shape[0], np.float32)
    h = np.ascontiguousarray(h, np.float32)
    lib().orc_gemv_f32(C.byref(q), ptr(h, f32p), ptr(y, f32p))
    return y


def mtp_heads_forward(heads, d, V, table, hidden):
    """heads: list of n (gate, up, down) triples of (fmt, codes, scales);
    table: fp32 [V][d] or None.  Returns logits [n][V]."""
    n = len(heads)
    arr = (QMat * (3 * n))()
    keep = []
    for k, trip in enumerate(heads):
        for w, (fmt, codes, scales) in enumerate(trip):
            q = qmat(fmt, codes, scales)
            keep.append(q)
            arr[3 * k + w] = q
    out = np.zeros((n, V), np.float32)
    t = None if table is None else np.ascontiguousarray(table, np.float32)
    h = np.ascontiguousarray(hidden, np.float32)
    lib().orc_mtp_heads_forward(arr, n, d, V, ptr(t, f32p) if t is not None else None, ptr(h, f32p),
                                ptr(out, f32p))
    return out


def quantize_activation_row(x):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(x.shape[0], np.int8)
    s = np.zeros(1, np.float32)
    lib().orc_quantize_activation_row(ptr(x, f32p), ptr(q, i8p), ptr(s, f32p), x.shape[0])
    return q, float(s[0])


class Model:
    """Oracle engine over a weight set produced by pocketforge_amd.weights
    (or any dict with the same keys)."""

    def __init__(self, cfg, w):
        self.cfg = cfg
        self.w = w
        L = cfg["n_layers"]
        mats = (QMat * (L * 7))()
        names = ["wq", "wk", "wv", "wo", "wgate", "wup", "wdown"]
        for l in range(L):
            for j, n in enumerate(names):
                fmt, codes, scales = w["layers"][l][n]
                mats[l * 7 + j] = qmat(fmt, codes, scales)
        self._mats = mats
        fmt, codes, scales = w["emb"]
        self._emb = qmat(fmt, codes, scales)
        nm = cfg["n_mtp"]
        mtp = (QMat * max(1, nm * 3))()
        for k in range(nm):
            for j, n in enumerate(["gate", "up", "down"]):
                fmt, codes, scales = w["mtp"][k][n]
                mtp[k * 3 + j] = qmat(fmt, codes, scales)
        self._mtp = mtp
        self._an = np.ascontiguousarray(w["attn_norm"], np.float32)
        self._fn = np.ascontiguousarray(w["ffn_norm"], np.float32)
        d = ModelDesc(L, cfg["n_embd"], cfg["n_heads"], cfg["head_dim"], cfg["n_ff"], cfg["n_vocab"],
                      nm, cfg["sink_size"], cfg["window_size"], cfg["pool_block"], cfg["max_context"],
                      C.cast(mats, C.POINTER(QMat)), C.pointer(self._emb),
                      C.cast(mtp, C.POINTER(QMat)), ptr(self._an, f32p), ptr(self._fn, f32p))
        self._desc = d
        self.h = lib().orc_engine_create(C.byref(d))

    def close(self):
        if self.h:
            lib().orc_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def reset(self):
        lib().orc_engine_reset(self.h)

    def set_layer_skip(self, threshold, interval=4):
        lib().orc_engine_set_layer_skip(self.h, float(threshold), int(interval))

    @property
    def skip_count(self):
        return lib().orc_engine_skip_count(self.h)

    @property
    def pos(self):
        return lib().orc_engine_pos(self.h)

    def forward(self, token, want_logits=True):
        V, D = self.cfg["n_vocab"], self.cfg["n_embd"]
        logits = np.zeros(V, np.float32) if want_logits else None
        hidden = np.zeros(D, np.float32)
        lib().orc_forward(self.h, int(token), ptr(logits, f32p) if want_logits else None,
                          ptr(hidden, f32p))
        return logits, hidden

    def mtp_forward(self, hidden):
        V, nm = self.cfg["n_vocab"], self.cfg["n_mtp"]
        out = np.zeros((nm, V), np.float32)
        hidden = np.ascontiguousarray(hidden, np.float32)
        lib().orc_mtp_forward(self.h, ptr(hidden, f32p), ptr(out, f32p))
        return out

    def step_mtp(self, token, hidden, has_table, sampling, seed=42, draw=0):
        """orc_step_mtp (Engine::step_mtp, src/engine.cpp:402-448) on this
        engine: (accepted, rejecting forward's logits or None,
        mtp_accepted_out, mtp_rejected_out, draw counter after)."""
        h = np.ascontiguousarray(hidden, np.float32)
        lg = np.zeros(self.cfg["n_vocab"], np.float32)
        d = C.c_uint64(draw)
        nl = C.c_uint32(0)
        a = C.c_int32(0)
        r = C.c_int32(0)
        k = lib().orc_step_mtp(self.h, int(token), ptr(h, f32p), int(has_table), C.byref(sampling), seed,
                               C.byref(d), ptr(lg, f32p), C.byref(nl), C.byref(a), C.byref(r))
        return k, (lg if nl.value else None), a.value, r.value, d.value

    def generate(self, prompt, max_new, sampling=None, seed=7):
        s = sampling or Sampling(0.8, 0.95, 40, 1)
        prompt = np.ascontiguousarray(prompt, np.int32)
        cap = len(prompt) + max_new + 8
        toks = np.zeros(cap, np.int32)
        n = C.c_uint32(0)
        acc = C.c_int32(0)
        rej = C.c_int32(0)
        rc = lib().orc_generate(self.h, ptr(prompt, i32p), len(prompt), max_new, C.byref(s), seed,
                                ptr(toks, i32p), cap, C.byref(n), C.byref(acc), C.byref(rej))
        assert rc == 0
        return toks[: n.value].copy(), acc.value, rej.value

    def kv_import(self, layer, head, counts, win_pos0, k, ks, v, vs):
        kv_import(lib().orc_engine_kv(self.h), layer, head, counts, win_pos0, k, ks, v, vs)

    def set_state(self, pos, hidden=None):
        """Next position and (optionally) the last hidden state, after
        kv_import of every plane."""
        h = None if hidden is None else np.ascontiguousarray(hidden, np.float32)
        lib().orc_engine_set_state(self.h, int(pos), ptr(h, f32p) if h is not None else None)

    def generate_continue(self, cur, max_new, sampling=None, seed=7):
        """Engine::generate's decode loop from the current state with current
        token `cur`; returns (generated tokens, accepted, rejected)."""
        s = sampling or Sampling(0.8, 0.95, 40, 1)
        cap = max_new + 8
        toks = np.zeros(cap, np.int32)
        n = C.c_uint32(0)
        acc = C.c_int32(0)
        rej = C.c_int32(0)
        rc = lib().orc_generate_continue(self.h, int(cur), max_new, C.byref(s), seed, ptr(toks, i32p), cap,
                                         C.byref(n), C.byref(acc), C.byref(rej))
        assert rc == 0
        return toks[: n.value].copy(), acc.value, rej.value


def kv_import(kv, layer, head, counts, win_pos0, k, ks, v, vs):
    """orc_kv_import on an orc_kv handle: counts = (sink, pooled, window,
    pending) rows, stacked in that order in k/ks/v/vs."""
    k = np.ascontiguousarray(k, np.int8)
    v = np.ascontiguousarray(v, np.int8)
    ks = np.ascontiguousarray(ks, np.float32)
    vs = np.ascontiguousarray(vs, np.float32)
    assert k.shape[0] == sum(counts)
    lib().orc_kv_import(kv, layer, head, counts[0], counts[1], counts[2], int(win_pos0), counts[3],
                        ptr(k, i8p), ptr(ks, f32p), ptr(v, i8p), ptr(vs, f32p))


def philox4x32_10(ctr, key):
    c = np.ascontiguousarray(ctr, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    out = np.zeros(4, np.uint32)
    lib().orc_philox4x32_10(ptr(c, u32p), ptr(k, u32p), ptr(out, u32p))
    return out


class ScriptedModel:
    """A model for the decode control flow whose logits come from Python
    callables: forward(token) -> logits [V] (records every call) and
    heads(hidden or None) -> [n_mtp][V].  hidden_valid follows the
    reference: false until the first forward (src/engine.cpp:551)."""

    def __init__(self, n_vocab, n_mtp, forward, heads):
        self.V, self.NH = n_vocab, n_mtp
        self.calls = []
        self.mtp_calls = 0
        self._valid = 0

        def fwd(_ctx, tok, out):
            lg = np.asarray(forward(int(tok)), np.float32)
            self.calls.append(int(tok))
            self._valid = 1
            if out:
                C.memmove(out, lg.ctypes.data, 4 * self.V)

        def valid(_ctx):
            return self._valid

        def mtp(_ctx, hidden, out):
            h = None if not hidden else np.ctypeslib.as_array(hidden, (1,)).copy()
            lg = np.ascontiguousarray(heads(h), np.float32).reshape(self.NH, self.V)
            self.mtp_calls += 1
            C.memmove(out, lg.ctypes.data, 4 * self.V * self.NH)

        self._cb = (FWD_FN(fwd), VALID_FN(valid), MTP_FN(mtp))
        self.ops = GenOps(None, n_vocab, n_mtp, *self._cb)

    def generate(self, prompt, max_new, sampling, seed=7, cap=None):
        prompt = np.ascontiguousarray(prompt, np.int32)
        cap = cap or len(prompt) + max_new + 8
        toks = np.zeros(max(cap, 1), np.int32)
        n = C.c_uint32(0)
        acc = C.c_int32(0)
        rej = C.c_int32(0)
        rc = lib().orc_generate_ops(C.byref(self.ops), ptr(prompt, i32p), len(prompt), max_new, C.byref(sampling),
                                    seed, ptr(toks, i32p), cap, C.byref(n), C.byref(acc), C.byref(rej))
        return rc, toks[: n.value].copy(), acc.value, rej.value

    def step_mtp(self, token, hidden, has_table, sampling, seed=42, draw=0):
        h = np.ascontiguousarray(hidden if hidden is not None else np.zeros(1), np.float32)
        lg = np.zeros(self.V, np.float32)
        d = C.c_uint64(draw)
        nl = C.c_uint32(0)
        a = C.c_int32(0)
        r = C.c_int32(0)
        k = lib().orc_step_mtp_ops(C.byref(self.ops), int(token), ptr(h, f32p), int(has_table), C.byref(sampling),
                                   seed, C.byref(d), ptr(lg, f32p), C.byref(nl), C.byref(a), C.byref(r))
        return k, (lg if nl.value else None), a.value, r.value, d.value


def sample(logits, cfg, seed, draw_idx):
    logits = np.ascontiguousarray(logits, np.float32)
    d = C.c_uint64(draw_idx)
    t = lib().orc_sample(ptr(logits, f32p), logits.shape[0], C.byref(cfg), seed, C.byref(d))
    return t, d.value
