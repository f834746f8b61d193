"""Python binding of libpocketforge_amd.so (include/pf_gpu.h) through ctypes.

The binding mirrors the reference's C++ API surface for the MTP hot path
(include/forge/{matmul_neon,kv_cache,mtp,engine}.hpp): every call goes to
the gfx950 kernels; there is no CPU fallback.  If the library is missing the
import raises.  Device buffers for the kernel-level entry points come from
the library's own pf_malloc (DeviceArray).
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libpocketforge_amd.so")

FMT_Q4, FMT_Q2, FMT_Q15, FMT_Q8 = 0, 1, 2, 3


def block_bytes(fmt):
    """Code bytes of one 32-element block in the interchange layout."""
    return {FMT_Q4: 16, FMT_Q8: 32}.get(fmt, 8)
MAT_Q, MAT_K, MAT_V, MAT_O, MAT_GATE, MAT_UP, MAT_DOWN = range(7)

f32p = C.POINTER(C.c_float)
i8p = C.POINTER(C.c_int8)
u8p = C.POINTER(C.c_uint8)
u16p = C.POINTER(C.c_uint16)
i32p = C.POINTER(C.c_int32)
u32p = C.POINTER(C.c_uint32)
vp = C.c_void_p


class PFError(RuntimeError):
    pass


class KvConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("n_layers", "n_kv_heads", "head_dim", "sink_size", "window_size",
                                          "pool_block", "max_context")]


class ModelDesc(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("n_layers", "n_embd", "n_heads", "head_dim", "n_ff", "n_vocab", "n_mtp")]


class Sampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_uint32), ("greedy", C.c_int32)]


class GenResult(C.Structure):
    _fields_ = [("n_tokens", C.c_uint32), ("mtp_accepted", C.c_int32), ("mtp_rejected", C.c_int32),
                ("oom_protected", C.c_int32), ("rounds", C.c_uint32), ("passes", C.c_uint32),
                ("continued", C.c_uint32), ("prefill_seconds", C.c_double), ("decode_seconds", C.c_double)]


class SqueezeInfo(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("version", "n_blocks", "n_layers", "n_embd", "n_heads", "n_kv_heads",
                                          "n_ff", "n_vocab", "max_seq_len", "mtp_heads")]


class CacheDesc(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("sink_size", "window_size", "pool_block", "max_context")]


# Symbol table: name -> (restype, argtypes).  Every entry point of
# include/pf_gpu.h is listed; tests check the library exports all of them.
SYMBOLS = {
    "pf_init": (C.c_int32, [C.c_int, C.POINTER(vp)]),
    "pf_destroy": (None, [vp]),
    "pf_last_error": (C.c_char_p, [vp]),
    "pf_device_info": (C.c_int32, [vp, C.c_char_p, C.c_size_t, C.POINTER(C.c_int)]),
    "pf_synchronize": (C.c_int32, [vp]),
    "pf_device_bytes": (C.c_size_t, [vp]),
    "pf_malloc": (C.c_int32, [vp, C.c_size_t, C.POINTER(vp)]),
    "pf_free": (C.c_int32, [vp, vp, C.c_size_t]),
    "pf_memcpy": (C.c_int32, [vp, vp, vp, C.c_size_t, C.c_int32]),
    "pf_gen_matrix": (C.c_int32, [C.c_uint64, C.c_uint32, C.c_float, C.c_uint32, C.c_uint32, C.c_int32, u8p, u16p]),
    "pf_quantize_matrix": (C.c_int32, [f32p, C.c_uint32, C.c_uint32, C.c_int32, u8p, u16p]),
    "pf_quantize_activation_rows": (C.c_int32, [vp, vp, vp, vp, C.c_uint32, C.c_uint32]),
    "pf_matmul_int8": (C.c_int32, [vp, vp, vp, vp, C.c_uint32, C.c_uint32, C.c_uint32]),
    "pf_matmul_quantized": (C.c_int32, [vp, vp, vp, vp, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp]),
    "pf_matrix_upload": (C.c_int32, [vp, C.c_int32, C.c_uint32, C.c_uint32, u8p, u16p, C.c_int32, C.POINTER(vp)]),
    "pf_matrix_free": (None, [vp]),
    "pf_gemv_q": (C.c_int32, [vp, vp, vp, vp, C.c_uint32]),
    "pf_gemv_q_noalloc": (C.c_int32, [vp, vp, vp, vp, C.c_uint32]),
    "pf_gemv_f32": (C.c_int32, [vp, vp, vp, vp, C.c_uint32]),
    "pf_dot_product": (C.c_int32, [vp, vp, vp, C.c_uint32, vp]),
    "pf_softmax": (C.c_int32, [vp, vp, C.c_uint32]),
    "pf_rmsnorm": (C.c_int32, [vp, vp, vp, vp, C.c_uint32]),
    "pf_argmax": (C.c_int32, [vp, vp, C.c_uint32, vp]),
    "pf_mtp_create": (C.c_int32, [vp, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(vp)]),
    "pf_mtp_destroy": (None, [vp]),
    "pf_mtp_set_head": (C.c_int32, [vp, C.c_uint32, C.c_int32, u8p, u16p]),
    "pf_mtp_set_table": (C.c_int32, [vp, f32p]),
    "pf_mtp_heads_forward": (C.c_int32, [vp, f32p, f32p]),
    "pf_mtp_memory": (C.c_size_t, [vp]),
    "pf_kv_create": (C.c_int32, [vp, C.POINTER(KvConfig), C.POINTER(vp)]),
    "pf_kv_destroy": (None, [vp]),
    "pf_kv_store": (C.c_int32, [vp, C.c_uint32, C.c_uint32, C.c_uint32, f32p, f32p]),
    "pf_kv_attention_scores": (C.c_int32, [vp, C.c_uint32, C.c_uint32, f32p, f32p, u32p]),
    "pf_kv_attention_weighted_sum": (C.c_int32, [vp, C.c_uint32, C.c_uint32, f32p, f32p, C.c_uint32]),
    "pf_kv_size": (C.c_uint32, [vp]),
    "pf_kv_clear": (C.c_int32, [vp]),
    "pf_kv_memory_usage": (C.c_size_t, [vp]),
    "pf_model_create": (C.c_int32, [vp, C.POINTER(ModelDesc), C.POINTER(vp)]),
    "pf_model_destroy": (None, [vp]),
    "pf_model_set_matrix": (C.c_int32, [vp, C.c_uint32, C.c_int32, C.c_int32, u8p, u16p]),
    "pf_model_set_embedding": (C.c_int32, [vp, u8p, u16p]),
    "pf_model_set_embedding_fmt": (C.c_int32, [vp, C.c_int32, u8p, u16p]),
    "pf_model_set_mtp": (C.c_int32, [vp, C.c_uint32, C.c_int32, u8p, u16p]),
    "pf_model_set_norm": (C.c_int32, [vp, C.c_uint32, C.c_int32, f32p]),
    "pf_engine_create": (C.c_int32, [vp, C.POINTER(CacheDesc), C.POINTER(vp)]),
    "pf_engine_destroy": (None, [vp]),
    "pf_engine_reset": (C.c_int32, [vp]),
    "pf_engine_position": (C.c_uint32, [vp]),
    "pf_engine_set_verify_full": (C.c_int32, [vp, C.c_int32]),
    "pf_engine_kv_export": (C.c_int32, [vp, C.c_uint32, C.c_uint32, C.c_uint32, vp, vp, vp, vp, C.c_uint32, vp]),
    "pf_forward": (C.c_int32, [vp, i32p, C.c_uint32, f32p, f32p]),
    "pf_mtp_forward": (C.c_int32, [vp, f32p, f32p]),
    "pf_sample": (C.c_int32, [vp, f32p, C.POINTER(Sampling), C.c_uint64, C.POINTER(C.c_uint64), i32p]),
    "pf_step_mtp": (C.c_int32, [vp, C.c_int32, f32p, C.POINTER(Sampling), C.c_uint64, C.POINTER(C.c_uint64), i32p,
                                i32p, i32p, f32p, i32p]),
    "pf_generate": (C.c_int32, [vp, i32p, C.c_uint32, C.c_uint32, C.POINTER(Sampling), C.c_uint64, i32p,
                                C.c_uint32, C.POINTER(GenResult)]),
    "pf_engine_set_max_memory": (C.c_int32, [vp, C.c_size_t]),
    "pf_engine_set_mtp_enabled": (C.c_int32, [vp, C.c_int32]),
    "pf_engine_set_layer_skip": (C.c_int32, [vp, C.c_float, C.c_uint32]),
    "pf_squeeze_open": (C.c_int32, [C.c_char_p, C.POINTER(vp)]),
    "pf_squeeze_close": (None, [vp]),
    "pf_squeeze_last_error": (C.c_char_p, [vp]),
    "pf_squeeze_get_info": (C.c_int32, [vp, C.POINTER(SqueezeInfo)]),
    "pf_squeeze_block_shape": (C.c_int32, [vp, C.c_uint32, C.c_uint32, u32p, u32p, u32p]),
    "pf_squeeze_load_block": (C.c_int32, [vp, C.c_uint32, C.c_uint32, vp, f32p]),
    "pf_squeeze_load_model": (C.c_int32, [vp, vp, C.POINTER(vp)]),
    "pf_engine_layer_skip_count": (C.c_int32, [vp, C.POINTER(C.c_uint64)]),
    "pf_engine_pass_times": (C.c_int32, [vp, C.POINTER(C.c_double), C.POINTER(C.c_double), u32p, u32p]),
    "pf_engine_profile": (C.c_int32, [vp, C.c_int32]),
    "pf_engine_round_time": (C.c_int32, [vp, C.POINTER(C.c_double), u32p]),
    "pf_engine_set_round_timing": (C.c_int32, [vp, C.c_int32]),
    "pf_engine_gemv_stats": (C.c_int32, [vp, u32p, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "pf_engine_attn_stats": (C.c_int32, [vp, u32p, C.POINTER(C.c_double)]),
    "pf_engine_gemv_by_size": (C.c_int32, [vp, C.c_uint32, C.POINTER(C.c_double), u32p, C.POINTER(C.c_double),
                                           u32p]),
    "pf_batch_create": (C.c_int32, [vp, C.POINTER(CacheDesc), C.c_uint32, C.POINTER(vp)]),
    "pf_batch_sequences": (C.c_uint32, [vp]),
    "pf_batch_position": (C.c_uint32, [vp, C.c_uint32]),
    "pf_batch_prefill": (C.c_int32, [vp, C.c_uint32, i32p, C.c_uint32]),
    "pf_batch_forward": (C.c_int32, [vp, u32p, C.c_uint32, C.c_uint32, i32p, f32p, f32p]),
    "pf_batch_generate": (C.c_int32, [vp, i32p, u32p, C.c_uint32, C.POINTER(Sampling), C.POINTER(C.c_uint64), i32p,
                                      C.c_uint32, C.POINTER(GenResult)]),
    "pf_batch_open": (C.c_int32, [vp, C.POINTER(Sampling), C.c_uint32]),
    "pf_batch_admit": (C.c_int32, [vp, C.c_uint32, i32p, C.c_uint32, C.c_uint32, C.c_uint64]),
    "pf_batch_step": (C.c_int32, [vp, u32p, u32p]),
    "pf_batch_take": (C.c_int32, [vp, C.c_uint32, i32p, C.c_uint32, C.POINTER(GenResult)]),
}

_lib = None


def lib():
    """The loaded C-ABI library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise PFError(f"{LIB_PATH} is missing: run `python -m pocketforge_amd.build` (no CPU fallback exists)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SYMBOLS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def P(a, t):
    return a.ctypes.data_as(t)


def _dptr(t):
    if t is None:
        return None
    if isinstance(t, DeviceArray):
        return C.c_void_p(t.ptr)
    return C.c_void_p(t.data_ptr())


class DeviceArray:
    """A device buffer owned by a Context (pf_malloc), holding one numpy
    dtype/shape.  Accepted wherever the C ABI takes *_dev pointers."""

    def __init__(self, ctx, shape, dtype):
        self.ctx = ctx
        self.shape = tuple(np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = vp()
        ctx.check(lib().pf_malloc(ctx.h, max(self.nbytes, 1), C.byref(p)), "pf_malloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, ctx, a):
        a = np.ascontiguousarray(a)
        d = cls(ctx, a.shape, a.dtype)
        ctx.check(lib().pf_memcpy(ctx.h, C.c_void_p(d.ptr), a.ctypes.data_as(vp), a.nbytes, 0), "pf_memcpy")
        return d

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        self.ctx.check(lib().pf_memcpy(self.ctx.h, out.ctypes.data_as(vp), C.c_void_p(self.ptr), self.nbytes, 1),
                       "pf_memcpy")
        return out

    def free(self):
        if self.ptr and self.ctx.h:
            lib().pf_free(self.ctx.h, C.c_void_p(self.ptr), max(self.nbytes, 1))
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ----------------------------------------------------- host-side weights

def gen_matrix(seed, stream, std, rows, cols, fmt):
    """N(0, std^2) weights quantized to a 32-block format (interchange layout)."""
    bb = block_bytes(fmt)
    codes = np.zeros((rows, cols // 32, bb), np.uint8)
    scales = np.zeros((rows, cols // 32), np.uint16)
    rc = lib().pf_gen_matrix(seed, stream, std, rows, cols, fmt, P(codes, u8p), P(scales, u16p))
    if rc:
        raise PFError(f"pf_gen_matrix failed ({rc})")
    return codes, scales


def quantize_matrix(w, fmt):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    bb = block_bytes(fmt)
    codes = np.zeros((rows, cols // 32, bb), np.uint8)
    scales = np.zeros((rows, cols // 32), np.uint16)
    rc = lib().pf_quantize_matrix(P(w, f32p), rows, cols, fmt, P(codes, u8p), P(scales, u16p))
    if rc:
        raise PFError(f"pf_quantize_matrix failed ({rc})")
    return codes, scales


# ------------------------------------------------------------- objects

class Context:
    def __init__(self, device=0):
        self.h = vp()
        rc = lib().pf_init(device, C.byref(self.h))
        if rc:
            msg = lib().pf_last_error(None)
            raise PFError(f"pf_init({device}) failed ({rc}): {msg.decode() if msg else ''}")

    def check(self, rc, what=""):
        if rc:
            raise PFError(f"{what} failed ({rc}): {lib().pf_last_error(self.h).decode()}")

    def close(self):
        if self.h:
            lib().pf_destroy(self.h)
            self.h = None

    def synchronize(self):
        self.check(lib().pf_synchronize(self.h), "pf_synchronize")

    def device_info(self):
        buf = C.create_string_buffer(256)
        cus = C.c_int(0)
        self.check(lib().pf_device_info(self.h, buf, 256, C.byref(cus)), "pf_device_info")
        return buf.value.decode(), cus.value

    @property
    def device_bytes(self):
        return lib().pf_device_bytes(self.h)

    # matmul_neon.hpp mirrors (device buffers: DeviceArray)
    def to_device(self, a):
        return DeviceArray.from_numpy(self, a)

    def empty(self, shape, dtype):
        return DeviceArray(self, shape, dtype)

    def quantize_activation_rows(self, x):
        M, K = x.shape
        q = self.empty((M, K), np.int8)
        s = self.empty((M,), np.float32)
        self.check(lib().pf_quantize_activation_rows(self.h, _dptr(x), _dptr(q), _dptr(s), M, K),
                   "pf_quantize_activation_rows")
        self.synchronize()
        return q, s

    def matmul_int8(self, A, B):
        M, K = A.shape
        N = B.shape[0]
        Cm = self.empty((M, N), np.int32)
        self.check(lib().pf_matmul_int8(self.h, _dptr(A), _dptr(B), _dptr(Cm), M, N, K), "pf_matmul_int8")
        self.synchronize()
        return Cm

    def matmul_quantized(self, A, B, w_scales, act_scales=None):
        M, K = A.shape
        N = B.shape[0]
        Cm = self.empty((M, N), np.float32)
        self.check(lib().pf_matmul_quantized(self.h, _dptr(A), _dptr(B), _dptr(Cm), M, N, K, _dptr(w_scales),
                                             _dptr(act_scales)), "pf_matmul_quantized")
        self.synchronize()
        return Cm

    def dot_product(self, a, b):
        out = self.empty((1,), np.float32)
        self.check(lib().pf_dot_product(self.h, _dptr(a), _dptr(b), a.shape[0], _dptr(out)), "pf_dot_product")
        return float(out.numpy()[0])

    def softmax(self, v):
        """In place on a DeviceArray of floats."""
        self.check(lib().pf_softmax(self.h, _dptr(v), v.shape[0]), "pf_softmax")
        self.synchronize()

    def rmsnorm(self, x, w):
        out = self.empty(x.shape, np.float32)
        self.check(lib().pf_rmsnorm(self.h, _dptr(out), _dptr(x), _dptr(w), x.shape[0]), "pf_rmsnorm")
        self.synchronize()
        return out

    def argmax(self, x):
        out = self.empty((1,), np.int32)
        self.check(lib().pf_argmax(self.h, _dptr(x), x.shape[0], _dptr(out)), "pf_argmax")
        return int(out.numpy()[0])

    def upload_matrix(self, fmt, codes, scales, rowmajor=False):
        return Matrix(self, fmt, codes, scales, rowmajor)

    def gemv_q(self, W, x):
        M = x.shape[0]
        y = self.empty((M, W.rows), np.float32)
        self.check(lib().pf_gemv_q(self.h, W.h, _dptr(x), _dptr(y), M), "pf_gemv_q")
        self.synchronize()
        return y

    def gemv_q_noalloc(self, W, x):
        """gemv_q through the entry point that allocates nothing (its M > 8
        path uses the library's fixed per-GPU scratch)."""
        M = x.shape[0]
        y = self.empty((M, W.rows), np.float32)
        self.check(lib().pf_gemv_q_noalloc(self.h, W.h, _dptr(x), _dptr(y), M), "pf_gemv_q_noalloc")
        self.synchronize()
        return y

    def gemv_f32(self, W, x):
        M = x.shape[0]
        y = self.empty((M, W.rows), np.float32)
        self.check(lib().pf_gemv_f32(self.h, W.h, _dptr(x), _dptr(y), M), "pf_gemv_f32")
        self.synchronize()
        return y


class Matrix:
    def __init__(self, ctx, fmt, codes, scales, rowmajor=False):
        self.ctx = ctx
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales, np.uint16)
        self.rows, nb = scales.shape
        self.cols = nb * 32
        self.h = vp()
        ctx.check(lib().pf_matrix_upload(ctx.h, fmt, self.rows, self.cols, P(codes, u8p), P(scales, u16p),
                                         int(rowmajor), C.byref(self.h)), "pf_matrix_upload")

    def close(self):
        if self.h:
            lib().pf_matrix_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


class MTPHeads:
    """include/forge/mtp.hpp:31-53 on the GPU: n chained heads of n_embd x
    n_embd Q4 gate/up/down, unembedded with an fp32 tied table (or the
    placeholder logits when none is set)."""

    def __init__(self, ctx, n_heads, n_embd, n_vocab):
        self.ctx = ctx
        self.n_heads, self.n_embd, self.n_vocab = n_heads, n_embd, n_vocab
        self.h = vp()
        ctx.check(lib().pf_mtp_create(ctx.h, n_heads, n_embd, n_vocab, C.byref(self.h)), "pf_mtp_create")

    def set_head(self, head, which, codes, scales):
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales, np.uint16)
        self.ctx.check(lib().pf_mtp_set_head(self.h, head, which, P(codes, u8p), P(scales, u16p)),
                       "pf_mtp_set_head")

    def set_table(self, table):
        t = None if table is None else np.ascontiguousarray(table, np.float32)
        self.ctx.check(lib().pf_mtp_set_table(self.h, P(t, f32p) if t is not None else None), "pf_mtp_set_table")

    def forward(self, hidden):
        hidden = np.ascontiguousarray(hidden, np.float32)
        out = np.zeros((self.n_heads, self.n_vocab), np.float32)
        self.ctx.check(lib().pf_mtp_heads_forward(self.h, P(hidden, f32p), P(out, f32p)), "pf_mtp_heads_forward")
        return out

    def memory_usage(self):
        return lib().pf_mtp_memory(self.h)

    def close(self):
        if self.h:
            lib().pf_mtp_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


class KVCache:
    """include/forge/kv_cache.hpp:33-56 on the GPU."""

    def __init__(self, ctx, n_layers=24, n_kv_heads=4, head_dim=64, sink_size=4, window_size=8192,
                 pool_block=64, max_context=131072):
        self.ctx = ctx
        self.head_dim = head_dim
        cfg = KvConfig(n_layers, n_kv_heads, head_dim, sink_size, window_size, pool_block, max_context)
        self.h = vp()
        ctx.check(lib().pf_kv_create(ctx.h, C.byref(cfg), C.byref(self.h)), "pf_kv_create")
        self.cap = 8 + window_size + max_context + 64

    def store(self, layer, head, pos, key, value):
        key = np.ascontiguousarray(key, np.float32)
        value = np.ascontiguousarray(value, np.float32)
        self.ctx.check(lib().pf_kv_store(self.h, layer, head, pos, P(key, f32p), P(value, f32p)), "pf_kv_store")

    def attention_scores(self, layer, head, q):
        q = np.ascontiguousarray(q, np.float32)
        out = np.zeros(self.cap, np.float32)
        n = C.c_uint32(0)
        self.ctx.check(lib().pf_kv_attention_scores(self.h, layer, head, P(q, f32p), P(out, f32p), C.byref(n)),
                       "pf_kv_attention_scores")
        return out[: n.value].copy()

    def attention_weighted_sum(self, layer, head, scores, count=None):
        scores = np.ascontiguousarray(scores, np.float32)
        out = np.zeros(self.head_dim, np.float32)
        cnt = len(scores) if count is None else count
        self.ctx.check(lib().pf_kv_attention_weighted_sum(self.h, layer, head, P(scores, f32p), P(out, f32p), cnt),
                       "pf_kv_attention_weighted_sum")
        return out

    def size(self):
        return lib().pf_kv_size(self.h)

    def clear(self):
        self.ctx.check(lib().pf_kv_clear(self.h), "pf_kv_clear")

    def memory_usage(self):
        return lib().pf_kv_memory_usage(self.h)

    def close(self):
        if self.h:
            lib().pf_kv_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


class Squeeze:
    """A .squeeze file (WeightLoader, include/forge/quant_format.hpp:92-140) read
    on the host; no GPU use."""

    def __init__(self, path):
        self.h = vp()
        rc = lib().pf_squeeze_open(str(path).encode(), C.byref(self.h))
        if rc:
            self.h = None
            raise PFError(f"pf_squeeze_open failed ({rc}): {lib().pf_squeeze_last_error(None).decode()}")
        self._info = SqueezeInfo()
        lib().pf_squeeze_get_info(self.h, C.byref(self._info))

    def _check(self, rc, what):
        if rc:
            raise PFError(f"{what} failed ({rc}): {lib().pf_squeeze_last_error(self.h).decode()}")

    def info(self):
        return {n: getattr(self._info, n) for n, _ in SqueezeInfo._fields_}

    def block_shape(self, layer, matrix):
        r, c, q = C.c_uint32(0), C.c_uint32(0), C.c_uint32(0)
        self._check(lib().pf_squeeze_block_shape(self.h, layer, matrix, C.byref(r), C.byref(c), C.byref(q)),
                    "pf_squeeze_block_shape")
        return r.value, c.value, q.value

    def load_block(self, layer, matrix):
        """(codes int8 [rows, cols], block multipliers float32 [ceil(rows*cols/32)], quant type)."""
        rows, cols, q = self.block_shape(layer, matrix)
        codes = np.zeros((rows, cols), np.int8)
        scales = np.zeros((rows * cols + 31) // 32, np.float32)
        self._check(lib().pf_squeeze_load_block(self.h, layer, matrix, codes.ctypes.data_as(vp), P(scales, f32p)),
                    "pf_squeeze_load_block")
        return codes, scales, q

    def close(self):
        if self.h:
            lib().pf_squeeze_close(self.h)
            self.h = None

    def __del__(self):
        self.close()


class Model:
    """Weights resident in HBM (pf_model_*)."""

    @classmethod
    def from_squeeze(cls, ctx, path, mtp=None):
        """Engine::load_model over a .squeeze file: every layer uploaded in the
        device layout.  mtp: optional [n_mtp] list of {gate, up, down} Q4
        (fmt, codes, scales) heads, which the file format does not hold."""
        sq = Squeeze(path)
        try:
            self = cls.__new__(cls)
            self.ctx = ctx
            i = sq.info()
            self.cfg = dict(n_layers=i["n_layers"], n_embd=i["n_embd"], n_heads=i["n_heads"],
                            head_dim=i["n_embd"] // max(1, i["n_heads"]), n_ff=i["n_ff"], n_vocab=i["n_vocab"],
                            n_mtp=i["mtp_heads"])
            self.h = vp()
            sq._check(lib().pf_squeeze_load_model(ctx.h, sq.h, C.byref(self.h)), "pf_squeeze_load_model")
            for k, hw in enumerate(mtp or []):
                for j, n in enumerate(["gate", "up", "down"]):
                    fmt, codes, scales = hw[n]
                    ctx.check(lib().pf_model_set_mtp(self.h, k, j, P(codes, u8p), P(scales, u16p)),
                              "pf_model_set_mtp")
            return self
        finally:
            sq.close()

    def __init__(self, ctx, cfg, weights):
        self.ctx = ctx
        self.cfg = cfg
        d = ModelDesc(cfg["n_layers"], cfg["n_embd"], cfg["n_heads"], cfg["head_dim"], cfg["n_ff"], cfg["n_vocab"],
                      cfg["n_mtp"])
        self.h = vp()
        ctx.check(lib().pf_model_create(ctx.h, C.byref(d), C.byref(self.h)), "pf_model_create")
        names = ["wq", "wk", "wv", "wo", "wgate", "wup", "wdown"]
        for l in range(cfg["n_layers"]):
            for j, n in enumerate(names):
                fmt, codes, scales = weights["layers"][l][n]
                ctx.check(lib().pf_model_set_matrix(self.h, l, j, fmt, P(codes, u8p), P(scales, u16p)),
                          f"pf_model_set_matrix({l},{n})")
        fmt, codes, scales = weights["emb"]
        ctx.check(lib().pf_model_set_embedding_fmt(self.h, fmt, P(codes, u8p), P(scales, u16p)),
                  "pf_model_set_embedding_fmt")
        for k in range(cfg["n_mtp"]):
            for j, n in enumerate(["gate", "up", "down"]):
                fmt, codes, scales = weights["mtp"][k][n]
                ctx.check(lib().pf_model_set_mtp(self.h, k, j, P(codes, u8p), P(scales, u16p)), "pf_model_set_mtp")
        an = np.ascontiguousarray(weights["attn_norm"], np.float32).reshape(cfg["n_layers"], -1)
        fn = np.ascontiguousarray(weights["ffn_norm"], np.float32).reshape(cfg["n_layers"], -1)
        for l in range(cfg["n_layers"]):
            ctx.check(lib().pf_model_set_norm(self.h, l, 7, P(np.ascontiguousarray(an[l]), f32p)), "set_norm")
            ctx.check(lib().pf_model_set_norm(self.h, l, 8, P(np.ascontiguousarray(fn[l]), f32p)), "set_norm")

    def close(self):
        if self.h:
            lib().pf_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


class Engine:
    """include/forge/engine.hpp:15-74 (forward, MTP, sample, generate) on the GPU."""

    def __init__(self, model, sink_size=4, window_size=8192, pool_block=64, max_context=4096):
        self.model = model
        self.ctx = model.ctx
        self.cfg = model.cfg
        cd = CacheDesc(sink_size, window_size, pool_block, max_context)
        self.h = vp()
        self.ctx.check(lib().pf_engine_create(model.h, C.byref(cd), C.byref(self.h)), "pf_engine_create")

    def reset(self):
        self.ctx.check(lib().pf_engine_reset(self.h), "pf_engine_reset")

    @property
    def pos(self):
        return lib().pf_engine_position(self.h)

    def forward(self, tokens, want_logits=True):
        toks = np.ascontiguousarray(np.atleast_1d(tokens), np.int32)
        n = len(toks)
        V, D = self.cfg["n_vocab"], self.cfg["n_embd"]
        logits = np.zeros((n, V), np.float32) if want_logits else None
        hidden = np.zeros((n, D), np.float32)
        self.ctx.check(lib().pf_forward(self.h, P(toks, i32p), n, P(logits, f32p) if want_logits else None,
                                        P(hidden, f32p)), "pf_forward")
        return logits, hidden

    def prefill(self, tokens):
        """Forward tokens (<= 8) at the next positions, no outputs copied."""
        toks = np.ascontiguousarray(np.atleast_1d(tokens), np.int32)
        self.ctx.check(lib().pf_forward(self.h, P(toks, i32p), len(toks), None, None), "pf_forward")

    def mtp_forward(self, hidden):
        hidden = np.ascontiguousarray(hidden, np.float32)
        out = np.zeros((self.cfg["n_mtp"], self.cfg["n_vocab"]), np.float32)
        self.ctx.check(lib().pf_mtp_forward(self.h, P(hidden, f32p), P(out, f32p)), "pf_mtp_forward")
        return out

    def step_mtp(self, token, hidden, sampling, seed=42, draw=0):
        """Engine::step_mtp on the device: (accepted, rejecting row's logits
        or None, mtp_accepted_out, mtp_rejected_out, draw counter after)."""
        hidden = np.ascontiguousarray(hidden, np.float32)
        lg = np.zeros(self.cfg["n_vocab"], np.float32)
        d = C.c_uint64(draw)
        a, acc, rej, has = C.c_int32(0), C.c_int32(0), C.c_int32(0), C.c_int32(0)
        self.ctx.check(lib().pf_step_mtp(self.h, int(token), P(hidden, f32p), C.byref(sampling), seed, C.byref(d),
                                         C.byref(a), C.byref(acc), C.byref(rej), P(lg, f32p), C.byref(has)),
                       "pf_step_mtp")
        return a.value, (lg if has.value else None), acc.value, rej.value, d.value

    def sample(self, logits, sampling, seed, draw_idx):
        logits = np.ascontiguousarray(logits, np.float32)
        d = C.c_uint64(draw_idx)
        t = C.c_int32(0)
        self.ctx.check(lib().pf_sample(self.h, P(logits, f32p), C.byref(sampling), seed, C.byref(d), C.byref(t)),
                       "pf_sample")
        return t.value, d.value

    def generate(self, prompt, max_new, sampling=None, seed=7):
        s = sampling or Sampling(0.8, 0.95, 40, 1)
        prompt = np.ascontiguousarray(prompt, np.int32)
        cap = len(prompt) + max_new + 8
        toks = np.zeros(cap, np.int32)
        res = GenResult()
        self.ctx.check(lib().pf_generate(self.h, P(prompt, i32p), len(prompt), max_new, C.byref(s), seed,
                                         P(toks, i32p), cap, C.byref(res)), "pf_generate")
        return toks[: res.n_tokens].copy(), res

    def set_max_memory(self, nbytes):
        self.ctx.check(lib().pf_engine_set_max_memory(self.h, nbytes), "pf_engine_set_max_memory")

    def set_verify_full(self, full):
        """1: every MTP round verifies all drafts in one pass; 0 (default):
        one-row first segment after a round with no accepted draft."""
        self.ctx.check(lib().pf_engine_set_verify_full(self.h, int(full)), "pf_engine_set_verify_full")

    def set_mtp_enabled(self, enabled):
        self.ctx.check(lib().pf_engine_set_mtp_enabled(self.h, int(enabled)), "pf_engine_set_mtp_enabled")

    def set_layer_skip(self, threshold, interval=4):
        self.ctx.check(lib().pf_engine_set_layer_skip(self.h, float(threshold), int(interval)),
                       "pf_engine_set_layer_skip")

    def layer_skip_count(self):
        n = C.c_uint64(0)
        self.ctx.check(lib().pf_engine_layer_skip_count(self.h, C.byref(n)), "pf_engine_layer_skip_count")
        return n.value

    def pass_times(self):
        v, b = C.c_double(0), C.c_double(0)
        vn, bn = C.c_uint32(0), C.c_uint32(0)
        self.ctx.check(lib().pf_engine_pass_times(self.h, C.byref(v), C.byref(b), C.byref(vn), C.byref(bn)),
                       "pf_engine_pass_times")
        return v.value, b.value, vn.value, bn.value

    def profile(self, enable=True):
        """Profiling level (pf_engine_profile): False/0 captured graphs, True/1
        kernels one by one with per-dispatch events on the verify passes, 2
        kernels one by one with events around each pass only."""
        self.ctx.check(lib().pf_engine_profile(self.h, int(enable)), "pf_engine_profile")

    def set_round_timing(self, on=True):
        """HIP events around every decode segment (pf_engine_set_round_timing),
        for round_time(); off by default."""
        self.ctx.check(lib().pf_engine_set_round_timing(self.h, int(bool(on))), "pf_engine_set_round_timing")

    def round_time(self):
        us, n = C.c_double(0), C.c_uint32(0)
        self.ctx.check(lib().pf_engine_round_time(self.h, C.byref(us), C.byref(n)), "pf_engine_round_time")
        return us.value, n.value

    def gemv_stats(self):
        n, us, by = C.c_uint32(0), C.c_double(0), C.c_double(0)
        self.ctx.check(lib().pf_engine_gemv_stats(self.h, C.byref(n), C.byref(us), C.byref(by)),
                       "pf_engine_gemv_stats")
        return n.value, us.value, by.value

    def gemv_by_size(self):
        """[(algorithmic bytes, launches, average us)] of the profiled GEMV
        launches, one entry per matrix shape."""
        n = C.c_uint32(0)
        self.ctx.check(lib().pf_engine_gemv_by_size(self.h, 0, None, None, None, C.byref(n)),
                       "pf_engine_gemv_by_size")
        k = n.value
        by, ln, us = (C.c_double * k)(), (C.c_uint32 * k)(), (C.c_double * k)()
        self.ctx.check(lib().pf_engine_gemv_by_size(self.h, k, by, ln, us, C.byref(n)), "pf_engine_gemv_by_size")
        return [(by[i], ln[i], us[i]) for i in range(min(k, n.value))]

    def kv_export(self, seq, layer, head, cap):
        """One KV plane's state at the sequence's position: (k, ks, v, vs,
        counts) with counts = (sink, pooled, window, pending) rows in that
        order (see pf_engine_kv_export)."""
        hd = self.cfg["n_embd"] // self.cfg["n_heads"]
        k = np.zeros((cap, hd), np.int8)
        v = np.zeros((cap, hd), np.int8)
        ks = np.zeros(cap, np.float32)
        vs = np.zeros(cap, np.float32)
        counts = np.zeros(4, np.uint32)
        self.ctx.check(lib().pf_engine_kv_export(self.h, seq, layer, head, P(k, vp), P(ks, vp), P(v, vp),
                                                 P(vs, vp), cap, P(counts, vp)), "pf_engine_kv_export")
        n = int(counts.sum())
        return k[:n], ks[:n], v[:n], vs[:n], tuple(int(x) for x in counts)

    def attn_stats(self):
        n, us = C.c_uint32(0), C.c_double(0)
        self.ctx.check(lib().pf_engine_attn_stats(self.h, C.byref(n), C.byref(us)), "pf_engine_attn_stats")
        return n.value, us.value

    def close(self):
        if self.h:
            lib().pf_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


class BatchEngine(Engine):
    """n_seq independent sequences over one model, decoded together: each
    sequence's tokens equal a single-sequence Engine's for the same prompt
    and seed, while every forward pass covers all sequences (no counterpart
    in the reference, which decodes one sequence per Engine)."""

    def __init__(self, model, n_seq, sink_size=4, window_size=8192, pool_block=64, max_context=4096):
        self.model = model
        self.ctx = model.ctx
        self.cfg = model.cfg
        self.n_seq = n_seq
        cd = CacheDesc(sink_size, window_size, pool_block, max_context)
        self.h = vp()
        self.ctx.check(lib().pf_batch_create(model.h, C.byref(cd), n_seq, C.byref(self.h)), "pf_batch_create")

    def position(self, seq):
        return lib().pf_batch_position(self.h, seq)

    def prefill_seq(self, seq, tokens):
        toks = np.ascontiguousarray(np.atleast_1d(tokens), np.int32)
        self.ctx.check(lib().pf_batch_prefill(self.h, seq, P(toks, i32p), len(toks)), "pf_batch_prefill")

    def forward_batch(self, seqs, tokens, want_logits=True):
        """tokens [len(seqs)][rows]: one pass; returns logits and hidden [len(seqs)][rows][...]."""
        seqs = np.ascontiguousarray(seqs, np.uint32)
        toks = np.ascontiguousarray(tokens, np.int32).reshape(len(seqs), -1)
        n, r = toks.shape
        V, D = self.cfg["n_vocab"], self.cfg["n_embd"]
        logits = np.zeros((n, r, V), np.float32) if want_logits else None
        hidden = np.zeros((n, r, D), np.float32)
        self.ctx.check(lib().pf_batch_forward(self.h, P(seqs, u32p), n, r, P(toks, i32p),
                                              P(logits, f32p) if want_logits else None, P(hidden, f32p)),
                       "pf_batch_forward")
        return logits, hidden

    def generate_batch(self, prompts, max_new, sampling=None, seeds=None):
        """prompts: list of n_seq int arrays; returns (list of token arrays, list of GenResult)."""
        s = sampling or Sampling(0.8, 0.95, 40, 1)
        assert len(prompts) == self.n_seq
        lens = np.array([len(p) for p in prompts], np.uint32)
        flat = np.ascontiguousarray(np.concatenate([np.asarray(p, np.int32) for p in prompts]) if lens.sum()
                                    else np.zeros(1, np.int32), np.int32)
        seeds = np.ascontiguousarray(seeds if seeds is not None else np.full(self.n_seq, 7), np.uint64)
        cap = int(lens.max()) + max_new + 8
        toks = np.zeros((self.n_seq, cap), np.int32)
        res = (GenResult * self.n_seq)()
        self.ctx.check(lib().pf_batch_generate(self.h, P(flat, i32p), P(lens, u32p), max_new, C.byref(s),
                                               seeds.ctypes.data_as(C.POINTER(C.c_uint64)), P(toks, i32p), cap,
                                               res), "pf_batch_generate")
        return [toks[i, : res[i].n_tokens].copy() for i in range(self.n_seq)], list(res)

    # continuous batching: requests join and leave between rounds
    def open(self, sampling=None, tokens_cap=1024):
        s = sampling or Sampling(0.8, 0.95, 40, 1)
        self._cap = tokens_cap
        self.ctx.check(lib().pf_batch_open(self.h, C.byref(s), tokens_cap), "pf_batch_open")

    def admit(self, seq, prompt, max_new, seed=7):
        p = np.ascontiguousarray(prompt, np.int32)
        self.ctx.check(lib().pf_batch_admit(self.h, seq, P(p, i32p), len(p), max_new, seed), "pf_batch_admit")

    def step(self):
        """One round of every generating slot; returns the slots that finished."""
        fin = np.zeros(self.n_seq, np.uint32)
        n = C.c_uint32(0)
        self.ctx.check(lib().pf_batch_step(self.h, P(fin, u32p), C.byref(n)), "pf_batch_step")
        return [int(x) for x in fin[: n.value]]

    def take(self, seq):
        """(tokens, GenResult) of a slot, which becomes free."""
        toks = np.zeros(self._cap, np.int32)
        r = GenResult()
        self.ctx.check(lib().pf_batch_take(self.h, seq, P(toks, i32p), self._cap, C.byref(r)), "pf_batch_take")
        return toks[: r.n_tokens].copy(), r
