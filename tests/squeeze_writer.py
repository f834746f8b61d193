""".squeeze writer for tests: a restatement of the reference's
Quantizer::quantize_matrix (src/quant_format.cpp:41-154),
Quantizer::compress_block (:156-168, zstd level 3) and
Quantizer::write_squeeze (:171-217), so tests can produce files in the
reference's format.  zstd is the system's libzstd.so.1.  Test
infrastructure only."""
import ctypes as C
import struct

import numpy as np

Q8, Q4, Q2, Q15 = 0, 1, 2, 3
BLOCK_BYTES = {Q8: 36, Q4: 20, Q2: 12, Q15: 16}

_z = None


def _zstd():
    global _z
    if _z is None:
        _z = C.CDLL("libzstd.so.1")
        _z.ZSTD_compressBound.restype = C.c_size_t
        _z.ZSTD_compressBound.argtypes = [C.c_size_t]
        _z.ZSTD_compress.restype = C.c_size_t
        _z.ZSTD_compress.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_int]
        _z.ZSTD_isError.restype = C.c_uint
        _z.ZSTD_isError.argtypes = [C.c_size_t]
    return _z


def _round_away(y):
    """std::round of float32 values (halves away from zero), exactly."""
    y = np.asarray(y, np.float32).astype(np.float64)
    return np.sign(y) * np.floor(np.abs(y) + 0.5)


def _to_int8(v):
    """(int8_t) of an integral value: two's-complement wrap, as x86 does for
    the conversion of 128."""
    return ((np.asarray(v, np.int64) + 128) % 256 - 128).astype(np.int8)


def quantize_matrix(w, qtype):
    """Bytes of one matrix (row-major, flattened, blocks of 32 elements)."""
    x = np.ascontiguousarray(w, np.float32).reshape(-1)
    n = x.size
    nb = (n + 31) // 32
    xp = np.zeros(nb * 32, np.float32)
    xp[:n] = x
    valid = np.arange(nb * 32) < n
    blocks = xp.reshape(nb, 32)
    vmask = valid.reshape(nb, 32)
    amax = np.where(vmask, np.abs(blocks), 0).max(axis=1).astype(np.float32)
    out = bytearray()
    if qtype == Q15:
        code = np.where(blocks > np.float32(0.35), 2, np.where(blocks < np.float32(-0.35), 0, 1))
        code = np.where(vmask, code, 0).astype(np.uint8)
        for b in range(nb):
            for i in range(0, 32, 2):
                byte = 0
                if vmask[b, i]:
                    byte |= int(code[b, i])
                if i + 1 < 32 and vmask[b, i + 1]:
                    byte |= int(code[b, i + 1]) << 2
                out.append(byte)
        return bytes(out)
    num = {Q8: 127.0, Q4: 7.0, Q2: 1.0}[qtype]
    with np.errstate(divide="ignore"):
        scale = np.where(amax == 0, np.float32(0), np.float32(num) / amax).astype(np.float32)
    y = (blocks * scale[:, None]).astype(np.float32)
    if qtype == Q8:
        c = _to_int8(_round_away((y + np.float32(0.5)).astype(np.float32)))
    elif qtype == Q4:
        c = np.clip(_to_int8(_round_away(y)), -8, 7)
    else:
        c = np.clip(_to_int8(_round_away(y)), -2, 1)
    for b in range(nb):
        out += struct.pack("<f", float(scale[b]))
        if qtype == Q8:
            row = [int(c[b, i]) & 255 if vmask[b, i] else 0 for i in range(32)]
            out += bytes(row)
        elif qtype == Q4:
            for i in range(0, 32, 2):
                if not vmask[b, i]:
                    continue
                byte = int(c[b, i]) + 8
                if vmask[b, i + 1]:
                    byte |= (int(c[b, i + 1]) + 8) << 4
                out.append(byte)
        else:
            for i in range(0, 32, 4):
                if not vmask[b, i]:
                    continue
                byte = 0
                for j in range(4):
                    if vmask[b, i + j]:
                        byte |= (int(c[b, i + j]) + 2) << (2 * j)
                out.append(byte)
    return bytes(out)


def compress_block(data):
    z = _zstd()
    cap = z.ZSTD_compressBound(len(data))
    dst = C.create_string_buffer(cap)
    src = C.create_string_buffer(data, len(data))
    r = z.ZSTD_compress(dst, cap, src, len(data), 3)
    if z.ZSTD_isError(r):
        return data
    return dst.raw[:r]


def write_squeeze(path, cfg, blocks):
    """cfg: n_layers, n_embd, n_heads, n_kv_heads, n_ff, n_vocab, max_seq_len,
    mtp_heads.  blocks: list of (layer, matrix, float array [rows, cols],
    quant type).  Returns the raw (uncompressed) bytes of each block."""
    raws, comps, recs = [], [], []
    for layer, matrix, w, qt in blocks:
        rows, cols = w.shape
        raw = quantize_matrix(w, qt)
        comp = compress_block(raw)
        raws.append(raw)
        comps.append(comp)
        recs.append([layer, matrix, rows, cols, len(comp), len(raw), qt, 0])
    off = 256
    for r, comp in zip(recs, comps):
        r[7] = off
        off += len(comp)
    index_offset = off

    def header(ioff, isize):
        h = b"FORGE\0\0\0" + struct.pack("<II", 1, len(blocks))
        h += struct.pack("<8I", cfg["n_layers"], cfg["n_embd"], cfg["n_heads"], cfg.get("n_kv_heads", cfg["n_heads"]),
                         cfg["n_ff"], cfg["n_vocab"], cfg.get("max_seq_len", 2048), cfg.get("mtp_heads", 0))
        h += struct.pack("<QQ", ioff, isize)
        return h + bytes(256 - len(h))

    with open(path, "wb") as f:
        f.write(header(index_offset, 32 * len(blocks)))
        for comp in comps:
            f.write(comp)
        for r in recs:
            # WeightBlock: six uint32, the quant type byte, 3 padding bytes,
            # the uint32 offset (include/forge/types.hpp:205-214)
            f.write(struct.pack("<6IB3xI", *r))
    return raws
