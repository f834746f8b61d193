"""Host side of the library without a GPU: it loads, exports every entry
point of include/pf_gpu.h, and its weight synthesis / quantizer matches the
oracle's restatement of the reference code rules byte for byte."""
import os
import re

import numpy as np
import pytest

import oracle as O
import pocketforge_amd as pf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "pf_gpu.h")).read()
    return sorted(set(re.findall(r"\b(pf_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    L = pf.lib()
    decl = declared_symbols()
    assert len(decl) >= 35
    for name in decl:
        assert hasattr(L, name), name
    assert set(decl) == set(pf.SYMBOLS), set(decl) ^ set(pf.SYMBOLS)


def test_init_without_gpu_fails_cleanly():
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("GPU present")
    except ImportError:
        pass
    with pytest.raises(pf.PFError):
        pf.Context(0)


@pytest.mark.parametrize("fmt", [pf.FMT_Q4, pf.FMT_Q2, pf.FMT_Q15, pf.FMT_Q8])
def test_quantizer_matches_oracle(fmt):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((96, 512)) * 0.02).astype(np.float32)
    w[3, :32] = 0.0                      # all-zero block
    w[4, 40] = 0.5                       # outlier block
    w[5, 64:96] *= 1e-7                  # block far below the row maximum (zeroed)
    w[6, ::2] = 0.015                    # ties at the rounding boundary
    c1, s1 = pf.quantize_matrix(w, fmt)
    c2, s2 = O.quantize_matrix(w, fmt)
    np.testing.assert_array_equal(c1, c2)
    np.testing.assert_array_equal(s1, s2)


def test_quantizer_code_rules():
    # Q4: v = clamp(round(x * 7/amax), -8, 7), byte = (v0+8) | (v1+8) << 4
    w = np.zeros((64, 256), np.float32)
    w[0, :4] = [0.7, -0.7, 0.35, 0.0]
    codes, scales = pf.quantize_matrix(w, pf.FMT_Q4)
    assert codes[0, 0, 0] == (7 + 8) | ((-7 + 8) << 4)
    assert codes[0, 0, 1] == (4 + 8) | (8 << 4)          # round(3.5) = 4 (half away from zero)
    assert np.float16(scales[0, 0].view(np.float16)) == np.float16(0.1)
    # Q2: v = clamp(round(x / amax), -2, 1), code = v + 2 at bits 2t
    codes, scales = pf.quantize_matrix(w, pf.FMT_Q2)
    assert codes[0, 0, 0] == (3 | (1 << 2) | (3 << 4) | (2 << 6))
    # Q1.5: 2 if x > 0.35 amax, 0 if x < -0.35 amax, else 1
    codes, scales = pf.quantize_matrix(w, pf.FMT_Q15)
    assert codes[0, 0, 0] == (2 | (0 << 2) | (2 << 4) | (1 << 6))
    np.testing.assert_allclose(scales[0, 0:1].view(np.float16).astype(np.float32), [0.5833], rtol=1e-3)
    # Q8: v = clamp(round(x * 127/amax), -127, 127), one signed byte per element, d = amax/127
    codes, scales = pf.quantize_matrix(w, pf.FMT_Q8)
    assert codes.shape == (64, 8, 32)
    assert list(codes[0, 0, :4].view(np.int8)) == [127, -127, 64, 0]      # round(63.5) = 64
    assert np.float16(scales[0, 0].view(np.float16)) == np.float16(0.7 / 127)


def test_gen_matrix_deterministic_and_normal():
    c1, s1 = pf.gen_matrix(1234, 3, 0.02, 256, 512, pf.FMT_Q4)
    c2, s2 = pf.gen_matrix(1234, 3, 0.02, 256, 512, pf.FMT_Q4)
    np.testing.assert_array_equal(c1, c2)
    np.testing.assert_array_equal(s1, s2)
    c3, _ = pf.gen_matrix(1234, 4, 0.02, 256, 512, pf.FMT_Q4)
    assert (c1 != c3).mean() > 0.5
    # dequantized values: mean ~0, std ~0.02 (within quantization error)
    q = pf.FMT_Q4
    W = O.qmat(q, c1, s1)
    import ctypes as C
    row = np.zeros(512, np.float32)
    vals = []
    for r in range(0, 256, 8):
        O.lib().orc_dequant_row(C.byref(W), r, O.ptr(row, O.f32p))
        vals.append(row.copy())
    v = np.concatenate(vals)
    assert abs(v.mean()) < 2e-3 and 0.016 < v.std() < 0.024
