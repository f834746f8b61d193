"""pf_gemv_q_noalloc, the entry point that allocates nothing, against
pf_gemv_q through the C ABI, bit for bit: two calls in a row through its
fixed per-GPU scratch (the second with fewer rows, so stale rows of the
first call are still in the array), the GEMV path (M <= 8, no scratch),
and the capacity check that turns an oversized call into an error before
any kernel runs."""
import numpy as np
import pytest

import pocketforge_amd as pf

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fmt", [pf.FMT_Q4, pf.FMT_Q2])
def test_gemv_q_noalloc_matches_gemv_q(gpu, fmt):
    N, K = 320, 2048
    codes, scales = pf.gen_matrix(77, 5 + fmt, 0.02, N, K, fmt)
    W = gpu.upload_matrix(fmt, codes, scales)
    rng = np.random.default_rng(11 + fmt)
    try:
        xs, want = [], []
        for M in (300, 45, 5):
            x = (rng.standard_normal((M, K)) * 0.5).astype(np.float32)
            x[M // 3] = 0.0                               # an all-zero row (scale 1, codes 0)
            xd = pf.DeviceArray.from_numpy(gpu, x)
            xs.append(xd)
            want.append(gpu.gemv_q(W, xd).numpy())
        print(f"pf_gemv_q_noalloc fmt {fmt} N {N} K {K}: M 300, 45, 5", flush=True)
        got = [gpu.gemv_q_noalloc(W, xd).numpy() for xd in xs]
        for M, g, w in zip((300, 45, 5), got, want):
            np.testing.assert_array_equal(g, w, err_msg=f"fmt {fmt} M {M}")
    finally:
        W.close()


def test_gemv_q_noalloc_rejects_oversize(gpu):
    N, K = 64, 4096
    codes, scales = pf.gen_matrix(78, 1, 0.02, N, K, pf.FMT_Q4)
    W = gpu.upload_matrix(pf.FMT_Q4, codes, scales)
    try:
        # 288 rows (padded to 288) x 4096 codes > 1 MiB: refused on the host
        xd = pf.DeviceArray.from_numpy(gpu, np.zeros((288, K), np.float32))
        with pytest.raises(pf.PFError, match=r"\(-6\).*fixed scratch"):
            gpu.gemv_q_noalloc(W, xd)
        # 256 rows x 4096 codes = 1 MiB exactly: accepted, equal to pf_gemv_q
        x = (np.random.default_rng(5).standard_normal((256, K)) * 0.5).astype(np.float32)
        xd = pf.DeviceArray.from_numpy(gpu, x)
        np.testing.assert_array_equal(gpu.gemv_q_noalloc(W, xd).numpy(), gpu.gemv_q(W, xd).numpy())
    finally:
        W.close()
