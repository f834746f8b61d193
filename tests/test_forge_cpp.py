"""The forge:: C++ classes (include/forge/*.hpp over the C ABI): the C++
tests in tests/cpp, written like the reference's own tests, run on the GPU;
on the CPU, the library's exports and its error path."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "pocketforge_amd", "_lib")
BIN = os.path.join(LIBDIR, "tests")
TESTS = ["test_forge_matmul", "test_forge_kv_cache", "test_forge_mtp", "test_forge_engine", "test_forge_batch"]


def _built(name):
    exe = os.path.join(BIN, name)
    if not os.path.exists(exe):
        pytest.skip("C++ tests not built (python -m pocketforge_amd.build)")
    return exe


def test_forge_library_exports_the_reference_api():
    lib = os.path.join(LIBDIR, "libforge_amd.so")
    if not os.path.exists(lib):
        pytest.skip("libforge_amd.so not built")
    out = subprocess.run(["nm", "-DC", "--defined-only", lib], capture_output=True, text=True, check=True).stdout
    for sym in ["forge::Engine::generate(", "forge::Engine::forward_with_hidden(", "forge::Engine::step_mtp(",
                "forge::Engine::sample_top_p(", "forge::KVCache::attention_scores(",
                "forge::KVCache::attention_weighted_sum(", "forge::MTPHeads::forward(",
                "forge::MTPHeads::speculative_accept(", "forge::matmul_int8(", "forge::matmul_quantized(",
                "forge::quantize_activation_row(", "forge::softmax(", "forge::rmsnorm(", "forge::dot_product(",
                "forge::BatchEngine::generate(", "forge::BatchEngine::load_random_model("]:
        assert sym in out, sym


def test_forge_fails_loudly_without_a_gpu():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    r = subprocess.run([_built("test_forge_matmul")], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "pf_init" in r.stderr


def _squeeze_file(path):
    """A 2-layer model (n_embd 256, n_ff 512, vocab 1024, 4 MTP heads) in the
    reference's .squeeze format."""
    import numpy as np
    import squeeze_writer as SW
    rng = np.random.default_rng(1)
    D, F, V = 256, 512, 1024
    shapes = [(D, D)] * 4 + [(F, D), (F, D), (D, F)]
    blocks = [(l, m, (0.02 * rng.standard_normal(s)).astype(np.float32), SW.Q4)
              for l in range(2) for m, s in enumerate(shapes)]
    blocks.append((0, 10, (0.02 * rng.standard_normal((V, D))).astype(np.float32), SW.Q4))
    SW.write_squeeze(str(path), dict(n_layers=2, n_embd=D, n_heads=4, n_kv_heads=4, n_ff=F, n_vocab=V,
                                     max_seq_len=512, mtp_heads=4), blocks)


@pytest.mark.gpu
@pytest.mark.parametrize("name", TESTS)
def test_forge_cpp(gpu, name, tmp_path):
    env = dict(os.environ)
    if name == "test_forge_engine":
        _squeeze_file(tmp_path / "m.squeeze")
        env["PF_TEST_SQUEEZE"] = str(tmp_path / "m.squeeze")
    r = subprocess.run([_built(name)], capture_output=True, text=True, timeout=300, env=env)
    print(r.stdout[-3000:])
    print(r.stderr[-3000:])
    assert r.returncode == 0, f"{name} failed:\n{r.stderr[-2000:]}"
