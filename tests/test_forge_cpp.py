"""The forge:: C++ classes (include/forge/*.hpp over the C ABI): the C++
tests in tests/cpp, written like the reference's own tests, run on the GPU;
on the CPU, the library's exports and its error path."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "pocketforge_amd", "_lib")
BIN = os.path.join(LIBDIR, "tests")
TESTS = ["test_forge_matmul", "test_forge_kv_cache", "test_forge_mtp", "test_forge_engine"]


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
                "forge::quantize_activation_row(", "forge::softmax(", "forge::rmsnorm(", "forge::dot_product("]:
        assert sym in out, sym


def test_forge_fails_loudly_without_a_gpu():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    r = subprocess.run([_built("test_forge_matmul")], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "pf_init" in r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("name", TESTS)
def test_forge_cpp(gpu, name):
    r = subprocess.run([_built(name)], capture_output=True, text=True, timeout=300)
    print(r.stdout[-3000:])
    print(r.stderr[-3000:])
    assert r.returncode == 0, f"{name} failed:\n{r.stderr[-2000:]}"
