"""Builds libpocketforge_amd.so (gfx950 kernels + C ABI + host runtime) in
tree with hipcc.  Usage: python -m pocketforge_amd.build [--jobs N]"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "_lib")
LIB = os.path.join(LIBDIR, "libpocketforge_amd.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

# -ffp-contract=off: fused multiply-adds only where written (bit parity with
# the CPU restatement).  -munsafe-fp-atomics: hardware fp64 atomic add (the
# GEMV's split sums are exact, so their order never changes a bit; device
# memory from hipMalloc only).  Denormals are kept and fp32 divide/sqrt are
# correctly rounded.  Packed fp32 instructions are disabled.  The leading
# scalar and pointer arguments of a kernel (up to 16 SGPRs) are preloaded
# into SGPRs at wave launch, which saves the first kernel-argument load
# (about 0.6 us) where a kernel's first decision needs them.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off", "-munsafe-fp-atomics",
    "-fno-gpu-flush-denormals-to-zero", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wno-unused-result", "-I" + os.path.join(ROOT, "include"),
]
CXX_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-ffp-contract=off", "-I" + os.path.join(ROOT, "include")]

UNITS = [
    ("pf_runtime.hip", "hip"),
    ("pf_host.cpp", "cxx"),
    ("pf_squeeze.cpp", "cxx"),
]


def _compile(unit):
    src, kind = unit
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    if kind == "hip":
        cmd = [HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj]
    else:
        cmd = ["g++"] + CXX_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


HOST = os.path.join(HERE, "host")
FORGE_LIB = os.path.join(LIBDIR, "libforge_amd.so")
CPP_TESTS = os.path.join(ROOT, "tests", "cpp")
TEST_BIN = os.path.join(LIBDIR, "tests")
ORACLE_BUILD = os.path.join(ROOT, "oracle", "_build")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def build_forge():
    """libforge_amd.so: the forge:: C++ classes over the C ABI (g++ only)."""
    tmp = FORGE_LIB + ".tmp"
    _run(["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-I" + os.path.join(ROOT, "include"),
          os.path.join(HOST, "forge_api.cpp"), "-o", tmp, "-L" + LIBDIR, "-lpocketforge_amd",
          "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, FORGE_LIB)
    return FORGE_LIB


def build_cpp_tests():
    """The forge:: C++ tests, linked against libforge_amd.so and the oracle
    (their checker).  Binaries go to _lib/tests/."""
    os.makedirs(TEST_BIN, exist_ok=True)
    out = []
    for f in sorted(os.listdir(CPP_TESTS)):
        if not f.endswith(".cpp"):
            continue
        exe = os.path.join(TEST_BIN, f[:-4])
        _run(["g++", "-O2", "-std=c++17", "-I" + os.path.join(ROOT, "include"), "-I" + CPP_TESTS,
              "-I" + os.path.join(ROOT, "oracle"), os.path.join(CPP_TESTS, f), "-o", exe,
              "-L" + LIBDIR, "-lforge_amd", "-lpocketforge_amd", "-L" + ORACLE_BUILD, "-loracle",
              "-Wl,-rpath,$ORIGIN/..", "-Wl,-rpath,$ORIGIN/../../../oracle/_build"])
        out.append(exe)
    return out


def build(jobs=4, verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, UNITS))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-o", tmp] + objs + ["-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    build_forge()
    if os.path.exists(os.path.join(ORACLE_BUILD, "liboracle.so")):
        build_cpp_tests()
    if verbose:
        print("built", LIB, FORGE_LIB)
    return LIB


if __name__ == "__main__":
    jobs = 4
    if "--jobs" in sys.argv:
        jobs = int(sys.argv[sys.argv.index("--jobs") + 1])
    build(jobs=jobs, verbose=True)
