"""The C-ABI layer's host code under AddressSanitizer, without a GPU.

`make -C causal-conv1d-triton_amd asan` builds _build/libccv1d_asan.so: ccv1d_api.hip's host code
(argument checks, tiling and workspace planning, error reporting) instrumented with ASan, linked
with the shipped kernel objects. This test runs the library-level CPU tests of test_abi.py against
it in a child Python process that preloads clang's ASan runtime; an invalid host memory access on
any of those paths aborts the child with an ASan report, which fails the test. The CPython binding
tests of test_abi.py are left out: that extension links the shipped library, not this one.
"""

import os
import subprocess
import sys

import pytest

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_PKG = os.path.join(_ROOT, "causal-conv1d-triton_amd")
_LIB = os.path.join(_PKG, "_build", "libccv1d_asan.so")
_CLANG = "/opt/rocm/llvm/bin/clang"


def _asan_runtime():
    if not os.path.exists(_CLANG):
        return None
    path = subprocess.run([_CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"],
                          capture_output=True, text=True).stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


def test_abi_checks_under_asan():
    runtime = _asan_runtime()
    if runtime is None:
        pytest.skip("clang's shared ASan runtime is not installed")
    if not os.path.exists(_LIB):
        pytest.skip("host ASan build missing: run `make -C causal-conv1d-triton_amd asan`")
    code = (
        "import sys\n"
        f"sys.path[:0] = [{_PKG!r}, {os.path.join(_ROOT, 'tests')!r}]\n"
        "import causal_conv1d_triton._ffi as F\n"
        f"F._LIB_PATH = {_LIB!r}\n"
        "import pytest\n"
        f"sys.exit(pytest.main([{os.path.join(_ROOT, 'tests', 'test_abi.py')!r}, '-q', '-m',"
        " 'not gpu', '-k', 'not native', '-p', 'no:cacheprovider']))\n"
    )
    env = dict(os.environ, LD_PRELOAD=runtime,
               # Leaks of the uninstrumented runtime libraries (HIP, Python) are not this layer's.
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1")
    r = subprocess.run([sys.executable, "-c", code], cwd=_ROOT, env=env, capture_output=True,
                       text=True, timeout=600)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    assert " passed" in out and " failed" not in out, out[-2000:]
