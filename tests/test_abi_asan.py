"""The C ABI tests (test_abi.py) against a host AddressSanitizer build of the library.

pope-pytorch_amd/build_asan.py compiles the ABI shim and the profiler with
-fsanitize=address and links them with the regular kernel objects; test_abi.py then
runs in a child process with the clang ASan runtime preloaded, so every host-side
validation path, workspace computation and error-text write it exercises is checked for
out-of-bounds and use-after-free accesses.  CPU only: no test here calls a kernel.
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_abi_tests_pass_under_address_sanitizer(tmp_path):
    sys.path.insert(0, os.path.join(ROOT, "pope-pytorch_amd"))
    import build_asan
    rt = build_asan.asan_runtime()
    if rt is None or not os.path.exists(build_asan.CLANGXX):
        pytest.skip("clang ASan runtime not available")
    if not build_asan.device_objects():
        pytest.skip("kernel objects not built (run pope-pytorch_amd/build.py)")
    lib = build_asan.build(str(tmp_path / "libpope_hip_asan.so"))
    env = dict(os.environ, LD_PRELOAD=rt, POPE_AMD_TEST_LIB=lib,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
                        os.path.join(ROOT, "tests", "test_abi.py")],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    assert " passed" in out
