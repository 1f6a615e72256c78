"""Host AddressSanitizer build of libpope_hip.so for the C ABI tests (CPU only).

    python pope-pytorch_amd/build_asan.py OUT.so

The host-side sources (the ABI shim and the profiler) are compiled with clang++ and
``-fsanitize=address``; the kernel objects are the regular gfx950 build's (``build.py``
must have run: they are taken from ``_build/``), linked unchanged.  Only host code is
instrumented.  Load the result with the clang ASan runtime preloaded (``asan_runtime()``)
and ``ASAN_OPTIONS=detect_leaks=0`` (the Python interpreter is not instrumented).
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
CLANGXX = os.path.join(ROCM, "llvm", "bin", "clang++")
HOST_SOURCES = ("pope_abi.cpp", "profile.cpp")
SAN_FLAGS = ["-fsanitize=address", "-fno-omit-frame-pointer", "-shared-libsan"]


def asan_runtime() -> str | None:
    """Path of the clang ASan runtime matching CLANGXX, or None."""
    hits = sorted(glob.glob(os.path.join(ROCM, "llvm", "lib", "clang", "*", "lib", "linux",
                                         "libclang_rt.asan-x86_64.so")))
    return hits[-1] if hits else None


def device_objects() -> list[str]:
    return sorted(glob.glob(os.path.join(OBJ_DIR, "*.hip.o")))


def build(out: str) -> str:
    if not os.path.exists(CLANGXX):
        raise RuntimeError(f"{CLANGXX} not found")
    objs = device_objects()
    if not objs:
        raise RuntimeError(f"no kernel objects under {OBJ_DIR}: run build.py first")
    work = os.path.dirname(os.path.abspath(out))
    host_objs = []
    for src in HOST_SOURCES:
        obj = os.path.join(work, src + ".asan.o")
        cmd = [CLANGXX, "-x", "c++", "-std=c++17", "-O1", "-g", "-fPIC", *SAN_FLAGS, "-D__HIP_PLATFORM_AMD__",
               "-I", os.path.join(ROCM, "include"), "-I", CSRC, "-c", os.path.join(CSRC, src), "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"compile failed: {src}\n{r.stderr}")
        host_objs.append(obj)
    cmd = [CLANGXX, "-shared", *SAN_FLAGS, "-o", out, *host_objs, *objs, "-L", os.path.join(ROCM, "lib"),
           "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed\n" + r.stderr)
    return out


if __name__ == "__main__":
    print(build(sys.argv[1] if len(sys.argv) > 1 else os.path.join(OBJ_DIR, "libpope_hip_asan.so")))
