"""ctypes binding of libpope_hip.so (the C ABI declared in include/pope_abi.h).

The library is built in-tree (``python pope-pytorch_amd/build.py``) and loaded
from this package directory.  There is no fallback: a missing or unloadable
library raises ``RuntimeError`` on first use, so GPU calls never silently run
anything but the HIP kernels.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpope_hip.so")
ABI_VERSION = 3
FLAG_PREPARED, FLAG_ZERO_GRADS, FLAG_SPLIT_BF16, FLAG_COMPLEX, FLAG_DETERMINISTIC = 1, 2, 4, 8, 16

POPE_F32, POPE_F16, POPE_BF16 = 0, 1, 2
OP_SIM_FWD, OP_SIM_BWD, OP_FLASH_FWD, OP_FLASH_BWD, OP_FLASH_DECODE, OP_POLAR_BWD = range(6)

_DTYPE_CODE = {torch.float32: POPE_F32, torch.float16: POPE_F16, torch.bfloat16: POPE_BF16}

_I64x3 = ctypes.c_int64 * 3


class PopeDesc(ctypes.Structure):
    """Mirror of ``struct pope_desc`` (include/pope_abi.h)."""

    _fields_ = [
        ("B", ctypes.c_int32), ("Hq", ctypes.c_int32), ("Hk", ctypes.c_int32),
        ("Nq", ctypes.c_int32), ("Nk", ctypes.c_int32), ("D", ctypes.c_int32), ("R", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("causal", ctypes.c_int32), ("softmax_scale", ctypes.c_float),
        ("flags", ctypes.c_int32), ("q_s", _I64x3), ("k_s", _I64x3), ("v_s", _I64x3), ("o_s", _I64x3),
        ("do_s", _I64x3), ("dq_s", _I64x3), ("dk_s", _I64x3), ("dv_s", _I64x3),
        ("sim_s", _I64x3), ("f_s", _I64x3), ("df_s", _I64x3),
        ("bias_sh", ctypes.c_int64), ("mask_sb", ctypes.c_int64),
    ]


EXPORTS = (
    "pope_abi_version", "pope_last_error", "pope_workspace_bytes", "pope_sim_fwd", "pope_sim_bwd",
    "pope_flash_fwd", "pope_flash_bwd", "pope_flash_decode", "pope_flash_decode_noalloc", "pope_polar_fwd",
    "pope_polar_bwd", "pope_profile_enable", "pope_profile_read", "pope_profile_reset",
)

_lib = None
_lock = threading.Lock()


def _declare(lib):
    vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    dp = ctypes.POINTER(PopeDesc)
    lib.pope_abi_version.restype = i32
    lib.pope_abi_version.argtypes = []
    lib.pope_last_error.restype = i32
    lib.pope_last_error.argtypes = [ctypes.c_char_p, sz]
    lib.pope_workspace_bytes.restype = i32
    lib.pope_workspace_bytes.argtypes = [i32, dp, ctypes.POINTER(sz)]
    lib.pope_sim_fwd.restype = i32
    lib.pope_sim_fwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.pope_sim_bwd.restype = i32
    lib.pope_sim_bwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.pope_flash_fwd.restype = i32
    lib.pope_flash_fwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.pope_flash_bwd.restype = i32
    lib.pope_flash_bwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.pope_flash_decode.restype = i32
    lib.pope_flash_decode.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.pope_flash_decode_noalloc.restype = i32
    lib.pope_flash_decode_noalloc.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.pope_polar_fwd.restype = i32
    lib.pope_polar_fwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp]
    lib.pope_polar_bwd.restype = i32
    lib.pope_polar_bwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.pope_profile_enable.restype = i32
    lib.pope_profile_enable.argtypes = [i32]
    lib.pope_profile_read.restype = i32
    lib.pope_profile_read.argtypes = [ctypes.c_char_p, sz]
    lib.pope_profile_reset.restype = i32
    lib.pope_profile_reset.argtypes = []


def lib():
    """The loaded library; raises RuntimeError when it is missing or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"pope_amd: HIP library not found at {LIB_PATH}; "
                    "build it with `python pope-pytorch_amd/build.py`")
            try:
                handle = ctypes.CDLL(LIB_PATH)
            except OSError as e:
                raise RuntimeError(f"pope_amd: cannot load {LIB_PATH}: {e}") from e
            _declare(handle)
            v = handle.pope_abi_version()
            if v != ABI_VERSION:
                raise RuntimeError(f"pope_amd: library ABI {v} != expected {ABI_VERSION}")
            _lib = handle
    return _lib


def last_error() -> str:
    buf = ctypes.create_string_buffer(512)
    lib().pope_last_error(buf, 512)
    return buf.value.decode(errors="replace")


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"pope_amd {what} failed (status {status}): {last_error()}")


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_ptr(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def strides3(t) -> tuple:
    """(b, h, n) element strides of a (B, H, N, D) tensor view with unit feature stride."""
    s = t.stride()
    return (s[0], s[1], s[2])


def workspace_bytes(op: int, desc: PopeDesc) -> int:
    n = ctypes.c_size_t(0)
    check(lib().pope_workspace_bytes(op, ctypes.byref(desc), ctypes.byref(n)), "workspace query")
    return int(n.value)


def workspace(op: int, desc: PopeDesc, device) -> torch.Tensor | None:
    n = workspace_bytes(op, desc)
    if n == 0:
        return None
    # torch's caching allocator returns 512-byte aligned blocks
    return torch.empty(n, dtype=torch.uint8, device=device)


def profile_enable(on: bool = True) -> None:
    """Time every kernel launch of the library with an event pair its dispatch stamps."""
    check(lib().pope_profile_enable(1 if on else 0), "profile enable")


def profile_reset() -> None:
    check(lib().pope_profile_reset(), "profile reset")


def profile_read() -> dict:
    """Per-kernel totals since the last reset: {name: (count, total_ms, min_ms, max_ms)}.
    Waits for the recorded events."""
    buf = ctypes.create_string_buffer(1 << 16)
    check(lib().pope_profile_read(buf, len(buf)), "profile read")
    out = {}
    for line in buf.value.decode().splitlines():
        name, cnt, tot, mn, mx = line.split()
        out[name] = (int(cnt), float(tot), float(mn), float(mx))
    return out


def deterministic_flag() -> int:
    """FLAG_DETERMINISTIC when torch.use_deterministic_algorithms(True) is in effect."""
    return FLAG_DETERMINISTIC if torch.are_deterministic_algorithms_enabled() else 0


def dtype_code(dtype: torch.dtype) -> int:
    if dtype not in _DTYPE_CODE:
        raise TypeError(f"pope_amd: unsupported dtype {dtype}")
    return _DTYPE_CODE[dtype]
