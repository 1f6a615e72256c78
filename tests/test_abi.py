"""The C ABI library on the CPU: it loads, exports every symbol include/pope_abi.h
declares, reports workspace sizes, and rejects bad arguments on the host before
any HIP call (so none of these tests needs or touches a GPU)."""
import ctypes
import os
import re

import pytest

from pope_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "pope_abi.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^int\s+(pope_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_exports():
    assert _declared() == sorted(_lib.EXPORTS)


def test_library_loads_and_exports_every_symbol():
    L = _lib.lib()
    for name in _declared():
        assert hasattr(L, name), name
    assert L.pope_abi_version() == _lib.ABI_VERSION


def _desc(B=2, Hq=8, Hk=8, Nq=256, Nk=256, D=64, R=32, dtype=_lib.POPE_BF16):
    d = _lib.PopeDesc()
    d.B, d.Hq, d.Hk, d.Nq, d.Nk, d.D, d.R, d.dtype = B, Hq, Hk, Nq, Nk, D, R, dtype
    d.softmax_scale = D ** -0.5
    for f in ("q_s", "k_s", "v_s", "o_s", "do_s", "dq_s", "dk_s", "dv_s"):
        getattr(d, f)[:] = (Hq * Nq * D, Nq * D, D)
    d.sim_s[:] = (Hq * Nq * Nk, Nq * Nk, Nk)
    d.f_s[:] = (0, 0, R)
    d.bias_sh = R
    return d


def _ws(op, d):
    n = ctypes.c_size_t(0)
    st = _lib.lib().pope_workspace_bytes(op, ctypes.byref(d), ctypes.byref(n))
    return st, n.value


def test_workspace_sizes():
    al = lambda n: (n + 255) // 256 * 256
    d = _desc()
    # cos/sin(F) (Nk, R) float2 | cos/sin(bias) (Hk, R) float2 | K_hat, Q_hat (E = 96 columns)
    # | visibility words (B, Nk/64) u64 | kend (B) int32 | (lse, delta) (B, Hq, Nq) float2
    want = (al(256 * 32 * 8) + al(8 * 32 * 8) + 2 * al(2 * 8 * 256 * 96 * 2) + al(2 * 4 * 8) + al(2 * 4)
            + al(2 * 8 * 256 * 8))
    assert _ws(_lib.OP_FLASH_FWD, d) == (0, want)
    assert _ws(_lib.OP_FLASH_BWD, d) == (0, want)   # one layout: the backward reuses the forward's
    # wide heads (D > 128): E rounded up to 128 (here 192 + 96 -> 384 columns); the backward adds the
    # raw expanded-row gradients, fp32 (B, Hk, NkP, EP) and (B, Hq, NqP, EP)
    dw = _desc(D=192, R=96)
    want_w = (al(256 * 96 * 8) + al(8 * 96 * 8) + 2 * al(2 * 8 * 256 * 384 * 2) + al(2 * 4 * 8) + al(2 * 4)
              + al(2 * 8 * 256 * 8))
    assert _ws(_lib.OP_FLASH_FWD, dw) == (0, want_w)
    assert _ws(_lib.OP_FLASH_BWD, dw) == (0, want_w + 2 * al(2 * 8 * 256 * 384 * 4))
    d3 = _desc(R=0, Nk=200)                          # no tables; K_hat rows padded to 256, E = 64
    want3 = 2 * al(2 * 8 * 256 * 64 * 2) + al(2 * 4 * 8) + al(2 * 4) + al(2 * 8 * 256 * 8)
    assert _ws(_lib.OP_FLASH_FWD, d3) == (0, want3)
    ds = _desc(dtype=_lib.POPE_F32, R=64)
    st, n = _ws(_lib.OP_SIM_FWD, ds)
    assert st == 0 and n == 8 * 256 * 64 * 8 + 256 * 64 * 8         # key table per kv head + query table
    # split-bf16 similarity: + hi / lo planes of Q_hat and K_hat (rows padded to 128, EP = 128 columns)
    ds.flags = _lib.FLAG_SPLIT_BF16
    planes = 2 * al(2 * 8 * 256 * 128 * 2) + 2 * al(2 * 8 * 256 * 128 * 2)
    assert _ws(_lib.OP_SIM_FWD, ds) == (0, n + planes)
    # backward: U, W (fp32, EP columns) and, split, their second partial sums
    uw = al(2 * 8 * 256 * 128 * 4) + al(2 * 8 * 256 * 128 * 4)
    ds.flags = 0
    assert _ws(_lib.OP_SIM_BWD, ds) == (0, n + uw)
    ds.flags = _lib.FLAG_SPLIT_BF16
    assert _ws(_lib.OP_SIM_BWD, ds) == (0, n + uw + planes + uw)


def _fake(n=1 << 20):
    # Host memory stands in for device pointers: every call below must fail in
    # host validation, before any HIP call would dereference them.
    return ctypes.create_string_buffer(n)


_BUF = _fake()
_P = ctypes.cast(_BUF, ctypes.c_void_p)
# 256-aligned view inside the buffer
_A = ctypes.c_void_p(((_P.value + 255) // 256) * 256)


def _flash_fwd(d, **over):
    args = dict(q=_A, k=_A, v=_A, freqs=_A, bias=_A, mask=None, o=_A, lse=_A, ws=_A, wsz=1 << 16)
    args.update(over)
    return _lib.lib().pope_flash_fwd(ctypes.byref(d), args["q"], args["k"], args["v"], args["freqs"],
                                     args["bias"], args["mask"], args["o"], args["lse"], args["ws"],
                                     args["wsz"], None)


@pytest.mark.parametrize("field,value,needle", [
    ("Hq", 6, "multiple of kv heads"),
    ("D", 60, "multiple of 8"),
    ("R", 72, "rotate dim"),
    ("Nq", 512, "exceeds key length"),
    ("B", 0, ">= 1"),
])
def test_flash_rejects_bad_shapes(field, value, needle):
    d = _desc()
    setattr(d, field, value)
    st = _flash_fwd(d)
    assert st != 0
    assert needle in _lib.last_error()


def test_flash_rejects_bad_dtype_strides_pointers_workspace():
    d = _desc(dtype=_lib.POPE_F32)
    assert _flash_fwd(d) == 2 and "bf16 or fp16" in _lib.last_error()
    d = _desc(D=264, R=0)
    assert _flash_fwd(d) == 2 and "head dim <= 256" in _lib.last_error()
    d = _desc()
    d.q_s[2] = 65
    assert _flash_fwd(d) == 1 and "stride" in _lib.last_error()
    d = _desc()
    assert _flash_fwd(d, q=None) == 1 and "non-NULL" in _lib.last_error()
    assert _flash_fwd(d, freqs=None) == 1 and "needs freqs and bias" in _lib.last_error()
    assert _flash_fwd(d, k=ctypes.c_void_p(_A.value + 2)) == 1 and "aligned" in _lib.last_error()
    assert _flash_fwd(d, ws=None) == 3 and "workspace" in _lib.last_error()
    assert _flash_fwd(d, wsz=16) == 3 and "workspace" in _lib.last_error()


def test_flash_bwd_rejects_unknown_flags():
    d = _desc()
    d.flags = 4
    st = _lib.lib().pope_flash_bwd(ctypes.byref(d), _A, _A, _A, _A, _A, _A, _A, _A, None, _A, _A, _A, None, None,
                                   _A, 1 << 16, None)
    assert st == 1 and "flags" in _lib.last_error()


def test_sim_and_decode_validation():
    L = _lib.lib()
    d = _desc(dtype=_lib.POPE_BF16)
    st = L.pope_sim_fwd(ctypes.byref(d), _A, _A, _A, _A, _A, _A, 1 << 16, None)
    assert st == 2 and "fp32" in _lib.last_error()
    d = _desc(Nq=64, dtype=_lib.POPE_BF16)
    st = L.pope_flash_decode(ctypes.byref(d), _A, _A, _A, _A, _A, None, _A, _A, _A, 1 << 16, None)
    assert st == 2 and "one non-causal query row" in _lib.last_error()
    d = _desc(dtype=_lib.POPE_F32, D=64, R=64)
    d.flags = 1   # the flash backward's PREPARED: not a similarity flag
    st = L.pope_sim_fwd(ctypes.byref(d), _A, _A, _A, _A, _A, _A, 1 << 16, None)
    assert st == 1 and "flags" in _lib.last_error()
    d = _desc(dtype=_lib.POPE_F32, D=64, R=64)
    d.bias_sh = -1
    st = L.pope_sim_bwd(ctypes.byref(d), _A, _A, _A, _A, _A, _A, _A, None, None, _A, 1 << 16, None)
    assert st == 1 and "negative" in _lib.last_error()
    # ZERO_GRADS is a backward flag: the similarity backward takes it (the check moves on to the
    # bias stride), the forward refuses it
    d.flags = _lib.FLAG_ZERO_GRADS
    st = L.pope_sim_bwd(ctypes.byref(d), _A, _A, _A, _A, _A, _A, _A, None, None, _A, 1 << 16, None)
    assert st == 1 and "negative" in _lib.last_error()
    d = _desc(dtype=_lib.POPE_F32, D=64, R=64)
    d.flags = _lib.FLAG_ZERO_GRADS
    st = L.pope_sim_fwd(ctypes.byref(d), _A, _A, _A, _A, _A, _A, 1 << 16, None)
    assert st == 1 and "flags" in _lib.last_error()


def test_last_error_is_per_thread():
    import threading
    d = _desc()
    d.D = 60
    _flash_fwd(d)
    seen = {}

    def other():
        seen["msg"] = _lib.last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert "multiple of 8" in _lib.last_error()
    assert seen["msg"] == ""


def test_flash_wrappers_check_shapes_before_any_call():
    """Shapes the kernels index by but the descriptor does not carry (v, mask, lse, o, do) are
    checked on the host when a call plan is built; CPU tensors never reach the library."""
    import torch
    from pope_amd.hip_pope_flash_attn import _bwd_impl, _fwd_impl
    B, H, N, D, R = 1, 2, 64, 32, 16
    q = torch.zeros(B, H, N, D, dtype=torch.bfloat16)
    k, v = torch.zeros_like(q), torch.zeros_like(q)
    f, b = torch.zeros(N, R), torch.zeros(1, R)
    with pytest.raises(ValueError, match="v "):
        _fwd_impl(q, k, v[:, :, :N - 1], f, b, None, False, 0.1)
    with pytest.raises(ValueError, match="mask"):
        _fwd_impl(q, k, v, f, b, torch.ones(B, N + 1, dtype=torch.bool), False, 0.1)
    with pytest.raises(ValueError, match="positions"):
        _fwd_impl(q, k, v, f[: N - 1], b, None, False, 0.1)
    lse = torch.zeros(B, H, N)
    with pytest.raises(ValueError, match="lse"):
        _bwd_impl(q, q, k, v, q, lse[:, :, 1:], f, b, None, True, 0.1, False, False)
    with pytest.raises(ValueError, match="must match q"):
        _bwd_impl(q[:, :, 1:], q, k, v, q, lse, f, b, None, True, 0.1, False, False)


def test_noalloc_decode_rejects_sizes_beyond_its_scratch():
    """The allocation-free decode holds its split partials in a 16 MiB array of the library: a call
    whose partials need more fails on the host, before any HIP call, with a clear error."""
    d = _desc(B=64, Hq=64, Hk=64, Nq=1, Nk=32768, D=64, R=64)
    st = _lib.lib().pope_flash_decode_noalloc(ctypes.byref(d), _A, _A, _A, _A, _A, None, _A, _A, None)
    assert st == 3 and "scratch array" in _lib.last_error()


def test_deterministic_mode_workspace():
    """POPE_FLAG_DETERMINISTIC adds the per-row phase-derivative region to the backwards' workspaces:
    dpsi (B, Hk, Nk, R) | dphi (B, Hq, Nq, R) | 64 dbias slices per (bias row, dim), fp32."""
    al = lambda n: (n + 255) // 256 * 256
    d = _desc()
    base = _ws(_lib.OP_FLASH_BWD, d)[1]
    assert _ws(_lib.OP_POLAR_BWD, d) == (0, 0)
    d.flags = _lib.FLAG_DETERMINISTIC
    det = al(2 * 8 * 256 * 32 * 4) + al(2 * 8 * 256 * 32 * 4) + al(8 * 32 * 64 * 4)
    assert _ws(_lib.OP_FLASH_BWD, d) == (0, base + det)
    assert _ws(_lib.OP_FLASH_FWD, d)[1] == base           # the forward's layout is unchanged
    assert _ws(_lib.OP_POLAR_BWD, d) == (0, det)
    ds = _desc(dtype=_lib.POPE_F32, R=64)
    plain = _ws(_lib.OP_SIM_BWD, ds)[1]
    ds.flags = _lib.FLAG_DETERMINISTIC
    assert _ws(_lib.OP_SIM_BWD, ds)[1] == plain + al(2 * 8 * 256 * 64 * 4) * 2 + al(8 * 64 * 64 * 4)
