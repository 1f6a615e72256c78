"""pope_flash_decode_noalloc (the decode entry point that allocates nothing) through the C ABI.

It runs the decode kernels on the library's own scratch array instead of a caller workspace.
Two calls in a row -- the second smaller, so stale partials of the first sit in the array --
must match pope_flash_decode (the same kernels on a torch-allocated workspace) bit for bit,
and the CPU oracle within the bf16 tolerance, 2e-2 absolute.
"""
import ctypes

import pytest
import torch

from gpu_common import make_pope_inputs, max_abs, oracle_attention

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _call(inp, noalloc):
    from pope_amd import _lib
    from pope_amd.hip_pope_flash_attn import _desc
    q, k, v, freqs, bias, mask = (inp[n] for n in ("q", "k", "v", "freqs", "bias", "mask"))
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
    d = _desc(q, k, freqs, bias, False, q.shape[-1] ** -0.5)
    d.q_s[:], d.k_s[:], d.v_s[:], d.o_s[:] = (_lib.strides3(t) for t in (q, k, v, o))
    d.mask_sb = mask.stride(0)
    L = _lib.lib()
    args = (ctypes.byref(d), q.data_ptr(), k.data_ptr(), v.data_ptr(), freqs.data_ptr(), bias.data_ptr(),
            mask.data_ptr(), o.data_ptr(), lse.data_ptr())
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        st = L.pope_flash_decode_noalloc(*args, stream)
    else:
        n = _lib.workspace_bytes(_lib.OP_FLASH_DECODE, d)
        ws = torch.empty(n, dtype=torch.uint8, device=q.device)
        st = L.pope_flash_decode(*args, ws.data_ptr(), n, stream)
    _lib.check(st, "decode" + (" (no allocation)" if noalloc else ""))
    torch.cuda.synchronize()
    return o, lse


def _inputs(seed, B, H, Nk):
    inp = make_pope_inputs(seed, B, H, H, 1, Nk, 64, 64, torch.bfloat16, "none")
    g = torch.Generator().manual_seed(seed + 1)
    lengths = torch.randint(Nk // 8, Nk + 1, (B,), generator=g)
    inp["mask"] = (torch.arange(Nk)[None, :] < lengths[:, None]).to("cuda")
    return inp


def test_noalloc_decode_matches_workspace_decode(cuda):
    for seed, B, H, Nk in ((31, 4, 16, 16384), (32, 2, 8, 4096)):   # the second call is smaller
        print(f"case seed={seed} B={B} H={H} Nk={Nk}", flush=True)
        inp = _inputs(seed, B, H, Nk)
        o_na, lse_na = _call(inp, noalloc=True)
        o_ws, lse_ws = _call(inp, noalloc=False)
        assert torch.equal(o_na, o_ws) and torch.equal(lse_na, lse_ws)
        ref = oracle_attention(inp, causal=False, grads=False)
        assert max_abs(o_na, ref["o"]) <= TOL
        assert (lse_na.cpu() - ref["lse"]).abs().max().item() <= TOL
