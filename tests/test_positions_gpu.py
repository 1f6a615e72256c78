"""Per-sample positions and position offsets through the fused kernels vs the oracle.

The phase table can be 2-D (N, R) -- shared by every batch and head --, 3-D (B, N, R) from a
(B, N) positions tensor (``PoPE(pos)``, pope.py:131-141, and ``b n d -> b 1 n d`` in
apply_pope_to_qk, pope.py:53-54), offset by ``pope(n, offset)`` (pope.py:135-137), or 4-D
(B, N, H, R) in the reference's (batch, seq, heads) operator layout
(triton_pope_flash_attn.py:237-245; one table per head, so query and kv heads coincide there).
Each layout runs through the flash attention (forward and backward, dfreqs included), the
decode kernel and the similarity, against the oracle on the same inputs.
Tolerances: 2e-2 absolute (beyond the bf16 rounding of the exact value) for bf16 flash and decode
outputs and per-element gradients,
2e-2 * max(1, ||ref||_inf) for the summed dbias / dfreqs; 1e-4 relative for the fp32 similarity.
"""
import math

import pytest
import torch

from gpu_common import excess_over, make_pope_inputs, max_abs, oracle_attention
from oracle import pope_oracle as orc

pytestmark = pytest.mark.gpu

TOL = 2e-2
SUMMED = ("dbias", "dfreqs")


def _check(got, ref, names):
    """Per-element bf16 outputs: 2e-2 beyond the bf16 rounding of the exact value (half a bf16 ulp
    alone is 1.6e-2 at |x| >= 4; gpu_common.excess_over).  Summed gradients: 2e-2 * max(1, ||ref||)."""
    for n in names:
        e = max_abs(got[n], ref[n])
        if n in SUMMED:
            ex = e - TOL * max(1.0, ref[n].abs().max().item())
        else:
            ex = excess_over(got[n], ref[n], TOL)
        print(f"{n}={e:.2e}", end=" ")
        assert ex <= 0, f"{n}: {e:.3e}, {ex:.3e} over the bound"
    print()


def _batch_positions(B, N, seed):
    """(B, N) positions: per-batch starts and uneven gaps (not an arange)."""
    g = torch.Generator().manual_seed(seed)
    steps = torch.randint(1, 4, (B, N), generator=g).float()
    return steps.cumsum(-1) + 100.0 * torch.arange(B).float()[:, None]


def _flash(inp, causal, layout="head_first"):
    import pope_amd
    from pope_amd.hip_pope_flash_attn import flash_attn
    t = [inp[n].detach().clone().requires_grad_(True) for n in ("q", "k", "v", "freqs", "bias")]
    if layout == "head_first":
        o = pope_amd.flash_attn_with_pope(t[0], t[1], t[2], pos_emb=(t[3], t[4]), mask=inp["mask"], causal=causal)
        o.backward(inp["do"])
        return dict(o=o, dq=t[0].grad, dk=t[1].grad, dv=t[2].grad, dfreqs=t[3].grad, dbias=t[4].grad)
    # the reference's operator layout: (B, N, H, D) tensors and (B, N, H, R) freqs
    tr = lambda x: x.detach().transpose(1, 2).contiguous().requires_grad_(True)
    qb, kb, vb, fb = tr(inp["q"]), tr(inp["k"]), tr(inp["v"]), tr(inp["freqs"])
    bias = inp["bias"].detach().clone().requires_grad_(True)
    o = flash_attn(qb, kb, vb, fb, bias, inp["mask"], causal)
    o.backward(inp["do"].transpose(1, 2))
    back = lambda x: x.transpose(1, 2)
    return dict(o=back(o), dq=back(qb.grad), dk=back(kb.grad), dv=back(vb.grad), dfreqs=back(fb.grad), dbias=bias.grad)


@pytest.mark.parametrize("causal", [True, False])
def test_flash_per_batch_positions(cuda, causal):
    B, H, N, D, R = 2, 4, 320, 64, 32
    inp = make_pope_inputs(61, B, H, H, N, N, D, R, torch.bfloat16, "prefix")
    inp["freqs"] = orc.pope_freqs(_batch_positions(B, N, 62), orc.inv_freqs(R)).cuda()   # (B, N, R)
    assert inp["freqs"].shape == (B, N, R)
    _check(_flash(inp, causal), oracle_attention(inp, causal), ["o", "dq", "dk", "dv", "dfreqs", "dbias"])


def test_flash_position_offset_matches_shifted_positions(cuda):
    """pope(n, offset): the rows of a longer table starting at `offset` (pope.py:135-137); with 2-D
    freqs the attention depends on position differences only, so the output matches offset 0."""
    import pope_amd
    B, H, N, D, R = 1, 4, 256, 64, 32
    inp = make_pope_inputs(63, B, H, H, N, N, D, R, torch.bfloat16, "none")
    pope = pope_amd.PoPE(R, heads=H).cuda()
    with torch.no_grad():
        pope.bias.copy_(inp["bias"])
    f_off, bias = pope(N, offset=1000)
    torch.testing.assert_close(f_off.cpu(), orc.pope_freqs(N, orc.inv_freqs(R), offset=1000), rtol=0, atol=0)
    inp_off = dict(inp, freqs=f_off.detach(), bias=bias.detach())
    got = _flash(inp_off, True)
    _check(got, oracle_attention(inp_off, True), ["o", "dq", "dk", "dv", "dfreqs", "dbias"])
    base = _flash(dict(inp, freqs=pope(N)[0].detach(), bias=bias.detach()), True)
    assert max_abs(got["o"], base["o"]) <= TOL


def test_flash_attn_per_head_tables_in_reference_layout(cuda):
    B, H, N, D, R = 2, 4, 192, 64, 32
    inp = make_pope_inputs(64, B, H, H, N, N, D, R, torch.bfloat16, "prefix")
    pos = _batch_positions(B * H, N, 65).view(B, H, N)
    inp["freqs"] = orc.pope_freqs(pos, orc.inv_freqs(R)).cuda()            # (B, H, N, R) head-first
    _check(_flash(inp, True, layout="bnhd"), oracle_attention(inp, True), ["o", "dq", "dk", "dv", "dfreqs", "dbias"])


def test_decode_per_batch_positions(cuda):
    import pope_amd
    from pope_amd import _lib
    B, H, N, D, R = 3, 4, 2048, 64, 64
    inp = make_pope_inputs(66, B, H, H, 1, N, D, R, torch.bfloat16, "prefix")
    inp["freqs"] = orc.pope_freqs(_batch_positions(B, N, 67), orc.inv_freqs(R)).cuda()
    _lib.profile_reset()
    _lib.profile_enable(True)
    o = pope_amd.flash_attn_with_pope(inp["q"], inp["k"], inp["v"], pos_emb=(inp["freqs"], inp["bias"]),
                                      mask=inp["mask"])
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    assert "flash_decode_split" in _lib.profile_read()
    _check(dict(o=o), oracle_attention(inp, False, grads=False), ["o"])


@pytest.mark.parametrize("allow_tf32", [True, False], ids=["split_bf16", "fp32"])
def test_similarity_per_batch_positions_and_offset(cuda, allow_tf32):
    import pope_amd
    g = torch.Generator().manual_seed(68)
    B, H, Nq, Nk, D, R = 2, 4, 100, 160, 64, 32
    q = torch.randn(B, H, Nq, D, generator=g)
    k = torch.randn(B, H, Nk, D, generator=g)
    bias = torch.rand(H, R, generator=g) * (-2 * math.pi)
    G = torch.randn(B, H, Nq, Nk, generator=g)
    for freqs in (orc.pope_freqs(_batch_positions(B, Nk, 69), orc.inv_freqs(R)),
                  orc.pope_freqs(Nk, orc.inv_freqs(R), offset=3000)):
        t = [x.clone().cuda().requires_grad_(True) for x in (q, k, freqs, bias)]
        S = pope_amd.compute_attn_similarity(t[0], t[1], (t[2], t[3]), allow_tf32=allow_tf32)
        S.backward(G.cuda())
        r = [x.clone().requires_grad_(True) for x in (q, k, freqs, bias)]
        S_ref = orc.sim_nonfused(*r)
        (S_ref * G).sum().backward()
        for a, b in zip([S] + [x.grad for x in t], [S_ref] + [x.grad for x in r]):
            rel = ((a.detach().double().cpu() - b.detach().double()).abs().max() / b.abs().max()).item()
            assert rel <= 1e-4, rel
