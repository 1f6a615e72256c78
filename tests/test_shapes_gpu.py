"""Head dims and rotate dims that are not multiples of 8, and heads wider than the flash kernels,
through the public API on the GPU vs the oracle.

The reference's kernels take any D and R (Triton blocks of next_pow2(D) with a rotate mask,
triton_pope.py:58-60, triton_pope_flash_attn.py:44,252).  Here the Python entry points pad such
shapes on the device before the kernels run (pope_amd._pad; the padding itself is pinned on the
CPU by test_pad_cpu.py).  Heads of 136 to 256 run the wide flash kernels (flash_wide.hip), through
flash_attn_with_pope and the reference-named operators alike; heads wider than 256 take
flash_attn_with_pope's materialising path (polar transform kernel, fp32 attention products).  Each case runs forward and
backward (dfreqs / dbias included) against the float64 oracle on the same rounded inputs.
Tolerances: 2e-2 absolute beyond the bf16 rounding of the exact value for bf16 outputs and
per-element gradients, 2e-2 * max(1, ||ref||_inf) for the summed dbias / dfreqs; 1e-4 relative
(normwise) for the fp32 similarity.
"""
import pytest
import torch

from gpu_common import excess_over, make_pope_inputs, max_abs, oracle_attention
from oracle import pope_oracle as orc

pytestmark = pytest.mark.gpu

TOL = 2e-2
SUMMED = ("dbias", "dfreqs")
ALL = ("o", "dq", "dk", "dv", "dfreqs", "dbias")


def _check(got, ref, names):
    for n in names:
        if ref.get(n) is None or not ref[n].numel():
            continue
        e = max_abs(got[n], ref[n])
        ex = e - TOL * max(1.0, ref[n].abs().max().item()) if n in SUMMED else excess_over(got[n], ref[n], TOL)
        print(f"{n}={e:.2e}", end=" ")
        assert ex <= 0, f"{n}: {e:.3e}, {ex:.3e} over the bound"
    print()


def _api(inp, causal):
    import pope_amd
    t = [inp[n].detach().clone().requires_grad_(True) for n in ("q", "k", "v", "freqs", "bias")]
    R = t[3].shape[-1]
    o = pope_amd.flash_attn_with_pope(t[0], t[1], t[2], pos_emb=(t[3], t[4]) if R else None, mask=inp["mask"],
                                      causal=causal)
    o.backward(inp["do"])
    return dict(o=o, dq=t[0].grad, dk=t[1].grad, dv=t[2].grad, dfreqs=t[3].grad, dbias=t[4].grad)


FLASH_CASES = [   # (B, Hq, Hk, Nq, Nk, D, R, causal, mask)
    (1, 2, 1, 100, 100, 20, 3, True, "none"),
    (2, 4, 2, 64, 130, 44, 12, False, "prefix"),
    (1, 2, 2, 77, 77, 12, 0, True, "none"),
    (1, 2, 2, 128, 128, 40, 36, False, "random"),
    (1, 2, 1, 96, 96, 100, 28, True, "none"),
]


@pytest.mark.parametrize("cfg", FLASH_CASES, ids=lambda c: "x".join(map(str, c)))
def test_flash_dims_not_multiple_of_8(cuda, cfg):
    *shape, causal, mask = cfg
    inp = make_pope_inputs(71, *shape, torch.bfloat16, mask)
    _check(_api(inp, causal), oracle_attention(inp, causal), ALL)


def test_decode_dims_not_multiple_of_8(cuda):
    """One query row against a long cache: the split-K decode kernel runs on the padded rows."""
    from pope_amd import _lib
    inp = make_pope_inputs(72, 2, 4, 2, 1, 1500, 44, 12, torch.bfloat16, "prefix")
    _lib.profile_reset()
    _lib.profile_enable(True)
    got = _api(inp, False)
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    assert "flash_decode_split" in _lib.profile_read()
    _check(got, oracle_attention(inp, False), ALL)


def test_reference_operator_api_dims_not_multiple_of_8(cuda):
    """flash_attn_forward / flash_attn_backward in the (B, N, H, D) layout, gradients into the
    caller's buffers (triton_pope_flash_attn.py:222-335)."""
    from pope_amd.hip_pope_flash_attn import flash_attn_backward, flash_attn_forward
    inp = make_pope_inputs(73, 2, 4, 2, 90, 90, 20, 3, torch.bfloat16, "prefix")
    ref = oracle_attention(inp, True)
    tr = lambda x: x.detach().transpose(1, 2).contiguous()
    q, k, v, do = tr(inp["q"]), tr(inp["k"]), tr(inp["v"]), tr(inp["do"])
    freqs, bias = inp["freqs"], inp["bias"]
    o, lse = flash_attn_forward(q, k, v, freqs, bias, inp["mask"], causal=True)
    assert o.shape == q.shape
    assert max_abs(lse, ref["lse"]) <= 1e-2
    dq, dk, dv = torch.zeros_like(q), torch.empty_like(k), torch.empty_like(v)
    dfreqs, dbias = torch.zeros_like(freqs), torch.zeros_like(bias)
    flash_attn_backward(do, q, k, v, o, lse, dq, dk, dv, dfreqs, dbias, freqs, bias, inp["mask"], causal=True)
    back = lambda x: x.transpose(1, 2)
    _check(dict(o=back(o), dq=back(dq), dk=back(dk), dv=back(dv), dfreqs=dfreqs, dbias=dbias), ref, ALL)


WIDE_CASES = [   # (B, Hq, Hk, Nq, Nk, D, R, causal, mask, dtype)
    (1, 2, 1, 96, 96, 160, 32, True, "prefix", torch.bfloat16),
    (1, 2, 2, 64, 64, 256, 64, False, "none", torch.bfloat16),
    (2, 8, 1, 59, 60, 129, 88, True, "none", torch.bfloat16),   # 8 query heads per kv head
    (2, 4, 2, 150, 300, 192, 192, False, "random", torch.bfloat16),   # E = 384, Nq < Nk
    (1, 2, 2, 200, 200, 256, 256, True, "prefix", torch.float16),     # E = 512, full rotation
    (2, 3, 3, 70, 70, 160, 0, False, "dead_row", torch.bfloat16),     # no rotation, a dead batch row
]


def _ran(names):
    from pope_amd import _lib
    ran = _lib.profile_read()
    return {n for n in names if n in ran}


@pytest.mark.parametrize("cfg", WIDE_CASES, ids=lambda c: "x".join(map(str, c[:9])) + "-" + str(c[9])[6:])
def test_flash_wide_heads(cuda, cfg):
    """Heads of 136 to 256: the wide flash kernels run (no materialised scores) and match the
    oracle, forward and backward."""
    from pope_amd import _lib
    *shape, causal, mask, dtype = cfg
    inp = make_pope_inputs(74, *shape, dtype, mask)
    _lib.profile_reset()
    _lib.profile_enable(True)
    got = _api(inp, causal)
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    assert _ran(("flash_wide_fwd", "flash_wide_kv", "flash_wide_q", "flash_wide_chain")) == {
        "flash_wide_fwd", "flash_wide_kv", "flash_wide_q", "flash_wide_chain"}
    _check(got, oracle_attention(inp, causal), ALL)


@pytest.mark.parametrize("D,R", [(160, 160), (192, 64), (256, 128)])
def test_reference_operator_api_wide_heads(cuda, D, R):
    """flash_attn / flash_attn_forward / flash_attn_backward / FlashAttnFunction in the (B, N, H, D)
    layout at head dims 160, 192 and 256 (the reference's Triton flash takes any D,
    triton_pope_flash_attn.py:252-254)."""
    from pope_amd.hip_pope_flash_attn import FlashAttnFunction, flash_attn, flash_attn_backward, flash_attn_forward
    inp = make_pope_inputs(75, 2, 4, 2, 120, 120, D, R, torch.bfloat16, "prefix")
    ref = oracle_attention(inp, True)
    tr = lambda x: x.detach().transpose(1, 2).contiguous()
    back = lambda x: x.transpose(1, 2)
    q, k, v, do = tr(inp["q"]), tr(inp["k"]), tr(inp["v"]), tr(inp["do"])
    freqs, bias = inp["freqs"], inp["bias"]
    o, lse = flash_attn_forward(q, k, v, freqs, bias, inp["mask"], causal=True)
    assert max_abs(lse, ref["lse"]) <= 1e-2
    dq, dk, dv = torch.zeros_like(q), torch.empty_like(k), torch.empty_like(v)
    dfreqs, dbias = torch.zeros_like(freqs), torch.zeros_like(bias)
    flash_attn_backward(do, q, k, v, o, lse, dq, dk, dv, dfreqs, dbias, freqs, bias, inp["mask"], causal=True)
    _check(dict(o=back(o), dq=back(dq), dk=back(dk), dv=back(dv), dfreqs=dfreqs, dbias=dbias), ref, ALL)
    # the autograd entry points
    for fn in (flash_attn, FlashAttnFunction.apply):
        t = [x.clone().requires_grad_(True) for x in (q, k, v)]
        fb = [freqs.clone().requires_grad_(True), bias.clone().requires_grad_(True)]
        o2 = fn(t[0], t[1], t[2], fb[0], fb[1], inp["mask"], True)
        o2.backward(do)
        _check(dict(o=back(o2), dq=back(t[0].grad), dk=back(t[1].grad), dv=back(t[2].grad), dfreqs=fb[0].grad,
                    dbias=fb[1].grad), ref, ALL)


@pytest.mark.parametrize("cfg", [
    (1, 2, 1, 64, 64, 264, 32, True, "prefix"),
    (1, 2, 2, 40, 40, 300, 300, False, "none"),
], ids=lambda c: "x".join(map(str, c)))
def test_flash_heads_wider_than_kernels(cuda, cfg):
    """Heads wider than 256: flash_attn_with_pope's materialising path."""
    *shape, causal, mask = cfg
    inp = make_pope_inputs(74, *shape, torch.bfloat16, mask)
    _check(_api(inp, causal), oracle_attention(inp, causal), ALL)


@pytest.mark.parametrize("D,R", [(20, 12), (44, 3), (24, 0), (300, 37), (512, 256)])   # the C ABI takes D <= 512
@pytest.mark.parametrize("allow_tf32", [True, False], ids=["split_bf16", "fp32"])
def test_similarity_dims_not_multiple_of_8(cuda, D, R, allow_tf32):
    from pope_amd.hip_pope import hip_compute_qk_similarity
    g = torch.Generator().manual_seed(75)
    B, Hq, Hk, Nq, Nk = 2, 4, 2, 70, 90
    q = torch.randn(B, Hq, Nq, D, generator=g)
    k = torch.randn(B, Hk, Nk, D, generator=g)
    freqs = torch.randn(Nk, R, generator=g) * 3.0
    bias = torch.randn(Hk, R, generator=g)
    G = torch.randn(B, Hq, Nq, Nk, generator=g)
    t = [x.clone().cuda().requires_grad_(True) for x in (q, k, freqs, bias)]
    S = hip_compute_qk_similarity(t[0], t[1], t[2], t[3], R, allow_tf32=allow_tf32)
    S.backward(G.cuda())
    r = [x.clone().requires_grad_(True) for x in (q, k, freqs, bias)]
    S_ref = orc.sim_nonfused(*r)
    (S_ref * G).sum().backward()
    for n, a, b in zip(("S", "dq", "dk", "dfreqs", "dbias"), [S] + [x.grad for x in t], [S_ref] + [x.grad for x in r]):
        if b is None or not b.numel():
            continue
        rel = ((a.detach().double().cpu() - b.detach().double()).abs().max() / b.abs().max()).item()
        print(f"{n}={rel:.2e}", end=" ")
        assert rel <= 1e-4, (n, rel)
    print()
