"""Single-query decode against a long KV cache on the GPU: the split-K decode
kernel (flash_decode) vs the CPU oracle.

Tolerance: the north star's 2e-2 absolute against an fp32+ reference for bf16
flash, with the oracle in float64 on the same bf16/fp16-rounded inputs.  Cases
follow BASELINE config C5 in miniature (one query row, PoPE with full rotation,
valid prefix lengths per batch via the key-padding mask) plus ragged cache
lengths, head dims 32..128 (including 96, whose 12 chunks of 8 dims leave lanes
idle), GQA, a batch row with every key masked, fp16, bf16 keys at and beyond the
range of the kernel's softplus table, and the backward through the decode's
log-sum-exp.
"""
import pytest
import torch

from gpu_common import make_pope_inputs, max_abs, oracle_attention

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _decode_inputs(seed, B, Hq, Hk, Nk, D, R, dtype, lengths=None, dead_row=False):
    inp = make_pope_inputs(seed, B, Hq, Hk, 1, Nk, D, R, dtype, "none")
    mask = torch.ones(B, Nk, dtype=torch.bool)
    g = torch.Generator().manual_seed(seed + 1)
    for b in range(B):
        L = lengths[b] if lengths is not None else int(torch.randint(Nk // 8, Nk + 1, (1,), generator=g))
        mask[b, L:] = False
    if dead_row:
        mask[0] = False
    inp["mask"] = mask.to("cuda")
    return inp


def _run(inp, need_grads=False):
    import pope_amd
    q, k, v = (inp[n].detach().clone().requires_grad_(need_grads) for n in ("q", "k", "v"))
    rot = inp["freqs"].shape[-1] > 0
    freqs = inp["freqs"].detach().clone().requires_grad_(need_grads and rot)
    bias = inp["bias"].detach().clone().requires_grad_(need_grads and rot)
    pos = (freqs, bias) if rot else None
    o = pope_amd.flash_attn_with_pope(q, k, v, pos_emb=pos, mask=inp["mask"], causal=False)
    res = dict(o=o)
    if need_grads:
        o.backward(inp["do"])
        res.update(dq=q.grad, dk=k.grad, dv=v.grad, dbias=bias.grad)
    return res


CASES = [
    # B, Hq, Hk, Nk, D, R, dtype
    (2, 4, 4, 8192, 64, 64, torch.bfloat16),
    (3, 4, 4, 5000 + 37, 64, 64, torch.bfloat16),     # ragged cache length
    (2, 8, 2, 4096, 64, 32, torch.bfloat16),          # GQA 4:1, partial rotation
    (2, 2, 2, 3000, 128, 64, torch.bfloat16),         # D = 128
    (2, 2, 2, 3000, 96, 96, torch.bfloat16),          # D = 96 (axial-style)
    (2, 2, 2, 2048, 32, 16, torch.float16),           # D = 32, fp16
    (1, 5, 5, 2500, 48, 16, torch.bfloat16),          # 5 heads over 4 waves, D = 48 (idle chunk lanes)
    (2, 1, 1, 4100, 64, 0, torch.float16),            # one head (three idle waves), no rotation
    (1, 6, 3, 3333, 128, 128, torch.bfloat16),        # GQA 2:1, full rotation at D = 128, ragged
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(str(x) for x in c[:6]))
def test_decode_forward(cuda, case):
    B, Hq, Hk, Nk, D, R, dtype = case
    inp = _decode_inputs(31, B, Hq, Hk, Nk, D, R, dtype)
    res = _run(inp)
    ref = oracle_attention(inp, False, grads=False)
    err = max_abs(res["o"], ref["o"])
    print(f"o={err:.2e}")
    assert err <= TOL


def test_decode_extreme_key_magnitudes(cuda):
    """bf16 keys outside the tabulated softplus range (|x| >= 32, |x| < 2^-24, zeros) and at its
    edges, sprinkled over N(0, 1) keys: the kernel's table clamps must match the oracle's softplus."""
    inp = _decode_inputs(41, 2, 4, 4, 3000, 64, 64, torch.bfloat16)
    g = torch.Generator().manual_seed(43)
    k = inp["k"].float().cpu()
    vals = torch.tensor([0.0, -0.0, 2.0 ** -30, -(2.0 ** -30), 2.0 ** -24, 2.0 ** -20, 31.75, -31.75, 32.0, -32.0,
                         40.0, -40.0, 100.0, -100.0])
    pick = torch.rand(k.shape, generator=g) < 0.02
    k[pick] = vals[torch.randint(0, len(vals), (int(pick.sum()),), generator=g)]
    inp["k"] = k.to(torch.bfloat16).to("cuda")
    res = _run(inp)
    ref = oracle_attention(inp, False, grads=False)
    err = max_abs(res["o"], ref["o"])
    print(f"o={err:.2e}")
    assert err <= TOL


def test_decode_lse_and_dead_row(cuda):
    from pope_amd.hip_pope_flash_attn import flash_attn_forward
    inp = _decode_inputs(5, 3, 4, 4, 6000, 64, 64, torch.bfloat16, lengths=[6000, 1, 4097], dead_row=True)
    tr = lambda t: t.transpose(1, 2)
    o, lse = flash_attn_forward(tr(inp["q"]), tr(inp["k"]), tr(inp["v"]), inp["freqs"], inp["bias"], inp["mask"])
    ref = oracle_attention(inp, False, grads=False)
    assert max_abs(tr(o), ref["o"]) <= TOL
    finite = torch.isfinite(ref["lse"])
    assert torch.equal(torch.isfinite(lse.cpu()), finite)           # batch 0: every key masked
    assert (lse.cpu()[finite] - ref["lse"][finite]).abs().max().item() <= TOL
    assert tr(o)[0].abs().max().item() == 0.0


def test_decode_backward(cuda):
    inp = _decode_inputs(9, 2, 4, 4, 4096, 64, 64, torch.bfloat16)
    res = _run(inp, need_grads=True)
    ref = oracle_attention(inp, False)
    for n in ("o", "dq", "dk", "dv", "dbias"):
        e = max_abs(res[n], ref[n])
        t = TOL * (max(1.0, ref[n].abs().max().item()) if n == "dbias" else 1.0)
        print(f"{n}={e:.2e}")
        assert e <= t, n


@pytest.mark.parametrize("view", ["offset_rows", "batch_one", "heads_one", "odd_offset"])
def test_decode_freqs_views(cuda, view):
    """freqs tables that are views the decode kernel cannot read as given: rows starting past the
    table's first element (a KV-cache continuation), a (1, N, R) table broadcast over the batch,
    a (B, N, 1, R) table with one head, and a view whose start is not a whole 16-byte vector.
    Each must give the oracle's result (the kernel choice may differ, the result may not)."""
    import pope_amd
    B, H, Nk, D, R = 2, 4, 2048, 64, 64
    inp = _decode_inputs(61, B, H, H, Nk, D, R, torch.bfloat16)
    F = inp["freqs"]
    if view == "offset_rows":
        big = orc_freqs(Nk + 100, R).to("cuda")
        fv = big[100:]
        want = big[100:].cpu()
    elif view == "batch_one":
        fv = F[None]
        want = F.cpu()
    elif view == "heads_one":
        fv = F[None, None].expand(B, 1, Nk, R).contiguous()      # (B, H = 1, N, R), head-first
        want = F.cpu()
    else:
        flat = torch.zeros(Nk * R + 1, device="cuda")
        flat[1:] = F.reshape(-1)
        fv = flat[1:].view(Nk, R)
        want = F.cpu()
    ref_inp = dict(inp, freqs=want.to("cuda"))
    ref = oracle_attention(ref_inp, False, grads=False)
    o = pope_amd.flash_attn_with_pope(inp["q"], inp["k"], inp["v"], pos_emb=(fv, inp["bias"]), mask=inp["mask"])
    err = max_abs(o, ref["o"])
    print(f"{view}: o={err:.2e}")
    assert err <= TOL


def orc_freqs(n, R):
    from oracle import pope_oracle as orc
    return orc.pope_freqs(n, orc.inv_freqs(R))


def test_fp32_flash_rejects_values_beyond_fp16(cuda):
    """fp32 q / k / v run on fp16 operands; a finite value beyond 65504 raises instead of
    silently becoming inf."""
    import pope_amd
    inp = make_pope_inputs(3, 1, 2, 2, 64, 64, 64, 32, torch.float32)
    q = inp["q"].clone()
    q[0, 0, 0, 0] = 7.0e4
    with pytest.raises(ValueError, match="fp16"):
        pope_amd.flash_attn_with_pope(q, inp["k"], inp["v"], pos_emb=(inp["freqs"], inp["bias"]))


def test_decode_head_groups(cuda):
    """Nq = 1 with query heads x head dim = 8192, above what one split workgroup stages in LDS
    (4096 query-weight words): the split kernel runs with two groups of 32 heads per split, and
    must match the oracle."""
    from pope_amd import _lib
    inp = _decode_inputs(71, 2, 64, 16, 2048, 128, 64, torch.bfloat16)
    _lib.profile_reset()
    _lib.profile_enable(True)
    try:
        res = _run(inp)
        torch.cuda.synchronize()
    finally:
        _lib.profile_enable(False)
    assert "flash_decode_split" in _lib.profile_read()
    ref = oracle_attention(inp, False, grads=False)
    err = max_abs(res["o"], ref["o"])
    print(f"o={err:.2e}")
    assert err <= TOL


@pytest.mark.parametrize("lengths", [[0, 3000, 1], [1, 1, 1], [2048, 0, 2048], [5, 2048, 1000]],
                         ids=["dead-long-one", "ones", "dead-middle", "mixed"])
def test_decode_deal_edge_lengths(cuda, lengths):
    """Batches with no visible key (o = 0 and lse = -inf), one key, and very unequal lengths side
    by side."""
    from pope_amd.hip_pope_flash_attn import flash_attn_forward
    B, H, Nk = len(lengths), 4, 3000
    inp = _decode_inputs(73, B, H, H, Nk, 64, 64, torch.bfloat16, lengths=lengths)
    tr = lambda t: t.transpose(1, 2)
    o, lse = flash_attn_forward(tr(inp["q"]), tr(inp["k"]), tr(inp["v"]), inp["freqs"], inp["bias"], inp["mask"])
    ref = oracle_attention(inp, False, grads=False)
    assert max_abs(tr(o), ref["o"]) <= TOL
    finite = torch.isfinite(ref["lse"])
    assert torch.equal(torch.isfinite(lse.cpu()), finite)
    if finite.any():
        assert (lse.cpu()[finite] - ref["lse"][finite]).abs().max().item() <= TOL
    for b, L in enumerate(lengths):
        if L == 0:
            assert tr(o)[b].abs().max().item() == 0.0


def test_decode_dead_splits_ignore_workspace_contents(cuda):
    """A split whose keys are all masked writes only (m, l) = (-inf, 0); the combine must not read
    the partial output rows it leaves unwritten.  The same call on a workspace filled with NaN
    bytes and on a zeroed one gives the same o and lse bit for bit, and both meet the oracle.
    The mask leaves dead splits at the start, in the middle and at the end of sequences, and one
    sequence with no visible key."""
    import ctypes
    from pope_amd import _lib
    from pope_amd.hip_pope_flash_attn import _desc
    B, H, Nk = 3, 4, 6000
    inp = _decode_inputs(77, B, H, H, Nk, 64, 64, torch.bfloat16, lengths=[Nk, Nk, 0])
    mask = inp["mask"].cpu()
    mask[0, 300:4000] = False      # dead splits between live ones
    mask[1, :2500] = False         # dead splits before the first visible key
    mask[1, 2600:] = False         # and after the last
    inp["mask"] = mask.to("cuda")
    q, k, v, freqs, bias, m = (inp[n] for n in ("q", "k", "v", "freqs", "bias", "mask"))
    d = _desc(q, k, freqs, bias, False, q.shape[-1] ** -0.5)
    outs = []
    for fill in (0xFF, 0x00):
        o = torch.empty_like(q)
        lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
        d.q_s[:], d.k_s[:], d.v_s[:], d.o_s[:] = (_lib.strides3(t) for t in (q, k, v, o))
        d.mask_sb = m.stride(0)
        n = _lib.workspace_bytes(_lib.OP_FLASH_DECODE, d)
        ws = torch.full((n,), fill, dtype=torch.uint8, device=q.device)
        st = _lib.lib().pope_flash_decode(ctypes.byref(d), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                          freqs.data_ptr(), bias.data_ptr(), m.data_ptr(), o.data_ptr(),
                                          lse.data_ptr(), ws.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
        _lib.check(st, "decode")
        torch.cuda.synchronize()
        outs.append((o, lse))
    (o1, l1), (o0, l0) = outs
    assert torch.equal(o1, o0) and torch.equal(l1, l0)
    assert torch.isfinite(o1).all()
    ref = oracle_attention(inp, False, grads=False)
    assert max_abs(o1, ref["o"]) <= TOL
    finite = torch.isfinite(ref["lse"])
    assert torch.equal(torch.isfinite(l1.cpu()), finite)
    assert (l1.cpu()[finite] - ref["lse"][finite]).abs().max().item() <= TOL
