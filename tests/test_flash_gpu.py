"""Flash attention with PoPE on the GPU: HIP kernels vs the CPU oracle.

Tolerance (from the build's north star, 2e-2 absolute against an fp32+
reference for bf16 flash forward and backward), with the oracle run in float64
on the same bf16/fp16-rounded inputs:
  * per-element outputs O, dq, dk, dv: max-abs error <= 2e-2;
  * the summed parameter gradients dbias (a sum over batch, group heads and
    keys) and dfreqs (a sum over batch and heads): max-abs error
    <= 2e-2 * max(1, ||ref||_inf), i.e. 2e-2 absolute at unit scale and 2e-2
    relative beyond it, because their magnitude -- and the bf16 rounding error
    of the MFMA operands summed into them -- grows with the number of terms.  The case matrix follows the reference's test_flash_attn.py:10-76
(dtype x causal x Nq in {1, 256} x mask, B2 H4 Nk256 D64 R32, (b n h d) layout),
plus ragged lengths, GQA, partial / full / no rotation, D = 32..128, fully
masked rows and the reference's consistency check against the similarity path
(test_flash_attn.py:78-110).
"""
import pytest
import torch

from gpu_common import make_pope_inputs, max_abs, oracle_attention

pytestmark = pytest.mark.gpu

TOL = 2e-2
SUMMED = ("dbias", "dfreqs")


def _tol(name, ref):
    if name in SUMMED:
        return TOL * max(1.0, ref.detach().abs().max().item())
    return TOL


def _run(inp, causal, head_first=True, need_grads=True, scale=None):
    import pope_amd
    q, k, v = (inp[n].detach().clone().requires_grad_(need_grads) for n in ("q", "k", "v"))
    freqs = inp["freqs"].detach().clone().requires_grad_(need_grads)
    bias = inp["bias"].detach().clone().requires_grad_(need_grads)
    R = freqs.shape[-1]
    pos = (freqs, bias) if R > 0 else None
    if head_first:
        o = pope_amd.flash_attn_with_pope(q, k, v, pos_emb=pos, mask=inp["mask"], causal=causal,
                                          softmax_scale=scale)
    else:
        tr = lambda t: t.transpose(1, 2).contiguous().detach().requires_grad_(need_grads)
        qb, kb, vb = tr(q), tr(k), tr(v)
        o = pope_amd.flash_attn_with_pope(qb, kb, vb, pos_emb=pos, mask=inp["mask"], causal=causal,
                                          softmax_scale=scale, head_dimension_at_first=False)
        o = o.transpose(1, 2)
        q, k, v = qb, kb, vb
    res = dict(o=o)
    if need_grads:
        do = inp["do"] if head_first else inp["do"]
        o.backward(do)
        g = lambda t: t.grad if head_first else t.grad.transpose(1, 2)
        res.update(dq=g(q), dk=g(k), dv=g(v), dfreqs=freqs.grad, dbias=bias.grad)
    return res


def _check(res, ref, names, tol_fn=_tol):
    errs = {n: max_abs(res[n], ref[n]) for n in names if res.get(n) is not None and ref.get(n) is not None}
    print(" ".join(f"{n}={e:.2e}" for n, e in errs.items()))
    for n, e in errs.items():
        t = tol_fn(n, ref[n])
        assert e <= t, f"{n} max-abs error {e:.3e} > {t:.3e}"
    return errs


# ---- the reference's case matrix: dtype x causal x Nq x mask (forward) -------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("seq_len_q", [1, 256])
@pytest.mark.parametrize("has_mask", [True, False])
def test_forward_reference_matrix(cuda, dtype, causal, seq_len_q, has_mask):
    inp = make_pope_inputs(42, 2, 4, 4, seq_len_q, 256, 64, 32, dtype, "half" if has_mask else "none")
    res = _run(inp, causal, head_first=False, need_grads=False)
    ref = oracle_attention(inp, causal, grads=False)
    _check(res, ref, ["o"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("seq_len_q", [1, 256])
@pytest.mark.parametrize("has_mask", [True, False])
def test_backward_reference_matrix(cuda, dtype, causal, seq_len_q, has_mask):
    inp = make_pope_inputs(42, 2, 4, 4, seq_len_q, 256, 64, 32, dtype, "half" if has_mask else "none")
    res = _run(inp, causal, head_first=False)
    ref = oracle_attention(inp, causal)
    _check(res, ref, ["o", "dq", "dk", "dv", "dfreqs", "dbias"])


# ---- shapes beyond the reference matrix ---------------------------------------------------------

SHAPES = [
    # B, Hq, Hk, Nq, Nk, D, R, causal, mask
    (2, 8, 8, 384, 384, 64, 32, True, "prefix"),      # C3 pattern, small
    (1, 4, 4, 200, 200, 64, 32, True, "random"),      # ragged tiles, random mask
    (1, 2, 2, 77, 130, 64, 64, False, "none"),        # ragged, Nq < Nk, full rotation
    (2, 4, 4, 256, 256, 96, 96, False, "none"),       # axial-style D = 96
    (1, 4, 4, 128, 128, 32, 16, True, "none"),        # D = 32
    (1, 2, 2, 192, 192, 128, 64, False, "prefix"),    # D = 128
    (1, 8, 2, 256, 256, 64, 32, True, "prefix"),      # GQA 4:1
    (1, 4, 4, 128, 128, 64, 0, True, "none"),         # no rotation: plain attention
    (2, 2, 2, 64, 64, 64, 32, False, "dead_row"),     # fully masked batch row -> 0
    (1, 2, 2, 1, 2048, 64, 64, False, "prefix"),      # single-query decode, long cache
    (2, 2, 2, 3, 1500, 64, 32, False, "random"),      # short query block, long cache
    (1, 2, 2, 2048, 2048, 64, 32, True, "prefix"),    # causal, 8 key blocks of 256
    (1, 1, 1, 2100, 2100, 96, 96, True, "none"),      # causal, wide rows (128-key jobs), ragged end
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(str(x) for x in s))
def test_forward_shapes(cuda, shape):
    B, Hq, Hk, Nq, Nk, D, R, causal, mk = shape
    inp = make_pope_inputs(7, B, Hq, Hk, Nq, Nk, D, R, torch.bfloat16, mk)
    res = _run(inp, causal, need_grads=False)
    ref = oracle_attention(inp, causal, grads=False)
    _check(res, ref, ["o"])


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(str(x) for x in s))
def test_backward_shapes(cuda, shape):
    B, Hq, Hk, Nq, Nk, D, R, causal, mk = shape
    inp = make_pope_inputs(11, B, Hq, Hk, Nq, Nk, D, R, torch.bfloat16, mk)
    res = _run(inp, causal)
    ref = oracle_attention(inp, causal)
    _check(res, ref, ["o", "dq", "dk", "dv", "dfreqs", "dbias"])


def test_lse_and_raw_forward(cuda):
    from pope_amd.hip_pope_flash_attn import flash_attn_forward
    inp = make_pope_inputs(3, 2, 4, 4, 256, 256, 64, 32, torch.bfloat16, "dead_row")
    tr = lambda t: t.transpose(1, 2)
    o, lse = flash_attn_forward(tr(inp["q"]), tr(inp["k"]), tr(inp["v"]), inp["freqs"], inp["bias"],
                                inp["mask"], causal=True)
    ref = oracle_attention(inp, True, grads=False)
    assert max_abs(tr(o), ref["o"]) <= TOL
    finite = torch.isfinite(ref["lse"])
    assert torch.equal(torch.isfinite(lse.cpu()), finite)
    assert (lse.cpu()[finite] - ref["lse"][finite]).abs().max().item() <= TOL


def test_fp32_inputs_and_custom_scale(cuda):
    """fp32 inputs run the fp16 MFMA kernels on fp16-rounded q, k, v (10 significant bits, as the
    reference's TF32 products keep): against the oracle on those rounded inputs the half-precision
    tolerance holds; against the fp32 oracle on the unrounded inputs the reference's own fp32
    tolerance holds, 2e-2 absolute (test_flash_attn.py:63-76: 5e-2 for half types, 2e-2 for fp32)."""
    inp = make_pope_inputs(5, 1, 4, 4, 128, 128, 64, 32, torch.float32, "prefix")
    res = _run(inp, True, need_grads=True, scale=0.2)
    assert res["o"].dtype == torch.float32
    rounded = dict(inp, **{n: inp[n].to(torch.float16).float() for n in ("q", "k", "v")})
    _check(res, oracle_attention(rounded, True, scale=0.2), ["o", "dq", "dk", "dv", "dbias"])
    _check(res, oracle_attention(inp, True, scale=0.2), ["o", "dq", "dk", "dv", "dbias"])


@pytest.mark.parametrize("seq_len_q", [1, 1024])
def test_consistent_with_similarity_path(cuda, seq_len_q):
    """softmax(sim * scale) v from compute_attn_similarity == flash_attn_with_pope
    (reference test_flash_attn.py:78-110, which asserts < 5e-4 with fp32 inputs)."""
    import pope_amd
    from pope_amd import PoPE
    torch.manual_seed(0)
    q = torch.randn(1, seq_len_q, 8, 64, device="cuda")
    k = torch.randn(1, 1024, 8, 64, device="cuda")
    v = torch.randn(1, 1024, 8, 64, device="cuda")
    pope = PoPE(32, heads=8).cuda()(1024)
    sim = pope_amd.compute_attn_similarity(q, k, pope, head_dimension_at_first=False)
    attn = (sim * 64 ** -0.5).softmax(-1)
    out_sim = torch.einsum("bhij,bhjd->bhid", attn, v.transpose(1, 2)).transpose(1, 2)
    out = pope_amd.flash_attn_with_pope(q, k, v, pos_emb=pope, head_dimension_at_first=False)
    # fp32 inputs run on fp16 operands (TF32's 10 significant bits): the reference's bound holds
    err = max_abs(out, out_sim)
    print(f"flash vs softmax(sim * scale) v: {err:.2e}")
    assert err < 5e-4


def test_readme_fused_flash_attn(cuda):
    import pope_amd
    pope = pope_amd.PoPE(dim=32, heads=8).cuda()
    q = torch.randn(2, 8, 1024, 64).cuda()
    k = torch.randn(2, 8, 1024, 64).cuda()
    v = torch.randn(2, 8, 1024, 64).cuda()
    mask = torch.ones((2, 1024)).bool().cuda()
    out = pope_amd.flash_attn_with_pope(q, k, v, pos_emb=pope(1024), causal=True, mask=mask)
    assert out.shape == (2, 8, 1024, 64)


def test_registered_ops_match_eager_path(cuda):
    """The torch.library ops (used under torch.compile tracing) and the eager autograd path run the
    same kernels: outputs equal, gradients equal up to the order of the fp32 atomic adds."""
    from pope_amd.hip_pope_flash_attn import _flash, flash_fwd_op
    inp = make_pope_inputs(7, 2, 4, 2, 192, 256, 64, 32, torch.bfloat16, "prefix")

    def grads(fn):
        q, k, v, f, b = (inp[n].detach().clone().requires_grad_(True) for n in ("q", "k", "v", "freqs", "bias"))
        o = fn(q, k, v, f, b, inp["mask"], True, 0.125)
        o.backward(inp["do"])
        return [o] + [t.grad for t in (q, k, v, f, b)]

    eager = grads(_flash)
    via_ops = grads(lambda *a: flash_fwd_op(*a)[0])
    assert torch.equal(eager[0], via_ops[0])
    for a, b in zip(eager[1:], via_ops[1:]):
        assert (a.float() - b.float()).abs().max().item() <= 1e-3 * max(1.0, a.float().abs().max().item())


def test_compiled_call_records_ops(cuda):
    """torch.compile traces the registered ops (no graph break) and gives the eager results."""
    import pope_amd
    inp = make_pope_inputs(8, 1, 2, 2, 128, 128, 64, 32, torch.bfloat16, "none")

    def f(q, k, v, fr, b):
        return pope_amd.flash_attn_with_pope(q, k, v, pos_emb=(fr, b), causal=True)

    args = [inp[n].detach().clone() for n in ("q", "k", "v", "freqs", "bias")]
    ref = f(*args)
    out = torch.compile(f, backend="aot_eager", fullgraph=True)(*args)
    assert torch.equal(out, ref)


def test_registered_op_checks(cuda):
    """torch.library.opcheck on pope_amd::flash_fwd: schema, autograd registration and the fake
    (meta) implementation.  Its AOT-dispatch check is left out: it compares every output of a traced
    and an eager call bit for bit, and the third output, the workspace handed to the backward, holds
    regions the forward does not write (the backward's row terms, alignment gaps)."""
    from pope_amd.hip_pope_flash_attn import flash_fwd_op
    inp = make_pope_inputs(3, 1, 2, 2, 128, 128, 64, 32, torch.bfloat16, "prefix")
    q, k, v, f, b = (inp[n].detach().clone().requires_grad_(True) for n in ("q", "k", "v", "freqs", "bias"))
    torch.library.opcheck(flash_fwd_op, (q, k, v, f, b, inp["mask"], True, 0.125),
                          test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))


# ---- the reference's operator-level names (triton_pope_flash_attn.py:222-373) -------------------

def test_reference_named_operators(cuda):
    """flash_attn, FlashAttnFunction.apply and flash_attn_forward / flash_attn_backward in the
    reference's (B, N, H, D) layout, against the oracle -- the binding a maintainer plugs in at
    attention.py:21-26.  flash_attn_backward keeps the reference launcher's write semantics: dq,
    dfreqs and dpope_bias accumulate into caller-zeroed buffers, dk and dv are overwritten."""
    from pope_amd.hip_pope_flash_attn import (FlashAttnFunction, flash_attn, flash_attn_backward,
                                              flash_attn_forward)
    inp = make_pope_inputs(21, 2, 4, 4, 192, 192, 64, 32, torch.bfloat16, "prefix")
    ref = oracle_attention(inp, True)
    tr = lambda t: t.transpose(1, 2)
    for fn in (flash_attn, FlashAttnFunction.apply):
        q, k, v = (tr(inp[n]).detach().clone().requires_grad_(True) for n in ("q", "k", "v"))
        f, b = (inp[n].detach().clone().requires_grad_(True) for n in ("freqs", "bias"))
        o = fn(q, k, v, f, b, inp["mask"], True)
        assert o.shape == q.shape
        o.backward(tr(inp["do"]))
        got = dict(o=tr(o), dq=tr(q.grad), dk=tr(k.grad), dv=tr(v.grad), dfreqs=f.grad, dbias=b.grad)
        _check(got, ref, ["o", "dq", "dk", "dv", "dfreqs", "dbias"])

    q, k, v, do = (tr(inp[n]).contiguous() for n in ("q", "k", "v", "do"))
    o, lse = flash_attn_forward(q, k, v, inp["freqs"], inp["bias"], inp["mask"], causal=True)
    assert lse.shape == (2, 4, 192) and lse.dtype == torch.float32
    dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
    df, db = torch.zeros_like(inp["freqs"]), torch.zeros_like(inp["bias"])
    for _ in range(2):   # a second call adds to dq / dfreqs / dbias and rewrites dk / dv
        flash_attn_backward(do, q, k, v, o, lse, dq, dk, dv, df, db, inp["freqs"], inp["bias"], inp["mask"],
                            causal=True)
    got = dict(o=tr(o), dq=tr(dq) / 2, dk=tr(dk), dv=tr(dv), dfreqs=df / 2, dbias=db / 2)
    _check(got, ref, ["o", "dq", "dk", "dv", "dfreqs", "dbias"])
    with pytest.raises(ValueError):   # a mis-shaped lse is rejected on every call, cached plan or not
        flash_attn_backward(do, q, k, v, o, lse[:, :, :-1], dq, dk, dv, None, None, inp["freqs"], inp["bias"],
                            inp["mask"], causal=True)


def test_freqs_longer_than_keys_get_zero_rows(cuda):
    """freqs may hold more positions than there are keys (the kernels use rows n < Nk); the rows past
    Nk get a zero gradient, as the reference's zeros_like(f) buffer gives them (:359)."""
    inp = make_pope_inputs(23, 1, 2, 2, 96, 96, 64, 32, torch.bfloat16, "none")
    long_f = torch.cat([inp["freqs"], inp["freqs"][:40] + 1000.0])   # 136 rows for 96 keys
    inp_long = dict(inp, freqs=long_f)
    res = _run(inp_long, causal=False)
    assert res["dfreqs"].shape == (136, 32)
    assert torch.equal(res["dfreqs"][96:].cpu(), torch.zeros(40, 32))
    ref = oracle_attention(inp, causal=False)
    _check(dict(res, dfreqs=res["dfreqs"][:96]), ref, ["o", "dq", "dk", "dv", "dfreqs", "dbias"])


def test_operand_dtypes_must_match(cuda):
    from pope_amd.hip_pope_flash_attn import flash_fwd_op
    inp = make_pope_inputs(3, 1, 2, 2, 64, 64, 64, 32, torch.bfloat16, "none")
    with pytest.raises(TypeError):
        flash_fwd_op(inp["q"], inp["k"].half(), inp["v"], inp["freqs"], inp["bias"], None, False, 0.125)


def test_registered_op_checks_on_the_decode_path(cuda):
    """opcheck's fake-tensor test on a call the decode kernel serves (Nq = 1, Nk >= 1024): the fake
    implementation returns the same (empty) workspace as the real one."""
    from pope_amd.hip_pope_flash_attn import flash_fwd_op
    inp = make_pope_inputs(4, 2, 2, 2, 1, 1024, 64, 64, torch.bfloat16, "prefix")
    args = (inp["q"], inp["k"], inp["v"], inp["freqs"], inp["bias"], inp["mask"], False, 0.125)
    o, lse, ws = flash_fwd_op(*args)
    assert ws.numel() == 0
    torch.library.opcheck(flash_fwd_op, args, test_utils=("test_schema", "test_faketensor"))


def test_workspace_reuse_off_gives_the_same_gradients(cuda):
    """set_flash_workspace_reuse(False): the forward's workspace is not kept, the backward repeats
    the preparation, and o, dq, dk, dv are bitwise those of the default path (dfreqs / dbias add
    fp32 atomics in an arbitrary order, so they agree to rounding)."""
    import pope_amd
    from pope_amd import hip_pope_flash_attn as fa
    inp = make_pope_inputs(41, 2, 4, 2, 300, 300, 64, 32, torch.bfloat16, mask_kind="prefix")

    def run():
        t = [inp[n].detach().clone().cuda().requires_grad_(True) for n in ("q", "k", "v", "freqs", "bias")]
        mask = inp["mask"].cuda() if inp["mask"] is not None else None
        o = pope_amd.flash_attn_with_pope(t[0], t[1], t[2], pos_emb=(t[3], t[4]), mask=mask, causal=True)
        o.backward(inp["do"].cuda())
        torch.cuda.synchronize()
        return [o.detach()] + [x.grad for x in t], fa._LAST_BWD_PREPARED

    ref, prepared = run()
    assert prepared
    fa.set_flash_workspace_reuse(False)
    try:
        got, prepared = run()
    finally:
        fa.set_flash_workspace_reuse(True)
    assert not prepared
    for a, b in zip(got[:4], ref[:4]):
        assert torch.equal(a, b)
    for a, b in zip(got[4:], ref[4:]):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5 * b.abs().max().item())
