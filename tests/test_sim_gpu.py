"""Fused PoPE similarity on the GPU: the fp32 MFMA kernels (allow_tf32=False) and the
split-bf16 kernels (allow_tf32=True, the default) vs the CPU oracle.

Tolerance (from the build's north star): 1e-4 relative for fp32 similarity,
read as ||kernel - oracle||_inf <= 1e-4 * ||oracle||_inf for S and for each
gradient (dq, dk, dbias, dfreqs), and element by element as
allclose(rtol=1e-4, atol=1e-4 * rms(oracle)).  The oracle runs in fp32 on the same inputs
(reproducing the reference's fl(freqs + bias) phase rounding, pope.py:56).
Cases follow the reference's test_triton.py: multi-config incl. R = 0
(:15-54), non-contiguous slices (:56-85), dfreqs with random freqs/bias
(:87-109); plus GQA, ragged sizes and the README example.
"""
import math

import pytest
import torch

from oracle import pope_oracle as orc

pytestmark = pytest.mark.gpu

RTOL = 1e-4


def _rel_inf(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def _elementwise(a, b):
    """Largest |a - b| / (RTOL |b| + RTOL rms(b)): at most 1 means allclose(rtol=1e-4,
    atol=1e-4 rms(ref)) holds element by element."""
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    rms = b.pow(2).mean().sqrt().clamp_min(1e-30)
    return ((a - b).abs() / (RTOL * b.abs() + RTOL * rms)).max().item()


def _case(seed, B, Hq, Hk, Nq, Nk, D, R, rand_freqs=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Nq, D, generator=g)
    k = torch.randn(B, Hk, Nk, D, generator=g)
    if rand_freqs:
        freqs = torch.randn(Nk, R, generator=g)
        bias = torch.randn(Hk, R, generator=g)
    else:
        freqs = orc.pope_freqs(Nk, orc.inv_freqs(R)) if R else torch.empty(Nk, 0)
        bias = torch.rand(Hk, R, generator=g) * (-2 * math.pi)
    G = torch.randn(B, Hq, Nq, Nk, generator=g)
    return q, k, freqs, bias, G


def _oracle(q, k, freqs, bias, G):
    t = [x.detach().clone().requires_grad_(True) for x in (q, k, freqs, bias)]
    S = orc.sim_nonfused(*t)
    (S * G).sum().backward()
    return S.detach(), [x.grad for x in t]


def _kernel(q, k, freqs, bias, G, slicer=None, allow_tf32=True):
    import pope_amd
    t = [x.detach().clone().cuda().requires_grad_(True) for x in (q, k, freqs, bias)]
    qq, kk = t[0], t[1]
    S = pope_amd.compute_attn_similarity(qq, kk, (t[2], t[3]), allow_tf32=allow_tf32)
    S.backward(G.cuda())
    return S.detach(), [x.grad for x in t]


def _compare(S, grads, S_ref, grads_ref, names=("dq", "dk", "dfreqs", "dbias")):
    e = {"S": _rel_inf(S, S_ref)}
    el = {"S": _elementwise(S, S_ref)}
    for n, g, r in zip(names, grads, grads_ref):
        if r is not None and g is not None and r.numel():
            e[n] = _rel_inf(g, r)
            el[n] = _elementwise(g, r)
    print(" ".join(f"{n}={v:.2e}/{el[n]:.2f}" for n, v in e.items()))
    for n, v in e.items():
        assert v <= RTOL, f"{n}: relative error {v:.3e} > {RTOL}"
        assert el[n] <= 1.0, f"{n}: elementwise allclose(rtol=1e-4, atol=1e-4 rms) fails by {el[n]:.2f}x"


@pytest.mark.parametrize("cfg", [
    (1, 8, 8, 128, 128, 64, 0),      # reference test_triton.py:274-276
    (1, 8, 8, 128, 128, 64, 32),
    (2, 4, 4, 256, 256, 128, 64),
    (2, 8, 8, 256, 256, 64, 64),     # C2 pattern, small
    (1, 4, 2, 100, 300, 64, 32),     # GQA, ragged, Nq < Nk
    (1, 2, 2, 64, 64, 256, 128),     # E = 384: several expanded-column chunks
    (1, 2, 2, 33, 33, 48, 16),       # D = 48
    (1, 2, 1, 40, 72, 256, 253),     # D = 256 with a ragged rotate dim: padded to 264 wide
], ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("allow_tf32", [True, False], ids=["split_bf16", "fp32"])
def test_similarity_multi_config(cuda, cfg, allow_tf32):
    q, k, freqs, bias, G = _case(100, *cfg)
    S_ref, g_ref = _oracle(q, k, freqs, bias, G)
    S, g = _kernel(q, k, freqs, bias, G, allow_tf32=allow_tf32)
    _compare(S, g, S_ref, g_ref)


def test_similarity_large_grid_paths(cuda):
    """A shape whose grids take the split-bf16 kernels' large-problem paths: U / W jobs without the
    split reduction (at least 512 workgroups of one part each) and four S tiles per forward
    workgroup with a partial last group (nine key blocks), with grouped heads and ragged sizes."""
    q, k, freqs, bias, G = _case(101, 1, 64, 16, 1000, 1150, 64, 32)
    S_ref, g_ref = _oracle(q, k, freqs, bias, G)
    S, g = _kernel(q, k, freqs, bias, G, allow_tf32=True)
    _compare(S, g, S_ref, g_ref)


def test_similarity_non_contiguous(cuda):
    import pope_amd
    g = torch.Generator().manual_seed(5)
    qf = torch.randn(1, 8, 256, 64, generator=g)
    kf = torch.randn(1, 8, 256, 64, generator=g)
    freqs = orc.pope_freqs(256, orc.inv_freqs(32))[:128]
    bias = torch.rand(8, 32, generator=g) * (-2 * math.pi)
    Gd = torch.randn(1, 8, 128, 128, generator=g)
    q_nc, k_nc = qf[:, :, :128, :], kf[:, :, :128, :]
    S_ref, g_ref = _oracle(q_nc, k_nc, freqs, bias, Gd)
    qc = qf.cuda()[:, :, :128, :].detach().requires_grad_(True)
    kc = kf.cuda()[:, :, :128, :].detach().requires_grad_(True)
    assert not qc.is_contiguous()
    fb = [freqs.cuda().requires_grad_(True), bias.cuda().requires_grad_(True)]
    S = pope_amd.compute_attn_similarity(qc, kc, tuple(fb))
    S.backward(Gd.cuda())
    _compare(S, [qc.grad, kc.grad, fb[0].grad, fb[1].grad], S_ref, g_ref)


def test_similarity_dfreqs_random_tables(cuda):
    # reference test_triton.py:87-109: B1 H2 N64 D32 R16, random freqs and bias
    q, k, freqs, bias, G = _case(9, 1, 2, 2, 64, 64, 32, 16, rand_freqs=True)
    S_ref, g_ref = _oracle(q, k, freqs, bias, G)
    S, g = _kernel(q, k, freqs, bias, G)
    _compare(S, g, S_ref, g_ref)


def test_similarity_head_dim_assert(cuda):
    import pope_amd
    q = torch.randn(1, 2, 8, 40, device="cuda")
    with pytest.raises(AssertionError):
        pope_amd.compute_attn_similarity(q, q, (torch.zeros(8, 8, device="cuda"), torch.zeros(2, 8, device="cuda")))


def test_readme_fused_similarity(cuda):
    import pope_amd
    pope = pope_amd.PoPE(dim=64, heads=8).cuda()
    pos_emb = pope(1024)
    q = torch.randn(1, 8, 1024, 64).cuda()
    k = torch.randn(1, 8, 1024, 64).cuda()
    sim = pope_amd.compute_attn_similarity(q, k, pos_emb)
    assert sim.shape == (1, 8, 1024, 1024)
    ref = orc.sim_nonfused(q.cpu(), k.cpu(), pos_emb.freqs.cpu(), pos_emb.bias.detach().cpu())
    assert _rel_inf(sim, ref) <= RTOL


def test_reference_named_similarity_function(cuda):
    """PoPESimilarityFunction.apply(q, k, freqs, bias, rotate_dim, allow_tf32) and
    hip_compute_qk_similarity, the reference's operator names (triton_pope.py:258-372)."""
    from pope_amd.hip_pope import PoPESimilarityFunction, hip_compute_qk_similarity
    q, k, freqs, bias, G = _case(31, 1, 4, 2, 96, 128, 64, 32)
    S_ref, g_ref = _oracle(q, k, freqs, bias, G)
    for fn in (PoPESimilarityFunction.apply, hip_compute_qk_similarity):
        t = [x.detach().clone().cuda().requires_grad_(True) for x in (q, k, freqs, bias)]
        S = fn(t[0], t[1], t[2], t[3], 32, False)
        S.backward(G.cuda())
        _compare(S, [x.grad for x in t], S_ref, g_ref)


def test_similarity_registered_op_checks(cuda):
    """torch.library.opcheck on pope_amd::sim_fwd: schema, autograd registration and the fake
    implementation."""
    from pope_amd.hip_pope import sim_fwd_op
    q, k, freqs, bias, G = _case(103, 1, 2, 2, 128, 128, 64, 32)
    args = [x.cuda().requires_grad_(True) for x in (q, k, freqs, bias)]
    torch.library.opcheck(sim_fwd_op, (*args, True),
                          test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))


@pytest.mark.parametrize("deterministic", [True, False], ids=["deterministic", "atomics"])
@pytest.mark.parametrize("extra_rows", [0, 5], ids=["dense", "longer_table"])
@pytest.mark.parametrize("split", [True, False], ids=["split_bf16", "fp32"])
def test_similarity_zero_grads_flag(cuda, split, extra_rows, deterministic):
    """POPE_FLAG_ZERO_GRADS through the C-ABI: the backward overwrites dfreqs rows n < Nk and
    every dbias row whatever they held (NaN here), leaves the rows n >= Nk of a longer freqs
    table untouched, and gives the gradients of a call that accumulates into zeros: bitwise in
    deterministic mode, within fp32 atomic-order rounding otherwise.  A per-batch table with
    extra rows takes the kernels' strided clearing, one without them the flat one."""
    import ctypes
    from pope_amd import _lib
    from pope_amd.hip_pope import _desc
    from pope_amd.hip_pope_flash_attn import _freqs_strides
    B, Hq, Hk, Nq, Nk, D, R = 2, 4, 2, 40, 72, 64, 32
    g = torch.Generator().manual_seed(211)
    q = torch.randn(B, Hq, Nq, D, generator=g).cuda()
    k = torch.randn(B, Hk, Nk, D, generator=g).cuda()
    freqs = torch.randn(B, Nk + extra_rows, R, generator=g).cuda()
    bias = torch.randn(Hk, R, generator=g).cuda()
    dsim = torch.randn(B, Hq, Nq, Nk, generator=g).cuda()
    L = _lib.lib()

    def run(zero, fill):
        d = _desc(q, k, freqs, bias, split)
        d.flags |= (_lib.FLAG_ZERO_GRADS if zero else 0) | (_lib.FLAG_DETERMINISTIC if deterministic else 0)
        d.sim_s[:] = _lib.strides3(dsim)
        dq, dk = torch.empty_like(q), torch.empty_like(k)
        d.dq_s[:], d.dk_s[:] = _lib.strides3(dq), _lib.strides3(dk)
        dfreqs, dbias = torch.full_like(freqs, fill), torch.full_like(bias, fill)
        d.df_s[:] = _freqs_strides(dfreqs)
        ws = _lib.workspace(_lib.OP_SIM_BWD, d, q.device)
        st = L.pope_sim_bwd(ctypes.byref(d), _lib.ptr(dsim), _lib.ptr(q), _lib.ptr(k), _lib.ptr(freqs),
                            _lib.ptr(bias), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dfreqs), _lib.ptr(dbias),
                            _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_ptr(q.device))
        _lib.check(st, "similarity backward")
        torch.cuda.synchronize()
        return dq, dk, dfreqs, dbias

    got = run(True, float("nan"))
    want = run(False, 0.0)
    if extra_rows:
        assert torch.isnan(got[2][:, Nk:]).all(), "rows past Nk must keep their contents"
        got = (*got[:2], got[2][:, :Nk], got[3])
        want = (*want[:2], want[2][:, :Nk], want[3])
    for name, a, b in zip(("dq", "dk", "dfreqs", "dbias"), got, want):
        assert torch.isfinite(a).all(), name
        if deterministic:
            assert torch.equal(a, b), name
        else:
            assert _rel_inf(a, b) <= 1e-5, (name, _rel_inf(a, b))
