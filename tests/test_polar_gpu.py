"""Materialising polar transform on the GPU (apply_pope_to_qk, pope.py:30-86) vs the CPU oracle.

Outputs q_hat / k_hat (fp32) and the gradients of q, k, freqs and bias through a random
upstream gradient.  Tolerances: fp32 inputs 1e-5 relative to ||ref||_inf for the outputs and
dq / dk, 1e-4 relative for the summed dfreqs / dbias; half-precision inputs
2e-2 * max(1, ||ref||_inf): the reference rounds to the input dtype several times on the way
(softplus in the input dtype, pope.py:60, and the half-precision autograd of it), the kernels
once, and one ulp of bf16 is 2^-8 of the value -- at |dq| ~ 4 two ulps are 0.03.
"""
import math

import pytest
import torch

from oracle import pope_oracle as orc

pytestmark = pytest.mark.gpu

CASES = [
    # B, Hq, Hk, Nq, Nk, D, R, dtype, 3-D freqs, bias rows
    (1, 8, 8, 1024, 1024, 64, 64, torch.float32, False, 8),   # C1's transform
    (2, 4, 2, 100, 300, 64, 32, torch.bfloat16, False, 2),    # partial rotation, Nq < Nk, 2 kv heads
    (2, 2, 2, 64, 64, 48, 16, torch.float16, True, 2),        # D = 48, per-batch positions
    (1, 2, 2, 33, 33, 128, 128, torch.float32, True, 1),      # one bias row broadcast over the heads
    (1, 3, 3, 40, 40, 96, 96, torch.bfloat16, False, 3),      # D = 96 (12 units per row)
    (2, 4, 2, 50, 70, 20, 3, torch.float32, False, 2),        # D, R not multiples of 8 (padded rows)
    (1, 2, 2, 33, 33, 44, 12, torch.bfloat16, True, 1),       # ragged pass-through part
    (1, 2, 2, 40, 40, 23, 23, torch.float32, False, 2),       # every dim rotated, odd count
]


def _case(seed, B, Hq, Hk, Nq, Nk, D, R, dtype, f3, hb):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Nq, D, generator=g).to(dtype)
    k = torch.randn(B, Hk, Nk, D, generator=g).to(dtype)
    if f3:
        freqs = torch.stack([orc.pope_freqs(Nk, orc.inv_freqs(R), offset=3 * b) for b in range(B)])
    else:
        freqs = orc.pope_freqs(Nk, orc.inv_freqs(R))
    bias = torch.rand(hb, R, generator=g) * (-2 * math.pi)
    return q, k, freqs, bias


def _err(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return (a - b).abs().max().item(), b.abs().max().item()


@pytest.mark.parametrize("cfg", CASES, ids=lambda c: "x".join(str(v) for v in c[:7]) + f"-{str(c[7])[6:]}-{'f3' if c[8] else 'f2'}")
def test_polar_forward_backward(cuda, cfg):
    import pope_amd
    from pope_amd import _lib
    B, Hq, Hk, Nq, Nk, D, R, dtype, f3, hb = cfg
    q, k, freqs, bias = _case(11, *cfg)
    half = dtype != torch.float32
    # oracle on the same (rounded) inputs, in the inputs' dtype like the reference's torch ops
    t_ref = [x.clone().requires_grad_(True) for x in (q, k, freqs, bias)]
    qh_ref, kh_ref = orc.apply_pope_to_qk(t_ref[2], t_ref[3], t_ref[0], t_ref[1])
    g = torch.Generator().manual_seed(12)
    gq = torch.randn(qh_ref.shape, generator=g)
    gk = torch.randn(kh_ref.shape, generator=g)
    ((qh_ref.float() * gq).sum() + (kh_ref.float() * gk).sum()).backward()

    t = [x.clone().cuda().requires_grad_(True) for x in (q, k, freqs, bias)]
    _lib.profile_reset()
    _lib.profile_enable(True)
    qh, kh = pope_amd.apply_pope_to_qk(pope_amd.PolarEmbedReturn(t[2], t[3]), t[0], t[1])
    ((qh * gq.cuda()).sum() + (kh * gk.cuda()).sum()).backward()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    ran = _lib.profile_read()
    assert "polar_fwd" in ran and "polar_bwd" in ran, ran     # the HIP kernels, not the torch ops
    assert qh.dtype == torch.float32 and qh.shape == qh_ref.shape and kh.shape == kh_ref.shape

    for name, a, r in (("q_hat", qh, qh_ref), ("k_hat", kh, kh_ref), ("dq", t[0].grad, t_ref[0].grad),
                       ("dk", t[1].grad, t_ref[1].grad)):
        e, m = _err(a, r)
        tol = 2e-2 * max(1.0, m) if half else 1e-5 * m
        print(f"{name}: err {e:.3e} (max {m:.3e})")
        assert e <= tol, f"{name}: {e:.3e} > {tol:.3e}"
    for name, a, r in (("dfreqs", t[2].grad, t_ref[2].grad), ("dbias", t[3].grad, t_ref[3].grad)):
        e, m = _err(a, r)
        tol = 2e-2 * max(1.0, m) if half else 1e-4 * m
        print(f"{name}: err {e:.3e} (max {m:.3e})")
        assert e <= tol, f"{name}: {e:.3e} > {tol:.3e}"


@pytest.mark.parametrize("cfg", [(1, 2, 2, 16, 16, 32, 16, False), (2, 4, 2, 40, 72, 64, 64, True),
                                 (1, 2, 2, 24, 24, 20, 3, False)],
                         ids=["partial", "full-f3", "odd-dims"])
def test_polar_complex_output(cuda, cfg):
    """return_complex=True on the kernels: complex64 rows of (a cos, a sin) pairs with pass-through
    dims as (x, 0) (pope.py:49-51,66-67,74-75), forward and backward vs the oracle's torch.polar."""
    import pope_amd
    from pope_amd import _lib
    B, Hq, Hk, Nq, Nk, D, R, f3 = cfg
    q, k, freqs, bias = _case(3, B, Hq, Hk, Nq, Nk, D, R, torch.float32, f3, Hk)
    t_ref = [x.clone().requires_grad_(True) for x in (q, k, freqs, bias)]
    qr, kr = orc.apply_pope_to_qk(t_ref[2], t_ref[3], t_ref[0], t_ref[1], return_complex=True)
    g = torch.Generator().manual_seed(5)
    gq = torch.randn(*qr.shape, 2, generator=g)
    gk = torch.randn(*kr.shape, 2, generator=g)
    ((torch.view_as_real(qr) * gq).sum() + (torch.view_as_real(kr) * gk).sum()).backward()

    t = [x.clone().cuda().requires_grad_(True) for x in (q, k, freqs, bias)]
    _lib.profile_reset()
    _lib.profile_enable(True)
    qc, kc = pope_amd.apply_pope_to_qk(pope_amd.PolarEmbedReturn(t[2], t[3]), t[0], t[1], return_complex=True)
    ((torch.view_as_real(qc) * gq.cuda()).sum() + (torch.view_as_real(kc) * gk.cuda()).sum()).backward()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    ran = _lib.profile_read()
    assert "polar_fwd" in ran and "polar_bwd" in ran, ran
    assert qc.dtype == torch.complex64 and qc.shape == qr.shape and kc.shape == kr.shape
    for name, a, r, rel in (("q_hat", torch.view_as_real(qc), torch.view_as_real(qr), 1e-5),
                            ("k_hat", torch.view_as_real(kc), torch.view_as_real(kr), 1e-5),
                            ("dq", t[0].grad, t_ref[0].grad, 1e-5), ("dk", t[1].grad, t_ref[1].grad, 1e-5),
                            ("dfreqs", t[2].grad, t_ref[2].grad, 1e-4), ("dbias", t[3].grad, t_ref[3].grad, 1e-4)):
        e, m = _err(a, r)
        print(f"{name}: err {e:.3e} (max {m:.3e})")
        assert e <= rel * m, f"{name}: {e:.3e} > {rel * m:.3e}"
    if R < D:   # pass-through dims: (x, 0)
        assert torch.equal(qc[..., R:].real.cpu(), q[..., R:]) and torch.all(qc[..., R:].imag == 0)


def test_polar_other_calls_keep_torch_ops(cuda):
    """Custom magnitudes and half-precision complex outputs are outside the kernels: the torch ops
    answer (a bf16 magnitude with fp32 phases is the reference's torch.polar error, pope.py:67)."""
    import pope_amd
    import torch.nn.functional as F
    q, k, freqs, bias = _case(3, 1, 2, 2, 16, 16, 32, 16, torch.float32, False, 2)
    pos = pope_amd.PolarEmbedReturn(freqs.cuda(), bias.cuda())
    qe, _ = pope_amd.apply_pope_to_qk(pos, q.cuda(), k.cuda(), to_magnitude=F.relu)
    assert qe.shape == (1, 2, 16, 48)
    a = torch.relu(q[..., :16]).cuda()
    torch.testing.assert_close(qe[..., 0:32:2], a * freqs[-16:].cuda().cos())
    with pytest.raises(RuntimeError):
        pope_amd.apply_pope_to_qk(pos, q.cuda().bfloat16(), k.cuda().bfloat16(), return_complex=True)
