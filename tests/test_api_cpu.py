"""The public API on CPU tensors against the oracle -- CPU only.

pope_amd's modules and its torch path (the branch CPU tensors and ``fused=False`` take,
attention.py:30-47,106-145 of the reference) are compared with the pinned oracle in float64:
  * ``PoPE`` / ``AxialPoPE``: frequencies, clamped bias and ``state_dict`` keys, and a checkpoint
    written with the reference's key names loads unchanged (pope.py:106-113, pope_nd.py:48-56);
  * ``apply_pope_to_qk`` (real and complex outputs), ``compute_attn_similarity`` and its non-fused
    form, ``flash_attn_with_pope(fused=False)`` and its CPU default, with grouped heads, masks,
    causal and both layouts, forward and gradients;
  * the shape cases of the reference's own CPU tests (tests/test_pope.py:6-53,
    tests/test_readme.py:5-54).
"""
import math

import pytest
import torch

import pope_amd
from oracle import pope_oracle as orc


def _close(a, b, tol=1e-10):
    torch.testing.assert_close(a, b, rtol=tol, atol=tol)


# ---- modules ------------------------------------------------------------------------------------

def test_pope_module_matches_closed_form():
    m = pope_amd.PoPE(32, heads=8)
    assert sorted(m.state_dict()) == ["bias", "inv_freqs"]          # reference pope.py:109,113
    assert m.bias.shape == (8, 32) and not m.inv_freqs.requires_grad
    torch.testing.assert_close(m.inv_freqs, orc.inv_freqs(32), rtol=0, atol=0)
    with torch.no_grad():
        m.bias.uniform_(-10.0, 3.0)
    freqs, bias = m(1024)
    torch.testing.assert_close(freqs, orc.pope_freqs(1024, orc.inv_freqs(32)), rtol=0, atol=0)
    torch.testing.assert_close(bias, orc.clamp_bias(m.bias), rtol=0, atol=0)
    # offset and tensor positions (batched positions give 3-D freqs, pope.py:131-141)
    torch.testing.assert_close(m(1000, offset=24).freqs, freqs[24:], rtol=0, atol=0)
    pos = torch.stack([torch.arange(16).float(), torch.arange(16).float() + 5])
    f3 = m(pos).freqs
    assert f3.shape == (2, 16, 32)
    torch.testing.assert_close(f3, orc.pope_freqs(pos, orc.inv_freqs(32)), rtol=0, atol=0)
    # offsets: an explicit integer 0 (no add), a tensor offset, tensor positions shifted by an integer;
    # the returned freqs never alias the positions passed in
    torch.testing.assert_close(m(1024, offset=0).freqs, freqs, rtol=0, atol=0)
    torch.testing.assert_close(m(1000, offset=torch.tensor(24.0)).freqs, freqs[24:], rtol=0, atol=0)
    torch.testing.assert_close(m(pos, offset=3).freqs, orc.pope_freqs(pos + 3, orc.inv_freqs(32)), rtol=0, atol=0)
    p1 = torch.arange(8).float()
    assert m(p1).freqs.data_ptr() != p1.data_ptr()
    # the bias gradient passes where the clamp is inactive (and at its bounds)
    m.bias.grad = None
    m(8).bias.sum().backward()
    inside = (m.bias >= -2 * math.pi) & (m.bias <= 0)
    assert torch.equal(m.bias.grad, inside.float())


def test_bias_clamp_matches_torch_clamp():
    """The modules' bias clamp (a fused-backward autograd function) against torch's clamp: values and
    gradients at the exact bounds, inside, outside and for NaN, for PoPE and AxialPoPE."""
    vals = torch.tensor([-7.0, -2 * math.pi, -3.0, 0.0, 0.5, float("nan"), -1.0, 2.0])
    g = torch.randn(4, 16, generator=torch.Generator().manual_seed(5))
    for m in (pope_amd.PoPE(16, heads=4), pope_amd.AxialPoPE(16, heads=4, axial_dims=(8, 8))):
        with torch.no_grad():
            m.bias.copy_(vals.repeat(8).view(4, 16))
        ref = m.bias.detach().clone().requires_grad_(True)
        out = m(8).bias if isinstance(m, pope_amd.PoPE) else m((2, 4)).bias
        (out * g).sum().backward()
        want = ref.clamp(-2 * math.pi, 0.0)
        (want * g).sum().backward()
        assert torch.equal(torch.nan_to_num(out.detach(), 9.0), torch.nan_to_num(want.detach(), 9.0))
        assert torch.equal(m.bias.grad, ref.grad)
        # a planted mistake: a gradient blocked at the bounds must differ
        assert not torch.equal(m.bias.grad, g * ((ref > -2 * math.pi) & (ref < 0)))


def test_pope_state_dict_round_trip_and_options():
    src = pope_amd.PoPE(64, heads=4, bias_uniform_init=True)      # the reference raises here
    assert src.bias.min() >= -2 * math.pi and src.bias.max() <= 0 and src.bias.abs().sum() > 0
    dst = pope_amd.PoPE(64, heads=4)
    dst.load_state_dict({"inv_freqs": src.inv_freqs.clone(), "bias": src.bias.detach().clone()})
    torch.testing.assert_close(dst(33).freqs, src(33).freqs, rtol=0, atol=0)
    torch.testing.assert_close(dst(33).bias, src(33).bias, rtol=0, atol=0)
    custom = pope_amd.PoPE(4, heads=1, inv_freqs=[1.0, 0.5, 0.25, 0.125])   # list accepted
    assert custom.inv_freqs.dtype == torch.float32
    torch.testing.assert_close(custom(3).freqs[2], torch.tensor([2.0, 1.0, 0.5, 0.25]))


def test_axial_pope_matches_oracle_and_reference_keys():
    m = pope_amd.AxialPoPE(96, heads=8, axial_dims=(32, 32, 32))
    assert sorted(m.state_dict()) == ["bias", "inv_freqs.0", "inv_freqs.1", "inv_freqs.2"]   # pope_nd.py:48-56
    freqs, bias = m((8, 16, 16))
    assert freqs.shape == (2048, 96)                               # reference test_readme.py:47
    want = orc.axial_freqs(orc.axial_grid_positions(8, 16, 16), orc.axial_inv_freqs((32, 32, 32)))
    torch.testing.assert_close(freqs, want, rtol=0, atol=0)
    torch.testing.assert_close(bias, orc.clamp_bias(m.bias), rtol=0, atol=0)
    m2 = pope_amd.AxialPoPE(64, heads=8, axial_dims=(32, 32))
    assert m2((32, 32)).freqs.shape == (1024, 64)                  # reference test_readme.py:36
    with pytest.raises(AssertionError):
        pope_amd.AxialPoPE(64, heads=8, axial_dims=(32, 16))
    # a checkpoint with the reference's keys loads
    sd = {k: v.clone() for k, v in m.state_dict().items()}
    m3 = pope_amd.AxialPoPE(96, heads=8, axial_dims=(32, 32, 32))
    m3.load_state_dict(sd)
    torch.testing.assert_close(m3((8, 16, 16)).freqs, freqs, rtol=0, atol=0)


# ---- the reference's CPU test shapes --------------------------------------------------------------

@pytest.mark.parametrize("partial", [False, True])
def test_reference_test_pope_shapes(partial):
    pope = pope_amd.PoPE(32 if partial else 64, heads=8)
    pos = pope(1024)
    q, k = torch.randn(1, 8, 1024, 64), torch.randn(1, 8, 1024, 64)
    rq, rk = pope.apply_pope_to_qk(pos, q, k)
    final = 128 if not partial else 96
    assert rq.shape == rk.shape == (1, 8, 1024, final)
    rq, rk = pope.apply_pope_to_qk(pos, q[..., -1:, :], k)
    assert rq.shape == (1, 8, 1, final) and rk.shape == (1, 8, 1024, final)


@pytest.mark.parametrize("partial", [False, True])
@pytest.mark.parametrize("q_len", [1, 1024])
def test_reference_similarity_shapes(partial, q_len):
    pos = pope_amd.PoPE(32 if partial else 64, heads=8)(1024)
    sim = pope_amd.compute_attn_similarity(torch.randn(1, 8, q_len, 64), torch.randn(1, 8, 1024, 64), pos)
    assert sim.shape == (1, 8, q_len, 1024)


def test_reference_readme_usage():
    pope = pope_amd.PoPE(64, heads=8)
    pos_emb = pope(1024)
    q, k = torch.randn(1, 8, 1024, 64), torch.randn(1, 8, 1024, 64)
    rq, rk = pope.apply_pope_to_qk(pos_emb, q, k)
    assert rq.shape == rk.shape == (1, 8, 1024, 128)
    rq, rk = pope.apply_pope_to_qk(pos_emb, q[..., -1:, :], k)
    assert rq.shape == (1, 8, 1, 128) and rk.shape == (1, 8, 1024, 128)
    video = pope_amd.AxialPoPE(dim=96, heads=8, axial_dims=(32, 32, 32))
    pv = video((8, 16, 16))
    rq, _ = pope_amd.AxialPoPE.apply_pope_to_qk(pv, torch.randn(1, 8, 2048, 96), torch.randn(1, 8, 2048, 96))
    assert rq.shape == (1, 8, 2048, 192)


# ---- transform and attention on the torch path vs the oracle ---------------------------------------

def _inputs(seed, B=2, Hq=4, Hk=2, Nq=9, Nk=13, D=16, R=8, three_d=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Nq, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, Hk, Nk, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, Hk, Nk, D, generator=g, dtype=torch.float64)
    if three_d:
        pos = torch.rand(B, Nk, generator=g, dtype=torch.float64) * 50
        freqs = orc.pope_freqs(pos, orc.inv_freqs(R).double())
    else:
        freqs = orc.pope_freqs(Nk, orc.inv_freqs(R).double(), offset=3)
    bias = torch.rand(Hk, R, generator=g, dtype=torch.float64) * -2 * math.pi
    mask = torch.rand(B, Nk, generator=g) > 0.3
    mask[:, 0] = True
    return q, k, v, freqs, bias, mask


@pytest.mark.parametrize("three_d", [False, True])
@pytest.mark.parametrize("return_complex", [False, True])
def test_apply_pope_to_qk_matches_oracle(three_d, return_complex):
    q, k, v, freqs, bias, _ = _inputs(1, three_d=three_d)
    got = pope_amd.apply_pope_to_qk((freqs, bias), q, k, return_complex=return_complex)
    want = orc.apply_pope_to_qk(freqs, bias, q, k, return_complex=return_complex)
    for a, b in zip(got, want):
        assert a.dtype == b.dtype and a.shape == b.shape
        # F.softplus (product) and the oracle's softplus differ in the last bit
        torch.testing.assert_close(a, b, rtol=1e-14, atol=1e-14)


@pytest.mark.parametrize("head_first", [True, False])
def test_similarity_cpu_matches_oracle(head_first):
    q, k, v, freqs, bias, _ = _inputs(2, D=32, R=16)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, freqs, bias)]
    tr = (lambda t: t) if head_first else (lambda t: t.transpose(1, 2))
    sim = pope_amd.compute_attn_similarity(tr(leaves[0]), tr(leaves[1]), (leaves[2], leaves[3]),
                                           head_dimension_at_first=head_first)
    refs = [t.clone().requires_grad_(True) for t in (q, k, freqs, bias)]
    want = orc.sim_nonfused(*refs)
    _close(sim, want)
    G = torch.randn(sim.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(9))
    (sim * G).sum().backward()
    (want * G).sum().backward()
    for a, b in zip(leaves, refs):
        _close(a.grad, b.grad)
    nf = pope_amd.compute_attn_similarity_non_fused(tr(q), tr(k), (freqs, bias), head_dimension_at_first=head_first)
    _close(nf, want.detach())
    with pytest.raises(AssertionError):   # the reference's head-dim assert (attention.py:61)
        pope_amd.compute_attn_similarity(torch.randn(1, 2, 4, 24), torch.randn(1, 2, 4, 24), (freqs[:4, :8], bias[:, :8]))


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("head_first", [True, False])
@pytest.mark.parametrize("three_d", [False, True])
def test_flash_torch_path_matches_oracle(causal, head_first, three_d):
    q, k, v, freqs, bias, mask = _inputs(3, Nq=13, Nk=13, three_d=three_d)
    mask[1, :] = False   # a fully masked batch row -> 0
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v, freqs, bias)]
    tr = (lambda t: t) if head_first else (lambda t: t.transpose(1, 2))
    for fused in (False, None):   # None: the default for CPU tensors is the torch path
        for t in leaves:
            t.grad = None
        o = pope_amd.flash_attn_with_pope(tr(leaves[0]), tr(leaves[1]), tr(leaves[2]), pos_emb=(leaves[3], leaves[4]),
                                          mask=mask, causal=causal, fused=fused, head_dimension_at_first=head_first)
        o = tr(o)
        refs = [t.clone().requires_grad_(True) for t in (q, k, v, freqs, bias)]
        want = orc.flash_nonfused(*refs, mask=mask, causal=causal)
        _close(o, want)
        assert torch.all(o[1] == 0)
        dO = torch.randn(o.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(4))
        (o * dO).sum().backward()
        (want * dO).sum().backward()
        for a, b in zip(leaves, refs):
            _close(a.grad, b.grad)


def test_flash_torch_path_half_precision_casts_like_the_reference():
    """bf16 inputs: softplus in bf16, promotion to fp32 against the fp32 phases, v cast to the
    promoted dtype and the output cast back to v's dtype (attention.py:125-127,140)."""
    q, k, v, freqs, bias, mask = _inputs(5, Nq=8, Nk=8)
    qb, kb, vb = (t.to(torch.bfloat16) for t in (q, k, v))
    o = pope_amd.flash_attn_with_pope(qb, kb, vb, pos_emb=(freqs.float(), bias.float()), mask=mask, causal=True)
    assert o.dtype == torch.bfloat16
    want = orc.flash_nonfused(qb.double(), kb.double(), vb.double(), freqs, bias, mask=mask, causal=True)
    assert (o.double() - want).abs().max().item() < 2e-2


def test_format_aware_bound_helper():
    """gpu_common.excess_over (the GPU tests' bound for bf16 outputs): exact values rounded to bf16
    are within 0 beyond the format's half ulp; a 3e-2 error on values near 1 exceeds 2e-2."""
    from gpu_common import excess_over
    ref = torch.randn(4096, dtype=torch.float64) * 10
    assert excess_over(ref.to(torch.bfloat16), ref, 0.0) <= 0
    small = torch.rand(4096, dtype=torch.float64) * 0.5 + 0.5
    assert excess_over((small + 0.03).to(torch.bfloat16), small, 2e-2) > 0
    assert excess_over(small.float(), small, 0.0) <= 1e-7


def test_flash_host_predicates_use_shapes_not_pointers():
    """The decode choice and the freqs strides the library sees depend on shapes, strides and
    storage offsets only (so the fake implementation decides as the real one does): extents of 1
    broadcast with stride 0, per-head tables and rows that are not whole 16-byte vectors leave the
    decode kernel, and tables whose view starts mid-vector are copied before any kernel sees them."""
    from pope_amd import hip_pope_flash_attn as fa
    B, H, Nk, D, R = 2, 4, 2048, 64, 64
    q, k = torch.zeros(B, H, 1, D), torch.zeros(B, H, Nk, D)
    F = torch.zeros(Nk, R)
    assert fa._freqs_strides(F) == (0, 0, R)
    assert fa._freqs_strides(F[None]) == (0, 0, R)                       # (1, N, R): one table
    assert fa._freqs_strides(torch.zeros(B, 1, Nk, R)) == (Nk * R, 0, R)  # (B, 1, N, R): per batch
    assert fa._freqs_strides(torch.zeros(B, Nk, 1, R), head_first=False) == (Nk * R, 0, R)
    assert fa._decode_eligible(q, k, k, F, False)
    assert fa._decode_eligible(q, k, k, torch.zeros(B, 1, Nk, R), False)
    assert not fa._decode_eligible(q, k, k, torch.zeros(B, H, Nk, R), False)      # per-head table
    assert not fa._decode_eligible(q, k, k, torch.zeros(Nk, R + 2)[:, :R], False)  # rows of 66 floats
    assert not fa._decode_eligible(q, k, k, F, True)
    # a view starting one float into its storage is copied; a whole-vector offset is kept
    flat = torch.zeros(Nk * R + 4)
    odd = flat[1:1 + Nk * R].view(Nk, R)
    even = flat[4:].view(Nk, R)
    bias = torch.zeros(H, R)
    f_odd, _ = fa._prep_pope(odd, bias)
    f_even, _ = fa._prep_pope(even, bias)
    assert f_odd.storage_offset() == 0 and f_odd.data_ptr() != odd.data_ptr()
    assert f_even.data_ptr() == even.data_ptr()
