"""BASELINE.json's GPU configs at their full sizes: the HIP path vs the CPU oracle.

Every config runs once on the GPU through the public API with the config's own seeded inputs
(seeds 1000 + i, drawn in fp32 on the CPU in the order q, k, v, upstream grad, mask lengths,
then cast), and the oracle recomputes it on the CPU in fp32 on the same rounded inputs, one
(batch, pair of heads) at a time; dbias and dfreqs sum the chunks' contributions.

  C2  compute_attn_similarity fwd+bwd, fp32, B2 H8 N2048 D64, PoPE(64, 8), both product
      arithmetics (allow_tf32 True: split-bf16 MFMA, False: fp32 MFMA)
  C3  flash_attn_with_pope fwd+bwd, bf16, causal, B2 H8 N4096 D64, PoPE(32, 8), key-padding
      mask with the last 0..512 keys of each batch masked
  C4  flash_attn_with_pope fwd+bwd, bf16, non-causal, B4 H8 N2048 D96, freqs from
      AxialPoPE(96, heads=8, axial_dims=(32, 32, 32))((8, 16, 16)) -- the multi-axis table
  C5  decode: q (8, 16, 1, 64) against a 32768-key bf16 cache, PoPE(64, 16), valid lengths
      U{4096..32768}; forward (the split-K decode kernel) and the backward through its LSE

Tolerances, written per check below:
  * fp32 similarity (C2): ||d||_inf <= 1e-4 ||ref||_inf and allclose(rtol=1e-4, atol=1e-4 rms)
    for S, dq, dk, dbias (the reference's fl(freqs + bias) rounding reproduced: oracle in fp32);
  * bf16 flash (C3, C4, C5): 2e-2 absolute for o, dq, dk, dv; 2e-2 * max(1, ||ref||_inf) for
    the summed parameter gradients dbias and dfreqs (sums over all keys of bf16-rounded
    products, whose error grows with the number of terms);
  * lse (C5): 2e-2 absolute on finite rows, -inf exactly where every key is masked.
"""
import math

import pytest
import torch

from oracle import pope_oracle as orc

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _flash_inputs(seed, B, H, N, D, max_pad=0, Nq=None):
    """q, k, v, dO iid N(0, 1) in that order, then the mask pad lengths U{0..max_pad}."""
    Nq = N if Nq is None else Nq
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Nq, D, generator=g)
    k = torch.randn(B, H, N, D, generator=g)
    v = torch.randn(B, H, N, D, generator=g)
    do = torch.randn(B, H, Nq, D, generator=g)
    mask = None
    if max_pad:
        pads = torch.randint(0, max_pad + 1, (B,), generator=g)
        mask = torch.ones(B, N, dtype=torch.bool)
        for b in range(B):
            if pads[b] > 0:
                mask[b, N - int(pads[b]):] = False
    bf = lambda t: t.to(torch.bfloat16)
    return bf(q), bf(k), bf(v), bf(do), mask


def _gpu_flash(q, k, v, do, freqs, bias, mask, causal):
    import pope_amd
    dev = torch.device("cuda")
    leaves = [t.to(dev).requires_grad_(True) for t in (q, k, v, freqs, bias)]
    o = pope_amd.flash_attn_with_pope(leaves[0], leaves[1], leaves[2], pos_emb=(leaves[3], leaves[4]),
                                      mask=None if mask is None else mask.to(dev), causal=causal)
    o.backward(do.to(dev))
    torch.cuda.synchronize()
    return dict(o=o.detach().cpu(), dq=leaves[0].grad.cpu(), dk=leaves[1].grad.cpu(), dv=leaves[2].grad.cpu(),
                dfreqs=leaves[3].grad.cpu(), dbias=leaves[4].grad.cpu())


def _oracle_flash_chunked(q, k, v, do, freqs, bias, mask, causal, heads=2):
    """fp32 oracle one (batch, `heads` heads) at a time; returns the GPU result's keys."""
    B, H = q.shape[:2]
    out = dict(o=torch.empty(q.shape), dq=torch.empty(q.shape), dk=torch.empty(k.shape), dv=torch.empty(v.shape),
               dfreqs=torch.zeros(freqs.shape), dbias=torch.zeros(bias.shape), lse=torch.empty(q.shape[:3]))
    for b in range(B):
        for h0 in range(0, H, heads):
            sl = (slice(b, b + 1), slice(h0, h0 + heads))
            t = [x[sl].float().requires_grad_(True) for x in (q, k, v)]
            f = freqs.detach().clone().float().requires_grad_(True)
            bs = bias[h0:h0 + heads].float().requires_grad_(True)
            m = None if mask is None else mask[b:b + 1]
            o = orc.flash_nonfused(t[0], t[1], t[2], f, bs, mask=m, causal=causal)
            (o * do[sl].float()).sum().backward()
            with torch.no_grad():
                out["lse"][sl] = orc.flash_lse(t[0], t[1], f, bs, mask=m, causal=causal)
            out["o"][sl] = o.detach()
            out["dq"][sl], out["dk"][sl], out["dv"][sl] = t[0].grad, t[1].grad, t[2].grad
            out["dfreqs"] += f.grad
            out["dbias"][h0:h0 + heads] += bs.grad
    return out


SUMMED = ("dbias", "dfreqs")


def _check(got, ref, names):
    """Per-element outputs: 2e-2 absolute.  dbias / dfreqs sum bf16-rounded products over every
    key (and batch, and head): their error grows with the number of terms, so their bound is
    2e-2 * max(1, ||ref||_inf) -- 2e-2 absolute at unit scale.  The measured errors print."""
    errs = {n: (got[n].double() - ref[n].double()).abs().max().item() for n in names}
    mags = {n: ref[n].abs().max().item() for n in names}
    print(" ".join(f"{n}={errs[n]:.2e}(|ref| {mags[n]:.1f})" for n in names))
    tol = {n: TOL * max(1.0, mags[n]) if n in SUMMED else TOL for n in names}
    bad = {n: (e, tol[n]) for n, e in errs.items() if not e <= tol[n]}
    assert not bad, f"max-abs errors above their bounds: {bad}"


def test_c3_causal_training_full_size(cuda):
    B, H, N, D, R = 2, 8, 4096, 64, 32
    q, k, v, do, mask = _flash_inputs(1003, B, H, N, D, max_pad=512)
    import pope_amd
    pope = pope_amd.PoPE(R, heads=H)
    with torch.no_grad():   # a non-zero clamped bias exercises the phase bias path
        pope.bias.uniform_(-2 * math.pi, 0.0)
    freqs, bias = (t.detach() for t in pope(N))
    got = _gpu_flash(q, k, v, do, freqs, bias, mask, causal=True)
    ref = _oracle_flash_chunked(q, k, v, do, freqs, bias, mask, causal=True)
    _check(got, ref, ["o", "dq", "dk", "dv", "dbias", "dfreqs"])


def test_c4_axial_full_size(cuda):
    import pope_amd
    B, H, D = 4, 8, 96
    axial = pope_amd.AxialPoPE(96, heads=H, axial_dims=(32, 32, 32))
    with torch.no_grad():
        axial.bias.uniform_(-2 * math.pi, 0.0)
    freqs, bias = (t.detach() for t in axial((8, 16, 16)))
    N = freqs.shape[0]
    assert N == 2048 and freqs.shape[1] == 96
    # the module's multi-axis table is the oracle's closed form
    want = orc.axial_freqs(orc.axial_grid_positions(8, 16, 16), orc.axial_inv_freqs((32, 32, 32)))
    assert torch.equal(freqs, want)
    q, k, v, do, _ = _flash_inputs(1004, B, H, N, D)
    got = _gpu_flash(q, k, v, do, freqs, bias, None, causal=False)
    ref = _oracle_flash_chunked(q, k, v, do, freqs, bias, None, causal=False)
    _check(got, ref, ["o", "dq", "dk", "dv", "dbias", "dfreqs"])


def test_c5_decode_full_size(cuda):
    import pope_amd
    from pope_amd import _lib
    B, H, N, D, R = 8, 16, 32768, 64, 64
    g = torch.Generator().manual_seed(1005)
    q = torch.randn(B, H, 1, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16)
    do = torch.randn(B, H, 1, D, generator=g).to(torch.bfloat16)
    lengths = torch.randint(4096, N + 1, (B,), generator=g)
    mask = torch.arange(N)[None, :] < lengths[:, None]
    pope = pope_amd.PoPE(R, heads=H)
    with torch.no_grad():
        pope.bias.uniform_(-2 * math.pi, 0.0)
    freqs, bias = (t.detach() for t in pope(N))
    dev = torch.device("cuda")
    leaves = [t.to(dev).requires_grad_(True) for t in (q, k, v, bias)]
    _lib.profile_reset()
    _lib.profile_enable(True)
    o = pope_amd.flash_attn_with_pope(leaves[0], leaves[1], leaves[2], pos_emb=(freqs.to(dev), leaves[3]),
                                      mask=mask.to(dev))
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    assert "flash_decode_split" in _lib.profile_read()   # the split-K decode kernel ran
    o.backward(do.to(dev))
    torch.cuda.synchronize()
    got = dict(o=o.detach().cpu(), dq=leaves[0].grad.cpu(), dk=leaves[1].grad.cpu(), dv=leaves[2].grad.cpu(),
               dbias=leaves[3].grad.cpu())
    from pope_amd.hip_pope_flash_attn import flash_attn_forward
    _, lse = flash_attn_forward(*(t.to(dev).transpose(1, 2) for t in (q, k, v)), freqs.to(dev), bias.to(dev),
                                mask.to(dev))
    ref = _oracle_flash_chunked(q, k, v, do, freqs, bias, mask, causal=False, heads=16)
    _check(got, ref, ["o", "dq", "dk", "dv", "dbias"])
    lse = lse.cpu()
    assert torch.isfinite(lse).all()
    assert (lse - ref["lse"]).abs().max().item() <= TOL


RTOL = 1e-4


@pytest.mark.parametrize("allow_tf32", [True, False], ids=["split_bf16", "fp32"])
def test_c2_similarity_full_size(cuda, allow_tf32):
    import pope_amd
    B, H, N, D, R = 2, 8, 2048, 64, 64
    g = torch.Generator().manual_seed(1002)
    q = torch.randn(B, H, N, D, generator=g)
    k = torch.randn(B, H, N, D, generator=g)
    G = torch.randn(B, H, N, N, generator=g)
    pope = pope_amd.PoPE(R, heads=H)
    with torch.no_grad():
        pope.bias.uniform_(-2 * math.pi, 0.0)
    freqs, bias = (t.detach() for t in pope(N))
    dev = torch.device("cuda")
    leaves = [t.to(dev).requires_grad_(True) for t in (q, k, freqs, bias)]
    S = pope_amd.compute_attn_similarity(leaves[0], leaves[1], (leaves[2], leaves[3]), allow_tf32=allow_tf32)
    S.backward(G.to(dev))
    torch.cuda.synchronize()
    got = [S.detach().cpu()] + [t.grad.cpu() for t in leaves]
    refs = [t.clone().requires_grad_(True) for t in (q, k, freqs, bias)]
    S_ref = orc.sim_nonfused(*refs)
    (S_ref * G).sum().backward()
    want = [S_ref.detach()] + [t.grad for t in refs]
    for name, a, r in zip(("S", "dq", "dk", "dfreqs", "dbias"), got, want):
        a, r = a.double(), r.double()
        rel = ((a - r).abs().max() / r.abs().max()).item()
        el = ((a - r).abs() / (RTOL * r.abs() + RTOL * r.pow(2).mean().sqrt())).max().item()
        print(f"{name}: rel-inf {rel:.2e}, elementwise {el:.2f}")
        assert rel <= RTOL, f"{name}: {rel:.3e}"
        assert el <= 1.0, f"{name}: elementwise allclose(rtol=1e-4, atol=1e-4 rms) fails by {el:.2f}x"
