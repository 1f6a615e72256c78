"""Device padding of head / rotate dims that are not multiples of 8 (pope_amd._pad), on the CPU.

The padded problem must have the same scores, outputs and gradients as the unpadded one.  Both
sides run the float64 oracle (pope.py:30-86, attention.py:30-47,106-145 restated), so the check
pins the padding itself: a pad value whose softplus is not exactly 0, a pass-through dim moved to
the wrong column, a value column not zeroed or a softmax scale re-derived from the padded width
each changes the result (the planted variants below show that the comparison sees them).
"""
import math

import pytest
import torch

from oracle import pope_oracle as orc
from pope_amd._pad import PAD_LOGIT, pad_last, pad_plan, pad_qk, unpad_qk

CASES = [   # (D, R): odd rotate dim, rotate dim with a ragged pass-through part, no rotation, all rotated
    (20, 3), (44, 12), (12, 0), (40, 36), (23, 23), (100, 28),
]


def _inputs(D, R, seed=0, B=2, Hq=4, Hk=2, Nq=5, Nk=9):
    g = torch.Generator().manual_seed(seed)
    t = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    q, k, v, do = t(B, Hq, Nq, D), t(B, Hk, Nk, D), t(B, Hk, Nk, D), t(B, Hq, Nq, D)
    freqs = t(Nk, R) * 3.0
    bias = t(Hk, R)
    mask = torch.rand(B, Nk, generator=g) > 0.3
    mask[:, 0] = True
    return q, k, v, do, freqs, bias, mask


def _attn(q, k, v, freqs, bias, mask, causal, scale):
    R = freqs.shape[-1]
    return orc.flash_nonfused(q, k, v, freqs if R else None, bias if R else None, mask=mask, causal=causal,
                              softmax_scale=scale)


def _grads(f, tensors):
    ts = [x.detach().clone().requires_grad_(True) for x in tensors]
    out = f(*ts)
    return out, ts


@pytest.mark.parametrize("D,R", CASES)
@pytest.mark.parametrize("causal", [False, True])
def test_padding_preserves_attention(D, R, causal):
    q, k, v, do, freqs, bias, mask = _inputs(D, R)
    p = pad_plan(D, R)
    assert p is not None and p.Dp % 8 == 0 and p.R8 % 8 == 0 and p.Dp - p.R8 >= D - R
    scale = D ** -0.5

    def plain(q, k, v, f, b):
        return _attn(q, k, v, f, b, mask, causal, scale)

    def padded(q, k, v, f, b):
        o = _attn(pad_qk(q, p), pad_qk(k, p), pad_last(v, p.Dp), pad_last(f, p.R8), pad_last(b, p.R8), mask,
                  causal, scale)
        return o[..., :D]

    o_ref, t_ref = _grads(plain, (q, k, v, freqs, bias))
    o_pad, t_pad = _grads(padded, (q, k, v, freqs, bias))
    assert (o_pad - o_ref).abs().max().item() < 1e-12
    (o_ref * do).sum().backward()
    (o_pad * do).sum().backward()
    for a, b, n in zip(t_pad, t_ref, ("dq", "dk", "dv", "dfreqs", "dbias")):
        if b.grad is None or not b.numel():
            continue
        assert (a.grad - b.grad).abs().max().item() < 1e-12, n


@pytest.mark.parametrize("D,R", CASES)
def test_padding_preserves_similarity(D, R):
    q, k, _, _, freqs, bias, _ = _inputs(D, R, seed=1, Nq=9)
    p = pad_plan(D, R)
    G = torch.randn(2, 4, 9, 9, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    S_ref, t_ref = _grads(lambda q, k, f, b: orc.sim_nonfused(q, k, f, b), (q, k, freqs, bias))
    S_pad, t_pad = _grads(lambda q, k, f, b: orc.sim_nonfused(pad_qk(q, p), pad_qk(k, p), pad_last(f, p.R8),
                                                              pad_last(b, p.R8)), (q, k, freqs, bias))
    assert (S_pad - S_ref).abs().max().item() < 1e-12
    (S_ref * G).sum().backward()
    (S_pad * G).sum().backward()
    for a, b in zip(t_pad, t_ref):
        if b.numel():
            assert (a.grad - b.grad).abs().max().item() < 1e-12


def test_pad_layout_round_trip():
    p = pad_plan(20, 3)
    assert p == (20, 3, 8, 32)
    x = torch.randn(3, 20, dtype=torch.float64)
    xp = pad_qk(x, p)
    assert torch.equal(xp[:, :3], x[:, :3])
    assert torch.all(xp[:, 3:8] == PAD_LOGIT)
    assert torch.equal(xp[:, 8:25], x[:, 3:])
    assert torch.all(xp[:, 25:] == 0)
    assert torch.equal(unpad_qk(xp, p), x)
    assert pad_plan(64, 32) is None and pad_plan(64, 0) is None


def test_padding_mistakes_are_seen():
    """Planted variants of the padding change the result: a zero rotated pad (softplus(0) = ln 2
    adds ln(2)^2 per pad dim to every score -- a constant per row, which the softmax hides but the
    similarity and the log-sum-exp show) and the softmax scale taken from the padded width."""
    D, R = 20, 3
    q, k, v, _, freqs, bias, mask = _inputs(D, R)
    p = pad_plan(D, R)

    def zero_pad(x):
        z = lambda n: torch.zeros(*x.shape[:-1], n, dtype=x.dtype)
        return torch.cat([x[..., :R], z(p.R8 - R), x[..., R:], z(p.Dp - p.R8 - (D - R))], -1)

    f8, b8 = pad_last(freqs, p.R8), pad_last(bias, p.R8)
    S_ref = orc.sim_nonfused(q, k, freqs, bias)
    S_good = orc.sim_nonfused(pad_qk(q, p), pad_qk(k, p), f8, b8)
    S_zero = orc.sim_nonfused(zero_pad(q), zero_pad(k), f8, b8)
    assert (S_good - S_ref).abs().max().item() < 1e-12
    assert (S_zero - S_ref).abs().min().item() > 0.9 * (p.R8 - R) * math.log(2) ** 2
    lse_ref = orc.flash_lse(q, k, freqs, bias, mask=mask, softmax_scale=D ** -0.5)
    lse_zero = orc.flash_lse(zero_pad(q), zero_pad(k), f8, b8, mask=mask, softmax_scale=D ** -0.5)
    assert (lse_zero - lse_ref).abs().min().item() > 1e-3
    ref = _attn(q, k, v, freqs, bias, mask, False, D ** -0.5)
    wrong_scale = _attn(pad_qk(q, p), pad_qk(k, p), pad_last(v, p.Dp), f8, b8, mask, False,
                        p.Dp ** -0.5)[..., :D]
    assert (wrong_scale - ref).abs().max().item() > 1e-3
    assert float(orc.softplus(torch.tensor(PAD_LOGIT, dtype=torch.float32))) == 0.0
