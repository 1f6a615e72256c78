"""Shared helpers of the GPU parity tests: seeded inputs and oracle references."""
import math

import torch

from oracle import pope_oracle as orc


def make_pope_inputs(seed, B, Hq, Hk, Nq, Nk, D, R, dtype, mask_kind="none", device="cuda",
                     random_bias=True):
    """Seeded q, k, v, dO (head-first), PoPE freqs/bias (fp32) and a key-padding mask.

    Inputs are drawn in fp32 on the CPU, then cast to ``dtype``; the oracle later
    reads the SAME rounded values upcast to fp32/fp64."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Nq, D, generator=g)
    k = torch.randn(B, Hk, Nk, D, generator=g)
    v = torch.randn(B, Hk, Nk, D, generator=g)
    do = torch.randn(B, Hq, Nq, D, generator=g)
    freqs = orc.pope_freqs(Nk, orc.inv_freqs(R)) if R > 0 else torch.empty(Nk, 0)
    if random_bias and R > 0:
        bias = torch.rand(Hk, R, generator=g) * (-2 * math.pi)
    else:
        bias = torch.zeros(Hk, R)
    mask = None
    if mask_kind == "prefix":        # last 0..Nk/4 keys masked per batch
        mask = torch.ones(B, Nk, dtype=torch.bool)
        for b in range(B):
            p = int(torch.randint(0, Nk // 4 + 1, (1,), generator=g))
            if p:
                mask[b, Nk - p:] = False
    elif mask_kind == "half":        # reference test_flash_attn.py:35-36
        mask = torch.ones(B, Nk, dtype=torch.bool)
        mask[:, Nk // 2:] = False
    elif mask_kind == "random":
        mask = torch.rand(B, Nk, generator=g) > 0.3
    elif mask_kind == "dead_row":    # batch 0 has every key masked
        mask = torch.ones(B, Nk, dtype=torch.bool)
        mask[0] = False
    cast = lambda t: t.to(dtype).to(device)
    out = dict(q=cast(q), k=cast(k), v=cast(v), do=cast(do), freqs=freqs.to(device), bias=bias.to(device),
               mask=None if mask is None else mask.to(device))
    return out


def oracle_attention(inp, causal, scale=None, dtype=torch.float64, grads=True):
    """O (and grads of sum(O * dO)) from the CPU oracle on the kernel's exact inputs."""
    up = lambda t: t.detach().to("cpu", dtype).requires_grad_(grads)
    q, k, v = up(inp["q"]), up(inp["k"]), up(inp["v"])
    freqs, bias = up(inp["freqs"]), up(inp["bias"])
    mask = None if inp["mask"] is None else inp["mask"].cpu()
    R = freqs.shape[-1]
    o = orc.flash_nonfused(q, k, v, freqs if R else None, bias if R else None, mask=mask, causal=causal,
                           softmax_scale=scale)
    lse = orc.flash_lse(q, k, freqs if R else None, bias if R else None, mask=mask, causal=causal,
                        softmax_scale=scale).detach()
    res = dict(o=o.detach(), lse=lse)
    if grads:
        (o * inp["do"].detach().to("cpu", dtype)).sum().backward()
        res.update(dq=q.grad, dk=k.grad, dv=v.grad, dfreqs=freqs.grad, dbias=bias.grad)
    return res


def max_abs(a, b):
    return (a.detach().float().cpu() - b.detach().float().cpu()).abs().max().item()


def excess_over(got, ref, atol):
    """Largest |got - ref| - (atol + half an ulp of ref in got's dtype), elementwise; <= 0 means
    every element is within atol of the exact value beyond the rounding of got's own format (a
    bf16 output cannot be closer than half an ulp: 1.6e-2 at |x| in [4, 8), 3.1e-2 in [8, 16))."""
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    if got.dtype in (torch.bfloat16, torch.float16):
        mant = 7 if got.dtype == torch.bfloat16 else 10
        e = torch.floor(torch.log2(r.abs().clamp_min(1e-30)))
        half_ulp = torch.pow(2.0, e - mant - 1)
    else:
        half_ulp = torch.zeros_like(r)
    return ((g - r).abs() - (atol + half_ulp)).max().item()
