"""Seeded random shapes through the public API on the GPU against the float64 oracle.

Each case draws its shape from its own seeded generator, so the case list and every input are fixed; the case id
names the shape.  Flash forward + backward: batch 1-2, up to 8 query heads over 1, 2 or 4 kv heads, Nq <= Nk up
to 700, head dims 8-136 and 160 / 192, plus 32 cases with head dims 137-256 and up to 400 keys (head dims above
128 run the wide-head kernels), rotate dims 0..D whether or not multiples of 8, bf16 and fp16, causal or not, no / prefix / random / half masks, both layouts, 2-D or per-batch 3-D freqs.  Decode:
up to 32 query heads, 1,024-6,000 keys, views into a longer KV cache, per-batch positions.  Similarity (both
product paths) and the polar transform: ragged sizes, grouped heads, odd dims.

Tolerances, as in the other GPU tests: flash and decode 2e-2 absolute beyond the rounding of the exact value to
the output format (gpu_common.excess_over) for O, dq, dk, dv and 2e-2 * max(1, ||ref||_inf) for the summed dbias /
dfreqs; the fp32 similarity 1e-4 relative to ||ref||_inf; the fp32 polar transform 1e-5 + 2^-23 max|F + beta|
relative (one ulp of the largest fp32 phase on top) for outputs, dq, dk and 1e-4 for dfreqs / dbias.  The shapes stay where bf16 operand rounding keeps within the bf16 bound: head
dims of at least 8 (a softmax scale of at most 0.35; at D = 1 the logits reach 12 and rounding q_hat / k_hat to bf16
alone moves them by 0.03), and at most 8 * 700 query rows summed into one dk element.
"""
import math
import random

import pytest
import torch

from gpu_common import excess_over, make_pope_inputs, max_abs, oracle_attention
from oracle import pope_oracle as orc

pytestmark = pytest.mark.gpu

TOL = 2e-2
SUMMED = ("dfreqs", "dbias")


def _rot(rng, D):
    kind = rng.random()
    if kind < 0.1:
        return 0
    if kind < 0.35:
        return D
    if kind < 0.7 and D >= 8:
        return rng.randrange(8, D + 1, 8)
    return rng.randrange(1, D + 1)


def _flash_case(i):
    rng = random.Random(7100 + i)
    Hk = rng.choice([1, 2, 4])
    Hq = Hk * rng.choice([1, 1, 2, 4] if Hk < 4 else [1, 2])
    B = rng.choice([1, 2])
    Nk = rng.randint(1, 700)
    Nq = Nk if rng.random() < 0.5 else rng.randint(1, Nk)
    D = rng.choice([rng.randint(8, 136), rng.choice([64, 96, 128, 160, 192])])
    return dict(seed=7100 + i, B=B, Hq=Hq, Hk=Hk, Nq=Nq, Nk=Nk, D=D, R=_rot(rng, D),
                dtype=rng.choice([torch.bfloat16, torch.float16]), causal=rng.random() < 0.5,
                mask=rng.choice(["none", "prefix", "random", "half"]), head_first=rng.random() < 0.6,
                per_batch=rng.random() < 0.3)


def _wide_case(i):
    """Heads of 137 to 256 (the wide flash kernels), with the same draws otherwise."""
    rng = random.Random(7900 + i)
    Hk = rng.choice([1, 2])
    Hq = Hk * rng.choice([1, 2, 4])
    Nk = rng.randint(1, 400)
    Nq = Nk if rng.random() < 0.5 else rng.randint(1, Nk)
    D = rng.randint(137, 256)
    return dict(seed=7900 + i, B=rng.choice([1, 2]), Hq=Hq, Hk=Hk, Nq=Nq, Nk=Nk, D=D, R=_rot(rng, D),
                dtype=rng.choice([torch.bfloat16, torch.float16]), causal=rng.random() < 0.5,
                mask=rng.choice(["none", "prefix", "random", "half"]), head_first=rng.random() < 0.6,
                per_batch=rng.random() < 0.3)


def _decode_case(i):
    rng = random.Random(7300 + i)
    Hk = rng.choice([1, 2, 4, 8])
    D = rng.choice([rng.randint(8, 128), 64, 128])
    return dict(seed=7300 + i, B=rng.choice([1, 2, 4]), Hk=Hk, Hq=Hk * rng.choice([1, 2, 4]),
                Nk=rng.randint(1024, 6000), D=D, R=_rot(rng, D), dtype=rng.choice([torch.bfloat16, torch.float16]),
                mask=rng.choice(["none", "prefix", "random"]), sliced=rng.random() < 0.5,
                per_batch=rng.random() < 0.3)


def _sim_case(i):
    rng = random.Random(7500 + i)
    Hk = rng.choice([1, 2])
    Nk = rng.randint(2, 400)
    D = rng.choice([32, 48, 64, 128, 256])
    return dict(seed=7500 + i, B=rng.choice([1, 2]), Hk=Hk, Hq=Hk * rng.choice([1, 2]), Nq=rng.randint(1, Nk), Nk=Nk,
                D=D, R=rng.choice([D, rng.randrange(8, D + 1, 8), rng.randrange(1, D + 1)]),
                allow_tf32=rng.random() < 0.5)


def _polar_case(i):
    rng = random.Random(7700 + i)
    Hk = rng.choice([1, 2, 3])
    Nk = rng.randint(1, 300)
    D = rng.randint(1, 192)
    return dict(seed=7700 + i, B=rng.choice([1, 2]), Hk=Hk, Hq=Hk * rng.choice([1, 2]), Nq=rng.randint(1, Nk), Nk=Nk,
                D=D, R=rng.randint(1, D), per_batch=rng.random() < 0.4, bias_rows=rng.choice([1, Hk]))


def _cid(c):
    return "-".join(f"{k}{str(v).replace('torch.', '')}" for k, v in c.items() if k != "seed")


FLASH = [_flash_case(i) for i in range(200)] + [_wide_case(i) for i in range(32)]
DECODE = [_decode_case(i) for i in range(64)]
SIM = [_sim_case(i) for i in range(64)]
POLAR = [_polar_case(i) for i in range(64)]


def _batch_freqs(B, N, R, seed):
    """(B, N, R) phase table from per-batch positions with uneven gaps and per-batch starts."""
    steps = torch.randint(1, 4, (B, N), generator=torch.Generator().manual_seed(seed)).float()
    pos = steps.cumsum(-1) + 100.0 * torch.arange(B).float()[:, None]
    return torch.stack([orc.pope_freqs(pos[b], orc.inv_freqs(R)) for b in range(B)])


def _bounded(got, ref, names):
    for n in names:
        if got.get(n) is None or ref.get(n) is None:
            continue
        if n in SUMMED:
            ex = max_abs(got[n], ref[n]) - TOL * max(1.0, ref[n].abs().max().item())
        else:
            ex = excess_over(got[n], ref[n], TOL)
        print(f"{n} excess {ex:.1e}", end="  ")
        assert ex <= 0, f"{n}: {ex:.3e} beyond the bound"
    print()


@pytest.mark.parametrize("c", FLASH, ids=_cid)
def test_random_flash(cuda, c):
    import pope_amd
    R = c["R"]
    inp = make_pope_inputs(c["seed"], c["B"], c["Hq"], c["Hk"], c["Nq"], c["Nk"], c["D"], R, c["dtype"], c["mask"])
    if R and c["per_batch"]:
        inp["freqs"] = _batch_freqs(c["B"], c["Nk"], R, c["seed"]).cuda()
    q, k, v = (inp[n].detach().clone().requires_grad_(True) for n in ("q", "k", "v"))
    freqs = inp["freqs"].detach().clone().requires_grad_(R > 0)
    bias = inp["bias"].detach().clone().requires_grad_(R > 0)
    pos = (freqs, bias) if R else None
    if c["head_first"]:
        o = pope_amd.flash_attn_with_pope(q, k, v, pos_emb=pos, mask=inp["mask"], causal=c["causal"])
        o.backward(inp["do"])
        got = dict(o=o, dq=q.grad, dk=k.grad, dv=v.grad)
    else:
        tr = lambda t: t.transpose(1, 2).contiguous().detach().requires_grad_(True)
        qb, kb, vb = tr(q), tr(k), tr(v)
        o = pope_amd.flash_attn_with_pope(qb, kb, vb, pos_emb=pos, mask=inp["mask"], causal=c["causal"],
                                          head_dimension_at_first=False)
        o.backward(inp["do"].transpose(1, 2))
        back = lambda t: t.transpose(1, 2)
        got = dict(o=back(o), dq=back(qb.grad), dk=back(kb.grad), dv=back(vb.grad))
    if R:
        got.update(dfreqs=freqs.grad, dbias=bias.grad)
    ref = oracle_attention(inp, c["causal"])
    _bounded(got, ref, ("o", "dq", "dk", "dv", "dfreqs", "dbias"))


@pytest.mark.parametrize("c", DECODE, ids=_cid)
def test_random_decode(cuda, c):
    import pope_amd
    R, D, Nk = c["R"], c["D"], c["Nk"]
    inp = make_pope_inputs(c["seed"], c["B"], c["Hq"], c["Hk"], 1, Nk, D, R, c["dtype"], c["mask"])
    if R and c["per_batch"]:
        inp["freqs"] = _batch_freqs(c["B"], Nk, R, c["seed"]).cuda()
    k, v = inp["k"], inp["v"]
    if c["sliced"]:   # views into a cache longer than the valid rows
        cap = Nk + 1 + c["seed"] % 500
        kc = torch.zeros(c["B"], c["Hk"], cap, D, dtype=c["dtype"], device="cuda")
        vc = torch.zeros_like(kc)
        kc[:, :, :Nk], vc[:, :, :Nk] = k, v
        k, v = kc[:, :, :Nk], vc[:, :, :Nk]
    with torch.no_grad():
        o = pope_amd.flash_attn_with_pope(inp["q"], k, v, pos_emb=(inp["freqs"], inp["bias"]) if R else None,
                                          mask=inp["mask"])
    _bounded(dict(o=o), oracle_attention(inp, False, grads=False), ("o",))


@pytest.mark.parametrize("c", SIM, ids=_cid)
def test_random_similarity(cuda, c):
    import pope_amd
    B, Hq, Hk, Nq, Nk, D, R = (c[n] for n in ("B", "Hq", "Hk", "Nq", "Nk", "D", "R"))
    g = torch.Generator().manual_seed(c["seed"])
    q, k = torch.randn(B, Hq, Nq, D, generator=g), torch.randn(B, Hk, Nk, D, generator=g)
    G = torch.randn(B, Hq, Nq, Nk, generator=g)
    freqs = orc.pope_freqs(Nk, orc.inv_freqs(R))
    bias = torch.rand(Hk, R, generator=g) * (-2 * math.pi)
    t = [x.cuda().requires_grad_(True) for x in (q, k, freqs, bias)]
    S = pope_amd.compute_attn_similarity(t[0], t[1], (t[2], t[3]), allow_tf32=c["allow_tf32"])
    S.backward(G.cuda())
    r = [x.double().requires_grad_(True) for x in (q, k, freqs, bias)]
    S_ref = orc.sim_nonfused(*r)
    S_ref.backward(G.double())
    for n, a, b in zip(("S", "dq", "dk", "dfreqs", "dbias"), [S] + [x.grad for x in t], [S_ref] + [x.grad for x in r]):
        rel = max_abs(a, b) / b.abs().max().item()
        print(f"{n}={rel:.1e}", end=" ")
        assert rel <= 1e-4, (n, rel)
    print()


@pytest.mark.parametrize("c", POLAR, ids=_cid)
def test_random_polar(cuda, c):
    import pope_amd
    B, Hq, Hk, Nq, Nk, D, R = (c[n] for n in ("B", "Hq", "Hk", "Nq", "Nk", "D", "R"))
    g = torch.Generator().manual_seed(c["seed"])
    q, k = torch.randn(B, Hq, Nq, D, generator=g), torch.randn(B, Hk, Nk, D, generator=g)
    freqs = (torch.stack([orc.pope_freqs(Nk, orc.inv_freqs(R), offset=5 * b) for b in range(B)]) if c["per_batch"]
             else orc.pope_freqs(Nk, orc.inv_freqs(R)))
    bias = torch.rand(c["bias_rows"], R, generator=g) * (-2 * math.pi)
    t = [x.cuda().requires_grad_(True) for x in (q, k, freqs, bias)]
    qh, kh = pope_amd.apply_pope_to_qk(pope_amd.PolarEmbedReturn(t[2], t[3]), t[0], t[1])
    gq, gk = torch.randn(qh.shape, generator=g), torch.randn(kh.shape, generator=g)
    ((qh * gq.cuda()).sum() + (kh * gk.cuda()).sum()).backward()
    r = [x.double().requires_grad_(True) for x in (q, k, freqs, bias)]
    qr, kr = orc.apply_pope_to_qk(r[2], r[3], r[0], r[1])
    ((qr * gq.double()).sum() + (kr * gk.double()).sum()).backward()
    # a key phase F + beta is rounded to fp32 before its cos / sin, as the reference's own fp32 `freqs + bias`
    # (pope.py:56) is: up to one ulp of itself (2^-23 |F + beta|), which the float64 oracle does not have, so the
    # key-side bound grows with the largest key phase.  Query phases are the fp32 table entries themselves
    # (pope.py:64), with no rounded sum: their bound stays 1e-5
    ph = 1e-5 + 2.0 ** -23 * (freqs.abs().max().item() + bias.abs().max().item())
    for n, a, b, tol in (("q_hat", qh, qr, 1e-5), ("k_hat", kh, kr, ph), ("dq", t[0].grad, r[0].grad, 1e-5),
                         ("dk", t[1].grad, r[1].grad, ph), ("dfreqs", t[2].grad, r[2].grad, 1e-4),
                         ("dbias", t[3].grad, r[3].grad, 1e-4)):
        rel = max_abs(a, b) / max(1e-30, b.abs().max().item())
        print(f"{n}={rel:.1e}", end=" ")
        assert rel <= tol, (n, rel)
    print()
