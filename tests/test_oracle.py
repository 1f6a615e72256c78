"""Pins the CPU oracle (oracle/pope_oracle.py) -- CPU only.

Checks, in order: the golden fixtures of tests/golden (independent float64
brute force + finite-difference gradients); closed forms of the frequency
tables and the reversed axial grid; the interleave / pass-through / right
alignment of the materialising transform and the shapes the reference's own
tests assert; invariants of the similarity (translation, global phase shift,
R = 0 reduces to q k^T); and that plausible mistakes planted in a copy of the
oracle are caught by these checks.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import pope_oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "pope_golden.npz")


def _golden_cases():
    z = np.load(GOLDEN)
    n = int(z["ncases"])
    out = []
    for c in range(n):
        d = {k[len(f"c{c}_"):]: z[k] for k in z.files if k.startswith(f"c{c}_")}
        out.append(d)
    return out


CASES = _golden_cases()


def _t(a, grad=False):
    return torch.tensor(a, dtype=torch.float64, requires_grad=grad)


@pytest.mark.parametrize("c", range(len(CASES)))
def test_golden_similarity_and_grads(c):
    g = CASES[c]
    q, k, F, bias = _t(g["q"], True), _t(g["k"], True), _t(g["F"], True), _t(g["bias"], True)
    S = orc.sim_nonfused(q, k, F, bias)
    np.testing.assert_allclose(S.detach().numpy(), g["S"], rtol=1e-12, atol=1e-12)
    (S * _t(g["G"])).sum().backward()
    for name, t in (("q", q), ("k", k), ("F", F), ("bias", bias)):
        np.testing.assert_allclose(t.grad.numpy(), g[f"sim_d{name}"], rtol=1e-6, atol=1e-6, err_msg=name)


@pytest.mark.parametrize("c", range(len(CASES)))
def test_golden_attention_and_grads(c):
    g = CASES[c]
    B, Hq, Hk, Nq, Nk, D, R, causal, masked = (int(x) for x in g["meta"])
    q, k, v = _t(g["q"], True), _t(g["k"], True), _t(g["v"], True)
    F, bias = _t(g["F"], True), _t(g["bias"], True)
    mask = torch.tensor(g["mask"]) if masked else None
    O = orc.flash_nonfused(q, k, v, F, bias, mask=mask, causal=bool(causal))
    np.testing.assert_allclose(O.detach().numpy(), g["O"], rtol=1e-12, atol=1e-12)
    lse = orc.flash_lse(q, k, F, bias, mask=mask, causal=bool(causal))
    np.testing.assert_allclose(lse.detach().numpy(), g["LSE"], rtol=1e-12, atol=1e-12)
    (O * _t(g["dO"])).sum().backward()
    for name, t in (("q", q), ("k", k), ("v", v), ("F", F), ("bias", bias)):
        np.testing.assert_allclose(t.grad.numpy(), g[f"attn_d{name}"], rtol=1e-6, atol=1e-6, err_msg=name)


def test_freqs_closed_form():
    inv = orc.inv_freqs(64)
    assert inv.shape == (64,)
    assert inv[0] == 1.0
    np.testing.assert_allclose(inv.numpy(), 10000.0 ** -(np.arange(64) / 64), rtol=1e-6)
    f = orc.pope_freqs(1024, inv)
    assert f.shape == (1024, 64)
    assert torch.all(f[0] == 0)
    assert torch.equal(f[:, 0], torch.arange(1024).float())
    # offset shifts positions: freqs(n, offset)[i] == freqs(n + offset)[i + offset]
    f2 = orc.pope_freqs(1000, inv, offset=24)
    assert torch.equal(f2, f[24:])


def test_axial_grid_reversed_order_and_shapes():
    pos = orc.axial_grid_positions(8, 16, 16)
    assert pos.shape == (2048, 3)
    n = torch.arange(2048)
    # column 0 is the LAST axis (fastest varying), column 2 the first
    assert torch.equal(pos[:, 0], (n % 16).float())
    assert torch.equal(pos[:, 1], ((n // 16) % 16).float())
    assert torch.equal(pos[:, 2], (n // 256).float())
    invs = orc.axial_inv_freqs((32, 32, 32))
    f = orc.axial_freqs(pos, invs)
    assert f.shape == (2048, 96)                            # reference test_readme.py:47
    assert torch.equal(f[:, :32], pos[:, 0:1] * invs[0])
    assert orc.axial_freqs(orc.axial_grid_positions(32, 32), orc.axial_inv_freqs((32, 32))).shape == (1024, 64)


# ---- axial tables against closed forms, and mistakes planted in copies of them ----

def _axial_closed_form(dims, axial_dims):
    """Float64 table built from scalars alone (pope_nd.py:48-52,65-68,84-100): token n of the
    row-major grid ``dims`` has coordinates (c_0, ..., c_{k-1}) with the last axis fastest;
    column block i holds the coordinate of axis k-1-i times 10000 ** -(j / axial_dims[i])."""
    k = len(dims)
    ntok = int(np.prod(dims))
    width = sum(axial_dims)
    out = np.zeros((ntok, width))
    for n in range(ntok):
        coords, rem = [0] * k, n
        for ax in reversed(range(k)):
            coords[ax], rem = rem % dims[ax], rem // dims[ax]
        col = 0
        for i, d in enumerate(axial_dims):
            p = coords[k - 1 - i]
            for j in range(d):
                out[n, col] = p * 10000.0 ** (-j / d)
                col += 1
    return out


# (grid, per-axis widths): unequal widths so that a denominator of sum(widths) or of another axis's
# width changes every block but the first entry; distinct grid sizes so that a wrong axis shows
AXIAL_PIN_CASES = [((3, 5, 7), (4, 2, 8)), ((8, 16, 16), (32, 32, 32)), ((6, 10), (8, 16)), ((9,), (12,))]


def _check_axial(inv_fn, grid_fn, freqs_fn):
    # fp32 pow: a few ulp (2^-23 = 1.2e-7) of relative error; every planted mistake is off by > 1e-2
    # per-axis inverse frequencies at widths where 10000 ** -(j / d) has short decimal forms
    exact = {1: [1.0], 2: [1.0, 1e-2], 4: [1.0, 1e-1, 1e-2, 1e-3], 8: [10.0 ** (-j / 2) for j in range(8)]}
    invs = inv_fn(tuple(exact))
    for inv, (d, want) in zip(invs, exact.items()):
        np.testing.assert_allclose(inv.double().numpy(), want, rtol=5e-7, atol=0)
    for dims, axial_dims in AXIAL_PIN_CASES:
        invs = inv_fn(axial_dims)
        for inv, d in zip(invs, axial_dims):
            np.testing.assert_allclose(inv.double().numpy(), 10000.0 ** (-np.arange(d) / d), rtol=5e-7, atol=0)
        got = freqs_fn(grid_fn(*dims), invs)
        np.testing.assert_allclose(got.double().numpy(), _axial_closed_form(dims, axial_dims),
                                   rtol=1e-6, atol=0)


def test_axial_tables_match_closed_form():
    """Every per-axis inverse frequency and every column block of the axial table, against
    float64 values computed from scalars (not from the oracle's own tensors)."""
    _check_axial(orc.axial_inv_freqs, orc.axial_grid_positions, orc.axial_freqs)


def _mutant_axial(kind):
    def inv_fn(axial_dims):
        if kind == "denominator_sum":
            s = sum(axial_dims)
            return [10000.0 ** -(torch.arange(d).float() / s) for d in axial_dims]
        if kind == "arange_step_two":                     # RoPE's arange(0, d, 2) / d, repeated
            return [(10000.0 ** -(torch.arange(0, d, 2).float() / d)).repeat_interleave(2)[:d]
                    for d in axial_dims]
        return orc.axial_inv_freqs(axial_dims)

    def grid_fn(*dims):
        if kind == "grid_not_reversed":
            grid = torch.meshgrid(*[torch.arange(d).float() for d in dims], indexing="ij")
            return torch.stack([g.flatten() for g in grid], dim=-1)
        return orc.axial_grid_positions(*dims)

    def freqs_fn(pos, invs):
        if kind == "first_axis_everywhere":
            return torch.cat([pos[..., 0, None] * inv for inv in invs], dim=-1)
        if kind == "blocks_reversed":
            return torch.cat([pos[..., i, None] * inv for i, inv in reversed(list(enumerate(invs)))], dim=-1)
        return orc.axial_freqs(pos, invs)
    return inv_fn, grid_fn, freqs_fn


@pytest.mark.parametrize("kind", ["denominator_sum", "arange_step_two", "grid_not_reversed",
                                  "first_axis_everywhere", "blocks_reversed"])
def test_planted_axial_mistakes_are_caught(kind):
    with pytest.raises(AssertionError):
        _check_axial(*_mutant_axial(kind))


@pytest.mark.parametrize("partial", [False, True])
def test_transform_layout_and_shapes(partial):
    torch.manual_seed(0)
    R = 32 if partial else 64
    F = orc.pope_freqs(1024, orc.inv_freqs(R))
    bias = torch.rand(8, R) * -2 * math.pi
    q, k = torch.randn(1, 8, 1024, 64), torch.randn(1, 8, 1024, 64)
    qh, kh = orc.apply_pope_to_qk(F, bias, q, k)
    final = 128 if not partial else 96                     # reference test_pope.py:21
    assert qh.shape == (1, 8, 1024, final) and kh.shape == (1, 8, 1024, final)
    a = orc.softplus(q[..., :R])
    torch.testing.assert_close(qh[..., 0:2 * R:2], a * F.cos())
    torch.testing.assert_close(qh[..., 1:2 * R:2], a * F.sin())
    c = orc.softplus(k[..., :R])
    torch.testing.assert_close(kh[..., 0:2 * R:2], c * (F + bias[:, None]).cos())
    assert torch.equal(qh[..., 2 * R:], q[..., R:])         # pass-through dims raw
    # decode: one query takes the LAST phase row (right aligned)
    q1, _ = orc.apply_pope_to_qk(F, bias, q[..., -1:, :], k)
    assert q1.shape == (1, 8, 1, final)                     # reference test_pope.py:26-29
    torch.testing.assert_close(q1, qh[..., -1:, :])
    # complex form carries the same numbers
    qc, kc = orc.apply_pope_to_qk(F, bias, q, k, return_complex=True)
    torch.testing.assert_close(qc[..., :R].real.float(), qh[..., 0:2 * R:2])
    torch.testing.assert_close(kc[..., :R].imag.float(), kh[..., 1:2 * R:2])


def _rand_case(seed, B=2, H=2, Nq=5, Nk=7, D=16, R=8, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Nq, D, generator=g, dtype=dtype)
    k = torch.randn(B, H, Nk, D, generator=g, dtype=dtype)
    v = torch.randn(B, H, Nk, D, generator=g, dtype=dtype)
    F = orc.pope_freqs(Nk, orc.inv_freqs(R).to(dtype))
    bias = torch.rand(H, R, generator=g, dtype=dtype) * -2 * math.pi
    return q, k, v, F, bias


def test_similarity_invariants():
    q, k, v, F, bias = _rand_case(1)
    S = orc.sim_nonfused(q, k, F, bias)
    # translation: positions offset by a constant leave S unchanged (2-D freqs)
    inv = orc.inv_freqs(8).double()
    S_off = orc.sim_nonfused(q, k, orc.pope_freqs(7, inv, offset=100), bias)
    torch.testing.assert_close(S, S_off, rtol=1e-9, atol=1e-9)
    # global phase shift of every row leaves S unchanged
    torch.testing.assert_close(S, orc.sim_nonfused(q, k, F + 0.37, bias), rtol=1e-12, atol=1e-12)
    # a bias is a key-side phase: equivalent to shifting the key rows only
    # R = 0 reduces to the plain q k^T
    S0 = orc.sim_nonfused(q, k, F[:, :0], bias[:, :0])
    torch.testing.assert_close(S0, q @ k.transpose(-1, -2))


def test_phase_gradient_identity():
    # S depends on phi - psi only, so sum_n dF[n, d] = 0 and dbias = -(sum of the query-row dF)
    q, k, v, F, bias = _rand_case(2, Nq=7, Nk=7)
    F.requires_grad_(True)
    bias.requires_grad_(True)
    S = orc.sim_nonfused(q, k, F, bias)
    G = torch.randn(S.shape, generator=torch.Generator().manual_seed(3), dtype=S.dtype)
    (S * G).sum().backward()
    torch.testing.assert_close(F.grad.sum(0), torch.zeros_like(F.grad[0]), atol=1e-10, rtol=0)
    # with Nq == Nk every F row is both a query and a key phase; bias grad is the key part
    Fq = F.detach().clone().requires_grad_(True)
    Fk = F.detach().clone().requires_grad_(True)
    qh, _ = orc.apply_pope_to_qk(Fq, bias.detach(), q, k)
    _, kh = orc.apply_pope_to_qk(Fk, bias.detach(), q, k)
    ((qh @ kh.transpose(-1, -2)) * G).sum().backward()
    torch.testing.assert_close(bias.grad.sum(0), Fk.grad.sum(0), rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(bias.grad.sum(0), -Fq.grad.sum(0), rtol=1e-9, atol=1e-9)


def test_flash_semantics():
    q, k, v, F, bias = _rand_case(4, Nq=4, Nk=6)
    mask = torch.tensor([[True] * 6, [False] * 6])
    O = orc.flash_nonfused(q, k, v, F, bias, mask=mask)
    assert torch.all(O[1] == 0)                             # fully-masked rows give 0
    lse = orc.flash_lse(q, k, F, bias, mask=mask)
    assert torch.all(torch.isinf(lse[1])) and torch.all(lse[1] < 0)
    # flash == softmax(scale * sim) v  (reference test_flash_attn.py:78-110)
    S = orc.sim_nonfused(q, k, F, bias) * q.shape[-1] ** -0.5
    torch.testing.assert_close(O[0], (S.softmax(-1) @ v)[0])
    # top-left causal with Nq < Nk: query i sees keys 0..i only
    Oc = orc.flash_nonfused(q, k, v, F, bias, causal=True)
    torch.testing.assert_close(Oc[:, :, 0], v[:, :, 0])


# ---- planted mistakes: each variant of the oracle must fail a golden check ----

def _mutant_sim(kind):
    def sim(q, k, F, bias):
        R = F.shape[-1]
        Nq = q.shape[-2]
        a, c = orc.softplus(q[..., :R]), orc.softplus(k[..., :R])
        if kind == "no_softplus":
            a, c = q[..., :R], k[..., :R]
        fq = F[-Nq:] if kind != "left_aligned" else F[:Nq]
        fk = F + (bias[:, None] if kind != "bias_sign" else -bias[:, None])
        if kind == "sum_phase":
            ang = fq[None, None, :, None, :] + fk[None, :, None, :, :]
        else:
            ang = fq[None, None, :, None, :] - fk[None, :, None, :, :]
        rot = (a[..., :, None, :] * c[..., None, :, :] * torch.cos(ang)).sum(-1)
        rest = q[..., R:] @ k[..., R:].transpose(-1, -2)
        if kind == "softplus_rest":
            rest = orc.softplus(q[..., R:]) @ orc.softplus(k[..., R:]).transpose(-1, -2)
        return rot + rest
    return sim


@pytest.mark.parametrize("kind", ["no_softplus", "left_aligned", "bias_sign", "sum_phase", "softplus_rest"])
def test_planted_mistakes_are_caught(kind):
    g = CASES[1]  # partial rotation, Nq < Nk, nonzero offset and bias
    q, k, F, bias = (_t(g[n]) for n in ("q", "k", "F", "bias"))
    # the faithful formula in the same shape matches the brute force ...
    good = _mutant_sim("none")(q, k, F, bias)
    np.testing.assert_allclose(good.numpy(), g["S"], rtol=1e-10, atol=1e-10)
    # ... and each plausible mistake does not
    bad = _mutant_sim(kind)(q, k, F, bias)
    assert np.abs(bad.numpy() - g["S"]).max() > 1e-3


# ---- functions the golden fixtures alone leave open ----

@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_softplus_matches_torch(dtype):
    """softplus with beta 1 and threshold 20 (x > 20 -> x): torch's F.softplus, the reference's
    magnitude function (pope.py:34,60), over both branches and the deep negative tail."""
    import torch.nn.functional as Fn
    x = torch.cat([torch.linspace(-100, 100, 20001, dtype=dtype),
                   torch.tensor([20.0, 20.0 + 1e-3, 19.999, -1e-30, 0.0], dtype=dtype)])
    tol = dict(rtol=1e-6, atol=1e-30) if dtype == torch.float32 else dict(rtol=1e-13, atol=1e-300)
    torch.testing.assert_close(orc.softplus(x), Fn.softplus(x), **tol)
    assert torch.equal(orc.softplus(x[x > 20]), x[x > 20])


@pytest.mark.parametrize("groups", [1, 2, 4])
def test_repeat_heads_matches_einops(groups):
    """The grouped-head repeat is einops' 'b h ... -> b (g h) ...' (attention.py:44-45,118-120)."""
    from einops import repeat
    t = torch.randn(2, 3, 5, 4)
    torch.testing.assert_close(orc._repeat_heads(t, groups), repeat(t, "b h ... -> b (g h) ...", g=groups),
                               rtol=0, atol=0)


def test_clamp_bias_closed_form_and_gradient():
    x = torch.tensor([-10.0, -2 * math.pi, -3.0, -1e-7, 0.0, 1e-7, 4.0], dtype=torch.float64,
                     requires_grad=True)
    y = orc.clamp_bias(x)
    want = torch.tensor([-2 * math.pi, -2 * math.pi, -3.0, -1e-7, 0.0, 0.0, 0.0], dtype=torch.float64)
    assert torch.equal(y.detach(), want)
    y.sum().backward()
    assert x.grad.tolist() == [0.0, 1.0, 1.0, 1.0, 1.0, 0.0, 0.0]


def test_planted_gqa_mapping_mistake_is_caught(monkeypatch):
    """Query head h must read kv head h % Hk; the blocked mapping h // (Hq / Hk) is a plausible
    mistake that the Hq = 4, Hk = 2 golden case must reject."""
    g = CASES[3]
    assert tuple(int(x) for x in g["meta"][1:3]) == (4, 2)
    q, k, F, bias = (_t(g[n]) for n in ("q", "k", "F", "bias"))
    np.testing.assert_allclose(orc.sim_nonfused(q, k, F, bias).numpy(), g["S"], rtol=1e-12, atol=1e-12)
    monkeypatch.setattr(orc, "_repeat_heads",
                        lambda t, groups: t.repeat_interleave(groups, dim=1) if groups > 1 else t)
    assert np.abs(orc.sim_nonfused(q, k, F, bias).numpy() - g["S"]).max() > 1e-3


def test_planted_softplus_threshold_mistake_is_caught(monkeypatch):
    """Clamping the input at the threshold instead of passing x > 20 through must fail the golden
    case whose inputs reach 25."""
    g = CASES[4]
    q, k, F, bias = (_t(g[n]) for n in ("q", "k", "F", "bias"))
    np.testing.assert_allclose(orc.sim_nonfused(q, k, F, bias).numpy(), g["S"], rtol=1e-12, atol=1e-12)
    monkeypatch.setattr(orc, "softplus", lambda x: torch.log1p(torch.exp(torch.clamp(x, max=20.0))))
    assert np.abs(orc.sim_nonfused(q, k, F, bias).numpy() - g["S"]).max() > 1e-3
