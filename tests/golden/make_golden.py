"""Writes tests/golden/pope_golden.npz: tiny PoPE cases computed by brute force.

Independent of the oracle's formulation: plain Python float64 loops over
  S_ij = sum_{d<R} softplus(q_id) softplus(k_jd) cos(phi_id - psi_jd) + sum_{d>=R} q_id k_jd
  phi_id = F[q_off + i, d],  psi_jd = F[j, d] + bias[h % Hk, d],  q_off = Nk - Nq
(the closed form behind pope.py:30-86 / triton_pope.py:70-81), the masked softmax
  O_i = sum_j p_ij v_j,  p_ij = exp(scale S_ij) / sum, over keys kept by
  (mask[b, j]) and (j <= i when causal)   (attention.py:106-145, top-left causal)
and central finite differences for every gradient.  No torch, no reference code.

    python tests/golden/make_golden.py      # rewrites the .npz (seeded, deterministic)
"""
from __future__ import annotations

import math
import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "pope_golden.npz")


def softplus(x):
    return x if x > 20.0 else math.log1p(math.exp(x))


def sim(q, k, F, bias, R):
    B, Hq, Nq, D = q.shape
    Hk, Nk = k.shape[1], k.shape[2]
    q_off = Nk - Nq
    S = np.zeros((B, Hq, Nq, Nk))
    for b in range(B):
        for h in range(Hq):
            hk = h % Hk
            for i in range(Nq):
                for j in range(Nk):
                    s = 0.0
                    for d in range(D):
                        if d < R:
                            phi = F[q_off + i, d]
                            psi = F[j, d] + bias[hk, d]
                            s += softplus(q[b, h, i, d]) * softplus(k[b, hk, j, d]) * math.cos(phi - psi)
                        else:
                            s += q[b, h, i, d] * k[b, hk, j, d]
                    S[b, h, i, j] = s
    return S


def attn(q, k, v, F, bias, R, mask, causal, scale):
    S = sim(q, k, F, bias, R)
    B, Hq, Nq, Nk = S.shape
    Hk, D = k.shape[1], v.shape[3]
    O = np.zeros((B, Hq, Nq, D))
    LSE = np.full((B, Hq, Nq), -np.inf)
    for b in range(B):
        for h in range(Hq):
            for i in range(Nq):
                keep = [j for j in range(Nk) if mask[b, j] and (not causal or j <= i)]
                if not keep:
                    continue
                m = max(scale * S[b, h, i, j] for j in keep)
                w = {j: math.exp(scale * S[b, h, i, j] - m) for j in keep}
                tot = sum(w.values())
                LSE[b, h, i] = m + math.log(tot)
                for d in range(D):
                    O[b, h, i, d] = sum(w[j] * v[b, h % Hk, j, d] for j in keep) / tot
    return O, LSE


def fd_grad(f, x, eps=1e-5):
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        idx = it.multi_index
        old = x[idx]
        x[idx] = old + eps
        fp = f()
        x[idx] = old - eps
        fm = f()
        x[idx] = old
        g[idx] = (fp - fm) / (2 * eps)
    return g


def make_case(rng, B, Hq, Hk, Nq, Nk, D, R, causal, masked, offset, big=False):
    q = rng.standard_normal((B, Hq, Nq, D))
    k = rng.standard_normal((B, Hk, Nk, D))
    v = rng.standard_normal((B, Hk, Nk, D))
    if big:
        # magnitudes past softplus's threshold (x > 20 -> x) and deep in its negative tail
        q[..., 0] = 25.0
        q[..., 1] = -23.0
        k[..., 2] = 21.5
        k[..., 3] = -30.0
    inv = 10000.0 ** -(np.arange(R) / max(R, 1))
    F = (np.arange(Nk)[:, None] + offset) * inv[None, :]
    bias = rng.uniform(-2 * math.pi, 0.0, (Hk, R))
    mask = np.ones((B, Nk), dtype=bool)
    if masked:
        for b in range(B):
            mask[b, Nk - 1 - b:] = False
    G = rng.standard_normal((B, Hq, Nq, Nk))
    dO = rng.standard_normal((B, Hq, Nq, D))
    scale = D ** -0.5

    S = sim(q, k, F, bias, R)
    O, LSE = attn(q, k, v, F, bias, R, mask, causal, scale)
    ls = lambda: float((sim(q, k, F, bias, R) * G).sum())
    la = lambda: float((attn(q, k, v, F, bias, R, mask, causal, scale)[0] * dO).sum())
    out = dict(q=q, k=k, v=v, F=F, bias=bias, mask=mask, G=G, dO=dO, S=S, O=O, LSE=LSE,
               meta=np.array([B, Hq, Hk, Nq, Nk, D, R, int(causal), int(masked)]))
    for name, x in (("q", q), ("k", k), ("F", F), ("bias", bias)):
        out[f"sim_d{name}"] = fd_grad(ls, x)
    for name, x in (("q", q), ("k", k), ("v", v), ("F", F), ("bias", bias)):
        out[f"attn_d{name}"] = fd_grad(la, x)
    return out


def main():
    rng = np.random.default_rng(20251201)
    cases = [
        dict(B=1, Hq=2, Hk=2, Nq=4, Nk=4, D=8, R=8, causal=False, masked=False, offset=0),
        dict(B=2, Hq=2, Hk=1, Nq=3, Nk=5, D=8, R=4, causal=True, masked=True, offset=3),
        dict(B=1, Hq=2, Hk=2, Nq=1, Nk=6, D=8, R=8, causal=False, masked=True, offset=0),
        # grouped heads with Hk > 1: query head h reads kv head h % Hk (not h // (Hq / Hk))
        dict(B=1, Hq=4, Hk=2, Nq=3, Nk=5, D=8, R=8, causal=False, masked=False, offset=2),
        # inputs beyond softplus's threshold, partial rotation
        dict(B=1, Hq=1, Hk=1, Nq=4, Nk=4, D=8, R=6, causal=True, masked=False, offset=0, big=True),
    ]
    arrays = {}
    for c, kw in enumerate(cases):
        for key, val in make_case(rng, **kw).items():
            arrays[f"c{c}_{key}"] = val
    arrays["ncases"] = np.array(len(cases))
    np.savez_compressed(OUT, **arrays)
    print(OUT, sum(a.size for a in arrays.values()), "values")


if __name__ == "__main__":
    main()
