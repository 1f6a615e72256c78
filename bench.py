"""Benchmark of the PoPE flash attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload (the config the headline metric is quoted
on): ``flash_attn_with_pope`` forward + backward in bf16, causal, B=2 H=8
N=4096 D=64, ``PoPE(32, heads=8)`` (partial rotation on D=64), key-padding
mask with the last 0..512 keys of each batch masked, q/k/v/dO iid N(0,1) from
seed 1003.  One step = o = flash_attn_with_pope(q, k, v, pos_emb, mask,
causal=True); o.backward(dO) -- the public API, the HIP kernels underneath.
pos_emb = pope(N) is the PoPE module's output, computed once before the timed
steps (its arange / outer product / clamp are torch ops outside the metric's
op); its bias is a leaf that requires grad, so every backward also computes
the bias gradient, as the reference's fused backward does.

Prints ONE JSON line.  ``value`` is TFLOP/s with the FA accounting of the
metric: 3.5 * 4 * B * H * N^2 * D / 2 flops per causal fwd+bwd step.
``roofline`` covers the kernel with the largest share of the step time, timed
by the library's own per-kernel hipEvents (recorded on the stream each kernel
runs on) over a second pass of the same steps (the events stay out of the
timed pass).  ``cpu_baseline`` times the CPU oracle (the
restatement of the reference's PyTorch path) fwd+bwd on a bounded sample of the
same workload on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "pope-pytorch_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "flash_attn_with_pope fwd+bwd TFLOP/s & % bf16 MFMA peak, B2 H8 N4096 D64"
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
B, H, N, D, R = 2, 8, 4096, 64, 32
SEED = 1003
MAX_PAD = 512


def fa_flops(kind: str) -> float:
    """Algorithmic flops of one launch (FA accounting, causal = half the N^2 pairs, head dim D).

    flash_fwd: 2 GEMMs (QK^T, PV); flash_bwd: 5 (dK/dV jobs: QK^T, dO V^T, P^T dO, dS^T Q; dQ jobs:
    dS K -- their recomputation of QK^T and dO V^T is not counted).  Together
    7 * 2 * B * H * N^2 * D / 2 = 3.5 * 4 * B * H * N^2 * D / 2."""
    pairs = B * H * N * N / 2
    gemms = {"flash_fwd": 2, "flash_bwd": 5}[kind]
    return gemms * 2 * pairs * D


STEP_FLOPS = 3.5 * 4 * B * H * N * N * D / 2


def make_inputs(device):
    import torch
    g = torch.Generator().manual_seed(SEED)
    q = torch.randn(B, H, N, D, generator=g)
    k = torch.randn(B, H, N, D, generator=g)
    v = torch.randn(B, H, N, D, generator=g)
    do = torch.randn(B, H, N, D, generator=g)
    pads = torch.randint(0, MAX_PAD + 1, (B,), generator=g)
    mask = torch.ones(B, N, dtype=torch.bool)
    for b in range(B):
        if pads[b] > 0:
            mask[b, N - int(pads[b]):] = False
    cast = lambda t: t.to(torch.bfloat16).to(device)
    return cast(q), cast(k), cast(v), cast(do), mask.to(device), [int(p) for p in pads]


def gpu_bench(steps: int, warmup: int):
    import torch

    import pope_amd
    from pope_amd import _lib

    dev = torch.device("cuda:0")
    q, k, v, do, mask, pads = make_inputs(dev)
    pope = pope_amd.PoPE(R, heads=H).to(dev)
    freqs, bias = pope(N)
    bias = bias.detach().requires_grad_(True)
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)

    def step():
        # fresh gradients each step (optimizer.zero_grad(set_to_none=True)), no accumulation kernels
        q.grad = k.grad = v.grad = bias.grad = None
        o = pope_amd.flash_attn_with_pope(q, k, v, pos_emb=(freqs, bias), mask=mask, causal=True)
        o.backward(do)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    # per-kernel times from a second pass of the same steps, with the library's hipEvents
    # around every launch (kept out of the timed pass above)
    _lib.profile_reset()
    _lib.profile_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    kernels = _lib.profile_read()
    return elapsed, kernels, pads


def cpu_baseline(min_seconds: float = 10.0, max_reps: int = 5):
    """The CPU oracle fwd+bwd on one (batch, head) slice x 2 heads of the workload, fp32 after the
    bf16 cast (the reference's PyTorch path promotes after softplus, pope.py:60,69-70)."""
    import torch

    from oracle import pope_oracle as orc

    # the host share this process is given (OMP_NUM_THREADS), else every core
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count() or 1
    torch.set_num_threads(threads)
    q, k, v, do, mask, _ = make_inputs("cpu")
    hs = 2
    up = lambda t: t[:1, :hs].float().clone().requires_grad_(True)
    freqs = orc.pope_freqs(N, orc.inv_freqs(R))
    bias = torch.zeros(hs, R, requires_grad=True)
    m1 = mask[:1]
    flops = 3.5 * 4 * 1 * hs * N * N * D / 2

    def one():
        qq, kk, vv = up(q), up(k), up(v)
        o = orc.flash_nonfused(qq, kk, vv, freqs, bias, mask=m1, causal=True)
        o.backward(do[:1, :hs].float())

    one()   # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < max_reps and (len(times) < 3 or time.perf_counter() - t_start < min_seconds):
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": round(flops / med / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle fwd+bwd (torch fp32, CPU) on batch 0, heads 0-{hs - 1} of the workload "
                  f"(1x{hs}x{N}x{D}, causal, mask); median of {len(times)} runs "
                  f"= {med * 1e3:.1f} ms; FA flop accounting as the GPU value",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {a.gpus} is not supported "
              "(the path shards over (batch x head); see the multi-GPU design notes)", file=sys.stderr)
        sys.exit(2)

    elapsed, kernels, pads = gpu_bench(a.steps, a.warmup)
    ms = elapsed / a.steps * 1e3
    value = STEP_FLOPS / (ms * 1e-3) / 1e12

    # dominant kernel: largest total time among the kernels with an algorithmic flop count
    cand = {n: kernels[n] for n in ("flash_fwd", "flash_bwd") if n in kernels}
    dom = max(cand, key=lambda n: cand[n][1])
    cnt, tot, _, _ = cand[dom]
    avg_s = tot / cnt * 1e-3
    achieved = fa_flops(dom) / avg_s / 1e12
    roofline = {
        "bound": "mfma", "kernel": dom, "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None,
        "avg_launch_us": round(avg_s * 1e6, 2),
    }
    breakdown = {n: {"launches": c, "avg_us": round(t / c * 1e3, 2)} for n, (c, t, _, _) in sorted(kernels.items())}

    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "C3 causal training flash attention: flash_attn_with_pope fwd+bwd, "
                               "PoPE(32, heads=8) partial rotation, key-padding mask",
                   "batch": B, "heads": H, "seq_len": N, "head_dim": D, "rotate_dim": R, "causal": True,
                   "mask_pad_per_batch": pads, "seed": SEED},
        "frac_of_peak": round(value / PEAK_BF16_TFLOPS, 4),
        "roofline": roofline,
        "kernels": breakdown,
    }
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
