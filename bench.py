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

Before the W warm-up steps, ``prewarm`` runs the step in 20-step windows until two
consecutive windows agree within 2% (at most 2 s; reported under ``prewarm``): the
GPU's clocks ramp for tens of milliseconds after idle, and a 20-step window right
after 5 warm-up steps reads about 18% slower than the steady state.  Then W
warm-up steps and exactly K timed steps between synchronisations, as before.

Prints ONE JSON line.  ``value`` is TFLOP/s with the FA accounting of the
metric: 3.5 * 4 * B * H * N^2 * D / 2 flops per causal fwd+bwd step.
``secondary`` carries the two other GPU configs of the path, measured in the
same run on their own inputs: C5 decode (one query row against a 32k KV cache,
HBM GB/s of the valid K/V rows), C2 fused similarity fwd+bwd in fp32 and C4
axial flash attention fwd+bwd (D = 96, non-causal).  ``--workload decode`` /
``sim`` / ``axial`` run only that config (used to profile one workload at a
time); the default ``train`` runs all four.
``roofline`` covers the kernel with the largest share of the step time, timed
by the library's own per-kernel hipEvents over a second pass of the same steps
(each launch's dispatch stamps its start and end into an event pair on the
stream it runs on; the events stay out of the timed pass).  Its ``traffic`` is
the HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
summary (profiles/flash_c3_traffic.md), calibrated against a copy kernel.
``cpu_baseline`` times the CPU oracle (the restatement of the reference's
PyTorch path) fwd+bwd on the whole workload on this host's cores; its ``configs``
object times the same oracle on C1, C2, C4 and C5 (forward, and forward + backward
where the config has one) on the GPU lines' seeded inputs.
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


TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "flash_c3_traffic.md")


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary (lines
    ``traffic: <kernel> <bytes>``), or None when it holds no figure for that kernel."""
    import re
    try:
        text = open(TRAFFIC_SUMMARY).read()
    except OSError:
        return None
    m = re.search(rf"^traffic: {re.escape(kernel)} (\d+)$", text, re.M)
    return int(m.group(1)) if m else None


def fa_flops(kind: str) -> float:
    """Algorithmic flops of one launch (FA accounting, causal = half the N^2 pairs, head dim D).

    flash_fwd: 2 GEMMs (QK^T, PV); flash_bwd: 5 (dK/dV jobs: QK^T, dO V^T, P^T dO, dS^T Q; dQ jobs:
    dS K -- their recomputation of QK^T and dO V^T is not counted).  Together
    7 * 2 * B * H * N^2 * D / 2 = 3.5 * 4 * B * H * N^2 * D / 2."""
    pairs = B * H * N * N / 2
    gemms = {"flash_fwd": 2, "flash_bwd": 5}[kind]
    return gemms * 2 * pairs * D


STEP_FLOPS = 3.5 * 4 * B * H * N * N * D / 2


# C5 decode: q (8,16,1,64), K/V (8,16,32768,64) bf16, PoPE(64, heads=16), valid lengths U{4096..32768}
DEC_B, DEC_H, DEC_N, DEC_D, DEC_SEED = 8, 16, 32768, 64, 1005
# C2 fused similarity: q, k (2,8,2048,64) fp32, PoPE(64, heads=8), dS N(0,1)
SIM_B, SIM_H, SIM_N, SIM_D, SIM_SEED = 2, 8, 2048, 64, 1002
AX_SEED = 1004
PEAK_HBM_GBS = 8000.0
PEAK_FP32_TFLOPS = 157.3


def prewarm(step, window: int = 20, tol: float = 0.02, max_s: float = 2.0) -> dict:
    """Runs the step in windows of `window` steps until two consecutive windows agree within `tol`
    (at most `max_s` seconds), before the W warm-up steps.  The GPU's clocks ramp up for tens of
    milliseconds after an idle spell: measured on MI355X, the first 20-step window after 5 warm-up
    steps reads about 18% slower per step than the steady state (285 vs 240 us at C3), and again
    after 0.5 s of idle.  Nothing of this phase is timed or reported as the value."""
    import torch

    t_start = time.perf_counter()
    prev, n, w = None, 0, 0.0
    while True:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(window):
            step()
        torch.cuda.synchronize()
        w = time.perf_counter() - t0
        n += window
        if (prev is not None and abs(w - prev) <= tol * prev) or time.perf_counter() - t_start > max_s:
            break
        prev = w
    return {"steps": n, "seconds": round(time.perf_counter() - t_start, 3),
            "last_window_us_per_step": round(w / window * 1e6, 2)}


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

    warm = prewarm(step)
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
    return elapsed, kernels, pads, warm


def _kernel_us(kernels, names):
    return {n: round(kernels[n][1] / kernels[n][0] * 1e3, 2) for n in names if n in kernels}


def decode_bench(steps: int, warmup: int):
    """C5: flash_attn_with_pope at Nq = 1 (the decode kernels).  GB/s counts the valid K and V rows
    once (sum_b L_b * H * D * 2 bytes * 2) -- the algorithmic bytes; masked rows are never read."""
    import torch

    import pope_amd
    from pope_amd import _lib

    g = torch.Generator().manual_seed(DEC_SEED)
    dev = torch.device("cuda:0")
    q = torch.randn(DEC_B, DEC_H, 1, DEC_D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(DEC_B, DEC_H, DEC_N, DEC_D, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(DEC_B, DEC_H, DEC_N, DEC_D, generator=g).to(torch.bfloat16).to(dev)
    lens = torch.randint(4096, DEC_N + 1, (DEC_B,), generator=g)
    mask = (torch.arange(DEC_N)[None, :] < lens[:, None]).to(dev)
    freqs, bias = pope_amd.PoPE(DEC_D, heads=DEC_H).to(dev)(DEC_N)
    run = lambda: pope_amd.flash_attn_with_pope(q, k, v, pos_emb=(freqs, bias), mask=mask)
    with torch.no_grad():
        prewarm(run)
        for _ in range(warmup):
            run()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            run()
        torch.cuda.synchronize()
        el = (time.perf_counter() - t0) / steps
        _lib.profile_reset()
        _lib.profile_enable(True)
        for _ in range(steps):
            run()
        torch.cuda.synchronize()
        _lib.profile_enable(False)
    ks = _lib.profile_read()
    valid = int(lens.sum()) * DEC_H * DEC_D * 2 * 2
    split = ks["flash_decode_split"]
    split_s = split[1] / split[0] * 1e-3
    kern_s = sum(c_t[1] / c_t[0] for c_t in ks.values()) * 1e-3
    return {
        "workload": "C5 decode: q (8,16,1,64) vs K/V (8,16,32768,64) bf16, PoPE(64, heads=16), "
                    "key-padding mask with valid lengths U{4096..32768}",
        "valid_lengths": [int(x) for x in lens], "algorithmic_bytes": valid,
        "us_per_call": round(el * 1e6, 2), "GBps": round(valid / el / 1e9, 1),
        "GBps_kernels": round(valid / kern_s / 1e9, 1),
        "roofline": {"bound": "hbm", "kernel": "flash_decode_split",
                     "achieved": round(valid / split_s / 1e9, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(valid / split_s / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": measured_traffic("flash_decode_split"),
                     "avg_launch_us": round(split_s * 1e6, 2)},
        "frac_of_hbm_peak": round(valid / el / 1e9 / PEAK_HBM_GBS, 4),
        "kernels_us": _kernel_us(ks, sorted(ks)),
    }


def sim_bench(steps: int, warmup: int):
    """C2: compute_attn_similarity fwd+bwd in fp32 (sim, dq, dk, dbias).  Flops: fwd 2*B*H*N^2*(D+R),
    bwd twice that; bytes: sim write + dS read + q, k read + dq, dk write + freqs."""
    import torch

    import pope_amd
    from pope_amd import _lib

    B_, H_, N_, D_ = SIM_B, SIM_H, SIM_N, SIM_D
    g = torch.Generator().manual_seed(SIM_SEED)
    dev = torch.device("cuda:0")
    q = torch.randn(B_, H_, N_, D_, generator=g).to(dev).requires_grad_(True)
    k = torch.randn(B_, H_, N_, D_, generator=g).to(dev).requires_grad_(True)
    ds = torch.randn(B_, H_, N_, N_, generator=g).to(dev)
    pope = pope_amd.PoPE(D_, heads=H_).to(dev)
    # pos_emb is the op's input, made once as in the C3 line (the clamped bias a leaf that
    # receives dbias): the step times compute_attn_similarity forward + backward
    freqs, bias = pope(N_)
    bias = bias.detach().requires_grad_(True)

    def step():
        q.grad = k.grad = bias.grad = None
        sim = pope_amd.compute_attn_similarity(q, k, (freqs, bias))
        sim.backward(ds)

    prewarm(step)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    el = (time.perf_counter() - t0) / steps
    _lib.profile_reset()
    _lib.profile_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    ks = _lib.profile_read()
    R_ = D_
    flops = 3 * 2 * B_ * H_ * N_ * N_ * (D_ + R_)
    nbytes = 2 * 4 * B_ * H_ * N_ * N_ + 2 * 4 * 2 * B_ * H_ * N_ * D_ + 4 * N_ * R_
    # the default arithmetic (allow_tf32=True) is three bf16 MFMA products per fp32 product:
    # its compute floor is 3 * flops at the bf16 peak, below the HBM floor
    t_mfma = 3 * flops / (PEAK_BF16_TFLOPS * 1e12)
    t_hbm = nbytes / (PEAK_HBM_GBS * 1e9)
    return {
        "workload": "C2 fused similarity fwd+bwd: q, k (2,8,2048,64) fp32, PoPE(64, heads=8), dS N(0,1); "
                    "compute_attn_similarity default allow_tf32=True (split-bf16 MFMA products)",
        "us_per_step": round(el * 1e6, 2), "TFLOPs": round(flops / el / 1e12, 2),
        "GBps": round(nbytes / el / 1e9, 1), "frac_of_hbm_peak": round(nbytes / el / 1e9 / PEAK_HBM_GBS, 4),
        "algorithmic_flops": flops, "algorithmic_bytes": nbytes,
        "roofline": {"bound": "hbm" if t_hbm >= t_mfma else "mfma", "t_min_us": round(max(t_hbm, t_mfma) * 1e6, 2),
                     "frac": round(max(t_hbm, t_mfma) / el, 4)},
        "fp32_peak_frac": round(flops / el / 1e12 / PEAK_FP32_TFLOPS, 4),
        "kernels_us": _kernel_us(ks, sorted(ks)),
    }


def axial_bench(steps: int, warmup: int):
    """C4: flash_attn_with_pope fwd+bwd in bf16, non-causal, no mask, AxialPoPE(96, heads=8,
    axial_dims=(32, 32, 32)) on an (8, 16, 16) grid (N = 2048), B = 4, H = 8, D = 96.  FA flop
    accounting: 3.5 * 4 * B * H * N^2 * D per step (non-causal)."""
    import torch

    import pope_amd
    from pope_amd import _lib

    B_, H_, D_, grid = 4, 8, 96, (8, 16, 16)
    N_ = grid[0] * grid[1] * grid[2]
    g = torch.Generator().manual_seed(AX_SEED)
    dev = torch.device("cuda:0")
    q, k, v, do = (torch.randn(B_, H_, N_, D_, generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
    for t in (q, k, v):
        t.requires_grad_(True)
    freqs, bias = pope_amd.AxialPoPE(D_, heads=H_, axial_dims=(32, 32, 32)).to(dev)(grid)
    bias = bias.detach().requires_grad_(True)

    def step():
        q.grad = k.grad = v.grad = bias.grad = None
        o = pope_amd.flash_attn_with_pope(q, k, v, pos_emb=(freqs, bias))
        o.backward(do)

    prewarm(step)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    el = (time.perf_counter() - t0) / steps
    _lib.profile_reset()
    _lib.profile_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    ks = _lib.profile_read()
    flops = 3.5 * 4 * B_ * H_ * N_ * N_ * D_
    return {
        "workload": "C4 axial flash attention fwd+bwd: q, k, v (4,8,2048,96) bf16, AxialPoPE(96, heads=8, "
                    "axial_dims=(32,32,32)) on an (8,16,16) grid, non-causal, no mask",
        "ms_per_step": round(el * 1e3, 4), "TFLOPs": round(flops / el / 1e12, 2),
        "frac_of_peak": round(flops / el / 1e12 / PEAK_BF16_TFLOPS, 4), "algorithmic_flops": flops,
        "kernels_us": _kernel_us(ks, sorted(ks)),
    }


def _cpu_model() -> str:
    """The host CPU's model name (the `model name` line lscpu reports, read from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(min_seconds: float = 10.0, max_reps: int = 10):
    """The CPU oracle fwd+bwd over the whole C3 workload (every batch and head, two heads per
    call), fp32 after the bf16 cast (the reference's PyTorch path promotes after softplus,
    pope.py:60,69-70).  Repeated until about ``min_seconds`` of CPU work; the median pass is
    reported."""
    import torch

    from oracle import pope_oracle as orc

    # the host share this process is given (OMP_NUM_THREADS, capped by the CPU affinity mask)
    avail = len(os.sched_getaffinity(0))
    threads = min(int(os.environ.get("OMP_NUM_THREADS", "0")) or avail, avail)
    torch.set_num_threads(threads)
    q, k, v, do, mask, _ = make_inputs("cpu")
    hs = 2
    freqs = orc.pope_freqs(N, orc.inv_freqs(R))
    bias = torch.zeros(hs, R, requires_grad=True)

    def one():
        for b in range(B):
            for h0 in range(0, H, hs):
                up = lambda t: t[b:b + 1, h0:h0 + hs].float().clone().requires_grad_(True)
                o = orc.flash_nonfused(up(q), up(k), up(v), freqs, bias, mask=mask[b:b + 1], causal=True)
                o.backward(do[b:b + 1, h0:h0 + hs].float())

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
        "value": round(STEP_FLOPS / med / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "cpu_model": _cpu_model(),
        "cpus_in_affinity_mask": avail,
        "kind": "port",
        "sample": f"the whole workload: oracle fwd+bwd (torch fp32, CPU) over B={B} x H={H} heads, "
                  f"N={N}, D={D}, causal, mask, two heads per call; median of {len(times)} passes "
                  f"= {med * 1e3:.1f} ms per step; FA flop accounting as the GPU value",
    }


def _time_cpu(fn, min_seconds: float, max_reps: int, min_reps: int = 3):
    """Median wall time of fn() over at least ``min_reps`` passes (after one warm-up pass),
    repeated until about ``min_seconds`` of CPU work or ``max_reps`` passes."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < max_reps and (len(times) < min_reps or time.perf_counter() - t_start < min_seconds):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_configs(min_seconds: float = 3.0, max_reps: int = 5) -> dict:
    """The CPU oracle on the other BASELINE configs, on the same seeded inputs as the GPU lines
    (C1 from seed 1001): forward, and forward + backward where the config has a backward, over
    the whole workload of each config in fp32 (bf16 inputs cast first, as the reference's
    PyTorch path promotes them, pope.py:60,69-70).  Each figure is the median of at least three
    passes; the value is in the unit the config's GPU figure uses."""
    import torch

    from oracle import pope_oracle as orc

    out = {}
    # C1: PoPE(64, heads=8), pope(1024), q, k, v (1, 8, 1024, 64) fp32: similarity and attention
    g = torch.Generator().manual_seed(1001)
    q1, k1, v1 = (torch.randn(1, 8, 1024, 64, generator=g) for _ in range(3))
    f1, b1 = orc.pope_freqs(1024, orc.inv_freqs(64)), torch.zeros(8, 64)

    def c1():
        orc.sim_nonfused(q1, k1, f1, b1)
        orc.flash_nonfused(q1, k1, v1, f1, b1)

    t, n = _time_cpu(c1, min_seconds, max_reps)
    c1_flops = 2 * 8 * 1024 * 1024 * (64 + 64) * 2 + 2 * 8 * 1024 * 1024 * 64
    out["C1"] = {"fwd_ms": round(t * 1e3, 2), "value": round(c1_flops / t / 1e12, 5), "unit": "TFLOP/s",
                 "passes": n, "sample": "whole workload: similarity (1,8,1024,1024) and attention output, fp32"}

    # C2: similarity fwd + bwd, q, k (2, 8, 2048, 64) fp32, dS N(0, 1) (the GPU line's seed and draws)
    g = torch.Generator().manual_seed(SIM_SEED)
    q2 = torch.randn(SIM_B, SIM_H, SIM_N, SIM_D, generator=g)
    k2 = torch.randn(SIM_B, SIM_H, SIM_N, SIM_D, generator=g)
    ds2 = torch.randn(SIM_B, SIM_H, SIM_N, SIM_N, generator=g)
    f2, b2 = orc.pope_freqs(SIM_N, orc.inv_freqs(SIM_D)), torch.zeros(SIM_H, SIM_D)
    qg, kg, bg = q2.clone().requires_grad_(True), k2.clone().requires_grad_(True), b2.clone().requires_grad_(True)
    tf, _ = _time_cpu(lambda: orc.sim_nonfused(q2, k2, f2, b2), min_seconds, max_reps)

    def c2():
        orc.sim_nonfused(qg, kg, f2, bg).backward(ds2)

    t, n = _time_cpu(c2, min_seconds, max_reps)
    c2_bytes = 2 * 4 * SIM_B * SIM_H * SIM_N * SIM_N + 2 * 4 * 2 * SIM_B * SIM_H * SIM_N * SIM_D + 4 * SIM_N * SIM_D
    out["C2"] = {"fwd_ms": round(tf * 1e3, 2), "fwd_bwd_ms": round(t * 1e3, 2),
                 "value": round(c2_bytes / t / 1e9, 3), "unit": "GB/s", "passes": n,
                 "sample": "whole workload: sim (2,8,2048,2048), dq, dk, dbias; bytes as the GPU line"}

    # C4: axial flash fwd + bwd, (4, 8, 2048, 96) bf16 -> fp32, AxialPoPE(96, 8, (32, 32, 32)) on (8, 16, 16)
    g = torch.Generator().manual_seed(AX_SEED)
    q4, k4, v4, do4 = (torch.randn(4, 8, 2048, 96, generator=g).to(torch.bfloat16).float() for _ in range(4))
    f4 = orc.axial_freqs(orc.axial_grid_positions(8, 16, 16), orc.axial_inv_freqs((32, 32, 32)))
    b4 = torch.zeros(8, 96)

    def c4(bwd):   # sample: batch 0 of 4 (a quarter of the workload), four heads per call
        def run():
            for b in range(1):
                for h0 in range(0, 8, 4):
                    sl = lambda t: t[b:b + 1, h0:h0 + 4].clone().requires_grad_(bwd)
                    o = orc.flash_nonfused(sl(q4), sl(k4), sl(v4), f4, b4[h0:h0 + 4])
                    if bwd:
                        o.backward(do4[b:b + 1, h0:h0 + 4])
        return run

    tf, _ = _time_cpu(c4(False), min_seconds, max_reps, 2)
    t, n = _time_cpu(c4(True), min_seconds, max_reps, 2)
    c4_flops = 3.5 * 4 * 1 * 8 * 2048 * 2048 * 96
    out["C4"] = {"fwd_ms": round(tf * 1e3, 2), "fwd_bwd_ms": round(t * 1e3, 2),
                 "value": round(c4_flops / t / 1e12, 5), "unit": "TFLOP/s", "passes": n,
                 "sample": "batch 0 of 4 (8 heads, a quarter of the workload), four heads per call; "
                           "times are for the sample, the value uses the sample's FA flops"}

    # C5: decode, q (8, 16, 1, 64) against K / V (8, 16, 32768, 64) bf16 -> fp32, valid lengths U{4096..32768}
    g = torch.Generator().manual_seed(DEC_SEED)
    q5 = torch.randn(DEC_B, DEC_H, 1, DEC_D, generator=g).to(torch.bfloat16).float()
    k5 = torch.randn(DEC_B, DEC_H, DEC_N, DEC_D, generator=g).to(torch.bfloat16)
    v5 = torch.randn(DEC_B, DEC_H, DEC_N, DEC_D, generator=g).to(torch.bfloat16)
    lens = torch.randint(4096, DEC_N + 1, (DEC_B,), generator=g)
    mask5 = torch.arange(DEC_N)[None, :] < lens[:, None]
    f5, b5 = orc.pope_freqs(DEC_N, orc.inv_freqs(DEC_D)), torch.zeros(DEC_H, DEC_D)

    def c5():   # sample: sequences 0 and 1 of 8, one per call
        for b in range(2):
            orc.flash_nonfused(q5[b:b + 1], k5[b:b + 1].float(), v5[b:b + 1].float(), f5, b5, mask=mask5[b:b + 1])

    t, n = _time_cpu(c5, min_seconds, max_reps, 2)
    valid = int(lens[:2].sum()) * DEC_H * DEC_D * 2 * 2
    out["C5"] = {"fwd_ms": round(t * 1e3, 2), "value": round(valid / t / 1e9, 3), "unit": "GB/s", "passes": n,
                 "sample": f"sequences 0 and 1 of 8 (valid lengths {int(lens[0])}, {int(lens[1])}), one "
                           "per call; GB/s of their valid bf16 K and V rows, as the GPU line counts"}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=("train", "decode", "sim", "axial"), default="train",
                    help="train (default): the C3 headline line with C5, C2 and C4 as secondary; "
                         "decode / sim / axial: only that config's measurement")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {a.gpus} is not supported "
              "(the path shards over (batch x head); see the multi-GPU design notes)", file=sys.stderr)
        sys.exit(2)

    if a.workload != "train":
        fn = {"decode": decode_bench, "sim": sim_bench, "axial": axial_bench}[a.workload]
        print(json.dumps({"workload": a.workload, "steps": a.steps, "warmup": a.warmup,
                          **fn(a.steps, a.warmup)}), flush=True)
        return

    elapsed, kernels, pads, warm = gpu_bench(a.steps, a.warmup)
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
        "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": measured_traffic(dom),
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
        "prewarm": warm,
        "roofline": roofline,
        "kernels": breakdown,
        "secondary": {"decode_c5": decode_bench(a.steps, a.warmup), "sim_c2": sim_bench(a.steps, a.warmup),
                      "axial_c4": axial_bench(a.steps, a.warmup)},
    }
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
        line["cpu_baseline"]["configs"] = cpu_configs()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
