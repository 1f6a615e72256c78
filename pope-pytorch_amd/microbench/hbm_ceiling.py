"""HBM rates that plain streaming reaches on one MI355X: torch's fill (write only), sum (read
only), copy and elementwise multiply (read + write) over 256 MiB fp32 tensors, timed with events.
They bound what the HBM-bound kernels of this library can expect in practice, below the 8 TB/s
of the published peak.

    python pope-pytorch_amd/microbench/hbm_ceiling.py
"""
import json

import torch


def timed_us(f, n=20):
    for _ in range(3):
        f()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(n):
        f()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / n * 1e3


def main():
    nbytes = 1 << 28
    x = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    x.normal_()
    tb = lambda moved, us: round(moved / us / 1e6, 2)
    out = {
        "bytes": nbytes,
        "fill_write_TBps": tb(nbytes, timed_us(lambda: y.fill_(1.0))),
        "sum_read_TBps": tb(nbytes, timed_us(lambda: x.sum())),
        "copy_read_write_TBps": tb(2 * nbytes, timed_us(lambda: y.copy_(x))),
        "mul_read_write_TBps": tb(2 * nbytes, timed_us(lambda: torch.mul(x, 2.0, out=y))),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
