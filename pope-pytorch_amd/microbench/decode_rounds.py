"""The decode split kernel against the number of live (batch, split) workgroups.

C5's shapes (q (8, 16, 1, 64), K / V (8, 16, 32768, 64) bf16, PoPE(64, heads=16)) with four
patterns of valid cache lengths: the bench's (U{4096..32768} from seed 1005), all full, all half and
all three quarters.  A split of 128 keys with a visible key is one live workgroup (all 16 heads,
512 KB of K and V); two workgroups fit on a CU, 512 on the chip.  The kernel time is the library's
per-launch events (the stream the kernel runs on).  Live workgroups / 512 is the number of rounds:
a partial last round costs about as long as a full one.

    python pope-pytorch_amd/microbench/decode_rounds.py
"""
import json
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import pope_amd  # noqa: E402
from pope_amd import _lib  # noqa: E402


def main():
    g = torch.Generator().manual_seed(1005)
    dev = torch.device("cuda:0")
    B, H, N, D, S = 8, 16, 32768, 64, 128
    q = torch.randn(B, H, 1, D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(dev)
    lens_bench = torch.randint(4096, N + 1, (B,), generator=g)
    freqs, bias = pope_amd.PoPE(D, heads=H).to(dev)(N)
    rows = []
    for name, lens in (("bench", lens_bench), ("half", torch.full((B,), N // 2)),
                       ("three_quarters", torch.full((B,), 3 * N // 4)), ("full", torch.full((B,), N))):
        mask = (torch.arange(N)[None, :] < lens[:, None]).to(dev)
        run = lambda: pope_amd.flash_attn_with_pope(q, k, v, pos_emb=(freqs, bias), mask=mask)
        with torch.no_grad():
            for _ in range(50):
                run()
            torch.cuda.synchronize()
            _lib.profile_reset()
            _lib.profile_enable(True)
            for _ in range(50):
                run()
            torch.cuda.synchronize()
            _lib.profile_enable(False)
        cnt, tot = _lib.profile_read()["flash_decode_split"][:2]
        us = tot / cnt * 1e3
        live = int(((lens + S - 1) // S).sum())
        kv = int(lens.sum()) * H * D * 2 * 2
        rows.append({"lengths": name, "live_workgroups": live, "rounds": round(live / 512, 2),
                     "split_us": round(us, 2), "us_per_round": round(us / -(-live // 512), 2),
                     "kv_TBps": round(kv / us / 1e6, 3)})
    for r in rows:
        print(json.dumps(r), flush=True)


if __name__ == "__main__":
    main()
