"""Top-K micro-benchmark (the shape of /root/reference/topk_test/benchmark.py:
33-46): 512 independent rows, top 512 of 8192 fp32 values, int32 payloads
0 / 1 / 8 per element.  Times htree_topk_rows (the block-wide radix select of
the wide forward, all 8192 keys resident in registers: the reference's
"direct" strategy; its "streaming" strategy exists to fit Triton's register
budget and has no counterpart here) against torch.topk, with HIP events on
the current stream.  One JSON line per payload count.

    python -m htree_amd.topk_bench [--rows 512] [--n 8192] [--k 512] [--reps 200]
"""
from __future__ import annotations

import argparse
import json

import torch

from .topk import topk_rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--rows", type=int, default=512)
    ap.add_argument("--n", type=int, default=8192)
    ap.add_argument("--k", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--reps", type=int, default=200)
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(args.rows, args.n, device=dev, generator=g)
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.reps * 1e3  # us

    for npay in (0, 1, 8):
        pay = None
        if npay:
            shape = (args.rows, args.n) if npay == 1 else (args.rows, args.n, npay)
            pay = torch.randint(0, 100000, shape, device=dev, dtype=torch.int32, generator=g)
        v, i, p = topk_rows(x, args.k, pay)
        ref = torch.topk(x, args.k, dim=-1, largest=True, sorted=True)
        ok = torch.equal(torch.sort(i.long(), dim=-1).values, torch.sort(ref.indices, dim=-1).values)
        us = timed(lambda: topk_rows(x, args.k, pay))
        us_t = timed(lambda: torch.topk(x, args.k, dim=-1, largest=True, sorted=False))
        print(json.dumps({
            "bench": "topk_rows", "rows": args.rows, "n": args.n, "k": args.k, "payload": npay,
            "us": us, "rows_per_s": args.rows / (us * 1e-6), "torch_topk_us": us_t,
            "speedup_vs_torch_topk": us_t / us, "matches_torch_topk": bool(ok),
            "input_GBps": x.numel() * 4 / (us * 1e-6) / 1e9,
        }), flush=True)


if __name__ == "__main__":
    main()
