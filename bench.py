"""Benchmark of the htree hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload C2] [--no-cpu] [--no-modes]

Other workloads (--workload): C3, C4, C5, REF_FWD (the
reference's speed_test.py defaults: T=120000, Hq=64, Hkv=4, D=32, fp32, CR=16,
top_k=512, MTN=8192; forward only, as that script) and REF_BWD (its
speed_test_bwd.py defaults: T=12000, the same heads and tree).

Workload ("C2"): B=1, T=32768, Hq=32, Hkv=2 (group
16), D=128, bf16, causal, CR=16, MTN=128, TK=16; q/k/v/dO iid N(0,1) drawn
on the host from a fixed seed and copied to HBM before timing.

A step is what the reference's speed_test_bwd.py times: the autograd
forward (`htree_forward_triton_autograd`: tree build + fused kernel) and
`out.backward(dO)`, gradients in the input dtype, with q/k/v's gradients
cleared before each step; forward-only workloads step `htree_forward`.  The
autograd mode is the drop-in's default: it keeps the reference's eight
tensors plus the parent lists and the packed tree
(`saved_bytes_beyond_reference`), so the backward replays no selection and
rebuilds the candidate scores.  `value` = B*T / wall-clock step time over
the timed steps (tokens/s); `fwd` / `bwd` split each step with HIP events
(speed_test_bwd.py:109-123).  `modes` repeats the measurement (up to 10
steps) in the two other autograd modes: `scores` (`_save_scores=True`: the
candidate scores kept too, the backward reads them) and `lean`
(`_save_parents=False`: the reference's eight tensors only; the backward
rebuilds the tree and replays the selection).  The roofline object is for
the largest kernel (the fused forward), timed with HIP events on the stream
it runs on, against the gathered-bytes model in htree_amd/workmodel.py.
The CPU baseline times the CPU restatement of src/naive.py (oracle/, C on
every host core up to 16) on a bounded random sample of the same workload's
query rows: their whole forward and their whole backward (dq and the dK/dV
of every candidate they accumulate), and, as cpu_baseline.c1, the whole of
the CPU config C1 (forward and backward, median of 3); it is a reported
baseline only.

After those, the default C2 run measures C3, C4, C5 and REF_BWD (inputs
drawn on the GPU, 2 warm-up + 20 timed steps, 10 for C4; forward /
backward / bare-kernel times with HIP events) into `other_workloads` of the
same line; `--also ''` skips them.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "fwd & bwd tokens/s at T=32K, Hq=32/Hkv=2, D=128, bf16; % of HBM roofline"
HBM_PEAK = 8.0e12

WORKLOADS = {
    # name: (B, T, Hq, Hkv, D, CR, TK, MTN), dtype, backward in the step
    "C2": ((1, 32768, 32, 2, 128, 16, 16, 128), "bfloat16", True),
    "C3": ((4, 16384, 32, 4, 128, 16, 16, 128), "bfloat16", True),
    "C4": ((1, 131072, 64, 8, 128, 32, 32, 256), "bfloat16", True),
    "C5": ((2, 65536, 32, 2, 128, 16, 16, 128), "bfloat16", True),
    "REF_FWD": ((1, 120000, 64, 4, 32, 16, 512, 8192), "float32", False),
    "REF_BWD": ((1, 12000, 64, 4, 32, 16, 512, 8192), "float32", True),
}
DT_SHORT = {"bfloat16": "bf16", "float16": "f16", "float32": "f32"}


def forward_kernel(workload: str) -> str:
    """The fused forward kernel a workload runs: the wide form for top_k > 64
    or more than 64 candidate tiles of 16 per level, the register form up to
    16 tiles, the streaming form between."""
    (_, _, _, _, _, CR, TK, _), _, _ = WORKLOADS[workload]
    tiles = TK * max(CR, 16) // 16
    if TK > 64 or tiles > 64:
        return "fwd_wide_kernel"
    return "fwd_reg_kernel" if tiles <= 16 else "fwd_kernel"


def measured_traffic(workload: str):
    """HBM bytes per launch of the fused forward kernel from the committed
    rocprofv3 PMC summary of this workload (FETCH_SIZE + WRITE_SIZE, each
    scaled by the same counter's reading of the calibration copy), or None."""
    kern = forward_kernel(workload)
    path = os.path.join(ROOT, "profiles", f"{kern}_{workload.lower()}_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    return {"bytes": rec["traffic_bytes_per_launch"], "source": os.path.relpath(path, ROOT)}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def host_threads() -> int:
    """Host threads for the CPU legs: every core os.cpu_count() reports, at
    most the 16 a one-GPU box's share holds."""
    return max(1, min(16, os.cpu_count() or 1))


def cpu_baseline(q, k, v, dO, out, gmax, gsum, parents, CR, TK, MTN, dtype, budget_s=10.0):
    """Oracle (CPU restatement of src/naive.py, C, on host_threads() threads)
    on random query rows of the workload until `budget_s` seconds of forward
    work have run, then the same rows through the whole backward
    (src/naive.py:320-386 for those rows: dq, and the dK / dV of every
    candidate they accumulate scattered into the per-level gradients)."""
    import numpy as np

    from oracle import oracle as orc

    B, T, H, D = q.shape
    th = host_threads()
    qn = q.float().cpu().numpy()
    tree = orc.Tree(k.float().cpu().numpy(), v.float().cpu().numpy(), CR, MTN, TK, dtype)
    rng = np.random.default_rng(0)
    done, t_fwd, rows_all = 0, 0.0, []
    while t_fwd < budget_s and done < B * T:
        rows = np.stack([rng.integers(0, B, 32 * th), rng.integers(0, T, 32 * th)], 1).astype(np.int32)
        t0 = time.perf_counter()
        orc.forward_threaded(qn, tree, D ** -0.5, th, rows=rows)
        t_fwd += time.perf_counter() - t0
        done += len(rows)
        rows_all.append(rows)
    rows = np.concatenate(rows_all)
    res = dict(fwd_tok_s=done / t_fwd, fwd_rows=done, fwd_s=t_fwd, threads=th)
    if parents is not None:
        par = parents.cpu().numpy()[:, rows[:, 0], rows[:, 1]]
        gm = gmax.cpu().numpy()[rows[:, 0], rows[:, 1]]
        gs = gsum.cpu().numpy()[rows[:, 0], rows[:, 1]]
        o = out.float().cpu().numpy()[rows[:, 0], rows[:, 1]]
        d = dO.float().cpu().numpy()[rows[:, 0], rows[:, 1]]
        delta = (o.astype(np.float64) * d).sum(-1).astype(np.float32)
        from concurrent.futures import ThreadPoolExecutor

        parts = orc.split_rows(np.arange(len(rows)), th)
        t0 = time.perf_counter()
        with ThreadPoolExecutor(len(parts)) as ex:
            list(ex.map(lambda i: orc.backward_rows(qn, tree, D ** -0.5, rows[i], par[:, i], gm[i],
                                                    gs[i], delta[i], d[i], with_dkv=False), parts))
        t_bwd = time.perf_counter() - t0
        res.update(bwd_tok_s=len(rows) / t_bwd, bwd_s=t_bwd)
    return res


def cpu_leg_c1(iters: int = 3):
    """The CPU baseline planned for the BASELINE.json CPU config C1 (B=1,
    T=2048, Hq=4, Hkv=1, D=64, fp32, CR=16, MTN=64, TK=8; q/k/v/dO iid N(0,1)
    from a fixed seed): the oracle's whole forward (tree build included) and
    whole analytical backward (src/naive.py:133-396 restated) on
    host_threads() threads, one warm-up and `iters` timed runs, median."""
    import numpy as np
    import torch

    from oracle import oracle as orc

    B, T, H, Hkv, D, CR, TK, MTN = 1, 2048, 4, 1, 64, 16, 8, 64
    g = torch.Generator().manual_seed(7)
    q, k, v, dO = (torch.randn(*s, generator=g).numpy()
                   for s in ((B, T, H, D), (B, T, Hkv, D), (B, T, Hkv, D), (B, T, H, D)))
    th = host_threads()
    tf, tb = [], []
    for _ in range(1 + iters):
        t0 = time.perf_counter()
        tree = orc.Tree(k, v, CR, MTN, TK, "float32")
        fw = orc.forward_threaded(q, tree, D ** -0.5, th)
        t1 = time.perf_counter()
        L = tree.L
        orc.backward_threaded(q, tree, D ** -0.5, fw["parents"].reshape(L, B, T, Hkv, TK),
                              fw["gmax"].reshape(B, T, H), fw["gsum"].reshape(B, T, H),
                              fw["out"].reshape(B, T, H, D), dO, th)
        t2 = time.perf_counter()
        tf.append(t1 - t0)
        tb.append(t2 - t1)
    f, b = float(np.median(tf[1:])), float(np.median(tb[1:]))
    return {"config": f"C1: B={B} T={T} Hq={H} Hkv={Hkv} D={D} f32 CR={CR} MTN={MTN} TK={TK}",
            "threads": th, "fwd_s": f, "bwd_s": b, "fwd_tokens_per_s": B * T / f,
            "bwd_tokens_per_s": B * T / b, "tokens_per_s": B * T / (f + b),
            "timing": f"1 warm-up + {iters} runs, median wall-clock"}


def make_inputs(workload, dev, on_gpu=False):
    """Seeded synthetic q, k, v, dO of a workload in HBM (drawn on the host
    for the headline run, on the GPU for the short extra runs)."""
    import torch

    (B, T, H, Hkv, D, CR, TK, MTN), dtype, _ = WORKLOADS[workload]
    tdt = getattr(torch, dtype)
    gdev = dev if on_gpu else torch.device("cpu")
    g = torch.Generator(device=gdev).manual_seed(1234)
    rn = lambda *shape: torch.randn(*shape, generator=g, device=gdev)
    where = "the GPU" if on_gpu else "the host"
    if workload == "C5":
        # C5: keys from a 64-component Gaussian mixture (means
        # N(0, 4 I), sigma 0.5), queries around 4 hot components, V and dO iid
        mu = 2.0 * rn(64, D)
        hot = torch.randperm(64, generator=g, device=gdev)[:4]
        k = mu[torch.randint(0, 64, (B, T, Hkv), generator=g, device=gdev)] + 0.5 * rn(B, T, Hkv, D)
        q = mu[hot[torch.randint(0, 4, (B, T, H), generator=g, device=gdev)]] + 0.5 * rn(B, T, H, D)
        v = rn(B, T, Hkv, D)
        dO = rn(B, T, H, D)
        q, k, v, dO = (x.to(tdt).to(dev) for x in (q, k, v, dO))
        data = (f"synthetic: C5 skewed keys/queries (64-component mixture, 4 hot), v,dO iid N(0,1), "
                f"seed 1234 on {where}")
    else:
        q = rn(B, T, H, D).to(tdt).to(dev)
        k = rn(B, T, Hkv, D).to(tdt).to(dev)
        v = rn(B, T, Hkv, D).to(tdt).to(dev)
        dO = rn(B, T, H, D).to(tdt).to(dev)
        data = f"synthetic: q,k,v,dO iid N(0,1) from torch.Generator seed 1234 on {where}"
    return q, k, v, dO, data


MODES = {
    # autograd mode: (htree_forward_triton_autograd keyword arguments, what it keeps)
    "default": ({}, "the reference's eight tensors + the parent lists and the packed tree; "
                    "the backward rebuilds the candidate scores"),
    "scores": ({"_save_scores": True}, "the default's tensors + every candidate tile's scores; "
                                       "the backward reads them"),
    "lean": ({"_save_parents": False}, "the reference's eight tensors only; the backward rebuilds "
                                       "the tree and replays the selection"),
}


def measure(workload, q, k, v, dO, steps, warmup, kernel_iters, mode_steps=0):
    """Times `steps` steps (wall clock, after `warmup`), with HIP events
    around each step's forward and backward (speed_test_bwd.py:109-123),
    then `mode_steps` steps in each other autograd mode, then `kernel_iters`
    bare launches of the fused forward kernel with HIP events on their
    stream.  A training step is the autograd forward
    (`htree_forward_triton_autograd`, default mode) and `out.backward(dO)`
    with the gradients of q, k, v cleared first, as the reference's
    speed_test_bwd.py times it.  Returns the figures and a forward's output
    and context."""
    import torch

    import htree_amd
    from htree_amd import _native as N
    from htree_amd.workmodel import work

    (B, T, H, Hkv, D, CR, TK, MTN), dtype, with_bwd = WORKLOADS[workload]
    dev = q.device
    has_bwd = with_bwd and hasattr(htree_amd, "htree_backward")
    if has_bwd:
        q, k, v = (x.detach().requires_grad_(True) for x in (q, k, v))
    stream = torch.cuda.current_stream(dev)
    ev = lambda: torch.cuda.Event(enable_timing=True)

    def step(marks=None, mode="default"):
        if marks:
            marks[0].record(stream)
        if not has_bwd:  # forward only (speed_test.py): nothing kept for a backward
            htree_amd.htree_forward(q, k, v, CR, MTN, TK)
            if marks:
                marks[1].record(stream)
            return
        q.grad = k.grad = v.grad = None
        out = htree_amd.htree_forward_triton_autograd(q, k, v, CR, MTN, TK, **MODES[mode][0])
        if marks:
            marks[1].record(stream)
        out.backward(dO)
        if marks:
            marks[2].record(stream)

    def timed(steps, warmup, mode="default"):
        for _ in range(warmup):
            step(mode=mode)
        torch.cuda.synchronize()
        marks = [[ev(), ev(), ev()] for _ in range(steps)]
        t0 = time.perf_counter()
        for i in range(steps):
            step(marks[i], mode)
        torch.cuda.synchronize()
        step_ms = (time.perf_counter() - t0) * 1e3 / steps
        fwd_ms = sum(m[0].elapsed_time(m[1]) for m in marks) / steps
        bwd_ms = sum(m[1].elapsed_time(m[2]) for m in marks) / steps if has_bwd else None
        print(f"# {workload} ({mode} mode): timed {steps} steps: {step_ms:.3f} ms/step "
              f"(forward {fwd_ms:.3f} ms" + (f", backward {bwd_ms:.3f} ms" if has_bwd else "") + ")",
              file=sys.stderr, flush=True)
        return step_ms, fwd_ms, bwd_ms

    step_ms, fwd_ms, bwd_ms = timed(steps, warmup)
    # the other autograd modes, after the above
    modes = {}
    if has_bwd and mode_steps:
        for mode in ("scores", "lean"):
            modes[mode] = dict(zip(("step_ms", "fwd_ms", "bwd_ms"), timed(mode_steps, 2, mode)))

    # the fused forward kernel alone, with HIP events
    with torch.no_grad():
        out, ctx = htree_amd.htree_forward(q.detach(), k.detach(), v.detach(), CR, MTN, TK,
                                           _save_for_backward=True, _save_scores=has_bwd)
    q = q.detach()
    d = ctx["dims"]
    ws = ctx["packed_tree"]
    cos, sin = ctx["cos_cache"], ctx["sin_cache"]
    gmax, gsum = ctx["global_max"], ctx["global_sum"]
    lib = N.lib()
    scale = float(D ** -0.5)
    sp = N.stream_ptr(dev)
    k0, k1 = ev(), ev()
    k0.record(stream)
    for _ in range(kernel_iters):
        rc = lib.htree_forward(d, scale, N.ptr(q), N.ptr(ws), ws.numel(), N.ptr(cos), N.ptr(sin),
                               N.ptr(out), N.ptr(gmax), N.ptr(gsum), None, sp)
        N.check(rc, "htree_forward")
    k1.record(stream)
    torch.cuda.synchronize()
    kern_ms = k0.elapsed_time(k1) / kernel_iters
    w = work(B, T, H, Hkv, D, CR, TK, MTN, getattr(torch, dtype).itemsize)
    saved = {}
    if has_bwd:  # bytes each mode keeps per call beyond the reference's eight tensors
        nb = lambda t: 0 if t is None else t.numel() * t.element_size()
        saved["default"] = nb(ctx["parents_stacked"]) + nb(ctx["packed_tree"])
        saved["scores"] = saved["default"] + nb(ctx.get("train_scores"))
        saved["lean"] = 0
    return dict(has_bwd=has_bwd, step_ms=step_ms, fwd_ms=fwd_ms, bwd_ms=bwd_ms, kern_ms=kern_ms,
                work=w, out=out, ctx=ctx, modes=modes, saved_bytes=saved)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="C2", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--kernel-iters", type=int, default=20)
    ap.add_argument("--no-modes", action="store_true",
                    help="skip the other autograd modes' measurement")
    ap.add_argument("--also", default=None,
                    help="comma-separated workloads measured after the main one "
                         "(20 steps each, 10 for C4; default for C2: C3,C4,C5,REF_BWD; '' for none)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported in this build "
              "(the path shards over (b, h_kv) with no communication between the shards)",
              file=sys.stderr)
        sys.exit(2)
    also = args.also if args.also is not None else ("C3,C4,C5,REF_BWD" if args.workload == "C2" else "")
    also = [w for w in also.split(",") if w]
    for w in also:
        if w not in WORKLOADS:
            ap.error(f"--also: unknown workload {w}")

    import torch

    (B, T, H, Hkv, D, CR, TK, MTN), dtype, with_bwd = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    q, k, v, dO, data = make_inputs(args.workload, dev)
    torch.cuda.synchronize()
    print(f"# workload {args.workload} B={B} T={T} H={H} Hkv={Hkv} D={D} {dtype} CR={CR} TK={TK} "
          f"MTN={MTN}", file=sys.stderr, flush=True)
    m = measure(args.workload, q, k, v, dO, args.steps, args.warmup, args.kernel_iters,
                mode_steps=min(args.steps, 10) if not args.no_modes else 0)
    has_bwd, fwd_ms, bwd_ms, kern_ms, w = m["has_bwd"], m["fwd_ms"], m["bwd_ms"], m["kern_ms"], m["work"]
    out, ctx = m["out"], m["ctx"]

    # Calibration copy for the PMC traffic measurement (outside every timed
    # region): 256 MiB read + 256 MiB written by torch's copy kernel, so that a
    # `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE` run of this script measures
    # the counters' scale on a transfer of known size.
    cal_src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
    cal_dst = torch.empty_like(cal_src)
    cal_dst.copy_(cal_src)
    torch.cuda.synchronize()
    del cal_src, cal_dst

    traffic = measured_traffic(args.workload)
    achieved = w.fwd_kernel_bytes / (kern_ms * 1e-3)
    fwd_tok = B * T / (fwd_ms * 1e-3)
    step_s = m["step_ms"] * 1e-3
    res = {
        "metric": METRIC if args.workload == "C2" else
        f"{'fwd & bwd' if has_bwd else 'fwd'} tokens/s at {args.workload}; % of HBM roofline",
        "value": B * T / step_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": m["step_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DT_SHORT[dtype],
        "data": data,
        "config": {
            "workload": f"{args.workload}: B={B} T={T} Hq={H} Hkv={Hkv} D={D} {DT_SHORT[dtype]} "
                        f"causal CR={CR} MTN={MTN} TK={TK}",
            "step": ("htree_forward_triton_autograd + out.backward(dO)" if has_bwd
                     else "htree_forward"),
            "autograd_mode": "default: " + MODES["default"][1] if has_bwd else None,
        },
        "fwd": {"ms": fwd_ms, "tokens_per_s": fwd_tok,
                "hbm_roofline_frac": w.fwd_bytes / (fwd_ms * 1e-3) / HBM_PEAK,
                "algorithmic_bytes": w.fwd_bytes},
        "bwd": None if not has_bwd else {
            "ms": bwd_ms, "tokens_per_s": B * T / (bwd_ms * 1e-3),
            "hbm_roofline_frac": w.bwd_bytes / (bwd_ms * 1e-3) / HBM_PEAK,
            "algorithmic_bytes": w.bwd_bytes},
        "event_ms_per_step": fwd_ms + (bwd_ms or 0.0),
        "saved_bytes_beyond_reference": m["saved_bytes"].get("default"),
        "modes": {
            mode: {
                "call": "htree_forward_triton_autograd(..., "
                        + ", ".join(f"{a}={b}" for a, b in MODES[mode][0].items()) + ")",
                "keeps": MODES[mode][1],
                "ms_per_step": r["step_ms"], "tokens_per_s": B * T / (r["step_ms"] * 1e-3),
                "fwd_ms": r["fwd_ms"], "bwd_ms": r["bwd_ms"],
                "bwd_hbm_roofline_frac": w.bwd_bytes / (r["bwd_ms"] * 1e-3) / HBM_PEAK,
                "saved_bytes_beyond_reference": m["saved_bytes"][mode]}
            for mode, r in m["modes"].items()} or None,
        "roofline": {
            "kernel": f"htree::{forward_kernel(args.workload)} (fused forward, all levels)",
            "bound": "hbm",
            "achieved": achieved / 1e9,
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK,
            "traffic": traffic["bytes"] if traffic else None,
            "traffic_source": traffic["source"] if traffic else None,
            "algorithmic_bytes_per_launch": w.fwd_kernel_bytes,
            "avg_launch_ms": kern_ms,
        },
    }
    if not args.no_cpu:
        cb = cpu_baseline(q, k, v, dO, out, ctx["global_max"], ctx["global_sum"],
                          ctx.get("parents_stacked") if has_bwd else None, CR, TK, MTN, dtype)
        tot = 1.0 / (1.0 / cb["fwd_tok_s"] + (1.0 / cb["bwd_tok_s"] if has_bwd and "bwd_tok_s" in cb else 0.0))
        res["cpu_baseline"] = {
            "value": tot, "unit": "tokens/s", "cores": cb["threads"], "kind": "port",
            "sample": f"{cb['fwd_rows']} random query rows (b,t) of {args.workload} through the "
                      f"oracle's whole forward ({cb['fwd_s']:.1f} s)"
                      + (f" and whole backward (dq, and the dK/dV of every candidate they "
                         f"accumulate, {cb['bwd_s']:.1f} s)" if "bwd_s" in cb else "")
                      + f", {cb['threads']} host threads; host CPU: {cpu_model()}, "
                      f"os.cpu_count()={os.cpu_count()}",
            "fwd_tokens_per_s": cb["fwd_tok_s"],
            "bwd_tokens_per_s": cb.get("bwd_tok_s"),
            "c1": cpu_leg_c1(),
        }
    else:
        res["cpu_baseline"] = None

    # the other BASELINE workloads, briefly (after every timed region above)
    if also:
        del q, k, v, dO, out, ctx, m
        torch.cuda.empty_cache()
        res["other_workloads"] = {}
    for wl in also:
        (B2, T2, H2, Hkv2, D2, CR2, TK2, MTN2), dt2, _ = WORKLOADS[wl]
        q2, k2, v2, dO2, data2 = make_inputs(wl, dev, on_gpu=True)
        n2 = 10 if wl == "C4" else 20
        m2 = measure(wl, q2, k2, v2, dO2, steps=n2, warmup=2, kernel_iters=3)
        w2 = m2["work"]
        res["other_workloads"][wl] = {
            "config": f"B={B2} T={T2} Hq={H2} Hkv={Hkv2} D={D2} {DT_SHORT[dt2]} CR={CR2} MTN={MTN2} "
                      f"TK={TK2}",
            "data": data2,
            "steps": n2, "warmup": 2,
            "tokens_per_s": B2 * T2 / (m2["step_ms"] * 1e-3),
            "fwd_ms": m2["fwd_ms"],
            "fwd_hbm_roofline_frac": w2.fwd_bytes / (m2["fwd_ms"] * 1e-3) / HBM_PEAK,
            "bwd_ms": m2["bwd_ms"],
            "bwd_hbm_roofline_frac": (w2.bwd_bytes / (m2["bwd_ms"] * 1e-3) / HBM_PEAK
                                      if m2["bwd_ms"] else None),
            "kernel_ms": m2["kern_ms"],
            "kernel_hbm_roofline_frac": w2.fwd_kernel_bytes / (m2["kern_ms"] * 1e-3) / HBM_PEAK,
            "ms_per_step": m2["step_ms"],
        }
        del q2, k2, v2, dO2, m2
        torch.cuda.empty_cache()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
