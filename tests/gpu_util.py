"""Helpers shared by the GPU parity tests: seeded CPU inputs (bit-identical
for the oracle and the device), oracle runs teacher-forced on the device's
own parent lists, and the tolerance bars."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as orc
from tests.helpers import compare_selection

DT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}

# output / gradient bars: |a - b| <= atol + rtol * |b|
TOL = {"bfloat16": (2e-2, 1e-2), "float32": (1e-4, 1e-4), "float16": (2e-3, 2e-3)}


def inputs(B, T, H, Hkv, D, dtype, seed, dO=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g).to(DT[dtype])
    k = torch.randn(B, T, Hkv, D, generator=g).to(DT[dtype])
    v = torch.randn(B, T, Hkv, D, generator=g).to(DT[dtype])
    if dO:
        return q, k, v, torch.randn(B, T, H, D, generator=g).to(DT[dtype])
    return q, k, v


def skewed_inputs(B, T, H, Hkv, D, dtype, seed, ncomp=64, nhot=4):
    """Keys from a 64-component Gaussian mixture (means N(0,4), sigma 0.5),
    queries around 4 hot components, V iid N(0,1) (the C5 workload)."""
    g = torch.Generator().manual_seed(seed)
    mu = 2.0 * torch.randn(ncomp, D, generator=g)
    hot = torch.randperm(ncomp, generator=g)[:nhot]
    ck = torch.randint(0, ncomp, (B, T, Hkv), generator=g)
    k = mu[ck] + 0.5 * torch.randn(B, T, Hkv, D, generator=g)
    cq = hot[torch.randint(0, nhot, (B, T, H), generator=g)]
    q = mu[cq] + 0.5 * torch.randn(B, T, H, D, generator=g)
    v = torch.randn(B, T, Hkv, D, generator=g)
    dO = torch.randn(B, T, H, D, generator=g)
    return q.to(DT[dtype]), k.to(DT[dtype]), v.to(DT[dtype]), dO.to(DT[dtype])


def close(a: np.ndarray, b: np.ndarray, dtype: str):
    atol, rtol = TOL[dtype]
    err = np.abs(a.astype(np.float64) - b.astype(np.float64))
    bound = atol + rtol * np.abs(b.astype(np.float64))
    return bool(np.all(err <= bound)), float(np.max(err / bound)) if err.size else 0.0


def check_forward(q, k, v, CR, TK, MTN, dtype, rows=None, out_dev=None, parents_dev=None,
                  tree=None):
    """Checks a device forward (out [B,T,H,D], parents [L,B,T,Hkv,TK]) against
    the oracle on `rows` ([n,2] of (b,t); default all), teacher-forced on the
    device's parent lists.  Returns a report dict; raises AssertionError on a
    selection outside the tie band or an output outside the bar."""
    B, T, H, D = q.shape
    Hkv = k.shape[2]
    if tree is None:
        tree = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, dtype)
    L = tree.L
    if rows is None:
        rows = orc.all_rows(B, T)
    rows = np.ascontiguousarray(rows, np.int32)
    par = parents_dev[:, rows[:, 0], rows[:, 1]]  # [L, n, Hkv, TK]
    fw = orc.forward(q.float().numpy(), tree, D ** -0.5, rows=rows, forced=par)
    rep = dict(rows=len(rows), levels=L, mismatch={}, excused={})
    # initial parents are data independent
    assert np.array_equal(fw["parents"][L - 1], par[L - 1]), "initial parent lists differ"
    for l in range(L - 1, 0, -1):
        res = compare_selection(par[l - 1], fw["sel"][l], fw["imp"][l], par[l], CR)
        rep["mismatch"][l] = res["n"] - res["exact"]
        rep["excused"][l] = res["excused"]
        assert not res["bad"], f"level {l}: selection outside the tie band: {res['bad'][:4]}"
    got = out_dev[rows[:, 0], rows[:, 1]]
    ok, worst = close(got, fw["out"], dtype)
    rep["out_worst"] = worst
    assert ok, f"output outside tolerance: worst {worst:.3f} of the bar"
    return rep


def oracle_grads(q, k, v, dO, CR, TK, MTN, dtype, parents_dev, out_dev, tree=None):
    """Oracle gradients (src/naive.py:320-396 restated) with the selection
    held at the device's parent lists: oracle forward teacher-forced on them
    (gmax, gsum), then the analytical backward.  The backward is a function
    of the `output` it is handed (delta = rowsum(dO * output),
    src/backward.py:966-976), so the oracle gets the device's output: a
    1-ulp difference of the two forwards' rounded outputs would otherwise
    reach dq through delta times the keys' common mean."""
    B, T, H, D = q.shape
    if tree is None:
        tree = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, dtype)
    L = tree.L
    rows = orc.all_rows(B, T)
    par = np.ascontiguousarray(parents_dev.reshape(L, B * T, *parents_dev.shape[3:]))
    fw = orc.forward(q.float().numpy(), tree, D ** -0.5, rows=rows, forced=par)
    bw = orc.backward(q.float().numpy(), tree, D ** -0.5, parents_dev, fw["gmax"].reshape(B, T, H),
                      fw["gsum"].reshape(B, T, H), out_dev.reshape(B, T, H, D), dO.float().numpy())
    return bw, fw


def check_backward(q, k, v, dO, CR, TK, MTN, dtype, out_dev, parents_dev, gmax_dev, gsum_dev,
                   dq, dk, dv, tree=None):
    """Device grads (fp32 numpy) vs the oracle's, same selection; bar as TOL."""
    bw, _ = oracle_grads(q, k, v, dO, CR, TK, MTN, dtype, parents_dev, out_dev, tree)
    rep = {}
    for name, got, ref in (("dq", dq, bw["dq"]), ("dk", dk, bw["dk"]), ("dv", dv, bw["dv"])):
        ok, worst = close(got, ref, dtype)
        rep[name] = worst
        assert np.all(np.isfinite(got)), f"{name} not finite"
        assert ok, f"{name} outside tolerance: worst {worst:.3f} of the bar"
    return rep
