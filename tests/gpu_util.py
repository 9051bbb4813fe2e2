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
                  tree=None, gmax_dev=None, gsum_dev=None):
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
    decisions = 0
    for l in range(L - 1, 0, -1):
        res = compare_selection(par[l - 1], fw["sel"][l], fw["imp"][l], par[l], CR,
                                arg_ref=fw["imparg"][l])
        rep["mismatch"][l] = res["n"] - res["exact"]
        rep["excused"][l] = res["excused"]
        decisions += res["n"]
        assert not res["bad"], f"level {l}: selection outside the tie band: {res['bad'][:4]}"
    # swaps inside the tie band are rare: at most one per 1000 decisions, plus one
    excused = sum(rep["excused"].values())
    assert excused <= 1 + decisions // 1000, f"{excused} excused swaps in {decisions} decisions"
    got = out_dev[rows[:, 0], rows[:, 1]]
    ok, worst = close(got, fw["out"], dtype)
    rep["out_worst"] = worst
    assert ok, f"output outside tolerance: worst {worst:.3f} of the bar"
    if gmax_dev is not None:
        rep.update(check_state(gmax_dev[rows[:, 0], rows[:, 1]], gsum_dev[rows[:, 0], rows[:, 1]],
                               fw["gmax"], fw["gsum"], dtype))
    return rep


# online-softmax state bars: the max is one score, |err| <= atol + rtol |max|
# (16-bit inputs: the split-bf16 score product); the sum's relative error
# follows the scores' (exp(s - max) moves by the score error)
STATE_TOL = {"bfloat16": (2e-3, 1e-3, 3e-3), "float16": (2e-3, 1e-3, 3e-3),
             "float32": (1e-4, 1e-4, 2e-4)}


def check_state(gmax, gsum, ref_max, ref_sum, dtype):
    """gmax / gsum [n, H] of the device against the oracle's: the max over
    the accumulated candidates and the sum of exp(s - max) over them."""
    atol, rtol, srtol = STATE_TOL[dtype]
    gm = np.abs(gmax.astype(np.float64) - ref_max) / (atol + rtol * np.abs(ref_max))
    gs = np.abs(gsum.astype(np.float64) - ref_sum) / (srtol * np.abs(ref_sum))
    rep = dict(gmax_worst=float(gm.max()), gsum_worst=float(gs.max()))
    assert rep["gmax_worst"] <= 1 and rep["gsum_worst"] <= 1, rep
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
                      fw["gsum"].reshape(B, T, H), out_dev.reshape(B, T, H, -1), dO.float().numpy())
    return bw, fw


def check_backward(q, k, v, dO, CR, TK, MTN, dtype, out_dev, parents_dev, gmax_dev, gsum_dev,
                   dq, dk, dv, tree=None, rope_base=10000.0):
    """Device grads (fp32 numpy) vs the oracle's, same selection; bar as TOL."""
    if tree is None:
        tree = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, dtype, rope_base)
    bw, _ = oracle_grads(q, k, v, dO, CR, TK, MTN, dtype, parents_dev, out_dev, tree)
    rep = {}
    for name, got, ref in (("dq", dq, bw["dq"]), ("dk", dk, bw["dk"]), ("dv", dv, bw["dv"])):
        ok, worst = close(got, ref, dtype)
        rep[name] = worst
        assert np.all(np.isfinite(got)), f"{name} not finite"
        assert ok, f"{name} outside tolerance: worst {worst:.3f} of the bar"
    return rep


def dkv_nodes_for_pair(tree, par_bh, T, CR, rng, n_random=8):
    """Level-0 nodes to check in one (b, h_kv): the children (up to 16,
    always the last) of a random level-1 parent and of the last one, plus
    random nodes; level-1 is the pooled parent of CR level-0 nodes."""
    L = tree.L
    nodes = set(rng.choice(T, min(T, n_random), replace=False).tolist())
    if L > 1:
        P0 = -(-T // CR)
        for p in (int(rng.integers(0, max(1, P0 - 1))), P0 - 1):
            kids = list(range(p * CR, min(p * CR + CR, T)))
            pick = kids if len(kids) <= 16 else sorted(
                set(rng.choice(kids[:-1], 15, replace=False).tolist()) | {kids[-1]})
            nodes |= set(pick)
    nodes |= {0, T - 1}
    return np.array(sorted(nodes), np.int64)


def check_dkv_sampled(q, dO, out, k, v, parents, gmax, gsum, dk, dv, CR, TK, MTN, dtype, pairs,
                      seed, scale=None):
    """Final dk / dv of the device at sampled level-0 nodes of the (b, h_kv)
    pairs listed, against the oracle's per-level terms combined with the
    mean-pool factors (src/naive.py:365-394), at the bar of `dtype`.

    The backward is a function of (q, k, v, dO, out, gmax, gsum, parents)
    (src/backward.py:941-1119): the oracle gets the device's forward state for
    those, so this checks the backward kernels alone; the forward state is
    checked against the oracle separately.  Arguments may be device tensors
    or host arrays ([B,T,H,D], [B,T,Hkv,D], [L,B,T,Hkv,TK], [B,T,H])."""
    tnp = lambda x, *ix: (x[ix].float().cpu().numpy() if hasattr(x, "cpu")
                          else np.asarray(x[ix], np.float32))
    B, T, H, D = q.shape
    Hkv = k.shape[2]
    G = H // Hkv
    if scale is None:
        scale = D ** -0.5
    rng = np.random.default_rng(seed)
    rep = {}
    for (b, h) in pairs:
        hs = slice(h * G, (h + 1) * G)
        qs = tnp(q, slice(b, b + 1), slice(None), hs)
        dOs = tnp(dO, slice(b, b + 1), slice(None), hs)
        os_ = tnp(out, slice(b, b + 1), slice(None), hs)
        dl = (os_.astype(np.float64) * dOs).sum(-1).astype(np.float32)
        gm = tnp(gmax, slice(b, b + 1), slice(None), hs)
        gs = tnp(gsum, slice(b, b + 1), slice(None), hs)
        ks = tnp(k, slice(b, b + 1), slice(None), slice(h, h + 1))
        vs = tnp(v, slice(b, b + 1), slice(None), slice(h, h + 1))
        ps = parents[:, b:b + 1, :, h:h + 1]
        ps = np.ascontiguousarray(ps.cpu().numpy() if hasattr(ps, "cpu") else ps, np.int32)
        tree = orc.Tree(ks, vs, CR, MTN, TK, dtype)
        nodes = dkv_nodes_for_pair(tree, ps, T, CR, rng)
        tg = np.stack([np.zeros_like(nodes), np.zeros_like(nodes), nodes], 1)
        rk, rv = orc.final_dkv_level0(qs, tree, scale, ps, gm, gs, dl, dOs, tg)
        ix = torch.from_numpy(nodes) if hasattr(dk, "cpu") else nodes
        gk = dk[b, ix.to(dk.device) if hasattr(dk, "cpu") else ix, h]
        gv = dv[b, ix.to(dv.device) if hasattr(dv, "cpu") else ix, h]
        gk = gk.float().cpu().numpy() if hasattr(gk, "cpu") else np.asarray(gk)
        gv = gv.float().cpu().numpy() if hasattr(gv, "cpu") else np.asarray(gv)
        okk, wk = close(gk, rk, dtype)
        okv, wv = close(gv, rv, dtype)
        rep[(b, h)] = dict(nodes=len(nodes), dk=wk, dv=wv)
        assert np.abs(rk).max() > 0 and np.abs(rv).max() > 0
        assert okk, f"dk at ({b}, {h}) outside tolerance: worst {wk:.3f} of the bar"
        assert okv, f"dv at ({b}, {h}) outside tolerance: worst {wv:.3f} of the bar"
    return rep
