"""Shared test helpers: fixture loading, dtype bit conversion and the
selection comparison rule used everywhere a Top-K result is compared.

Selection tie rule (the parity bar for node indices):
  At (level, row, kv head) two selections A (under test) and B (oracle) agree
  when A == B, or when every node in the symmetric difference has an oracle
  importance within a tie band of the oracle's TK-th largest importance th:
      |imp(x) - th| <= TIE_RTOL * th + TIE_ATOL
  Importances are the reference's sum_g exp(s_g - max s) (<= G, the forced
  rightmost is 1e6).  TIE_RTOL is the north star's 1e-3 score tie; TIE_ATOL
  covers candidates whose weight is below 1e-6 of the leading one.
  Rows are compared only where the previous level's parents matched (the
  cascade rule of the reference's compare_traces, correctness_test.py:409-431).

Exact ties are held exactly.  An importance is 0 exactly when every term
exp(s_g - max) underflows in fp32 (argument below ln 2^-150 = -103.97, with
subnormal results kept, as the oracle's expf and the kernels' exponential
both do).  Given the oracle's largest exponent argument a(x) of each
candidate, a candidate with a(x) < ZERO_ARG is 0 on both sides and one with
a(x) > NONZERO_ARG is positive on both (the margins are orders of magnitude
above any score error).  If the selection under test took x, a certain
zero, and left out y that the oracle took, it must have seen y as exactly 0
too (so y is not a certain nonzero), and then the stable order puts the
lower flat position first, so x must come before y; anything else is a
violation that the tie band does not excuse (src/naive.py:94).
"""
from __future__ import annotations

import os
from typing import Dict, Tuple

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TIE_RTOL = 1e-3
TIE_ATOL = 1e-6
# exp(x) rounds to 0 in fp32 below ln(2^-150) = -103.97; 0.5 of margin each side
ZERO_ARG = -104.47
NONZERO_ARG = -103.47

TORCH_DT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


def from_native(a: np.ndarray, dtype: str) -> np.ndarray:
    """uint16 bit patterns (bf16/fp16) or fp32 -> fp32 values."""
    if dtype == "float32":
        return a.astype(np.float32)
    t = torch.from_numpy(a.view(np.int16).copy()).view(TORCH_DT[dtype])
    return t.float().numpy()


def load_golden(name: str) -> Dict:
    from tests.golden.make_golden import golden_inputs, inputs_sha

    z = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    B, T, H, Hkv, D, CR, TK, MTN, seed = [int(x) for x in z["config"]]
    dtype = str(z["dtype"])
    q, k, v, dO = golden_inputs(B, T, H, Hkv, D, dtype, seed)
    assert inputs_sha(q, k, v, dO) == str(z["inputs_sha256"]), \
        "regenerated inputs differ from the ones the fixture was made with"
    L = int(z["num_layers"])
    rec = dict(B=B, T=T, H=H, Hkv=Hkv, D=D, CR=CR, TK=TK, MTN=MTN, dtype=dtype, L=L,
               q=q, k=k, v=v, dO=dO, scale=D ** -0.5)
    for key in ("out", "out_autograd", "dq", "dk", "dv"):
        rec[key] = from_native(z[key], dtype)
    for l in range(L):
        rec[f"lmax_l{l}"] = z[f"lmax_l{l}"]
        rec[f"lsum_l{l}"] = z[f"lsum_l{l}"]
        if f"parents_l{l}" in z:
            rec[f"parents_l{l}"] = z[f"parents_l{l}"].astype(np.int32)
    return rec


def compare_selection(sel_test: np.ndarray, sel_ref: np.ndarray, imp_ref: np.ndarray,
                      par_ref: np.ndarray, CR: int, prev_ok: np.ndarray = None,
                      rtol: float = TIE_RTOL, atol: float = TIE_ATOL,
                      arg_ref: np.ndarray = None) -> Dict:
    """Compare two selections [n, Hkv, TK] (ascending node ids, -1 padded).

    imp_ref [n, Hkv, TK*CR]: the oracle's importance per flat position (-1 past nc).
    par_ref [n, Hkv, TK]: the parent list the oracle expanded at this level
    (maps flat position j -> node = valid_parents[j // CR] * CR + j % CR).
    prev_ok [n, Hkv]: rows whose previous-level parents matched (cascade rule).
    arg_ref [n, Hkv, TK*CR]: the oracle's largest exponent argument per flat
    position (the oracle forward's `imparg`); with it, swaps that only the
    tie order decides are held to that order (module docstring).
    Returns counts and a boolean exact-match mask."""
    n, Hkv, TK = sel_test.shape
    exact = np.all(sel_test == sel_ref, axis=-1)
    if prev_ok is None:
        prev_ok = np.ones((n, Hkv), bool)
    bad = []
    excused = 0
    for r, h in zip(*np.nonzero(~exact & prev_ok)):
        A = set(int(x) for x in sel_test[r, h] if x >= 0)
        Bset = set(int(x) for x in sel_ref[r, h] if x >= 0)
        vp = [int(x) for x in par_ref[r, h] if x >= 0]
        imp = imp_ref[r, h]
        nc = int(np.sum(imp >= 0))
        node_imp, node_arg = {}, {}
        for j in range(nc):
            node = vp[j // CR] * CR + j % CR
            node_imp[node] = float(imp[j])
            if arg_ref is not None:
                node_arg[node] = float(arg_ref[r, h, j])
        srt = np.sort(imp[:nc])[::-1]
        th = float(srt[min(TK, nc) - 1])
        ok = True
        for x in A ^ Bset:
            if x not in node_imp or abs(node_imp[x] - th) > rtol * th + atol:
                ok = False
        if ok and arg_ref is not None:
            # (flat position order is node order: the parent lists ascend)
            for x in A - Bset:
                if node_arg[x] >= ZERO_ARG:
                    continue
                for y in Bset - A:
                    if node_arg[y] > NONZERO_ARG or y < x:
                        ok = False
        if ok:
            excused += 1
        else:
            bad.append((int(r), int(h), sorted(A - Bset), sorted(Bset - A), th))
    return dict(n=int(n * Hkv), exact=int(exact.sum()), excused=excused, bad=bad,
                exact_mask=exact)


def round_np(x: np.ndarray, dtype: str) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(TORCH_DT[dtype]).float().numpy()


def ulp_close(a: np.ndarray, b: np.ndarray, dtype: str, ulps: float = 2.0,
              atol: float = 0.0) -> Tuple[bool, float]:
    """|a-b| <= ulps * ulp(max(|a|,|b|)) + atol in the given dtype."""
    mant = {"float32": 23, "bfloat16": 7, "float16": 10}[dtype]
    mag = np.maximum(np.abs(a), np.abs(b)).astype(np.float64)
    e = np.floor(np.log2(np.maximum(mag, 1e-38)))
    ulp = np.exp2(e - mant)
    err = np.abs(a.astype(np.float64) - b)
    worst = float(np.max(err / (ulp + 1e-300))) if err.size else 0.0
    return bool(np.all(err <= ulps * ulp + atol)), worst
