"""The GPU parity checkers, run on the CPU with the oracle's own results in
place of the device's: they accept a correct result and reject planted
mistakes (rows of dV swapped inside one parent, a shifted gmax), so a green
GPU run means the check ran, not that it looked away."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import check_dkv_sampled, check_state, inputs


@pytest.fixture(scope="module")
def case():
    B, T, H, Hkv, D, CR, TK, MTN, dtype = 2, 700, 8, 2, 32, 8, 8, 64, "float32"
    q, k, v, dO = (x.numpy() for x in inputs(B, T, H, Hkv, D, dtype, 3, dO=True))
    tree = orc.Tree(k, v, CR, MTN, TK, dtype)
    fw = orc.forward(q, tree, D ** -0.5)
    L = tree.L
    par = fw["parents"].reshape(L, B, T, Hkv, TK)
    gm, gs = fw["gmax"].reshape(B, T, H), fw["gsum"].reshape(B, T, H)
    out = fw["out"].reshape(B, T, H, D)
    bw = orc.backward(q, tree, D ** -0.5, par, gm, gs, out, dO)
    return dict(q=q, k=k, v=v, dO=dO, out=out, par=par, gm=gm, gs=gs, bw=bw, CR=CR, TK=TK, MTN=MTN,
                B=B, Hkv=Hkv, T=T, fw=fw)


def run_check(c, dk, dv, dtype="float32"):
    return check_dkv_sampled(c["q"], c["dO"], c["out"], c["k"], c["v"], c["par"], c["gm"], c["gs"],
                             dk, dv, c["CR"], c["TK"], c["MTN"], dtype,
                             [(0, 0), (c["B"] - 1, c["Hkv"] - 1)], 9)


def test_dkv_checker_accepts_oracle(case):
    rep = run_check(case, case["bw"]["dk"], case["bw"]["dv"])
    for r in rep.values():
        assert r["nodes"] >= 20 and r["dk"] < 0.05 and r["dv"] < 0.05


def test_dkv_checker_accepts_device_tensors(case):
    """Same check with torch tensors for the device's arrays (the form the
    full-size tests pass), here on the CPU."""
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x))
    c = dict(case, q=t(case["q"]), dO=t(case["dO"]), out=t(case["out"]), k=t(case["k"]),
             v=t(case["v"]), gm=t(case["gm"]), gs=t(case["gs"]), par=t(case["par"]))
    run_check(c, t(case["bw"]["dk"]), t(case["bw"]["dv"]))


@pytest.mark.parametrize("which", ["dk", "dv"])
def test_dkv_checker_rejects_swapped_rows(case, which):
    """Two sibling rows swapped (the mass check over a (b, h_kv) cannot see
    this) at every sampled pair's last parent."""
    g = {n: case["bw"][n].copy() for n in ("dk", "dv")}
    T, CR = case["T"], case["CR"]
    p = (T - 1) // CR
    a, b = p * CR, T - 1
    for (bb, h) in [(0, 0), (case["B"] - 1, case["Hkv"] - 1)]:
        g[which][bb, [a, b], h] = g[which][bb, [b, a], h]
    with pytest.raises(AssertionError, match=which):
        run_check(case, g["dk"], g["dv"])


def test_state_checker(case):
    fw = case["fw"]
    check_state(fw["gmax"], fw["gsum"], fw["gmax"], fw["gsum"], "bfloat16")
    with pytest.raises(AssertionError):
        check_state(fw["gmax"] + 0.01, fw["gsum"], fw["gmax"], fw["gsum"], "bfloat16")
    with pytest.raises(AssertionError):
        check_state(fw["gmax"], fw["gsum"] * 1.01, fw["gmax"], fw["gsum"], "bfloat16")
