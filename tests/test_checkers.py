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


def test_selection_rule_holds_exact_ties():
    """compare_selection with the oracle's exponent arguments: among
    candidates whose importance underflows to exactly 0 on both sides the
    lowest flat position must win (src/naive.py:94); the tie band alone
    would excuse any order among them.  One row, parent list [0, 1] at CR 3
    (flat position j is node j), top_k 3."""
    from tests.helpers import compare_selection

    CR, TK = 3, 3
    par = np.array([[[0, 1, -1]]], np.int32)
    imp = np.full((1, 1, TK * CR), -1.0, np.float32)
    arg = np.full((1, 1, TK * CR), -1e30, np.float32)
    imp[0, 0, :6] = [0.5, 0.0, 0.0, 0.0, 0.0, 1e6]
    arg[0, 0, :6] = [-0.7, -300.0, -300.0, -300.0, -300.0, 0.0]
    ref = np.array([[[0, 1, 5]]], np.int32)  # the stable order: zeros by position
    sel = lambda *n: np.array([[list(n)]], np.int32)

    def check(got, a=arg, i=imp):
        return compare_selection(got, ref, i, par, CR, arg_ref=a)

    assert check(ref)["exact"] == 1
    # a higher-position zero in place of the lowest one: a tie-order violation
    assert check(sel(0, 3, 5))["bad"]
    assert not compare_selection(sel(0, 3, 5), ref, imp, par, CR)["bad"]  # the band alone excuses it
    # node 3 near the underflow cut (it may be a subnormal on the side under
    # test, which then prefers it to the certain zero 1)
    a2 = arg.copy()
    a2[0, 0, 3] = -104.0
    assert not check(sel(0, 3, 5), a2)["bad"]
    # ... but node 1 near the cut does not excuse a certain zero 3 taken in
    # its place: 1 is then 0 on that side too, and comes first
    a2 = arg.copy()
    a2[0, 0, 1] = -104.0
    assert check(sel(0, 3, 5), a2)["bad"]
    # node 1 a certain nonzero of weight 1e-7 (inside the absolute band), node
    # 3 a certain zero: taking 3 instead is never right
    i3, a3 = imp.copy(), arg.copy()
    i3[0, 0, 1], a3[0, 0, 1] = 1e-7, -16.1
    assert check(sel(0, 3, 5), a3, i3)["bad"]
    assert not compare_selection(sel(0, 3, 5), ref, i3, par, CR)["bad"]
