"""Pin the CPU oracle against the reference's own outputs (golden fixtures
written by tests/golden/make_golden.py from /root/reference/src/naive.py)."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import compare_selection, load_golden, round_np, ulp_close

FIXTURES = ["cr4_d16_fp32", "cr16_tk4_bf16", "cr8_tk16_fp32_g8", "cr16_tk4_fp16_b2"]


@pytest.fixture(scope="module", params=FIXTURES)
def golden_run(request):
    g = load_golden(request.param)
    tree = orc.Tree(g["k"], g["v"], g["CR"], g["MTN"], g["TK"], g["dtype"])
    fw = orc.forward(g["q"], tree, g["scale"], trace=True)
    return g, tree, fw


def test_levels_match(golden_run):
    g, tree, fw = golden_run
    assert tree.L == g["L"]
    assert [x.shape[1] for x in tree.lk] == orc.level_sizes(g["T"], g["CR"], g["MTN"])


def test_selection_matches_reference(golden_run):
    g, tree, fw = golden_run
    B, T, Hkv, TK = g["B"], g["T"], g["Hkv"], g["TK"]
    prev_ok = None
    for l in range(g["L"] - 1, 0, -1):
        ref = g[f"parents_l{l}"].reshape(B * T, Hkv, TK)
        res = compare_selection(fw["sel"][l], ref, fw["imp"][l], fw["parents"][l], g["CR"], prev_ok,
                                arg_ref=fw["imparg"][l])
        assert not res["bad"], f"level {l}: {res['bad'][:5]}"
        # the oracle follows the reference bit for bit at these sizes
        assert res["exact"] >= res["n"] - 2, res
        prev_ok = res["exact_mask"]


def test_forward_output_matches_reference(golden_run):
    g, tree, fw = golden_run
    out = fw["out"].reshape(g["out"].shape)
    ok, worst = ulp_close(out, g["out"], g["dtype"], ulps=2, atol=2e-6)
    assert ok, f"worst {worst:.2f} ulp"
    # the autograd path of the reference agrees with its own forward
    assert np.allclose(g["out_autograd"], g["out"], atol=1e-5, rtol=1e-2)


def test_layer_state_matches_reference(golden_run):
    g, tree, fw = golden_run
    B, T, H = g["B"], g["T"], g["H"]
    for l in range(g["L"]):
        lm = fw["lmax"][l].reshape(B, T, H)
        ls = fw["lsum"][l].reshape(B, T, H)
        np.testing.assert_allclose(lm, g[f"lmax_l{l}"], rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(ls, g[f"lsum_l{l}"], rtol=1e-4, atol=1e-5)


def test_backward_matches_reference(golden_run):
    g, tree, fw = golden_run
    B, T, H, Hkv, D, TK, L = g["B"], g["T"], g["H"], g["Hkv"], g["D"], g["TK"], g["L"]
    parents = fw["parents"].reshape(L, B, T, Hkv, TK)
    # delta = rowsum(dO * out) uses the reference's own (dtype-rounded) output,
    # so that 1-ulp rounding-boundary flips of `out` do not leak into the grads
    out = g["out_autograd"]
    bw = orc.backward(g["q"], tree, g["scale"], parents, fw["gmax"].reshape(B, T, H),
                      fw["gsum"].reshape(B, T, H), out, g["dO"])
    for name in ("dq", "dk", "dv"):
        mine = round_np(bw[name], g["dtype"])
        ref = g[name]
        # fp32: the reference's fp32 summation order; 16-bit dtypes: at most one
        # rounding-boundary flip of the final cast
        ok, worst = ulp_close(mine, ref, g["dtype"], ulps=1.01 if g["dtype"] != "float32" else 64,
                              atol=1e-5 * float(np.abs(ref).max()))
        assert ok, f"{name}: worst {worst:.2f} ulp, max|ref|={np.abs(ref).max():.3g}"
