"""Pin the CPU oracle with checks the mathematics fixes, independently of the
reference: exact tree means, closed-form candidate counts, brute-force
selection in float64, a dense softmax over the union of accumulated
candidates, and torch float64 autograd of that dense form (selection held
fixed).  Each check is built so a plausible slip (wrong RoPE position,
dropped tail child, wrong tie order, missing level) fails it."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.helpers import compare_selection

CASES = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype
    (1, 300, 4, 1, 16, 4, 8, 32, "float32"),
    (2, 530, 8, 2, 32, 8, 8, 64, "float32"),
    (1, 700, 16, 1, 64, 16, 4, 64, "bfloat16"),
]


def make_inputs(B, T, H, Hkv, D, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    dt = {"float32": torch.float32, "bfloat16": torch.bfloat16}[dtype]
    q = torch.randn(B, T, H, D, generator=g).to(dt).float().numpy()
    k = torch.randn(B, T, Hkv, D, generator=g).to(dt).float().numpy()
    v = torch.randn(B, T, Hkv, D, generator=g).to(dt).float().numpy()
    dO = torch.randn(B, T, H, D, generator=g).to(dt).float().numpy()
    return q, k, v, dO


def rope64(x, pos, cos, sin):
    """closed-form RoPE in float64 from cos/sin of the fp32 table."""
    h = x.shape[-1] // 2
    c = cos[pos].astype(np.float64)
    s = sin[pos].astype(np.float64)
    lo, hi = x[..., :h], x[..., h:]
    return np.concatenate([lo * c - hi * s, lo * s + hi * c], -1)


def test_rope_table_closed_form():
    cos, sin = orc.rope_tables(64, 1200, 10000.0)
    i = np.arange(32)
    inv = 1.0 / (10000.0 ** (2 * i / 64))
    p = np.arange(1200)[:, None]
    np.testing.assert_allclose(cos, np.cos(p * inv), atol=2e-4)
    np.testing.assert_allclose(sin, np.sin(p * inv), atol=2e-4)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_tree_build_is_rounded_mean(dtype):
    rng = np.random.default_rng(3)
    B, T, Hkv, D, CR = 2, 1000, 2, 16, 16  # 1000 = 62*16 + 8: partial tail
    dt = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}[dtype]
    k = torch.from_numpy(rng.standard_normal((B, T, Hkv, D)).astype(np.float32)).to(dt).float().numpy()
    lk, _ = orc.build_tree(k, k, CR, 32, dtype)
    assert [x.shape[1] for x in lk] == [1000, 63, 4]
    for l in range(1, len(lk)):
        child = lk[l - 1].astype(np.float64)
        n = child.shape[1]
        exact = np.stack([child[:, p * CR:min(p * CR + CR, n)].mean(1) for p in range(lk[l].shape[1])], 1)
        want = torch.from_numpy(exact.astype(np.float32)).to(dt).float().numpy()
        got = lk[l]
        ulp = {"float32": 2.0 ** -23, "bfloat16": 2.0 ** -7, "float16": 2.0 ** -10}[dtype]
        if dtype != "float32":
            # the fp32 running sum can move a 16-bit mean only at a rounding boundary
            assert np.mean(got == want) > 0.999
            assert np.all(np.abs(got - exact) <= 1.01 * ulp * np.maximum(np.abs(exact), 2.0 ** -14) + 1e-7)
        else:
            # sequential fp32 summation error bound: (n-1) u sum|x| / n, plus the final rounding
            absmean = np.stack([np.abs(child[:, p * CR:min(p * CR + CR, n)]).mean(1)
                                for p in range(lk[l].shape[1])], 1)
            assert np.all(np.abs(got - exact) <= 2.0 ** -24 * (CR * absmean + np.abs(exact)) + 1e-30)
        # the partial tail averages only its valid children
        tail = child[:, (lk[l].shape[1] - 1) * CR:].mean(1)
        np.testing.assert_allclose(got[:, -1], tail, rtol=ulp * 2, atol=1e-6)
    const = np.full((1, 37, 1, 4), 0.375, np.float32)
    lc, _ = orc.build_tree(const, const, 4, 4, dtype)
    assert all(np.all(x == 0.375) for x in lc)


@pytest.fixture(scope="module", params=CASES, ids=lambda c: f"T{c[1]}cr{c[5]}tk{c[6]}{c[8]}")
def run(request):
    B, T, H, Hkv, D, CR, TK, MTN, dtype = request.param
    q, k, v, dO = make_inputs(B, T, H, Hkv, D, dtype)
    tree = orc.Tree(k, v, CR, MTN, TK, dtype)
    fw = orc.forward(q, tree, D ** -0.5, trace=True)
    return dict(B=B, T=T, H=H, Hkv=Hkv, D=D, CR=CR, TK=TK, MTN=MTN, dtype=dtype,
                q=q, k=k, v=v, dO=dO, tree=tree, fw=fw)


def accumulated_sets(r, b, t, h):
    """(level, flat position j, node) of every accumulated candidate for one
    query group, derived from the parent lists only."""
    fw, tree, CR, TK = r["fw"], r["tree"], r["CR"], r["TK"]
    row = b * r["T"] + t
    out = []
    for l in range(tree.L - 1, -1, -1):
        vp = [int(x) for x in fw["parents"][l, row, h] if x >= 0]
        nc = (len(vp) - 1) * CR + (t // CR ** l) % CR + 1
        nxt = set(int(x) for x in fw["parents"][l - 1, row, h] if x >= 0) if l > 0 else set()
        for j in range(nc):
            node = vp[j // CR] * CR + j % CR
            if node not in nxt:
                out.append((l, j, node, nc))
    return out


def test_candidate_counts_closed_form(run):
    fw, tree, CR, TK = run["fw"], run["tree"], run["CR"], run["TK"]
    for row in range(0, run["B"] * run["T"], 7):
        t = row % run["T"]
        cc = orc.candidate_counts(t, CR, TK, tree.L)
        for h in range(run["Hkv"]):
            for l in range(tree.L - 1, -1, -1):
                npar = int(np.sum(fw["parents"][l, row, h] >= 0))
                nc = (npar - 1) * CR + (t // CR ** l) % CR + 1
                assert nc == cc[l][0]
                if l > 0:
                    assert int(np.sum(fw["sel"][l, row, h] >= 0)) == cc[l][1]
                    # the rightmost node (the one holding t) is always kept
                    assert (t // CR ** l) in set(fw["sel"][l, row, h].tolist())
                    # selections are ascending node ids, -1 padded
                    s = fw["sel"][l, row, h]
                    s = s[s >= 0]
                    assert np.all(np.diff(s) > 0)


def test_selection_is_bruteforce_topk(run):
    """float64 importance + stable descending sort reproduces the selection
    up to the documented tie band."""
    fw, tree, CR, TK, D = run["fw"], run["tree"], run["CR"], run["TK"], run["D"]
    G = run["H"] // run["Hkv"]
    rows = range(0, run["B"] * run["T"], 5)
    for l in range(tree.L - 1, 0, -1):
        sel_bf, imp_bf, par_bf, sel_or = [], [], [], []
        for row in rows:
            b, t = divmod(row, run["T"])
            for h in range(run["Hkv"]):
                vp = [int(x) for x in fw["parents"][l, row, h] if x >= 0]
                nc = (len(vp) - 1) * CR + (t // CR ** l) % CR + 1
                nodes = np.array([vp[j // CR] * CR + j % CR for j in range(nc)])
                kr = rope64(tree.lk[l][b, nodes, h].astype(np.float64), np.arange(nc), tree.cos, tree.sin)
                qg = run["q"][b, t, h * G:(h + 1) * G].astype(np.float64)
                qr = rope64(qg, np.full(G, nc - 1), tree.cos, tree.sin) * D ** -0.5
                s = qr @ kr.T
                imp = np.exp(s - s.max()).sum(0)
                imp[nc - 1] = 1e6
                order = np.argsort(-imp, kind="stable")[:min(TK, nc)]
                sel = np.full(TK, -1)
                sel[:len(order)] = np.sort(nodes[order])
                sel_bf.append(sel)
                ip = np.full(TK * CR, -1.0)
                ip[:nc] = imp
                imp_bf.append(ip)
                par_bf.append(fw["parents"][l, row, h])
                sel_or.append(fw["sel"][l, row, h])
        n = len(sel_bf)
        sh = lambda a: np.array(a).reshape(n, 1, -1)
        res = compare_selection(sh(sel_or), sh(sel_bf), sh(imp_bf), sh(par_bf), CR)
        assert not res["bad"], res["bad"][:3]


def test_output_is_dense_softmax_over_accumulated(run):
    """out = softmax over the union of accumulated candidates of all levels."""
    fw, tree, D = run["fw"], run["tree"], run["D"]
    G = run["H"] // run["Hkv"]
    for row in range(0, run["B"] * run["T"], 11):
        b, t = divmod(row, run["T"])
        for h in range(run["Hkv"]):
            acc = accumulated_sets(run, b, t, h)
            qg = run["q"][b, t, h * G:(h + 1) * G].astype(np.float64)
            S, V = [], []
            for (l, j, node, nc) in acc:
                kr = rope64(tree.lk[l][b, node, h].astype(np.float64), j, tree.cos, tree.sin)
                qr = rope64(qg, np.full(G, nc - 1), tree.cos, tree.sin) * D ** -0.5
                S.append(qr @ kr)
                V.append(tree.lv[l][b, node, h].astype(np.float64))
            S = np.stack(S, 1)
            P = np.exp(S - S.max(1, keepdims=True))
            o = (P @ np.stack(V)) / P.sum(1, keepdims=True)
            np.testing.assert_allclose(fw["out_f32"][row, h * G:(h + 1) * G], o, rtol=2e-5, atol=2e-5)
            np.testing.assert_allclose(fw["gmax"][row, h * G:(h + 1) * G], S.max(1), rtol=1e-5, atol=1e-5)


def dense_torch_forward(r, q, k, v, rows):
    """Differentiable float64 dense form: tree by mean pooling, then for each
    row one softmax over the accumulated candidates (selection fixed)."""
    tree, CR, D = r["tree"], r["CR"], r["D"]
    G = r["H"] // r["Hkv"]
    lk, lv = [k], [v]
    for n in [x.shape[1] for x in tree.lk[1:]]:
        cur_k, cur_v = lk[-1], lv[-1]
        N = cur_k.shape[1]
        lk.append(torch.stack([cur_k[:, p * CR:min(p * CR + CR, N)].mean(1) for p in range(n)], 1))
        lv.append(torch.stack([cur_v[:, p * CR:min(p * CR + CR, N)].mean(1) for p in range(n)], 1))
    cos = torch.from_numpy(tree.cos).double()
    sin = torch.from_numpy(tree.sin).double()

    def rope(x, pos):
        h = x.shape[-1] // 2
        c, s = cos[pos], sin[pos]
        return torch.cat([x[..., :h] * c - x[..., h:] * s, x[..., :h] * s + x[..., h:] * c], -1)

    outs = []
    for (b, t) in rows:
        for h in range(r["Hkv"]):
            acc = accumulated_sets(r, b, t, h)
            qg = q[b, t, h * G:(h + 1) * G]
            S, V = [], []
            for (l, j, node, nc) in acc:
                kr = rope(lk[l][b, node, h], j)
                qr = rope(qg, nc - 1) * D ** -0.5
                S.append(qr @ kr)
                V.append(lv[l][b, node, h])
            P = torch.softmax(torch.stack(S, 1), 1)
            outs.append(P @ torch.stack(V))
    return torch.stack(outs)


def test_backward_is_autograd_of_dense_form(run):
    if run["dtype"] != "float32" or run["T"] > 300:
        pytest.skip("float64 autograd reference is sized for the small fp32 cases")
    r = run
    B, T, H, Hkv, D, TK, L = r["B"], r["T"], r["H"], r["Hkv"], r["D"], r["TK"], r["tree"].L
    fw = r["fw"]
    bw = orc.backward(r["q"], r["tree"], D ** -0.5, fw["parents"].reshape(L, B, T, Hkv, TK),
                      fw["gmax"].reshape(B, T, H), fw["gsum"].reshape(B, T, H),
                      fw["out"].reshape(B, T, H, D), r["dO"])
    q = torch.from_numpy(r["q"]).double().requires_grad_(True)
    k = torch.from_numpy(r["k"]).double().requires_grad_(True)
    v = torch.from_numpy(r["v"]).double().requires_grad_(True)
    rows = [(b, t) for b in range(B) for t in range(T)]
    o = dense_torch_forward(r, q, k, v, rows).reshape(B, T, H, D)
    o.backward(torch.from_numpy(r["dO"]).double())
    for name, got, ref in (("dq", bw["dq"], q.grad), ("dk", bw["dk"], k.grad), ("dv", bw["dv"], v.grad)):
        ref = ref.numpy()
        err = np.abs(got - ref).max() / np.abs(ref).max()
        assert err < 1e-5, f"{name}: rel err {err:.2e}"
