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


# ------------------------------------------------------------ subset checkers
# The full-size GPU tests check the device against row- and node-subset forms
# of the oracle (backward_dq_rows, backward_dkv_nodes, final_dkv_level0) and
# against the forward teacher-forced on the device's lists.  These tie each of
# them to the full backward (itself pinned by the reference's gradients and by
# float64 autograd above) and to the dense softmax.

def full_backward(r):
    B, T, H, Hkv, D, TK, L = r["B"], r["T"], r["H"], r["Hkv"], r["D"], r["TK"], r["tree"].L
    fw = r["fw"]
    par = fw["parents"].reshape(L, B, T, Hkv, TK)
    gm, gs = fw["gmax"].reshape(B, T, H), fw["gsum"].reshape(B, T, H)
    out = fw["out"].reshape(B, T, H, D)
    bw = orc.backward(r["q"], r["tree"], D ** -0.5, par, gm, gs, out, r["dO"])
    return bw, par, gm, gs, orc.delta(out, r["dO"])


def sample_nodes(r, rng, per_level=12):
    """(level, b, h, node) targets: random nodes of every level plus each
    level's first and last node (the last parent's partial tail)."""
    tree = r["tree"]
    out = []
    for l in range(tree.L):
        n = int(tree.n[l])
        for b in range(r["B"]):
            for h in range(r["Hkv"]):
                picks = set(rng.choice(n, min(n, per_level), replace=False).tolist()) | {0, n - 1}
                out += [(l, b, h, x) for x in sorted(picks)]
    return np.array(out, np.int32)


def test_dq_rows_matches_full_backward(run):
    bw, par, gm, gs, dl = full_backward(run)
    B, T, H, D = run["B"], run["T"], run["H"], run["D"]
    rows = orc.all_rows(B, T)[::7]
    rows = np.concatenate([rows, [[B - 1, T - 1]]]).astype(np.int32)
    b, t = rows[:, 0], rows[:, 1]
    got = orc.backward_dq_rows(run["q"], run["tree"], D ** -0.5, rows, par[:, b, t], gm[b, t], gs[b, t],
                               dl[b, t], run["dO"][b, t])
    # same per-group routine on the same inputs: identical values
    np.testing.assert_array_equal(got, bw["dq"][b, t])


def test_backward_rows_matches_full_backward(run):
    """The row-subset full backward (the CPU baseline's backward leg): over
    every row in order it is the full backward, bit for bit; over two row
    chunks its dq rows are the full backward's and its scattered per-level
    dK / dV add up to the full backward's."""
    bw, par, gm, gs, dl = full_backward(run)
    B, T, H, D = run["B"], run["T"], run["H"], run["D"]
    rows = orc.all_rows(B, T)
    b, t = rows[:, 0], rows[:, 1]
    args = lambda i: (rows[i], par[:, b[i], t[i]], gm[b[i], t[i]], gs[b[i], t[i]], dl[b[i], t[i]],
                      run["dO"][b[i], t[i]])
    dq, dk, dv = orc.backward_rows(run["q"], run["tree"], D ** -0.5, *args(slice(None)))
    np.testing.assert_array_equal(dq, bw["dq"].reshape(-1, H, D))
    flat = lambda lv: np.concatenate([x.ravel() for x in lv])
    np.testing.assert_array_equal(dk, flat(bw["dk_levels"]))
    np.testing.assert_array_equal(dv, flat(bw["dv_levels"]))
    cut = len(rows) // 3
    parts = [orc.backward_rows(run["q"], run["tree"], D ** -0.5, *args(sl))
             for sl in (slice(0, cut), slice(cut, None))]
    np.testing.assert_array_equal(np.concatenate([p[0] for p in parts]), dq)
    for i, ref in ((1, dk), (2, dv)):
        got = parts[0][i] + parts[1][i]
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())
    # without the dK / dV outputs only dq comes back, the same
    dq2, none_k, none_v = orc.backward_rows(run["q"], run["tree"], D ** -0.5, *args(slice(0, cut)),
                                            with_dkv=False)
    assert none_k is None and none_v is None
    np.testing.assert_array_equal(dq2, parts[0][0])


def test_dkv_nodes_matches_full_backward(run):
    """Per-level dK/dV from each node's own scores (a different route from
    the full backward, which scores whole groups and scatters)."""
    bw, par, gm, gs, dl = full_backward(run)
    tg = sample_nodes(run, np.random.default_rng(1))
    dk, dv = orc.backward_dkv_nodes(run["q"], run["tree"], run["D"] ** -0.5, par, gm, gs, dl,
                                    run["dO"], tg, threads=4)
    ref_k = np.stack([bw["dk_levels"][l][b, x, h] for l, b, h, x in tg])
    ref_v = np.stack([bw["dv_levels"][l][b, x, h] for l, b, h, x in tg])
    for got, ref in ((dk, ref_k), (dv, ref_v)):
        scl = np.abs(ref).max()
        assert scl > 0
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=2e-6 * scl)
    # nodes that nothing accumulates (e.g. a level's nodes that every query
    # passes down) come out exactly zero in both
    zero = np.all(ref_k == 0, axis=1)
    assert np.all(dk[zero] == 0)


def test_final_dkv_level0_matches_full_backward(run):
    bw, par, gm, gs, dl = full_backward(run)
    rng = np.random.default_rng(2)
    T = run["T"]
    nodes = [(b, h, x) for b in range(run["B"]) for h in range(run["Hkv"])
             for x in set(rng.choice(T, 10, replace=False).tolist()) | {0, T - 1}]
    nodes = np.array(nodes, np.int32)
    dk, dv = orc.final_dkv_level0(run["q"], run["tree"], run["D"] ** -0.5, par, gm, gs, dl, run["dO"],
                                  nodes, threads=4)
    ref_k = np.stack([bw["dk"][b, x, h] for b, h, x in nodes])
    ref_v = np.stack([bw["dv"][b, x, h] for b, h, x in nodes])
    for got, ref in ((dk, ref_k), (dv, ref_v)):
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=2e-6 * np.abs(ref).max())


def test_subset_backward_matches_autograd():
    """dq rows and final dk/dv at level-0 nodes straight against float64
    autograd of the dense form (the first, small fp32 case)."""
    B, T, H, Hkv, D, CR, TK, MTN, dtype = CASES[0]
    q, k, v, dO = make_inputs(B, T, H, Hkv, D, dtype)
    tree = orc.Tree(k, v, CR, MTN, TK, dtype)
    fw = orc.forward(q, tree, D ** -0.5, trace=True)
    r = dict(B=B, T=T, H=H, Hkv=Hkv, D=D, CR=CR, TK=TK, MTN=MTN, dtype=dtype, q=q, k=k, v=v, dO=dO,
             tree=tree, fw=fw)
    L = tree.L
    qt = torch.from_numpy(q).double().requires_grad_(True)
    kt = torch.from_numpy(k).double().requires_grad_(True)
    vt = torch.from_numpy(v).double().requires_grad_(True)
    rows_all = [(b, t) for b in range(B) for t in range(T)]
    o = dense_torch_forward(r, qt, kt, vt, rows_all).reshape(B, T, H, D)
    o.backward(torch.from_numpy(dO).double())
    par = fw["parents"].reshape(L, B, T, Hkv, TK)
    gm, gs = fw["gmax"].reshape(B, T, H), fw["gsum"].reshape(B, T, H)
    dl = orc.delta(fw["out"].reshape(B, T, H, D), dO)
    rows = np.array([(0, t) for t in (0, 5, 77, 150, 299)], np.int32)
    b, t = rows[:, 0], rows[:, 1]
    dq = orc.backward_dq_rows(q, tree, D ** -0.5, rows, par[:, b, t], gm[b, t], gs[b, t], dl[b, t], dO[b, t])
    ref = qt.grad.numpy()[b, t]
    assert np.abs(dq - ref).max() < 1e-5 * np.abs(qt.grad.numpy()).max()
    nodes = np.array([(0, 0, x) for x in (0, 3, 64, 150, 298, 299)], np.int32)
    dk, dv = orc.final_dkv_level0(q, tree, D ** -0.5, par, gm, gs, dl, dO, nodes, threads=2)
    for got, ref in ((dk, kt.grad.numpy()[0, nodes[:, 2], 0]), (dv, vt.grad.numpy()[0, nodes[:, 2], 0])):
        assert np.abs(got - ref).max() < 1e-5 * np.abs(ref).max()


def perturbed_lists(r, rng, frac=0.5):
    """Parent lists [L, n, Hkv, TK] that differ from the oracle's own
    selection: level by level from the top, each list is the oracle's own
    Top-K from the (already perturbed) list above, and in about `frac` of the
    rows one selected node other than the rightmost is swapped for a
    candidate that was not selected.  Lists stay ascending, -1 padded, with
    the rightmost node kept, like every list the device writes."""
    tree, CR, TK, q, D = r["tree"], r["CR"], r["TK"], r["q"], r["D"]
    L = tree.L
    rows = orc.all_rows(r["B"], r["T"])
    forced = orc.forward(q, tree, D ** -0.5, rows=rows)["parents"].copy()
    swapped = 0
    for l in range(L - 1, 0, -1):
        fw = orc.forward(q, tree, D ** -0.5, rows=rows, forced=forced)
        sel = fw["sel"][l].copy()  # own Top-K at level l from the list used there
        for i in range(sel.shape[0]):
            t = int(rows[i, 1])
            for h in range(sel.shape[1]):
                if rng.random() >= frac:
                    continue
                vp = [int(x) for x in forced[l, i, h] if x >= 0]
                nc = (len(vp) - 1) * CR + (t // CR ** l) % CR + 1
                cand = [vp[j // CR] * CR + j % CR for j in range(nc)]
                cur = [int(x) for x in sel[i, h] if x >= 0]
                right = t // CR ** l
                out_ = [x for x in cand if x not in cur]
                inn = [x for x in cur if x != right]
                if not out_ or not inn:
                    continue
                cur.remove(inn[rng.integers(len(inn))])
                cur.append(out_[rng.integers(len(out_))])
                cur.sort()
                sel[i, h] = cur + [-1] * (TK - len(cur))
                swapped += 1
        forced[l - 1] = sel
    return forced, swapped


@pytest.mark.parametrize("case", CASES[:2], ids=lambda c: f"T{c[1]}cr{c[5]}tk{c[6]}")
def test_forced_forward_is_dense_softmax(case):
    """Teacher forcing with lists that are not the oracle's own choice: the
    output is one softmax over the candidates those lists leave accumulated,
    and gmax its max."""
    B, T, H, Hkv, D, CR, TK, MTN, dtype = case
    q, k, v, dO = make_inputs(B, T, H, Hkv, D, dtype, seed=5)
    tree = orc.Tree(k, v, CR, MTN, TK, dtype)
    r = dict(B=B, T=T, H=H, Hkv=Hkv, D=D, CR=CR, TK=TK, MTN=MTN, dtype=dtype, q=q, tree=tree)
    forced, swapped = perturbed_lists(r, np.random.default_rng(7))
    assert swapped > 50
    fw = orc.forward(q, tree, D ** -0.5, rows=orc.all_rows(B, T), forced=forced)
    assert np.array_equal(fw["parents"][:-1], forced[:-1])
    own = orc.forward(q, tree, D ** -0.5)
    assert not np.allclose(fw["out_f32"], own["out_f32"])  # the lists matter
    r["fw"] = fw
    test_output_is_dense_softmax_over_accumulated(r)


# ------------------------------------------------------------ K != V
# The reference carries the value head dim apart from the key head dim
# (src/naive.py:144 v_dim = v.shape[-1]).  The oracle restates that directly;
# pinned here by the dense softmax and float64 autograd of the dense form.

@pytest.mark.parametrize("kv", [(32, 16), (16, 32)], ids=lambda x: f"K{x[0]}V{x[1]}")
def test_oracle_separate_value_dim(kv):
    K, V = kv
    B, T, H, Hkv, CR, TK, MTN, dtype = 1, 260, 4, 2, 4, 8, 32, "float32"
    g = torch.Generator().manual_seed(11)
    q = torch.randn(B, T, H, K, generator=g).numpy()
    k = torch.randn(B, T, Hkv, K, generator=g).numpy()
    v = torch.randn(B, T, Hkv, V, generator=g).numpy()
    dO = torch.randn(B, T, H, V, generator=g).numpy()
    tree = orc.Tree(k, v, CR, MTN, TK, dtype)
    assert tree.DV == V and tree.lv[1].shape[-1] == V
    fw = orc.forward(q, tree, K ** -0.5, trace=True)
    assert fw["out"].shape == (B * T, H, V)
    r = dict(B=B, T=T, H=H, Hkv=Hkv, D=K, CR=CR, TK=TK, MTN=MTN, dtype=dtype, q=q, k=k, v=v, dO=dO,
             tree=tree, fw=fw)
    test_output_is_dense_softmax_over_accumulated(r)
    L = tree.L
    par = fw["parents"].reshape(L, B, T, Hkv, TK)
    gm, gs = fw["gmax"].reshape(B, T, H), fw["gsum"].reshape(B, T, H)
    out = fw["out"].reshape(B, T, H, V)
    bw = orc.backward(q, tree, K ** -0.5, par, gm, gs, out, dO)
    assert bw["dq"].shape == q.shape and bw["dk"].shape == k.shape and bw["dv"].shape == v.shape
    qt = torch.from_numpy(q).double().requires_grad_(True)
    kt = torch.from_numpy(k).double().requires_grad_(True)
    vt = torch.from_numpy(v).double().requires_grad_(True)
    o = dense_torch_forward(r, qt, kt, vt, [(b, t) for b in range(B) for t in range(T)])
    o.reshape(B, T, H, V).backward(torch.from_numpy(dO).double())
    for name, got, ref in (("dq", bw["dq"], qt.grad), ("dk", bw["dk"], kt.grad), ("dv", bw["dv"], vt.grad)):
        ref = ref.numpy()
        err = np.abs(got - ref).max() / np.abs(ref).max()
        assert err < 1e-5, f"{name}: rel err {err:.2e}"
    # the subset forms at K != V
    dl = orc.delta(out, dO)
    nodes = np.array([(0, h, x) for h in range(Hkv) for x in (0, 7, 130, 259)], np.int32)
    dk, dv = orc.final_dkv_level0(q, tree, K ** -0.5, par, gm, gs, dl, dO, nodes, threads=2)
    np.testing.assert_allclose(dk, bw["dk"][0, nodes[:, 2], nodes[:, 1]], rtol=1e-4,
                               atol=1e-6 * np.abs(bw["dk"]).max())
    np.testing.assert_allclose(dv, bw["dv"][0, nodes[:, 2], nodes[:, 1]], rtol=1e-4,
                               atol=1e-6 * np.abs(bw["dv"]).max())
    rows = np.array([(0, t) for t in (3, 100, 259)], np.int32)
    b, t = rows[:, 0], rows[:, 1]
    dq = orc.backward_dq_rows(q, tree, K ** -0.5, rows, par[:, b, t], gm[b, t], gs[b, t], dl[b, t], dO[b, t])
    np.testing.assert_array_equal(dq, bw["dq"][b, t])


def test_threaded_forms_match(run):
    """forward_threaded / backward_threaded (the CPU baseline's multi-core
    forms) against the single-threaded forward and full backward."""
    B, T, H, D = run["B"], run["T"], run["H"], run["D"]
    fw = orc.forward_threaded(run["q"], run["tree"], D ** -0.5, threads=3)
    for key in ("out", "gmax", "gsum", "parents"):
        np.testing.assert_array_equal(fw[key], run["fw"][key])
    bw, par, gm, gs, _ = full_backward(run)
    dq, dk, dv = orc.backward_threaded(run["q"], run["tree"], D ** -0.5, par, gm, gs,
                                       run["fw"]["out"].reshape(B, T, H, D), run["dO"], threads=3)
    np.testing.assert_array_equal(dq, bw["dq"])
    for got, ref in ((dk, bw["dk"]), (dv, bw["dv"])):
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=2e-6 * np.abs(ref).max())
