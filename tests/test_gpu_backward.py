"""GPU parity of the HIP backward (dq, dk, dv) against the CPU oracle's
analytical backward (restating src/naive.py:320-396) with the selection held
at the device's own parent lists, against the reference's own gradients
(golden fixtures), and at the training shape through sampled rows and a
size-independent checksum.  Bars: 2e-2 abs + 1e-2 rel (bf16), 1e-4 (fp32),
2e-3 (fp16)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import (check_backward, check_dkv_sampled, check_forward, close, inputs,
                            skewed_inputs)
from tests.helpers import load_golden

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def run(q, k, v, dO, CR, TK, MTN, scores=False):
    import htree_amd

    out, par, gmax, gsum, ctx = htree_amd.htree_forward_parents(
        q.to(DEV), k.to(DEV), v.to(DEV), CR, MTN, TK, _save_scores=scores)
    dq, dk, dv = htree_amd.htree_backward(dO.to(DEV), q.to(DEV), out, ctx)
    torch.cuda.synchronize()
    f = lambda x: x.float().cpu().numpy()
    return f(out), par.cpu().numpy(), f(gmax), f(gsum), f(dq), f(dk), f(dv)


CASES = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype, seed
    (1, 2048, 4, 1, 64, 16, 8, 64, "float32", 1),
    (1, 2048, 4, 1, 64, 16, 8, 64, "bfloat16", 1),
    (2, 1200, 16, 2, 128, 16, 16, 128, "bfloat16", 2),
    (1, 1100, 8, 1, 128, 16, 16, 128, "float16", 3),
    (1, 4100, 8, 1, 128, 16, 4, 64, "bfloat16", 4),
    (1, 700, 8, 2, 64, 8, 16, 128, "float32", 5),
    (1, 900, 4, 1, 128, 32, 8, 256, "bfloat16", 6),
    (1, 3000, 8, 1, 64, 4, 32, 64, "bfloat16", 7),
    (1, 2000, 16, 4, 32, 16, 16, 128, "float32", 8),   # D = 32
    (1, 1500, 16, 4, 32, 16, 8, 128, "float16", 9),
    (2, 1000, 8, 2, 32, 8, 16, 64, "bfloat16", 10),
    (1, 2500, 16, 4, 32, 4, 32, 64, "float32", 11),
    (1, 3000, 8, 1, 128, 32, 32, 256, "bfloat16", 12),  # the C4 workload's tree shape
    (1, 2000, 8, 1, 64, 64, 8, 512, "bfloat16", 14),   # CR 64: four tiles per parent
    (1, 1500, 4, 1, 128, 64, 4, 256, "float32", 15),
    (1, 2500, 16, 2, 128, 64, 4, 256, "bfloat16", 16),  # CR 64 with the stored scores (16 tiles)
    (1, 1100, 8, 1, 128, 32, 8, 256, "float16", 17),   # CR 32, fp16 (split dS, shared staging)
    (1, 4096, 8, 2, 64, 16, 16, 16, "bfloat16", 18),   # 16-node top level: accumulates nothing
    (2, 3000, 8, 1, 64, 16, 16, 16, "float32", 19),
    # 750 level-0 parents > 128 * top_k: a sparse level, whose bitmap is set
    # by atomics (bitmap_set_kernel); five levels
    (1, 3000, 8, 1, 64, 4, 4, 16, "bfloat16", 20),
    # CR 32 with stored scores: the top level (125 nodes) merged into 64-child
    # parents of two real ones, the last one partial
    (1, 4000, 8, 1, 64, 32, 8, 256, "bfloat16", 21),
    # CR 128: children 64..127 in the records' second mask; dq recomputes
    (1, 3000, 8, 2, 64, 128, 4, 512, "bfloat16", 22),  # 32 tiles per level
    (1, 1500, 8, 1, 32, 128, 2, 256, "float32", 23),    # 16 tiles per level
    # D = 256: stored scores and dS (bf16), recomputed dq (fp32, fp16)
    (1, 1200, 16, 2, 256, 16, 16, 128, "bfloat16", 24),
    (1, 1100, 8, 1, 256, 32, 8, 256, "float32", 25),
    (1, 900, 8, 2, 256, 8, 16, 128, "float16", 26),
]


@pytest.mark.parametrize("cfg", CASES, ids=lambda c: f"T{c[1]}H{c[2]}kv{c[3]}D{c[4]}cr{c[5]}tk{c[6]}{c[8]}")
def test_backward_matches_oracle(cfg):
    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v, dO = inputs(B, T, H, Hkv, D, dtype, seed, dO=True)
    out, par, gmax, gsum, dq, dk, dv = run(q, k, v, dO, CR, TK, MTN)
    rep = check_backward(q, k, v, dO, CR, TK, MTN, dtype, out, par, gmax, gsum, dq, dk, dv)
    print(rep, flush=True)


SCORE_CASES = [c for c in CASES if c[8] == "bfloat16"]


@pytest.mark.parametrize("cfg", SCORE_CASES,
                         ids=lambda c: f"T{c[1]}H{c[2]}kv{c[3]}D{c[4]}cr{c[5]}tk{c[6]}{c[8]}")
def test_backward_stored_scores_matches_oracle(cfg):
    """The same cases with the forward's stored scores (where the
    configuration keeps them: <= 16 candidate tiles per level, CR <= 64)."""
    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg} stored scores", flush=True)
    q, k, v, dO = inputs(B, T, H, Hkv, D, dtype, seed, dO=True)
    out, par, gmax, gsum, dq, dk, dv = run(q, k, v, dO, CR, TK, MTN, scores=True)
    rep = check_backward(q, k, v, dO, CR, TK, MTN, dtype, out, par, gmax, gsum, dq, dk, dv)
    print(rep, flush=True)


def test_backward_skewed():
    B, T, H, Hkv, D, CR, TK, MTN = 1, 2500, 16, 1, 128, 16, 16, 128
    q, k, v, dO = skewed_inputs(B, T, H, Hkv, D, "bfloat16", 5)
    out, par, gmax, gsum, dq, dk, dv = run(q, k, v, dO, CR, TK, MTN)
    print(check_backward(q, k, v, dO, CR, TK, MTN, "bfloat16", out, par, gmax, gsum, dq, dk, dv))


@pytest.mark.parametrize("skewed", [False, True], ids=["iid", "skewed"])
def test_backward_stored_and_rebuilt_scores(skewed):
    """The training forward keeps every candidate tile's scores (fp16,
    relative to the head's running max) for the backward; without them the
    backward rebuilds the scores from q and the tree.  Both meet the bar
    against the oracle on the same selection."""
    import htree_amd

    B, T, H, Hkv, D, CR, TK, MTN = 1, 2500, 16, 1, 128, 16, 16, 128
    if skewed:
        q, k, v, dO = skewed_inputs(B, T, H, Hkv, D, "bfloat16", 5)
    else:
        q, k, v, dO = inputs(B, T, H, Hkv, D, "bfloat16", 8, dO=True)
    out, par, gmax, gsum, ctx = htree_amd.htree_forward_parents(
        q.to(DEV), k.to(DEV), v.to(DEV), CR, MTN, TK, _save_scores=True)
    assert ctx["train_scores"] is not None
    f = lambda x: x.float().cpu().numpy()
    for stored in (True, False):
        c2 = dict(ctx, train_scores=ctx["train_scores"] if stored else None)
        dq, dk, dv = htree_amd.htree_backward(dO.to(DEV), q.to(DEV), out, c2)
        torch.cuda.synchronize()
        rep = check_backward(q, k, v, dO, CR, TK, MTN, "bfloat16", f(out), par.cpu().numpy(),
                             f(gmax), f(gsum), f(dq), f(dk), f(dv))
        print("stored" if stored else "rebuilt", rep, flush=True)


@pytest.mark.parametrize("name", ["cr16_tk4_bf16", "cr8_tk16_fp32_g8", "cr16_tk4_fp16_b2"])
def test_backward_matches_reference_golden(name):
    """Against the reference's own gradients (naive autograd), where the
    device selected exactly like the reference."""
    g = load_golden(name)
    print(f"golden {name}", flush=True)
    out, par, gmax, gsum, dq, dk, dv = run(g["q"], g["k"], g["v"], g["dO"], g["CR"], g["TK"], g["MTN"])
    B, T, Hkv, TK, L = g["B"], g["T"], g["Hkv"], g["TK"], g["L"]
    same = all(np.array_equal(par[l - 1], g[f"parents_l{l}"].reshape(B, T, Hkv, TK))
               for l in range(L - 1, 0, -1))
    if not same:
        pytest.skip("selection differs from the reference inside the tie band; oracle tests cover it")
    dt = g["dtype"]
    rnd = lambda x: torch.from_numpy(x).to({"float32": torch.float32, "bfloat16": torch.bfloat16,
                                             "float16": torch.float16}[dt]).float().numpy()
    for name_, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        ok, worst = close(rnd(got), g[name_], dt)
        print(name_, worst, flush=True)
        assert ok, f"{name_}: worst {worst:.3f} of the bar"


def test_backward_training_shape_c3():
    """The C3 workload (B=4, T=16384, Hq=32, Hkv=4, D=128, bf16): the forward
    (selection, output, gmax, gsum) and dq on sampled rows vs the oracle,
    final dk / dv at sampled level-0 nodes of two (b, h_kv) pairs; sum over
    nodes of dv equals sum over the group's queries and heads of dO (pooling
    conserves mass, P sums to 1)."""
    B, T, H, Hkv, D, CR, TK, MTN = 4, 16384, 32, 4, 128, 16, 16, 128
    q, k, v, dO = inputs(B, T, H, Hkv, D, "bfloat16", 31, dO=True)
    out, par, gmax, gsum, dq, dk, dv = run(q, k, v, dO, CR, TK, MTN)
    print("device forward + backward done", flush=True)
    assert np.all(np.isfinite(dq)) and np.all(np.isfinite(dk)) and np.all(np.isfinite(dv))
    G = H // Hkv
    dOf = dO.float().numpy().reshape(B, T, Hkv, G, D).astype(np.float64)
    want = dOf.sum(axis=(1, 3))                    # [B, Hkv, D]
    got = dv.astype(np.float64).sum(axis=1)        # [B, Hkv, D]
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-3 * np.sqrt(T * G))
    tree = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, "bfloat16")
    rng = np.random.default_rng(3)
    n = 120
    rows = np.stack([rng.integers(0, B, n), rng.integers(0, T, n)], 1).astype(np.int32)
    L = tree.L
    pr = par[:, rows[:, 0], rows[:, 1]]
    fw = orc.forward(q.float().numpy(), tree, D ** -0.5, rows=rows, forced=pr)
    o = out[rows[:, 0], rows[:, 1]]  # the output the device backward was handed
    d = dO.float().numpy()[rows[:, 0], rows[:, 1]]
    delta = (o.astype(np.float64) * d).sum(-1).astype(np.float32)
    ref = orc.backward_dq_rows(q.float().numpy(), tree, D ** -0.5, rows, pr, fw["gmax"], fw["gsum"],
                               delta, d)
    ok, worst = close(dq[rows[:, 0], rows[:, 1]], ref, "bfloat16")
    print("c3 dq worst", worst, flush=True)
    assert ok
    rep = check_forward(q, k, v, CR, TK, MTN, "bfloat16", rows=rows, out_dev=out, parents_dev=par,
                        tree=tree, gmax_dev=gmax, gsum_dev=gsum)
    print("c3 forward", rep, flush=True)
    rep = check_dkv_sampled(q.float().numpy(), dO.float().numpy(), out, k.float().numpy(),
                            v.float().numpy(), par, gmax, gsum, dk, dv, CR, TK, MTN, "bfloat16",
                            [(0, 0), (B - 1, Hkv - 1)], 33)
    print("c3 dk/dv at sampled nodes", rep, flush=True)


def test_backward_deterministic():
    q, k, v, dO = inputs(1, 3000, 16, 2, 128, "bfloat16", 9, dO=True)
    a = run(q, k, v, dO, 16, 16, 128)
    b = run(q, k, v, dO, 16, 16, 128)
    for x, y in zip(a[4:], b[4:]):
        assert np.array_equal(x, y)


def test_backward_replaced_parent_lists():
    """A bwd_ctx whose per_layer_parents (the reference's key) were replaced
    by equal copies runs on the caller's lists: the gradients equal, bitwise,
    those of the forward's own lists through the same path (no stored
    scores); a list naming a node past its level is rejected before launch."""
    import htree_amd

    q, k, v, dO = (x.to(DEV) for x in inputs(1, 1500, 8, 2, 64, "bfloat16", 41, dO=True))
    out, ctx = htree_amd.htree_forward(q, k, v, 16, 128, 16, _save_for_backward=True)
    a = htree_amd.htree_backward(dO, q, out, dict(ctx, train_scores=None))
    plp = {l: t.clone() for l, t in ctx["per_layer_parents"].items()}
    b = htree_amd.htree_backward(dO, q, out, dict(ctx, per_layer_parents=plp))
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    bad = {l: t.clone() for l, t in plp.items()}
    bad[0][0, 1499, 0, 0] = 94  # level 0 lists name level-1 nodes: 94 of them
    with pytest.raises(AssertionError, match="outside"):
        htree_amd.htree_backward(dO, q, out, dict(ctx, per_layer_parents=bad))


@pytest.mark.parametrize("H", [8, 32], ids=["G4", "G16pairs"])
def test_backward_lists_edited_in_place(H):
    """per_layer_parents edited in place (views of the forward's stacked
    lists, which share their version counter) are the caller's lists: the
    backward drops the scores the forward stored for its own lists, checks
    the edited lists and copies them to every KV-head copy (G 32 runs as
    pairs).  An edit that keeps the values gives bitwise the gradients of
    the rebuilt-score backward; an edit that breaks a list is rejected."""
    import htree_amd

    q, k, v, dO = (x.to(DEV) for x in inputs(1, 1500, H, 1, 128, "bfloat16", 42, dO=True))
    out, ctx = htree_amd.htree_forward(q, k, v, 16, 128, 16, _save_for_backward=True,
                                       _save_scores=True)
    assert ctx["train_scores"] is not None
    a = htree_amd.htree_backward(dO, q, out, dict(ctx, train_scores=None))
    plp = ctx["per_layer_parents"]
    plp[0][0, 700, 0, 3] = plp[0][0, 700, 0, 3].clone()  # same value, new version
    b = htree_amd.htree_backward(dO, q, out, ctx)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    plp[0][0, 1499, 0, 0] = 94  # a level-1 node past the level's 94
    with pytest.raises(AssertionError, match="outside"):
        htree_amd.htree_backward(dO, q, out, ctx)


AUTOGRAD = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype, seed, DS budget (None: default)
    (1, 1500, 8, 1, 128, 16, 16, 128, "bfloat16", 4, None),   # stored scores and dS
    (1, 1500, 8, 1, 128, 16, 16, 128, "bfloat16", 4, "0"),    # dq recomputes the scores
    (1, 1100, 8, 1, 128, 32, 8, 256, "float16", 5, None),
    (1, 900, 8, 2, 64, 8, 16, 128, "float32", 6, None),
    (1, 2000, 8, 2, 64, 16, 128, 1024, "bfloat16", 7, None),  # wide forward
    (1, 1200, 24, 1, 64, 16, 16, 128, "bfloat16", 8, None),   # G 24: KV-head pairs
    (1, 1000, 8, 2, (32, 64), 16, 16, 128, "float16", 9, None),  # K 32 padded to V 64
]


@pytest.mark.parametrize("cfg", AUTOGRAD, ids=lambda c: f"D{c[4]}G{c[2] // c[3]}tk{c[6]}{c[8]}"
                         .replace(", ", "x") + ("_recompute" if c[10] else ""))
def test_autograd_contract(cfg, monkeypatch):
    """HTreeTritonFunction: grads in the input dtype, None for non-tensors,
    equal bit for bit to htree_backward's fp32 gradients cast to the dtype
    (the reference's backward, src/backward.py:1193).  The kernels round
    them as they store them, except for KV-head pairs, whose halves are
    added in fp32 first."""
    import htree_amd

    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed, budget = cfg
    print(f"case {cfg}", flush=True)
    if budget is not None:
        monkeypatch.setenv("HTREE_DS_BUDGET_MB", budget)
    dt = getattr(torch, dtype)
    K, V = D if isinstance(D, tuple) else (D, D)
    q, k, _ = inputs(B, T, H, Hkv, K, dtype, seed)
    _, _, v, dO = inputs(B, T, H, Hkv, V, dtype, seed + 100, dO=True)
    qg, kg, vg = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
    out = htree_amd.htree_forward_triton_autograd(qg, kg, vg, CR, MTN, TK)
    out.backward(dO.to(DEV))
    for x in (qg, kg, vg):
        assert x.grad.dtype == dt and x.grad.shape == x.shape and x.grad.is_contiguous()
    _, _, _, _, dq, dk, dv = run(q, k, v, dO, CR, TK, MTN)
    for name, got, ref in (("dq", qg.grad, dq), ("dk", kg.grad, dk), ("dv", vg.grad, dv)):
        r = torch.from_numpy(ref).to(dt).float().numpy()
        assert np.array_equal(got.float().cpu().numpy(), r), name


WIDE = [
    # top_k > 64 or more than 64 candidate tiles per level
    (1, 1500, 8, 2, 32, 4, 128, 256, "float32", 41),    # CR 4, 3 levels, evictions at level 1
    (1, 2000, 8, 2, 64, 16, 128, 1024, "bfloat16", 42),  # 125 tiles at the bottom
    (1, 1500, 8, 2, 256, 16, 128, 1024, "bfloat16", 48),  # D = 256
    (1, 2000, 32, 1, 64, 16, 128, 1024, "bfloat16", 49),   # G = 32: the wide forward's KV-head pairs
    (1, 1500, 48, 2, 32, 4, 256, 256, "float32", 50),      # G = 24, CR 4, three levels
    (1, 1200, 64, 1, 64, 8, 128, 128, "bfloat16", 51),     # G = 64: KV-head quads, three levels
]


@pytest.mark.parametrize("cfg", WIDE, ids=lambda c: f"T{c[1]}D{c[4]}cr{c[5]}tk{c[6]}{c[8]}")
def test_backward_wide_matches_oracle(cfg):
    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v, dO = inputs(B, T, H, Hkv, D, dtype, seed, dO=True)
    out, par, gmax, gsum, dq, dk, dv = run(q, k, v, dO, CR, TK, MTN)
    rep = check_backward(q, k, v, dO, CR, TK, MTN, dtype, out, par, gmax, gsum, dq, dk, dv)
    print(rep, flush=True)


REGIME = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype, seed
    (1, 12000, 16, 4, 32, 16, 512, 8192, "float32", 43),  # correctness_test_bwd.py defaults
    (1, 20000, 8, 2, 32, 16, 1024, 16384, "float32", 45),  # top_k 1024: 16384 candidates
    (1, 20000, 8, 2, 64, 32, 512, 512, "bfloat16", 46),    # top_k 512 at CR 32, 3 levels
    (1, 20000, 8, 2, 32, 128, 128, 16384, "float16", 47),  # CR 128, 16384 candidates
]


@pytest.mark.parametrize("cfg", REGIME, ids=lambda c: f"T{c[1]}D{c[4]}cr{c[5]}tk{c[6]}{c[8]}")
def test_backward_reference_default_regime(cfg):
    """correctness_test_bwd.py defaults (T=12000, Hq=16, Hkv=4, K=V=32, fp32,
    CR=16, top_k=512, MTN=8192) and the largest candidate sets (16384 per
    level): dq on sampled rows and final dk / dv at sampled level-0 nodes vs
    the oracle; the sum of dv over the nodes equals the sum of dO over the
    group's queries and heads (every head's probabilities sum to 1, the
    pooling backward keeps sums)."""
    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v, dO = inputs(B, T, H, Hkv, D, dtype, seed, dO=True)
    out, par, gmax, gsum, dq, dk, dv = run(q, k, v, dO, CR, TK, MTN)
    assert np.all(np.isfinite(dq)) and np.all(np.isfinite(dk)) and np.all(np.isfinite(dv))
    G = H // Hkv
    want = dO.float().numpy().reshape(B, T, Hkv, G, D).astype(np.float64).sum(axis=(1, 3))
    got = dv.astype(np.float64).sum(axis=1)
    atol = 1e-4 * np.sqrt(T * G)
    if dtype != "float32":
        # each node's dv rounded once to bf16 (relative 2^-9): the rounding
        # errors of the sum stay within a few 2^-9 sqrt(sum dv^2)
        atol = atol + 4 * 2.0 ** -9 * np.sqrt((dv.astype(np.float64) ** 2).sum(axis=1))
    ratio = np.abs(got - want) / (atol + 1e-4 * np.abs(want))
    print("dv mass check: worst error / bound", float(ratio.max()), flush=True)
    assert ratio.max() <= 1.0
    tree = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, dtype)
    rng = np.random.default_rng(4)
    n = 40
    rows = np.stack([np.zeros(n, int), np.sort(rng.choice(T, n, replace=False))], 1).astype(np.int32)
    rows = np.concatenate([rows, [[0, T - 1]]]).astype(np.int32)
    pr = par[:, rows[:, 0], rows[:, 1]]
    fw = orc.forward(q.float().numpy(), tree, D ** -0.5, rows=rows, forced=pr)
    o = out[rows[:, 0], rows[:, 1]]
    d = dO.float().numpy()[rows[:, 0], rows[:, 1]]
    delta = (o.astype(np.float64) * d).sum(-1).astype(np.float32)
    ref = orc.backward_dq_rows(q.float().numpy(), tree, D ** -0.5, rows, pr, fw["gmax"], fw["gsum"],
                               delta, d)
    ok, worst = close(dq[rows[:, 0], rows[:, 1]], ref, dtype)
    print("default-regime dq worst", worst, flush=True)
    assert ok
    rep = check_dkv_sampled(q.float().numpy(), dO.float().numpy(), out, k.float().numpy(),
                            v.float().numpy(), par, gmax, gsum, dk, dv, CR, TK, MTN, dtype,
                            [(0, 0), (0, Hkv - 1)], seed + 1)
    print("default-regime dk/dv at sampled nodes", rep, flush=True)


@pytest.mark.parametrize("cfg", [(1, 1500, 16, 2, 128, 16, 16, 128, "bfloat16", 61),
                                 (1, 1100, 8, 1, 128, 32, 8, 256, "float16", 62),
                                 (1, 900, 8, 2, 64, 8, 16, 128, "float32", 63),
                                 (1, 4096, 8, 2, 64, 16, 16, 16, "bfloat16", 64)],
                         ids=lambda c: f"D{c[4]}cr{c[5]}{c[8]}")
def test_backward_recomputed_dq(cfg, monkeypatch):
    """The dq pass that recomputes the scores (taken when the stored dS
    would exceed its memory budget or the caller's workspace, and for
    top_k > 64), forced here by a zero budget."""
    monkeypatch.setenv("HTREE_DS_BUDGET_MB", "0")
    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v, dO = inputs(B, T, H, Hkv, D, dtype, seed, dO=True)
    out, par, gmax, gsum, dq, dk, dv = run(q, k, v, dO, CR, TK, MTN)
    print(check_backward(q, k, v, dO, CR, TK, MTN, dtype, out, par, gmax, gsum, dq, dk, dv), flush=True)


@pytest.mark.parametrize("cfg", [(1, 2048, 16, 1, 128, 16, 16, 128, 71),
                                 (1, 1500, 8, 2, 64, 8, 16, 64, 72),
                                 (1, 1200, 16, 4, 32, 16, 8, 128, 73)],
                         ids=lambda c: f"D{c[4]}cr{c[5]}")
def test_backward_power_of_two_scalings(cfg):
    """bf16 inputs keep the stored dS and the K~ blocks dq reads as fp16
    with a power-of-two scale per tile / block.  Gradients are linear in dO,
    and (q 2^-s, k 2^s) leaves every score unchanged while dq scales by 2^s
    and dk by 2^-s; power-of-two factors commute with every rounding step
    when nothing overflows or underflows, so the scaled runs reproduce the
    plain run's gradients exactly.  The factors take |dS| far past fp16's
    largest value (dO 2^15), deep below its smallest (dO 2^-30) and K~ past
    it (k 2^16): without the per-tile / per-block scales these runs would
    give inf, or lose the small values."""
    B, T, H, Hkv, D, CR, TK, MTN, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v, dO = inputs(B, T, H, Hkv, D, "bfloat16", seed, dO=True)
    base = run(q, k, v, dO, CR, TK, MTN)
    for s_do, s_k in ((15, 0), (-30, 0), (0, 16)):
        print(f"dO 2^{s_do}, k 2^{s_k}", flush=True)
        got = run(q * 2.0 ** -s_k, k * 2.0 ** s_k, v, dO * 2.0 ** s_do, CR, TK, MTN)
        assert np.array_equal(got[1], base[1])  # same selection
        for name, i, f in (("dq", 4, s_do + s_k), ("dk", 5, s_do - s_k), ("dv", 6, s_do)):
            g = got[i].astype(np.float64) * 2.0 ** -f
            assert np.all(np.isfinite(g)), name
            np.testing.assert_array_equal(g, base[i].astype(np.float64), err_msg=name)


def test_backward_min_workspace():
    """Given the smallest workspace (htree_backward_workspace_min_bytes) the
    backward recomputes the scores in its dq pass instead of storing dS; the
    gradients meet the bar against the oracle and agree with the
    full-workspace run (dk, dv bit-exact: only dq's product changes; the
    94-node top level is too small for the merged 64-child view), and one
    byte less is rejected before any launch."""
    import htree_amd
    from htree_amd import _native as N

    B, T, H, Hkv, D, CR, TK, MTN = 1, 1500, 16, 2, 128, 16, 16, 128
    q, k, v, dO = inputs(B, T, H, Hkv, D, "bfloat16", 81, dO=True)
    qd, dOd = q.to(DEV), dO.to(DEV)
    out, par, gmax, gsum, ctx = htree_amd.htree_forward_parents(qd, k.to(DEV), v.to(DEV), CR, MTN, TK)
    d = ctx["dims"]
    nfull, nmin = N.ctypes.c_int64(), N.ctypes.c_int64()
    N.check(N.lib().htree_backward_workspace_bytes(N.ctypes.byref(d), N.ctypes.byref(nfull)), "ws")
    N.check(N.lib().htree_backward_workspace_min_bytes(N.ctypes.byref(d), N.ctypes.byref(nmin)), "ws")
    assert 0 < nmin.value < nfull.value
    ws, cos, sin = ctx["packed_tree"], ctx["cos_cache"], ctx["sin_cache"]

    def call(nbytes):
        dq = torch.empty(B, T, H, D, dtype=torch.float32, device=DEV)
        dk = torch.empty(B, T, Hkv, D, dtype=torch.float32, device=DEV)
        dv = torch.empty_like(dk)
        bws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        rc = N.lib().htree_backward(d, float(ctx["scale"]), N.ptr(qd), N.ptr(out), N.ptr(dOd),
                                    N.ptr(gmax), N.ptr(gsum), N.ptr(ctx["parents_stacked"]), N.ptr(ws),
                                    ws.numel(), N.ptr(cos), N.ptr(sin), N.ptr(dq), N.ptr(dk), N.ptr(dv),
                                    N.ptr(bws), bws.numel(), N.stream_ptr(qd.device))
        torch.cuda.synchronize()
        return rc, [x.cpu().numpy() for x in (dq, dk, dv)]

    rc, full = call(nfull.value)
    N.check(rc, "htree_backward")
    rc, small = call(nmin.value)
    N.check(rc, "htree_backward")
    rc, _ = call(nmin.value - 1)
    assert rc < 0
    f = lambda x: x.float().cpu().numpy()
    print(check_backward(q, k, v, dO, CR, TK, MTN, "bfloat16", f(out), par.cpu().numpy(), f(gmax),
                         f(gsum), *small), flush=True)
    assert np.array_equal(small[1], full[1]) and np.array_equal(small[2], full[2])
    ok, worst = close(small[0], full[0], "bfloat16")
    assert ok, worst
