"""GPU parity of the drop-in's other entry paths, against the CPU oracle:

* a bwd_ctx holding exactly the reference's keys (src/parallel.py:1139-1158),
  made at a non-default rope_base: the backward rebuilds the operand tree and
  (without per_layer_parents) replays the selection with the context's own
  RoPE tables, as src/backward.py:848-934 does;
* the autograd modes: the default (the reference's eight saved tensors,
  src/backward.py:1141-1145, plus the parent lists and the packed tree), the
  lean mode (the eight alone: the same gradients from the selection-only
  replay, htree_select, whose lists are the forward's) and the stored-score
  mode; the backward's workspace choice under a memory limit;
* K != V head dims (src/parallel.py:904, src/naive.py:144): forward and
  backward against the oracle's native two-dim restatement."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import DT, check_backward, check_forward, close

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

REF_KEYS = ("global_max", "global_sum", "per_layer_parents", "layers_k", "layers_v", "cos_cache",
            "sin_cache", "num_layers", "compression_rate", "top_k_per_layer", "max_top_nodes",
            "scale", "NUM_GROUPS", "G_PAD", "TILE_P", "DROP_BLOCK")


def seeded(B, T, H, Hkv, K, V, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g).to(DT[dtype])
    return r(B, T, H, K), r(B, T, Hkv, K), r(B, T, Hkv, V), r(B, T, H, V)


@pytest.mark.parametrize("with_parents", [True, False], ids=["parents", "replay"])
@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_reference_keys_context(with_parents, dtype):
    import htree_amd

    B, T, H, Hkv, D, CR, TK, MTN, base = 1, 2000, 16, 2, 64, 16, 16, 128, 500.0
    print(f"case ref-keys ctx {dtype} parents={with_parents}", flush=True)
    q, k, v, dO = seeded(B, T, H, Hkv, D, D, dtype, 51)
    qd, kd, vd, dOd = (x.to(DEV) for x in (q, k, v, dO))
    out, ctx = htree_amd.htree_forward(qd, kd, vd, CR, MTN, TK, rope_base=base,
                                       _save_for_backward=True)
    full = htree_amd.htree_backward(dOd, qd, out, ctx)
    ref_ctx = {key: ctx[key] for key in REF_KEYS}
    if not with_parents:
        ref_ctx["per_layer_parents"] = None
    got = htree_amd.htree_backward(dOd, qd, out, ref_ctx)
    torch.cuda.synchronize()
    par = ctx["parents_stacked"].cpu().numpy()
    f = lambda x: x.float().cpu().numpy()
    tree = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, dtype, base)
    rep = check_backward(q, k, v, dO, CR, TK, MTN, dtype, f(out), par, f(ctx["global_max"]),
                         f(ctx["global_sum"]), *[f(x) for x in got], tree=tree)
    print(rep, flush=True)
    if not with_parents:
        # the selection-only replay selects the same lists; the backward then
        # rebuilds the scores, as the full context's does without its stored ones
        rebuilt = htree_amd.htree_backward(dOd, qd, out, dict(ctx, train_scores=None))
        for a, b in zip(got, rebuilt):
            assert torch.equal(a, b)
    # the forward at this base is the oracle's at this base, not at 10000
    rows = orc.all_rows(B, T)[::3]
    check_forward(q, k, v, CR, TK, MTN, dtype, rows=rows, out_dev=f(out), parents_dev=par, tree=tree,
                  gmax_dev=f(ctx["global_max"]), gsum_dev=f(ctx["global_sum"]))
    tree0 = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, dtype)
    with pytest.raises(AssertionError):
        check_forward(q, k, v, CR, TK, MTN, dtype, rows=rows, out_dev=f(out), parents_dev=par,
                      tree=tree0)


def test_reference_keys_context_without_max_top_nodes():
    """A context without max_top_nodes (it is not among the keys the
    reference's backward reads) still resolves the tree's levels."""
    import htree_amd

    B, T, H, Hkv, D, CR, TK, MTN = 1, 3000, 8, 1, 64, 8, 16, 64
    q, k, v, dO = (x.to(DEV) for x in seeded(B, T, H, Hkv, D, D, "bfloat16", 52))
    out, ctx = htree_amd.htree_forward(q, k, v, CR, MTN, TK, _save_for_backward=True)
    a = htree_amd.htree_backward(dO, q, out, dict(ctx, train_scores=None))
    ref_ctx = {key: ctx[key] for key in REF_KEYS if key != "max_top_nodes"}
    b = htree_amd.htree_backward(dO, q, out, ref_ctx)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_autograd_modes(dtype):
    """The three autograd modes.  Default: the reference's eight tensors plus
    the parent lists and the packed tree are saved, nothing more (no stored
    scores); `_save_parents=False` saves the eight alone and replays the
    selection in the backward: bitwise the default mode's gradients, and
    those of htree_backward on the forward's own lists with rebuilt scores.
    `_save_scores=True` also saves the scores (bf16 only) and agrees within
    the bar; the gradients are checked against the oracle."""
    import htree_amd

    B, T, H, Hkv, D, CR, TK, MTN = 1, 2500, 16, 2, 128, 16, 16, 128
    q, k, v, dO = seeded(B, T, H, Hkv, D, D, dtype, 53)
    dOd = dO.to(DEV)
    grads = {}
    for mode in ("default", "scores", "lean"):
        qg, kg, vg = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
        out = htree_amd.htree_forward_triton_autograd(qg, kg, vg, CR, MTN, TK, rope_base=2000.0,
                                                      _save_parents=mode != "lean",
                                                      _save_scores=mode == "scores")
        saved = [t for t in out.grad_fn.saved_tensors if t is not None]
        scores = mode == "scores" and dtype == "bfloat16"
        assert len(saved) == {"default": 10, "scores": 10 + scores, "lean": 8}[mode], len(saved)
        out.backward(dOd)
        torch.cuda.synchronize()
        grads[mode] = (out.detach(), qg.grad, kg.grad, vg.grad)
    for mode in ("scores", "lean"):
        assert torch.equal(grads[mode][0], grads["default"][0])
    qd, kd, vd = (x.to(DEV) for x in (q, k, v))
    out, ctx = htree_amd.htree_forward(qd, kd, vd, CR, MTN, TK, rope_base=2000.0,
                                       _save_for_backward=True)
    assert ctx["train_scores"] is None
    rebuilt = htree_amd.htree_backward(dOd, qd, out, ctx, _grad_dtype=q.dtype)
    torch.cuda.synchronize()
    f = lambda x: x.float().cpu().numpy()
    for a, b, c, s in zip(grads["lean"][1:], rebuilt, grads["default"][1:], grads["scores"][1:]):
        assert torch.equal(a, b)
        assert torch.equal(a, c)
        ok, w = close(f(s), f(c), dtype)
        assert ok, w
    par = ctx["parents_stacked"].cpu().numpy()
    tree = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, dtype, 2000.0)
    for mode in ("default", "scores"):
        g = [f(x) for x in grads[mode][1:]]
        rep = check_backward(q, k, v, dO, CR, TK, MTN, dtype, f(out), par, f(ctx["global_max"]),
                             f(ctx["global_sum"]), *g, tree=tree)
        print(mode, rep, flush=True)


def test_backward_workspace_limit():
    """The stored-dS workspace is taken only where it fits what may be
    spent (default: what the device can spare); below it the backward runs
    in the smallest workspace and dq recomputes the scores.  The plan taken
    is recorded in the context; both meet the bar against the oracle and
    agree with each other within it."""
    import htree_amd
    from htree_amd import _native as N

    B, T, H, Hkv, D, CR, TK, MTN = 1, 3000, 16, 2, 128, 16, 16, 128
    q, k, v, dO = seeded(B, T, H, Hkv, D, D, "bfloat16", 54)
    qd, kd, vd, dOd = (x.to(DEV) for x in (q, k, v, dO))
    out, ctx = htree_amd.htree_forward(qd, kd, vd, CR, MTN, TK, _save_for_backward=True)
    nb = N.ctypes.c_int64()
    N.check(N.lib().htree_backward_workspace_bytes(N.ctypes.byref(ctx["dims"]),
                                                   N.ctypes.byref(nb)), "bytes")
    full = nb.value
    a = htree_amd.htree_backward(dOd, qd, out, ctx)
    assert ctx["backward_plan"] == "stored_ds"
    b = htree_amd.htree_backward(dOd, qd, out, ctx, _workspace_limit=full - 1)
    assert ctx["backward_plan"] == "recompute"
    torch.cuda.synchronize()
    f = lambda x: x.float().cpu().numpy()
    par = ctx["parents_stacked"].cpu().numpy()
    for g in (a, b):
        rep = check_backward(q, k, v, dO, CR, TK, MTN, "bfloat16", f(out), par,
                             f(ctx["global_max"]), f(ctx["global_sum"]), *[f(x) for x in g])
        print(rep, flush=True)
    for x, y in zip(a, b):
        ok, w = close(f(x), f(y), "bfloat16")
        assert ok, w


SELECT_CASES = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype, seed: every forward and group form
    (1, 2500, 16, 2, 128, 16, 16, 128, "bfloat16", 91),   # register forward, 3 levels
    (1, 3001, 8, 1, 64, 8, 32, 64, "float16", 92),        # streaming forward, 3 levels
    (1, 3000, 16, 4, 32, 4, 128, 256, "float32", 93),     # wide forward, 3 levels
    (1, 20000, 8, 2, 32, 16, 1024, 16384, "bfloat16", 94),  # wide, 64 keys per thread
    (1, 1501, 32, 1, 128, 16, 16, 128, "bfloat16", 95),   # KV-head pairs (register)
    (1, 2200, 32, 1, 64, 8, 256, 256, "bfloat16", 96),    # KV-head pairs (wide), 3 levels
    (1, 3001, 32, 1, 128, 32, 32, 256, "bfloat16", 101),  # KV-head pairs (streaming)
    (1, 1500, 64, 1, 32, 4, 64, 64, "bfloat16", 97),      # KV-head quads, 4 levels
    (1, 1000, 17, 1, 64, 4, 16, 32, "float32", 98),       # padding heads (streaming), 4 levels
    (1, 1200, 33, 1, 32, 16, 128, 256, "float16", 99),    # quads with padding heads
    (2, 500, 8, 2, 64, 16, 32, 512, "bfloat16", 100),     # one level: no selection at all
]


@pytest.mark.parametrize("cfg", SELECT_CASES, ids=lambda c: f"G{c[2] // c[3]}D{c[4]}cr{c[5]}tk{c[6]}{c[8]}")
def test_select_matches_forward_lists(cfg):
    """htree_select (selection only) writes the forward's parent lists of
    every level, bit for bit, in every forward form and group layout."""
    import htree_amd
    from htree_amd.parallel import select_frame

    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v, _ = seeded(B, T, H, Hkv, D, D, dtype, seed)
    qd, kd, vd = (x.to(DEV) for x in (q, k, v))
    out, ctx = htree_amd.htree_forward(qd, kd, vd, CR, MTN, TK, _save_for_backward=True)
    hf = ctx["head_frame"]
    cos_k, sin_k = hf.tables(ctx["cos_cache"], ctx["sin_cache"])
    sel, _ = select_frame(hf.q_heads(hf.pad_qk(qd)), hf.kv_k(kd), hf.kv_v(vd), ctx["dims"], cos_k,
                          sin_k, ctx["scale"])
    torch.cuda.synchronize()
    assert sel.shape == ctx["parents_stacked"].shape
    assert torch.equal(sel, ctx["parents_stacked"])


KV_CASES = [
    # B, T, H, Hkv, K, V, CR, TK, MTN, dtype, seed
    (1, 2000, 16, 2, 128, 64, 16, 16, 128, "bfloat16", 61),
    (1, 1500, 8, 1, 64, 128, 16, 8, 128, "bfloat16", 62),
    (1, 1200, 8, 2, 32, 64, 8, 16, 128, "float32", 63),
    (2, 900, 4, 1, 64, 32, 4, 32, 64, "float16", 64),
    # head dims that are not a kernel head dim: zero-padded to the next one
    (1, 1500, 8, 1, 16, 16, 16, 16, 128, "bfloat16", 65),   # K = V = 16 on D = 32
    (1, 1200, 8, 2, 96, 96, 16, 16, 128, "float32", 66),    # K = V = 96 on D = 128
    (1, 1000, 4, 1, 80, 48, 8, 16, 64, "float16", 67),      # K = 80, V = 48 on D = 128
]


@pytest.mark.parametrize("cfg", KV_CASES, ids=lambda c: f"K{c[4]}V{c[5]}cr{c[6]}{c[9]}")
def test_separate_value_dim(cfg):
    import htree_amd

    B, T, H, Hkv, K, V, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v, dO = seeded(B, T, H, Hkv, K, V, dtype, seed)
    qd, kd, vd = (x.to(DEV) for x in (q, k, v))
    out, par, gmax, gsum, ctx = htree_amd.htree_forward_parents(qd, kd, vd, CR, MTN, TK)
    assert out.shape == (B, T, H, V) and out.dtype == q.dtype
    assert ctx["layers_k"][0] is kd and ctx["layers_v"][0] is vd
    assert all(x.shape[-1] == K for x in ctx["layers_k"]) and all(x.shape[-1] == V for x in ctx["layers_v"])
    dq, dk, dv = htree_amd.htree_backward(dO.to(DEV), qd, out, ctx)
    torch.cuda.synchronize()
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    f = lambda x: x.float().cpu().numpy()
    tree = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, dtype)
    for l in range(1, tree.L):  # the caller-frame levels are the oracle's, bit for bit
        assert np.array_equal(f(ctx["layers_k"][l]), tree.lk[l]) and np.array_equal(f(ctx["layers_v"][l]), tree.lv[l])
    par = par.cpu().numpy()
    rep = check_forward(q, k, v, CR, TK, MTN, dtype, out_dev=f(out), parents_dev=par, tree=tree,
                        gmax_dev=f(gmax), gsum_dev=f(gsum))
    rep.update(check_backward(q, k, v, dO, CR, TK, MTN, dtype, f(out), par, f(gmax), f(gsum), f(dq),
                              f(dk), f(dv), tree=tree))
    print(rep, flush=True)
    # the autograd path at K != V, lean and default: same gradients
    for save in (True, False):
        qg, kg, vg = (x.clone().requires_grad_(True) for x in (qd, kd, vd))
        o = htree_amd.htree_forward_triton_autograd(qg, kg, vg, CR, MTN, TK, _save_parents=save)
        o.backward(dO.to(DEV))
        for got, ref in ((qg.grad, dq), (kg.grad, dk), (vg.grad, dv)):
            ok, w = close(f(got), f(ref.to(got.dtype)), dtype)
            assert ok, w


G_CASES = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype, seed
    (1, 1501, 32, 1, 128, 16, 16, 128, "bfloat16", 71),  # G = 32; 1501 pairs: a last block half empty
    (1, 1500, 48, 2, 64, 8, 16, 128, "float32", 72),      # G = 24
    (2, 900, 64, 2, 32, 16, 8, 128, "float16", 73),       # G = 32, two batches, two KV heads
    # 64 candidate tiles per level: the streaming forward's paired waves
    (1, 3001, 32, 1, 128, 32, 32, 256, "bfloat16", 74),  # G = 32, C4's CR / top_k
    (1, 2500, 48, 2, 32, 8, 64, 256, "float16", 75),      # G = 24, top_k 64, three levels
    # top_k > 64: the wide forward's KV-head pairs (one block, two halves)
    (1, 3000, 48, 2, 32, 16, 128, 256, "float32", 76),    # G = 24
    (1, 2200, 32, 1, 64, 8, 256, 256, "bfloat16", 77),    # G = 32, CR 8, three levels
    # groups of 33..64 heads: KV-head quads, the wide forward at every level size
    (1, 1200, 64, 1, 64, 16, 16, 128, "bfloat16", 78),   # G = 64, 16 tiles per level
    (1, 1000, 80, 2, 32, 8, 32, 128, "float16", 79),     # G = 40: 10 heads per part
    (1, 1500, 64, 1, 32, 16, 128, 256, "float32", 80),   # G = 64, top_k 128
    # groups that 2 or 4 does not divide: padding heads left out of the selection
    (1, 1000, 17, 1, 64, 16, 16, 128, "bfloat16", 81),   # G = 17: pairs of 9, one padding head
    (1, 900, 62, 2, 32, 8, 32, 128, "float16", 82),      # G = 31: streaming forward's pairs
    (1, 1500, 23, 1, 32, 16, 128, 256, "float32", 83),   # G = 23: wide forward's pairs
    (1, 1200, 33, 1, 32, 16, 128, 256, "float32", 84),   # G = 33: quads of 9, three padding heads
    (1, 1000, 50, 1, 64, 4, 16, 64, "bfloat16", 85),     # G = 50: quads of 13, CR 4
]


@pytest.mark.parametrize("cfg", G_CASES, ids=lambda c: f"G{c[2] // c[3]}D{c[4]}cr{c[5]}{c[8]}")
def test_query_groups_over_16_heads(cfg):
    """Groups of 17..64 query heads (the reference pads them to G_PAD,
    src/parallel.py:1023): forward, backward, trace and both autograd modes
    against the oracle, which restates any group size directly."""
    import htree_amd

    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v, dO = seeded(B, T, H, Hkv, D, D, dtype, seed)
    qd, kd, vd, dOd = (x.to(DEV) for x in (q, k, v, dO))
    out, par, gmax, gsum, ctx = htree_amd.htree_forward_parents(qd, kd, vd, CR, MTN, TK)
    assert par.shape == (ctx["num_layers"], B, T, Hkv, TK)
    assert ctx["per_layer_parents"][0].shape == (B, T, Hkv, TK)
    dq, dk, dv = htree_amd.htree_backward(dOd, qd, out, ctx)
    torch.cuda.synchronize()
    assert dk.shape == k.shape and dv.shape == v.shape
    f = lambda x: x.float().cpu().numpy()
    tree = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, dtype)
    for l in range(1, tree.L):
        assert np.array_equal(f(ctx["layers_k"][l]), tree.lk[l])
    parn = par.cpu().numpy()
    rep = check_forward(q, k, v, CR, TK, MTN, dtype, out_dev=f(out), parents_dev=parn, tree=tree,
                        gmax_dev=f(gmax), gsum_dev=f(gsum))
    rep.update(check_backward(q, k, v, dO, CR, TK, MTN, dtype, f(out), parn, f(gmax), f(gsum), f(dq),
                              f(dk), f(dv), tree=tree))
    print(rep, flush=True)
    tout, tr = htree_amd.run_parallel_with_trace(qd, kd, vd, CR, MTN, TK, None, 10000.0)
    torch.cuda.synchronize()
    for l in range(1, tr["num_layers"]):
        assert torch.equal(tr["layers"][l].selected_parents, par[l - 1]), l
    ok, w = close(f(tout), f(out), dtype)
    assert ok, w
    for save in (True, False):
        qg, kg, vg = (x.clone().requires_grad_(True) for x in (qd, kd, vd))
        o = htree_amd.htree_forward_triton_autograd(qg, kg, vg, CR, MTN, TK, _save_parents=save)
        o.backward(dOd)
        for got, ref in ((qg.grad, dq), (kg.grad, dk), (vg.grad, dv)):
            ok, w = close(f(got), f(ref.to(got.dtype)), dtype)
            assert ok, w
