"""GPU parity of the split selection (htree_amd/csrc/htree_split.hip): the
configurations whose shared Top-K one block cannot hold.

  * query groups of more than 64 heads (kernel shares of 8 and 16 KV-head
    copies, padding heads where the share does not divide the group);
  * groups of 33..64 heads over 8192 candidates per level (quads whose four
    importance arrays exceed one block's LDS);
  * candidate sets above 16384 per level (32768 and 65536);
  * lists of more than 1024 parents (top_k 2048).

Forward: every level's selection against the oracle's from the same parent
list (ties as tests/helpers.py), outputs and state teacher-forced on the
device's lists, list invariants on every row, and htree_select's lists equal
to the forward's bit for bit.  Backward: the oracle's gradients on every row
where the oracle is cheap, else dq on sampled rows, dk / dv at sampled
level-0 nodes and the dv mass."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import (check_backward, check_dkv_sampled, check_forward, check_state, close,
                            inputs)

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def run_fwd(q, k, v, CR, TK, MTN):
    import htree_amd

    out, par, gmax, gsum, ctx = htree_amd.htree_forward_parents(
        q.to(DEV), k.to(DEV), v.to(DEV), compression_rate=CR, max_top_nodes=MTN,
        top_k_per_layer=TK)
    torch.cuda.synchronize()
    return (out.float().cpu().numpy(), par.cpu().numpy(), gmax.cpu().numpy(),
            gsum.cpu().numpy(), ctx)


def list_invariants(par, T, CR, TK):
    L = par.shape[0]
    t = np.arange(T)
    for l in range(L - 1, 0, -1):
        sel = par[l - 1]
        cnt = (sel >= 0).sum(-1)
        want = np.array([orc.candidate_counts(int(x), CR, TK, L)[l][1] for x in t])
        assert np.array_equal(cnt, np.broadcast_to(want[None, :, None], cnt.shape)), f"level {l} counts"
        right = (t // CR ** l).astype(np.int32)
        assert np.all(np.any(sel == right[None, :, None, None], axis=-1)), f"level {l} rightmost"
        nxt_valid = sel[..., 1:] >= 0
        assert np.all((np.diff(sel, axis=-1) > 0) | ~nxt_valid), f"level {l} ascending"


def sample_rows(B, T, n, seed):
    rng = np.random.default_rng(seed)
    rows = np.stack([rng.integers(0, B, n), np.sort(rng.choice(T, n, replace=False))], 1)
    return np.concatenate([rows, [[0, 0], [B - 1, T - 1]]]).astype(np.int32)


FWD = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype, seed
    (1, 4100, 128, 1, 64, 16, 16, 16, "bfloat16", 81),   # G = 128: share 8, three levels
    (2, 3000, 200, 2, 32, 16, 32, 256, "float32", 82),   # G = 100: share 8 of 13, 4 padding heads
    (1, 1500, 256, 1, 32, 8, 16, 64, "float16", 83),     # G = 256: share 16, CR 8, three levels
    (1, 3000, 72, 1, 128, 32, 8, 256, "bfloat16", 84),   # G = 72: share 8 of 9, CR 32
    # G = 48 (quads) over 16384 candidates per level: level 1 selects 512 of 1024
    (1, 32768, 48, 1, 32, 32, 512, 32, "bfloat16", 85),
    # 32768 candidates per level (G = 16, no share): level 1 selects 1024 of 2048
    (1, 65536, 16, 1, 32, 32, 1024, 64, "bfloat16", 86),
    # 65536 candidates per level at the bottom, 1024 threads in the selection
    (1, 65536, 8, 1, 32, 64, 1024, 16, "float16", 87),
    # lists of 2048 parents: level 1 selects 2048 of up to 3004 (CR 4)
    (1, 12000, 16, 1, 32, 4, 2048, 8192, "bfloat16", 88),
    # and 2048 of up to 2256 at CR 16, over 32768 candidates at the bottom
    (1, 36000, 16, 1, 64, 16, 2048, 32768, "float16", 89),
]


@pytest.mark.parametrize("cfg", FWD, ids=lambda c: f"T{c[1]}G{c[2] // c[3]}D{c[4]}cr{c[5]}tk{c[6]}{c[8]}")
def test_split_forward_matches_oracle(cfg):
    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v = inputs(B, T, H, Hkv, D, dtype, seed)
    out, par, gmax, gsum, ctx = run_fwd(q, k, v, CR, TK, MTN)
    assert np.all(np.isfinite(out))
    list_invariants(par, T, CR, TK)
    rows = sample_rows(B, T, 48 if T > 20000 else 120, seed)
    rep = check_forward(q, k, v, CR, TK, MTN, dtype, rows=rows, out_dev=out, parents_dev=par,
                        gmax_dev=gmax, gsum_dev=gsum)
    print(rep, flush=True)


@pytest.mark.parametrize("cfg", [FWD[1], FWD[4]], ids=["G100", "G48quads16384"])
def test_split_select_matches_forward(cfg):
    """htree_select (the backward's replay) runs the same scoring and select
    launches: its lists equal the forward's bit for bit; a second forward
    gives the same output bit for bit."""
    import htree_amd
    from htree_amd.parallel import select_frame

    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    q, k, v = (x.to(DEV) for x in inputs(B, T, H, Hkv, D, dtype, seed))
    out, ctx = htree_amd.htree_forward(q, k, v, CR, MTN, TK, _save_for_backward=True)
    hf = ctx["head_frame"]
    cos_k, sin_k = hf.tables(ctx["cos_cache"], ctx["sin_cache"])
    sel, _ = select_frame(hf.q_heads(hf.pad_qk(q)), hf.kv_k(k), hf.kv_v(v), ctx["dims"], cos_k,
                          sin_k, ctx["scale"])
    torch.cuda.synchronize()
    assert torch.equal(sel, ctx["parents_stacked"])
    out2, ctx2 = htree_amd.htree_forward(q, k, v, CR, MTN, TK, _save_for_backward=True)
    torch.cuda.synchronize()
    assert torch.equal(out2, out) and torch.equal(ctx2["parents_stacked"], ctx["parents_stacked"])


BWD = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype, seed
    (1, 1500, 128, 1, 64, 16, 16, 64, "bfloat16", 91),   # G = 128, every row vs the oracle
    (1, 1200, 100, 1, 32, 8, 16, 64, "float32", 92),     # G = 100: padding heads, CR 8
]


@pytest.mark.parametrize("cfg", BWD, ids=lambda c: f"T{c[1]}G{c[2] // c[3]}D{c[4]}cr{c[5]}{c[8]}")
def test_split_backward_matches_oracle(cfg):
    import htree_amd

    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v, dO = inputs(B, T, H, Hkv, D, dtype, seed, dO=True)
    out, par, gmax, gsum, ctx = htree_amd.htree_forward_parents(
        q.to(DEV), k.to(DEV), v.to(DEV), CR, MTN, TK)
    dq, dk, dv = htree_amd.htree_backward(dO.to(DEV), q.to(DEV), out, ctx)
    torch.cuda.synchronize()
    f = lambda x: x.float().cpu().numpy()
    rep = check_backward(q, k, v, dO, CR, TK, MTN, dtype, f(out), par.cpu().numpy(), f(gmax),
                         f(gsum), f(dq), f(dk), f(dv))
    print(rep, flush=True)


LARGE_BWD = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype, seed
    (1, 20000, 16, 1, 64, 32, 1024, 32, "bfloat16", 93),   # 20000 candidates at the bottom
    (1, 12000, 16, 1, 32, 4, 2048, 8192, "bfloat16", 94),  # lists of 2048 parents
]


@pytest.mark.parametrize("cfg", LARGE_BWD, ids=["pos20000", "tk2048"])
def test_split_backward_large_candidate_sets(cfg):
    """Above 16384 candidates per level (20000 at the last queries' bottom
    level, G = 16, D = 64), and lists of 2048 parents: the recomputing dq
    pass with 65536-position and 2048-entry lists; dq on sampled rows, dk /
    dv at sampled level-0 nodes, the dv mass (every head's probabilities sum
    to 1, the pooling backward keeps sums)."""
    import htree_amd

    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v, dO = inputs(B, T, H, Hkv, D, dtype, seed, dO=True)
    out, par, gmax, gsum, ctx = htree_amd.htree_forward_parents(
        q.to(DEV), k.to(DEV), v.to(DEV), CR, MTN, TK)
    dq, dk, dv = htree_amd.htree_backward(dO.to(DEV), q.to(DEV), out, ctx)
    torch.cuda.synchronize()
    f = lambda x: x.float().cpu().numpy()
    out, gmax, gsum, dq, dk, dv, par = f(out), f(gmax), f(gsum), f(dq), f(dk), f(dv), par.cpu().numpy()
    # the case covers what it names
    if TK > 1024:
        assert (par[0] >= 0).sum(-1).max() > 1024
    else:
        assert (par[0] >= 0).sum(-1).max() * CR > 16384
    assert np.all(np.isfinite(dq)) and np.all(np.isfinite(dk)) and np.all(np.isfinite(dv))
    G = H // Hkv
    want = dO.float().numpy().reshape(B, T, Hkv, G, D).astype(np.float64).sum(axis=(1, 3))
    got = dv.astype(np.float64).sum(axis=1)
    atol = 1e-4 * np.sqrt(T * G) + 4 * 2.0 ** -9 * np.sqrt((dv.astype(np.float64) ** 2).sum(axis=1))
    ratio = np.abs(got - want) / (atol + 1e-4 * np.abs(want))
    print("dv mass check: worst error / bound", float(ratio.max()), flush=True)
    assert ratio.max() <= 1.0
    tree = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, dtype)
    rows = sample_rows(B, T, 30, seed)
    pr = par[:, rows[:, 0], rows[:, 1]]
    fw = orc.forward(q.float().numpy(), tree, D ** -0.5, rows=rows, forced=pr)
    o = out[rows[:, 0], rows[:, 1]]
    d = dO.float().numpy()[rows[:, 0], rows[:, 1]]
    delta = (o.astype(np.float64) * d).sum(-1).astype(np.float32)
    ref = orc.backward_dq_rows(q.float().numpy(), tree, D ** -0.5, rows, pr, fw["gmax"], fw["gsum"],
                               delta, d)
    ok, worst = close(dq[rows[:, 0], rows[:, 1]], ref, dtype)
    print("dq worst", worst, flush=True)
    assert ok
    rep = check_dkv_sampled(q.float().numpy(), dO.float().numpy(), out, k.float().numpy(),
                            v.float().numpy(), par, gmax, gsum, dk, dv, CR, TK, MTN, dtype,
                            [(0, 0)], seed + 1)
    print("dk/dv at sampled nodes", rep, flush=True)
