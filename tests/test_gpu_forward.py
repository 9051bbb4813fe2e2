"""GPU parity of the HIP forward against the CPU oracle (and, through the
golden fixtures, against the reference's own src/naive.py outputs).

Selection: every level's Top-K must equal the oracle's choice from the same
parent list, except swaps inside the tie band (tests/helpers.py).
Outputs: teacher-forced on the device's parent lists, within
2e-2 abs + 1e-2 rel (bf16), 1e-4 (fp32), 2e-3 (fp16).
Tree levels: bit-exact."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import DT, check_forward, close, inputs, skewed_inputs
from tests.helpers import load_golden

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


SMALL = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype, seed
    (1, 2048, 4, 1, 64, 16, 8, 64, "float32", 1),      # the C1 workload shape
    (1, 2048, 4, 1, 64, 16, 8, 64, "bfloat16", 1),
    (2, 1500, 16, 2, 128, 16, 16, 128, "bfloat16", 2),
    (1, 1100, 8, 1, 128, 16, 16, 128, "float16", 3),
    (1, 4100, 16, 1, 128, 16, 4, 64, "bfloat16", 4),   # 3 levels, TK < CR
    (1, 700, 8, 2, 64, 8, 16, 128, "float32", 5),      # CR < 16
    (1, 900, 4, 1, 128, 32, 8, 256, "bfloat16", 6),    # CR > 16
    (1, 3000, 8, 1, 64, 4, 32, 64, "bfloat16", 7),     # CR = 4, 4 levels
    (1, 2000, 16, 4, 32, 16, 16, 128, "float32", 8),   # D = 32 (the reference's default head dim)
    (1, 1500, 16, 4, 32, 16, 8, 128, "float16", 9),
    (2, 1000, 8, 2, 32, 8, 16, 64, "bfloat16", 10),
    (1, 2500, 16, 4, 32, 4, 32, 64, "float32", 11),    # D = 32, 32 tiles: multi-pass kernel
    (1, 3000, 8, 1, 128, 32, 32, 256, "bfloat16", 12),  # CR 32, top_k 32 (the C4 workload's tree): 64 tiles
    (1, 2200, 8, 2, 64, 16, 32, 256, "float16", 13),    # 32 tiles, fp16 (split V)
    (2, 4096, 16, 2, 128, 16, 16, 16, "bfloat16", 14),  # 16-node top level (keeps every candidate), as C5
    (1, 3000, 8, 2, 64, 128, 4, 512, "bfloat16", 15),  # CR 128: 32 tiles per level
    (1, 1500, 8, 1, 32, 128, 2, 256, "float32", 16),    # CR 128: 16 tiles per level
    (1, 1200, 16, 2, 256, 16, 16, 128, "bfloat16", 17),  # D = 256 (register forward)
    (1, 1500, 8, 1, 256, 16, 32, 256, "float32", 18),    # D = 256, 32 tiles (streaming forward)
]


@pytest.mark.parametrize("cfg", SMALL, ids=lambda c: f"T{c[1]}H{c[2]}kv{c[3]}D{c[4]}cr{c[5]}tk{c[6]}{c[8]}")
def test_forward_matches_oracle(cfg):
    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v = inputs(B, T, H, Hkv, D, dtype, seed)
    out, par, gmax, gsum, ctx = run_fwd(q, k, v, CR, TK, MTN)
    tree = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, dtype)
    # tree levels are bit-exact
    for l in range(1, tree.L):
        got_k = ctx["layers_k"][l].float().cpu().numpy()
        got_v = ctx["layers_v"][l].float().cpu().numpy()
        assert np.array_equal(got_k, tree.lk[l]), f"level {l} K differs"
        assert np.array_equal(got_v, tree.lv[l]), f"level {l} V differs"
    rows = orc.all_rows(B, T)
    if len(rows) > 1500:
        rng = np.random.default_rng(seed)
        rows = rows[np.sort(rng.choice(len(rows), 1500, replace=False))]
        rows = np.concatenate([rows, orc.all_rows(B, T)[:64], orc.all_rows(B, T)[-64:]])
    rep = check_forward(q, k, v, CR, TK, MTN, dtype, rows=rows, out_dev=out, parents_dev=par,
                        tree=tree)
    print(rep, flush=True)
    assert np.all(np.isfinite(out))
    assert np.all(gsum >= 1.0 - 1e-6)  # the max term contributes exp(0) = 1


@pytest.mark.parametrize("name", ["cr16_tk4_bf16", "cr8_tk16_fp32_g8", "cr16_tk4_fp16_b2"])
def test_forward_matches_reference_golden(name):
    """Device forward vs the reference's own outputs (fixtures written from
    src/naive.py).  Selection must match the reference's per-level parents
    up to the tie band; outputs within the dtype bar where selection matched."""
    g = load_golden(name)
    print(f"golden {name}", flush=True)
    out, par, _, _, _ = run_fwd(g["q"], g["k"], g["v"], g["CR"], g["TK"], g["MTN"])
    B, T, Hkv, TK, L = g["B"], g["T"], g["Hkv"], g["TK"], g["L"]
    ok_rows = np.ones((B, T, Hkv), bool)
    for l in range(L - 1, 0, -1):
        ref = g[f"parents_l{l}"].reshape(B, T, Hkv, TK)
        ok_rows &= np.all(par[l - 1] == ref, axis=-1)
    frac = ok_rows.mean()
    assert frac > 0.995, f"only {frac:.4f} of the query groups select like the reference"
    G = g["H"] // Hkv
    m = np.repeat(ok_rows, G, axis=2)  # [B,T,H]
    ok, worst = close(out[m], g["out"][m], g["dtype"])
    assert ok, f"worst {worst:.3f} of the bar"


def test_forward_c2_sample():
    """The C2 workload (T=32768, Hq=32, Hkv=2, D=128, bf16, CR16 MTN128
    TK16): sampled rows against the oracle; every row through invariants."""
    B, T, H, Hkv, D, CR, TK, MTN = 1, 32768, 32, 2, 128, 16, 16, 128
    q, k, v = inputs(B, T, H, Hkv, D, "bfloat16", 2024)
    out, par, gmax, gsum, ctx = run_fwd(q, k, v, CR, TK, MTN)
    assert np.all(np.isfinite(out))
    L = par.shape[0]
    assert L == 3
    # selected lists: ascending, -1 padded, closed-form counts, rightmost kept
    t = np.arange(T)
    for l in range(L - 1, 0, -1):
        sel = par[l - 1]
        cnt = (sel >= 0).sum(-1)
        want = np.array([orc.candidate_counts(int(x), CR, TK, L)[l][1] for x in t])
        assert np.array_equal(cnt, np.broadcast_to(want[None, :, None], cnt.shape))
        right = (t // CR ** (l)).astype(np.int32)
        assert np.all(np.any(sel == right[None, :, None, None], axis=-1))
        nxt_valid = sel[..., 1:] >= 0
        assert np.all((np.diff(sel, axis=-1) > 0) | ~nxt_valid)
        assert np.all(sel[..., 1:][~(sel[..., :-1] >= 0)] < 0)  # -1 padding is a suffix
    rng = np.random.default_rng(0)
    rows = np.stack([np.zeros(300, int), np.sort(rng.choice(T, 300, replace=False))], 1)
    rep = check_forward(q, k, v, CR, TK, MTN, "bfloat16", rows=rows, out_dev=out, parents_dev=par)
    print(rep, flush=True)


def test_forward_skewed_sample():
    """Skewed keys (the C5 distribution, reduced T): many exact-zero
    importances, ties broken by position."""
    B, T, H, Hkv, D, CR, TK, MTN = 1, 8192, 32, 2, 128, 16, 16, 128
    q, k, v, _ = skewed_inputs(B, T, H, Hkv, D, "bfloat16", 77)
    out, par, gmax, gsum, ctx = run_fwd(q, k, v, CR, TK, MTN)
    assert np.all(np.isfinite(out))
    rng = np.random.default_rng(1)
    rows = np.stack([np.zeros(400, int), np.sort(rng.choice(T, 400, replace=False))], 1)
    rep = check_forward(q, k, v, CR, TK, MTN, "bfloat16", rows=rows, out_dev=out, parents_dev=par)
    print(rep, flush=True)


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_forward_clustered_importances(dtype):
    """Keys of small spread (0.05 N(0,1)): every candidate's importance lies
    within a few percent of the others', so many keys share the top 16 bits
    of the selection threshold and the radix select's low 15 bits decide.
    Selections against the oracle (tie band and exact ties as everywhere)."""
    B, T, H, Hkv, D, CR, TK, MTN = 1, 6000, 32, 2, 128, 16, 16, 128
    q, k, v = inputs(B, T, H, Hkv, D, dtype, 78)
    k = (k.float() * 0.05).to(k.dtype)
    out, par, gmax, gsum, ctx = run_fwd(q, k, v, CR, TK, MTN)
    assert np.all(np.isfinite(out))
    rng = np.random.default_rng(2)
    rows = np.stack([np.zeros(300, int), np.sort(rng.choice(T, 300, replace=False))], 1)
    rep = check_forward(q, k, v, CR, TK, MTN, dtype, rows=rows, out_dev=out, parents_dev=par,
                        gmax_dev=gmax, gsum_dev=gsum)
    print(rep, flush=True)


def test_forward_deterministic():
    q, k, v = inputs(1, 3000, 16, 2, 128, "bfloat16", 9)
    a = run_fwd(q, k, v, 16, 16, 128)
    b = run_fwd(q, k, v, 16, 16, 128)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


WIDE = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype, seed, skewed: top_k > 64 or more than
    # 64 candidate tiles per level (one block of four waves per query group)
    (1, 3000, 16, 4, 32, 16, 128, 2048, "float32", 21, False),
    (1, 12000, 16, 4, 32, 16, 512, 8192, "float16", 22, False),  # correctness_test.py defaults
    (1, 5000, 8, 2, 64, 4, 256, 1024, "bfloat16", 23, False),     # CR < 16: one tile per parent
    (1, 6000, 8, 1, 128, 32, 128, 4096, "bfloat16", 24, False),   # CR > 16
    (1, 8192, 16, 2, 64, 16, 256, 4096, "bfloat16", 25, True),    # many exact-zero importances
    # 16384 candidates per level (64 keys per thread in the selection)
    (1, 20000, 8, 2, 32, 16, 1024, 16384, "float32", 26, False),  # top_k 1024
    (1, 20000, 8, 2, 64, 32, 512, 512, "bfloat16", 27, False),    # top_k 512 at CR 32, 3 levels
    (1, 20000, 8, 2, 32, 128, 128, 16384, "float16", 28, False),  # CR 128
    (1, 3000, 8, 2, 256, 16, 128, 2048, "bfloat16", 29, False),   # D = 256
    # groups of 17..32 heads: KV-head pairs, one block of two 2-wave halves
    (1, 12000, 64, 2, 32, 16, 512, 8192, "float32", 30, False),  # speed_test defaults, G = 32
    (1, 20000, 48, 2, 32, 16, 1024, 16384, "bfloat16", 31, False),  # G = 24, 64 keys per thread
    (1, 6000, 32, 1, 128, 32, 128, 4096, "bfloat16", 32, True),  # G = 32, D = 128, CR 32
    # groups of 33..64 heads: KV-head quads, one block of four one-wave parts
    (1, 12000, 64, 1, 32, 16, 512, 8192, "float32", 33, False),  # speed_test's 64 heads over 1 KV head
    (1, 8192, 96, 2, 64, 8, 256, 1024, "bfloat16", 34, True),   # G = 48, CR 8, 3 levels
    (1, 12000, 57, 1, 32, 16, 512, 8192, "bfloat16", 35, False),  # G = 57: quads of 15, 3 padding heads
]


@pytest.mark.parametrize("cfg", WIDE, ids=lambda c: f"T{c[1]}D{c[4]}cr{c[5]}tk{c[6]}{c[8]}{'skew' if c[10] else ''}")
def test_forward_wide_matches_oracle(cfg):
    """The reference's default regime and beyond (top_k up to 1024, up to
    16384 candidates per level): sampled rows against the oracle,
    teacher-forced on the device's lists; every row through the list
    invariants."""
    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed, skewed = cfg
    print(f"case {cfg}", flush=True)
    if skewed:
        q, k, v, _ = skewed_inputs(B, T, H, Hkv, D, dtype, seed)
    else:
        q, k, v = inputs(B, T, H, Hkv, D, dtype, seed)
    out, par, gmax, gsum, ctx = run_fwd(q, k, v, CR, TK, MTN)
    assert np.all(np.isfinite(out))
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
    rng = np.random.default_rng(seed)
    n = 160
    rows = np.stack([rng.integers(0, B, n), np.sort(rng.choice(T, n, replace=False))], 1)
    rows = np.concatenate([rows, [[0, 0], [0, T - 1]]]).astype(np.int32)
    rep = check_forward(q, k, v, CR, TK, MTN, dtype, rows=rows, out_dev=out, parents_dev=par)
    print(rep, flush=True)
