"""Parity at the full C2, C4 and C5 workload sizes (the forward's streaming and
register kernels, the shared-staging dkv, the stored-dS dq at tens of GB and
the skewed tree with its 16-node top level): sampled query rows against the
oracle, teacher-forced on the device's parent lists, plus size-independent
properties over every row: the parent lists' closed-form lengths, ascending
order and forced rightmost child, and the mass of dV (pooling conserves it and
every P row sums to 1, so the sum of dV over all nodes equals the sum of dO
over the group's queries and heads); and final dK / dV at sampled level-0
nodes of two (b, h_kv) pairs (every query that accumulates them or their
ancestors), against the oracle's per-level terms and the pooling factors.

Inputs are drawn on the device (seeded) so that a test fits its time limit;
the oracle gets K and V whole and Q/dO only at the sampled rows (it reads no
other row)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import DT, check_dkv_sampled, check_forward, close

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def device_inputs(B, T, H, Hkv, D, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, device=DEV).to(DT[dtype])
    return r(B, T, H, D), r(B, T, Hkv, D), r(B, T, Hkv, D), r(B, T, H, D)


def device_skewed_inputs(B, T, H, Hkv, D, dtype, seed, ncomp=64, nhot=4):
    """Keys from a 64-component Gaussian mixture (means N(0,4), sigma 0.5),
    queries around 4 hot components, V and dO iid N(0,1)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    mu = 2.0 * torch.randn(ncomp, D, generator=g, device=DEV)
    hot = torch.randperm(ncomp, generator=g, device=DEV)[:nhot]
    ck = torch.randint(0, ncomp, (B, T, Hkv), generator=g, device=DEV)
    k = mu[ck] + 0.5 * torch.randn(B, T, Hkv, D, generator=g, device=DEV)
    cq = hot[torch.randint(0, nhot, (B, T, H), generator=g, device=DEV)]
    q = mu[cq] + 0.5 * torch.randn(B, T, H, D, generator=g, device=DEV)
    v = torch.randn(B, T, Hkv, D, generator=g, device=DEV)
    dO = torch.randn(B, T, H, D, generator=g, device=DEV)
    return tuple(x.to(DT[dtype]) for x in (q, k, v, dO))


def lists_invariants(par, T, CR, TK):
    L = par.shape[0]
    t = np.arange(T)
    for l in range(L - 1, 0, -1):
        sel = par[l - 1]
        cnt = (sel >= 0).sum(-1)
        want = np.array([orc.candidate_counts(int(x), CR, TK, L)[l][1] for x in t])
        assert np.array_equal(cnt, np.broadcast_to(want[None, :, None], cnt.shape)), l
        right = (t // CR ** l).astype(np.int32)
        assert np.all(np.any(sel == right[None, :, None, None], axis=-1)), l
        valid = sel[..., 1:] >= 0
        assert np.all((np.diff(sel, axis=-1) > 0) | ~valid), l


def sparse_rows(x_dev, rows):
    """[B,T,H,D] float32 host array holding x only at `rows` (zero pages
    elsewhere, which the allocator maps lazily)."""
    B, T, H, D = x_dev.shape
    out = np.zeros((B, T, H, D), np.float32)
    idx = torch.from_numpy(rows.astype(np.int64)).to(DEV)
    out[rows[:, 0], rows[:, 1]] = x_dev[idx[:, 0], idx[:, 1]].float().cpu().numpy()
    return out


def run_case(q, k, v, dO, CR, TK, MTN, nrows, seed, autograd=False):
    """autograd: the gradients of the drop-in's training step (the default
    autograd mode, input-dtype gradients), the forward state from a second,
    identical forward (the forward is deterministic, checked on its output);
    else htree_forward + htree_backward (fp32 gradients)."""
    import htree_amd

    B, T, H, D = q.shape
    Hkv = k.shape[2]
    out, par, gmax, gsum, ctx = htree_amd.htree_forward_parents(q, k, v, CR, MTN, TK)
    if autograd:
        qg, kg, vg = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
        o2 = htree_amd.htree_forward_triton_autograd(qg, kg, vg, CR, MTN, TK)
        o2.backward(dO)
        assert torch.equal(o2.detach(), out)
        dq, dk, dv = qg.grad, kg.grad, vg.grad
        assert dq.dtype == q.dtype and dk.dtype == k.dtype
        del qg, kg, vg, o2
    else:
        dq, dk, dv = htree_amd.htree_backward(dO, q, out, ctx)
    torch.cuda.synchronize()
    print("device forward + backward done", flush=True)
    for x in (out, dq, dk, dv):
        assert bool(torch.isfinite(x).all())
    want = dO.reshape(B, T, Hkv, H // Hkv, D).to(torch.float64).sum(dim=(1, 3)).cpu().numpy()
    got = dv.to(torch.float64).sum(dim=1).cpu().numpy()
    atol = 1e-3 * np.sqrt(T * H / Hkv)
    if dv.dtype != torch.float32:
        # each node's dv rounded once to its dtype (relative 2^-9 for bf16)
        atol = atol + 4 * 2.0 ** -9 * np.sqrt((dv.to(torch.float64) ** 2).sum(dim=1).cpu().numpy())
    ratio = np.abs(got - want) / (atol + 1e-3 * np.abs(want))
    print("dv mass check: worst error / bound", float(ratio.max()), flush=True)
    assert ratio.max() <= 1.0
    del ctx
    torch.cuda.empty_cache()
    par = par.cpu().numpy()
    lists_invariants(par, T, CR, TK)
    print("parent-list invariants hold", flush=True)
    rep = check_dkv_sampled(q, dO, out, k, v, par, gmax, gsum, dk, dv, CR, TK, MTN, "bfloat16",
                            [(0, 0), (B - 1, Hkv - 1)], seed)
    print("dk/dv at sampled level-0 nodes:", rep, flush=True)
    del dk, dv
    torch.cuda.empty_cache()
    rng = np.random.default_rng(seed)
    rows = np.stack([rng.integers(0, B, nrows), np.sort(rng.choice(T, nrows, replace=False))],
                    1).astype(np.int32)
    rows = np.concatenate([rows, [[0, 0], [B - 1, T - 1]]]).astype(np.int32)
    qn = sparse_rows(q, rows)
    dOn = sparse_rows(dO, rows)
    idx = torch.from_numpy(rows.astype(np.int64)).to(DEV)
    out_r = out[idx[:, 0], idx[:, 1]].float().cpu().numpy()
    dq_r = dq[idx[:, 0], idx[:, 1]].float().cpu().numpy()
    tree = orc.Tree(k.float().cpu().numpy(), v.float().cpu().numpy(), CR, MTN, TK, "bfloat16")
    print("oracle tree built", flush=True)
    # check_forward indexes the device outputs at `rows`: hand it arrays that
    # hold those rows in place
    out_s = np.zeros((B, T, H, D), np.float32)
    out_s[rows[:, 0], rows[:, 1]] = out_r
    gm_s = np.zeros((B, T, H), np.float32)
    gs_s = np.ones((B, T, H), np.float32)
    gm_s[rows[:, 0], rows[:, 1]] = gmax[idx[:, 0], idx[:, 1]].cpu().numpy()
    gs_s[rows[:, 0], rows[:, 1]] = gsum[idx[:, 0], idx[:, 1]].cpu().numpy()
    rep = check_forward(torch.from_numpy(qn), k[:, :1, :, :1], None, CR, TK, MTN, "bfloat16",
                        rows=rows, out_dev=out_s, parents_dev=par, tree=tree, gmax_dev=gm_s,
                        gsum_dev=gs_s)
    pr = par[:, rows[:, 0], rows[:, 1]]
    fw = orc.forward(qn, tree, D ** -0.5, rows=rows, forced=pr)
    d = dOn[rows[:, 0], rows[:, 1]]
    delta = (out_r.astype(np.float64) * d).sum(-1).astype(np.float32)
    ref = orc.backward_dq_rows(qn, tree, D ** -0.5, rows, pr, fw["gmax"], fw["gsum"], delta, d)
    ok, worst = close(dq_r, ref, "bfloat16")
    print(rep, "dq worst", worst, flush=True)
    assert ok, worst


def test_c2_full_size_training_step():
    """C2: B=1, T=32768, Hq=32, Hkv=2, D=128, bf16, CR=16, MTN=128, TK=16,
    the headline workload, through the default autograd mode (the bench's
    training step): sampled rows (selection, output, state, dq) and final
    dk / dv at sampled level-0 nodes of both KV heads."""
    B, T, H, Hkv, D, CR, TK, MTN = 1, 32768, 32, 2, 128, 16, 16, 128
    print("case C2 seed 202 (autograd)", flush=True)
    q, k, v, dO = device_inputs(B, T, H, Hkv, D, "bfloat16", 202)
    run_case(q, k, v, dO, CR, TK, MTN, 200, 2, autograd=True)


def test_c4_full_size():
    """C4: B=1, T=131072, Hq=64, Hkv=8, D=128, bf16, CR=32, MTN=256, TK=32."""
    B, T, H, Hkv, D, CR, TK, MTN = 1, 131072, 64, 8, 128, 32, 32, 256
    print("case C4 seed 404", flush=True)
    q, k, v, dO = device_inputs(B, T, H, Hkv, D, "bfloat16", 404)
    run_case(q, k, v, dO, CR, TK, MTN, 192, 4)


def test_c5_full_size():
    """C5: B=2, T=65536, Hq=32, Hkv=2, D=128, bf16, CR=16, MTN=128, TK=16,
    skewed keys and queries (16-node top level, exact-zero importances)."""
    B, T, H, Hkv, D, CR, TK, MTN = 2, 65536, 32, 2, 128, 16, 16, 128
    print("case C5 seed 505", flush=True)
    q, k, v, dO = device_skewed_inputs(B, T, H, Hkv, D, "bfloat16", 505)
    run_case(q, k, v, dO, CR, TK, MTN, 256, 5)
