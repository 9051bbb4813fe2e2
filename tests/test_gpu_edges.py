"""Edge shapes through the forward and the backward, against the oracle:
a single query (T = 1), a single level (T <= max_top_nodes: full causal
attention), one query head per KV head (G = 1), several batches, lengths
that are not multiples of 16 or of the compression rate, and the
block-per-group kernels (top_k > 64) on one and on two levels."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.gpu_util import DT, check_backward, check_forward, inputs

pytestmark = pytest.mark.gpu

DEV = "cuda:0"

EDGES = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype, seed
    (1, 1, 4, 1, 64, 16, 8, 128, "float32", 51),        # one query
    (2, 100, 4, 1, 64, 16, 8, 128, "bfloat16", 52),     # one level: full causal attention
    (3, 700, 4, 4, 64, 16, 8, 64, "float32", 53),       # G = 1, three batches
    (1, 1037, 8, 2, 128, 8, 16, 64, "float16", 54),     # T not a multiple of 16 or CR
    (1, 513, 8, 2, 32, 16, 512, 8192, "float32", 55),   # top_k 512 on one level
    (2, 2100, 4, 2, 32, 16, 128, 2048, "float16", 56),  # top_k 128, two batches, two levels
]


@pytest.mark.parametrize("cfg", EDGES, ids=lambda c: f"B{c[0]}T{c[1]}H{c[2]}kv{c[3]}D{c[4]}cr{c[5]}tk{c[6]}{c[8]}")
def test_edges_forward_backward(cfg):
    import htree_amd

    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    print(f"case {cfg}", flush=True)
    q, k, v, dO = inputs(B, T, H, Hkv, D, dtype, seed, dO=True)
    out, par, gmax, gsum, ctx = htree_amd.htree_forward_parents(
        q.to(DEV), k.to(DEV), v.to(DEV), compression_rate=CR, max_top_nodes=MTN, top_k_per_layer=TK)
    dq, dk, dv = htree_amd.htree_backward(dO.to(DEV), q.to(DEV), out, ctx)
    torch.cuda.synchronize()
    f = lambda x: x.float().cpu().numpy()
    tree = orc.Tree(k.float().numpy(), v.float().numpy(), CR, MTN, TK, dtype)
    if tree.L == 1:
        assert par.shape[0] == 1
    rep = check_forward(q, k, v, CR, TK, MTN, dtype, out_dev=f(out), parents_dev=par.cpu().numpy(),
                        tree=tree)
    rep.update(check_backward(q, k, v, dO, CR, TK, MTN, dtype, f(out), par.cpu().numpy(), f(gmax),
                              f(gsum), f(dq), f(dk), f(dv), tree=tree))
    print(rep, flush=True)
    assert dq.dtype == torch.float32 and dq.shape == q.shape and dk.shape == k.shape


@pytest.mark.parametrize("B,T", [(0, 300), (2, 0)])
def test_empty_inputs(B, T):
    """No batch or no tokens: empty outputs and gradients of the right
    shapes and dtypes, with no launch; the library's limits still apply."""
    import htree_amd

    q = torch.randn(B, T, 8, 64, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    k = torch.randn(B, T, 2, 64, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    v = torch.randn(B, T, 2, 64, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    out, ctx = htree_amd.htree_forward(q.detach(), k.detach(), v.detach(), 16, 128, 16,
                                       _save_for_backward=True)
    assert out.shape == q.shape and out.dtype == q.dtype
    dq, dk, dv = htree_amd.htree_backward(torch.zeros_like(out), q.detach(), out, ctx)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    assert dq.dtype == dk.dtype == dv.dtype == torch.float32
    o = htree_amd.htree_forward_triton_autograd(q, k, v, 16, 128, 16)
    o.sum().backward()
    assert q.grad.shape == q.shape and k.grad.dtype == k.dtype
    wide = lambda x: torch.zeros(*x.shape[:-1], 512, device=DEV, dtype=x.dtype)  # head dim 512
    with pytest.raises(AssertionError, match="configuration outside"):
        htree_amd.htree_forward(wide(q), wide(k), wide(v), 16, 128, 16)
