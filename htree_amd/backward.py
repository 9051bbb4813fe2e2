"""htree backward on MI355X: drop-in for `htree_backward`,
`HTreeTritonFunction` and `htree_forward_triton_autograd` of
/root/reference/src/backward.py:941-1208.

`htree_backward(dO, q, output, bwd_ctx) -> (dq, dk, dv)` in fp32, reading
the reference's bwd_ctx keys.  The selection is taken from
`per_layer_parents` (saved by the forward); when the context holds none
(the reference's autograd path saves none, src/backward.py:1138) the
forward's selection is replayed once to recover them.  The autograd
Function saves the parent lists (B*T*H_kv*TK int32 per level) instead of
recomputing them.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native as N
from .parallel import build_tree, htree_forward, make_dims
from .workmodel import level_sizes


def _stack_parents(per_layer_parents, L):
    return torch.stack([per_layer_parents[l] for l in range(L)]).contiguous()


def _check_parents(parents, B, T, H_kv, TK, CR, MTN, device):
    """Caller-supplied lists go to the kernels as they are: hold them to what
    the forward produces (src/naive.py:88-118, :204-207): list l names nodes
    of level l + 1 (the virtual top parents at the top level), ascending,
    padded with -1 at the end."""
    sizes = level_sizes(T, CR, MTN)
    L = len(sizes)
    assert parents.shape == (L, B, T, H_kv, TK) and parents.dtype == torch.int32, \
        f"parent lists must be int32 [{L}, {B}, {T}, {H_kv}, {TK}], got {parents.dtype} {list(parents.shape)}"
    assert parents.device == device, "parent lists must be on the inputs' device"
    for l in range(L):
        p = parents[l]
        lim = -(-sizes[l] // CR)
        assert bool(((p >= -1) & (p < lim)).all()), f"level {l}: parent index outside [-1, {lim})"
        valid = p >= 0
        assert bool((valid[..., 1:] <= valid[..., :-1]).all()), f"level {l}: -1 padding must come last"
        assert bool(((p[..., 1:] > p[..., :-1]) | ~valid[..., 1:]).all()), \
            f"level {l}: parent lists must be ascending"


def htree_backward(dO: torch.Tensor, q: torch.Tensor, output: torch.Tensor, bwd_ctx: dict):
    """Gradients of the htree forward wrt q, k, v (fp32), selection fixed.

    dO and output are read in q's dtype; the reference upcasts both to fp32
    (src/backward.py:966-967), so the two agree when dO comes in q's dtype,
    as autograd hands it."""
    B, T, H, K = q.shape
    layers_k, layers_v = bwd_ctx["layers_k"], bwd_ctx["layers_v"]
    k, v = layers_k[0], layers_v[0]
    if B == 0 or T == 0:  # empty inputs: empty gradients, no launch
        f32 = dict(dtype=torch.float32, device=q.device)
        return (torch.empty(B, T, H, K, **f32), torch.empty(B, T, k.shape[2], K, **f32),
                torch.empty(B, T, k.shape[2], K, **f32))
    CR = bwd_ctx["compression_rate"]
    TK = bwd_ctx["top_k_per_layer"]
    MTN = bwd_ctx.get("max_top_nodes", TK * CR)
    scale = bwd_ctx["scale"]
    L = bwd_ctx["num_layers"]
    d = bwd_ctx.get("dims")
    if d is None:
        d, _ = make_dims(q, k, CR, MTN, TK)
    ws = bwd_ctx.get("packed_tree")
    cos, sin = bwd_ctx["cos_cache"], bwd_ctx["sin_cache"]
    if ws is None:
        rope_base = bwd_ctx.get("rope_base", 10000.0)
        _, _, ws, cos, sin = build_tree(k, v, d, d.rope_rows, rope_base)
    parents = bwd_ctx.get("parents_stacked")
    plp = bwd_ctx.get("per_layer_parents")
    # per_layer_parents (what the reference reads) are views of the forward's
    # stacked lists; a caller that replaced them gets its own lists
    if parents is not None and plp is not None and any(
            plp[l].data_ptr() != parents[l].data_ptr() for l in range(L)):
        parents = None
    # the training forward's stored scores go with its own parent lists
    scores = bwd_ctx.get("train_scores") if parents is not None else None
    if parents is None:
        if plp is not None:
            parents = _stack_parents(plp, L)
            _check_parents(parents, B, T, k.shape[2], TK, CR, MTN, q.device)
        else:
            _, ctx2 = htree_forward(q, k, v, CR, MTN, TK, scale, bwd_ctx.get("rope_base", 10000.0),
                                    _save_for_backward=True, _save_parents=True)
            parents = ctx2["parents_stacked"]
    q = q.contiguous()
    dO = dO.contiguous().to(q.dtype)
    output = output.contiguous().to(q.dtype)
    dev = q.device
    dq = torch.empty(B, T, H, K, dtype=torch.float32, device=dev)
    dk = torch.empty(B, T, k.shape[2], K, dtype=torch.float32, device=dev)
    dv = torch.empty_like(dk)
    nb = N.ctypes.c_int64()
    N.check(N.lib().htree_backward_workspace_bytes(N.ctypes.byref(d), N.ctypes.byref(nb)),
            "htree_backward_workspace_bytes")
    try:
        bws = torch.empty(nb.value, dtype=torch.uint8, device=dev)
    except torch.OutOfMemoryError:
        # no room for the stored dS: the smallest workspace, dq recomputes
        N.check(N.lib().htree_backward_workspace_min_bytes(N.ctypes.byref(d), N.ctypes.byref(nb)),
                "htree_backward_workspace_min_bytes")
        bws = torch.empty(nb.value, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        if scores is not None:
            rc = N.lib().htree_backward_train(
                d, float(scale), N.ptr(q), N.ptr(output), N.ptr(dO), N.ptr(bwd_ctx["global_max"]),
                N.ptr(bwd_ctx["global_sum"]), N.ptr(parents), N.ptr(ws), ws.numel(), N.ptr(cos),
                N.ptr(sin), N.ptr(scores), scores.numel(), N.ptr(dq), N.ptr(dk), N.ptr(dv),
                N.ptr(bws), bws.numel(), N.stream_ptr(dev))
            N.check(rc, "htree_backward_train")
        else:
            rc = N.lib().htree_backward(
                d, float(scale), N.ptr(q), N.ptr(output), N.ptr(dO), N.ptr(bwd_ctx["global_max"]),
                N.ptr(bwd_ctx["global_sum"]), N.ptr(parents), N.ptr(ws), ws.numel(), N.ptr(cos),
                N.ptr(sin), N.ptr(dq), N.ptr(dk), N.ptr(dv), N.ptr(bws), bws.numel(),
                N.stream_ptr(dev))
            N.check(rc, "htree_backward")
    return dq, dk, dv


class HTreeTritonFunction(torch.autograd.Function):
    """Autograd contract of the reference (src/backward.py:1126-1193): grads
    in the input dtypes and None for the five non-tensor arguments."""

    @staticmethod
    def forward(ctx, q, k, v, compression_rate, max_top_nodes, top_k_per_layer, scale, rope_base):
        out, bwd_ctx = htree_forward(q, k, v, compression_rate=compression_rate,
                                     max_top_nodes=max_top_nodes, top_k_per_layer=top_k_per_layer,
                                     scale=scale, rope_base=rope_base, _save_for_backward=True,
                                     _save_parents=True)
        ctx.save_for_backward(q, k, v, out, bwd_ctx["global_max"], bwd_ctx["global_sum"],
                              bwd_ctx["cos_cache"], bwd_ctx["sin_cache"],
                              bwd_ctx["parents_stacked"], bwd_ctx["packed_tree"],
                              bwd_ctx["train_scores"])
        ctx.meta = dict(num_layers=bwd_ctx["num_layers"], compression_rate=compression_rate,
                        top_k_per_layer=top_k_per_layer, max_top_nodes=max_top_nodes,
                        scale=bwd_ctx["scale"], dims=bwd_ctx["dims"], rope_base=rope_base)
        return out

    @staticmethod
    def backward(ctx, dO):
        q, k, v, out, gmax, gsum, cos, sin, parents, ws, scores = ctx.saved_tensors
        bwd_ctx = dict(ctx.meta, global_max=gmax, global_sum=gsum, layers_k=[k], layers_v=[v],
                       cos_cache=cos, sin_cache=sin, parents_stacked=parents, packed_tree=ws,
                       train_scores=scores)
        dq, dk, dv = htree_backward(dO, q, out, bwd_ctx)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None, None, None, None


HTreeFunction = HTreeTritonFunction


def htree_forward_triton_autograd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                  compression_rate: int = 16, max_top_nodes: int = 8192,
                                  top_k_per_layer: int = 512, scale: Optional[float] = None,
                                  rope_base: float = 10000.0) -> torch.Tensor:
    """Differentiable htree forward (name of src/backward.py:1196 kept for
    drop-in use; the kernels are the HIP ones)."""
    if scale is None:
        scale = q.shape[-1] ** -0.5
    return HTreeTritonFunction.apply(q.contiguous(), k.contiguous(), v.contiguous(),
                                     compression_rate, max_top_nodes, top_k_per_layer, scale,
                                     rope_base)


htree_forward_autograd = htree_forward_triton_autograd
