"""htree backward on MI355X: drop-in for `htree_backward`,
`HTreeTritonFunction` and `htree_forward_triton_autograd` of
/root/reference/src/backward.py:941-1208.

`htree_backward(dO, q, output, bwd_ctx) -> (dq, dk, dv)` in fp32, reading
the reference's bwd_ctx keys.  The selection is taken from
`per_layer_parents` when the context holds them; otherwise (the reference's
own autograd path saves none, src/backward.py:1138) the forward's selection
is replayed once by the selection-only launch (`htree_select`), with the
context's own RoPE tables (`cos_cache`, `sin_cache`), as the reference's
`_recompute_parents` does (src/backward.py:881-934,1163-1171).  A context without `packed_tree` gets
its operand tree rebuilt from `layers_k[0]` / `layers_v[0]` with those same
tables (src/backward.py:848-878).

Three autograd modes (htree_forward_triton_autograd):
  * default: the Function saves the reference's eight tensors (q, k, v, out,
    global max / sum, cos / sin, src/backward.py:1141-1145) plus the parent
    lists and the packed operand tree (C2: 13 MB + 54 MB), so the backward
    replays no selection and rebuilds only the candidate scores;
  * `_save_scores=True`: also the candidate scores (bf16 configurations with
    <= 16 candidate tiles per level; C2: 1.6 GB), so the backward reads them
    instead of rebuilding them;
  * `_save_parents=False`: the reference's eight tensors only; the backward
    rebuilds the tree, replays the selection alone and rebuilds the scores.

Workspace: the backward keeps every entry's dS for the dq pass when the
stored-dS workspace fits what the device can spare (free memory plus what
torch's caching allocator holds unused, less a margin); otherwise it runs in
the smallest workspace and dq recomputes the scores.  The plan taken is
written into the context under `backward_plan`.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native as N
from .parallel import (HeadFrame, build_tree, check_tables, htree_forward, make_dims,
                       select_frame)
from .workmodel import level_sizes


def _stack_parents(per_layer_parents, L):
    return torch.stack([per_layer_parents[l] for l in range(L)]).contiguous()


def _check_parents(parents, B, T, H_kv, TK, CR, MTN, device):
    """Caller-supplied lists go to the kernels as they are: hold them to what
    the forward produces (src/naive.py:88-118, :204-207): list l names nodes
    of level l + 1 (the virtual top parents at the top level), ascending,
    padded with -1 at the end.  The list of the highest level that
    accumulates is fixed by the algorithm, whatever the data: the virtual
    parents 0 .. (t / CR^l) / CR (src/naive.py:108-118), which is also every
    top node up to t's when a top level of <= top_k nodes keeps them all."""
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
    ltop = L - 2 if L > 1 and sizes[-1] <= TK else L - 1
    t = torch.arange(T, device=device)
    nvp = (t // CR ** ltop) // CR + 1
    slot = torch.arange(TK, device=device)
    fixed = torch.where(slot[None, :] < nvp[:, None], slot[None, :], -1).to(torch.int32)
    assert bool((parents[ltop] == fixed[None, :, None, :]).all()), \
        f"level {ltop}: the top list must be the virtual parents 0 .. (t / CR^{ltop}) / CR"


def infer_max_top_nodes(T: int, CR: int, TK: int, L: int) -> int:
    """A max_top_nodes that gives the context's level count L (for a context
    without the key): the smallest power of two >= the top level's size is
    below the level under it, so the level rule stops at the same level."""
    n = T
    for _ in range(L - 1):
        n = -(-n // CR)
    if L == 1:
        return TK * CR
    return 1 << max(0, (n - 1).bit_length())


# memory left free on the device after the backward's workspace: the larger
# of 2 GiB and 5% of the device
WORKSPACE_MARGIN_FRACTION = 0.05
WORKSPACE_MARGIN_MIN = 2 << 30


def spare_device_bytes(device) -> int:
    """Bytes a workspace can take on `device`: free device memory plus what
    torch's caching allocator holds without using, less the margin."""
    free, total = torch.cuda.mem_get_info(device)
    idle = torch.cuda.memory_reserved(device) - torch.cuda.memory_allocated(device)
    margin = max(WORKSPACE_MARGIN_MIN, int(WORKSPACE_MARGIN_FRACTION * total))
    return max(0, free + idle - margin)


def backward_workspace(d, device, limit: Optional[int] = None):
    """Allocates the backward's workspace: the stored-dS plan where it fits
    `limit` bytes (default: what the device can spare), else the smallest
    plan (dq recomputes the scores).  Returns (workspace, plan name)."""
    nb = N.ctypes.c_int64()
    N.check(N.lib().htree_backward_workspace_bytes(N.ctypes.byref(d), N.ctypes.byref(nb)),
            "htree_backward_workspace_bytes")
    full = nb.value
    N.check(N.lib().htree_backward_workspace_min_bytes(N.ctypes.byref(d), N.ctypes.byref(nb)),
            "htree_backward_workspace_min_bytes")
    small = nb.value
    if limit is None:
        limit = spare_device_bytes(device)
    if full > small and full <= limit:
        try:
            return torch.empty(full, dtype=torch.uint8, device=device), "stored_ds"
        except torch.OutOfMemoryError:
            pass
    # (full == small: the configuration has no stored-dS plan: top_k > 64,
    # CR 128, or dS beyond the library's own cap of a third of the device)
    return torch.empty(small, dtype=torch.uint8, device=device), "recompute"


def htree_backward(dO: torch.Tensor, q: torch.Tensor, output: torch.Tensor, bwd_ctx: dict,
                   _grad_dtype: Optional[torch.dtype] = None,
                   _workspace_limit: Optional[int] = None):
    """Gradients of the htree forward wrt q, k, v (fp32 unless `_grad_dtype`),
    selection fixed.

    dO and output are read in q's dtype; the reference upcasts both to fp32
    (src/backward.py:966-967), so the two agree when dO comes in q's dtype,
    as autograd hands it.  `_grad_dtype` (the autograd path's input dtype)
    has the kernels round the fp32 gradients into that dtype as they store
    them: the values `.to(_grad_dtype)` of the fp32 results would give.
    `_workspace_limit` caps the workspace in bytes (default: what the device
    can spare)."""
    B, T, H, K = q.shape
    layers_k, layers_v = bwd_ctx["layers_k"], bwd_ctx["layers_v"]
    k, v = layers_k[0], layers_v[0]
    H_kv, V = k.shape[2], v.shape[3]
    dev = q.device
    gdt = _grad_dtype or torch.float32
    if B == 0 or T == 0:  # empty inputs: empty gradients, no launch
        e = dict(dtype=gdt, device=dev)
        return (torch.empty(B, T, H, K, **e), torch.empty(B, T, H_kv, K, **e),
                torch.empty(B, T, H_kv, V, **e))
    hf = bwd_ctx.get("head_frame") or HeadFrame(K, V, H // H_kv)
    CR = bwd_ctx["compression_rate"]
    TK = bwd_ctx["top_k_per_layer"]
    L = bwd_ctx["num_layers"]
    MTN = bwd_ctx.get("max_top_nodes") or infer_max_top_nodes(T, CR, TK, L)
    scale = bwd_ctx["scale"]
    cos, sin = bwd_ctx["cos_cache"], bwd_ctx["sin_cache"]
    ws = bwd_ctx.get("packed_tree")
    d = bwd_ctx.get("dims")
    if ws is None or d is None:
        # a context of the reference's keys: the kernels run with its own tables
        check_tables(cos, sin, K // 2, max(TK * CR, CR + 1), dev)
        d = make_dims(B, T, H, H_kv, hf.D, CR, MTN, TK, q.dtype, cos.shape[0], hf.share, hf.gpad)
        assert len(N.levels(d)) == L, f"num_layers {L} does not match T={T}, CR={CR}, MTN={MTN}"
        ws = None
    cos_k, sin_k = hf.tables(cos, sin)
    q = q.contiguous()
    qf = hf.q_heads(hf.pad_qk(q))
    parents = bwd_ctx.get("parents_stacked")
    plp = bwd_ctx.get("per_layer_parents")
    # per_layer_parents (what the reference reads) are views of the forward's
    # stacked lists.  Lists a caller replaced, or edited in place (views
    # share their base's version counter), are the caller's own: checked,
    # copied to every KV-head copy, and without the forward's stored scores.
    own = parents is not None and parents._version == bwd_ctx.get("parents_version",
                                                                   parents._version)
    if parents is not None and plp is not None and any(
            plp[l].data_ptr() != parents[l].data_ptr() for l in range(L)):
        own, parents = False, None
    # the training forward's stored scores go with its own parent lists
    scores = bwd_ctx.get("train_scores") if own else None
    if not own and plp is not None:
        parents = _stack_parents(plp, L)
    elif not own and parents is not None:
        parents = hf.pick(parents, 3).contiguous()
    if not own and parents is not None:
        _check_parents(parents, B, T, H_kv, TK, CR, MTN, dev)
        parents = hf.dup(parents, 3)
    if parents is None:
        # replay the selection alone (the lists of every level, no output);
        # the backward then rebuilds the scores
        parents, ws = select_frame(qf, hf.kv_k(k.contiguous()), hf.kv_v(v.contiguous()), d, cos_k,
                                   sin_k, scale)
        scores = None
    elif ws is None:
        _, _, ws = build_tree(hf.kv_k(k.contiguous()), hf.kv_v(v.contiguous()), d, cos_k, sin_k)
    # padding heads of a group: zero dO (they add nothing to dk / dv), and
    # any finite out / max / sum
    dOf = hf.q_heads(hf.pad_v(dO.contiguous().to(q.dtype)))
    outf = hf.q_heads(hf.pad_v(output.contiguous().to(q.dtype)))
    gmax = hf.q_heads(bwd_ctx["global_max"].contiguous(), fill=0.0)
    gsum = hf.q_heads(bwd_ctx["global_sum"].contiguous(), fill=1.0)
    D = hf.D
    # KV-head pairs add their halves' dk / dv in fp32 before the rounding
    kdt = gdt if hf.share == 1 else torch.float32
    if kdt != torch.float32:
        d = N.with_grad_dtype(d, kdt)
    g = dict(dtype=kdt, device=dev)
    dq = torch.empty(B, T, qf.shape[2], D, **g)
    dk = torch.empty(B, T, H_kv * hf.share, D, **g)
    dv = torch.empty_like(dk)
    with torch.cuda.device(dev):
        bws, plan = backward_workspace(d, dev, _workspace_limit)
        bwd_ctx["backward_plan"] = plan
        if scores is not None:
            rc = N.lib().htree_backward_train(
                d, float(scale), N.ptr(qf), N.ptr(outf), N.ptr(dOf), N.ptr(gmax),
                N.ptr(gsum), N.ptr(parents), N.ptr(ws), ws.numel(), N.ptr(cos_k),
                N.ptr(sin_k), N.ptr(scores), scores.numel(), N.ptr(dq), N.ptr(dk), N.ptr(dv),
                N.ptr(bws), bws.numel(), N.stream_ptr(dev))
            N.check(rc, "htree_backward_train")
        else:
            rc = N.lib().htree_backward(
                d, float(scale), N.ptr(qf), N.ptr(outf), N.ptr(dOf), N.ptr(gmax),
                N.ptr(gsum), N.ptr(parents), N.ptr(ws), ws.numel(), N.ptr(cos_k),
                N.ptr(sin_k), N.ptr(dq), N.ptr(dk), N.ptr(dv), N.ptr(bws), bws.numel(),
                N.stream_ptr(dev))
            N.check(rc, "htree_backward")
    return (hf.unpad_qk(hf.q_heads_back(dq)).to(gdt), hf.unpad_qk(hf.pair_sum(dk)).to(gdt),
            hf.unpad_v(hf.pair_sum(dv)).to(gdt))


_REF_META = ("num_layers", "compression_rate", "top_k_per_layer", "max_top_nodes", "scale",
             "rope_base", "NUM_GROUPS", "G_PAD", "TILE_P", "DROP_BLOCK")


def _save_forward(ctx, q, k, v, compression_rate, max_top_nodes, top_k_per_layer, scale,
                  rope_base, save_scores):
    out, bwd_ctx = htree_forward(q, k, v, compression_rate=compression_rate,
                                 max_top_nodes=max_top_nodes, top_k_per_layer=top_k_per_layer,
                                 scale=scale, rope_base=rope_base, _save_for_backward=True,
                                 _save_parents=True, _save_scores=save_scores)
    ctx.save_for_backward(q, k, v, out, bwd_ctx["global_max"], bwd_ctx["global_sum"],
                          bwd_ctx["cos_cache"], bwd_ctx["sin_cache"],
                          bwd_ctx["parents_stacked"], bwd_ctx["packed_tree"],
                          bwd_ctx["train_scores"])
    ctx.meta = {key: bwd_ctx[key] for key in _REF_META}
    ctx.meta.update(dims=bwd_ctx["dims"], head_frame=bwd_ctx["head_frame"])
    return out


def _saved_backward(ctx, dO):
    q, k, v, out, gmax, gsum, cos, sin, parents, ws, scores = ctx.saved_tensors
    bwd_ctx = dict(ctx.meta, global_max=gmax, global_sum=gsum, layers_k=[k], layers_v=[v],
                   cos_cache=cos, sin_cache=sin, parents_stacked=parents,
                   parents_version=parents._version, per_layer_parents=None, packed_tree=ws,
                   train_scores=scores)
    dq, dk, dv = htree_backward(dO, q, out, bwd_ctx, _grad_dtype=q.dtype)
    return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None, None, None, None


class HTreeTritonFunction(torch.autograd.Function):
    """Autograd contract of the reference (src/backward.py:1126-1193): grads
    in the input dtypes and None for the five non-tensor arguments.  Saves
    the reference's eight tensors plus the parent lists and the packed
    operand tree (C2: 67 MB beyond the eight), so that the backward replays
    no selection; it rebuilds the candidate scores."""

    @staticmethod
    def forward(ctx, q, k, v, compression_rate, max_top_nodes, top_k_per_layer, scale, rope_base):
        return _save_forward(ctx, q, k, v, compression_rate, max_top_nodes, top_k_per_layer, scale,
                             rope_base, False)

    @staticmethod
    def backward(ctx, dO):
        return _saved_backward(ctx, dO)


class HTreeScoresFunction(torch.autograd.Function):
    """HTreeTritonFunction that also keeps every candidate tile's scores
    (bf16 configurations with <= 16 candidate tiles per level; C2: 1.6 GB),
    so that the backward reads them instead of rebuilding them."""

    @staticmethod
    def forward(ctx, q, k, v, compression_rate, max_top_nodes, top_k_per_layer, scale, rope_base):
        return _save_forward(ctx, q, k, v, compression_rate, max_top_nodes, top_k_per_layer, scale,
                             rope_base, True)

    @staticmethod
    def backward(ctx, dO):
        return _saved_backward(ctx, dO)


class HTreeLeanFunction(torch.autograd.Function):
    """The reference's memory trade-off (src/backward.py:1130-1171): saves
    only q, k, v, out, global max / sum and the RoPE tables; the backward
    rebuilds the tree and replays the selection.  Same contract as
    HTreeTritonFunction."""

    @staticmethod
    def forward(ctx, q, k, v, compression_rate, max_top_nodes, top_k_per_layer, scale, rope_base):
        out, bwd_ctx = htree_forward(q, k, v, compression_rate=compression_rate,
                                     max_top_nodes=max_top_nodes, top_k_per_layer=top_k_per_layer,
                                     scale=scale, rope_base=rope_base, _save_for_backward=True,
                                     _save_parents=False)
        ctx.save_for_backward(q, k, v, out, bwd_ctx["global_max"], bwd_ctx["global_sum"],
                              bwd_ctx["cos_cache"], bwd_ctx["sin_cache"])
        ctx.meta = {key: bwd_ctx[key] for key in _REF_META}
        return out

    @staticmethod
    def backward(ctx, dO):
        q, k, v, out, gmax, gsum, cos, sin = ctx.saved_tensors
        bwd_ctx = dict(ctx.meta, global_max=gmax, global_sum=gsum, layers_k=[k], layers_v=[v],
                       cos_cache=cos, sin_cache=sin, per_layer_parents=None)
        dq, dk, dv = htree_backward(dO, q, out, bwd_ctx, _grad_dtype=q.dtype)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None, None, None, None


HTreeFunction = HTreeTritonFunction


def htree_forward_triton_autograd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                  compression_rate: int = 16, max_top_nodes: int = 8192,
                                  top_k_per_layer: int = 512, scale: Optional[float] = None,
                                  rope_base: float = 10000.0, _save_parents: bool = True,
                                  _save_scores: bool = False) -> torch.Tensor:
    """Differentiable htree forward (name of src/backward.py:1196 kept for
    drop-in use; the kernels are the HIP ones).  Default: the reference's
    eight tensors plus the parent lists and the packed tree are kept between
    forward and backward (HTreeTritonFunction).  `_save_scores=True` also
    keeps the candidate scores (HTreeScoresFunction, faster backward);
    `_save_parents=False` keeps only the eight tensors (HTreeLeanFunction:
    the backward replays the selection)."""
    if scale is None:
        scale = q.shape[-1] ** -0.5
    if not _save_parents:
        fn = HTreeLeanFunction
    else:
        fn = HTreeScoresFunction if _save_scores else HTreeTritonFunction
    return fn.apply(q.contiguous(), k.contiguous(), v.contiguous(), compression_rate, max_top_nodes,
                    top_k_per_layer, scale, rope_base)


htree_forward_autograd = htree_forward_triton_autograd
