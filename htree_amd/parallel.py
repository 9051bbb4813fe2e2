"""htree forward on MI355X: the drop-in for `htree_forward` of
/root/reference/src/parallel.py:874-1159.

Same signature, argument meaning, defaults, return values and `bwd_ctx` keys.
Differences, all deliberate:
  * `max_top_nodes <= top_k_per_layer * compression_rate` is accepted (the
    reference asserts equality, src/parallel.py:917); the algorithm never
    relies on equality.  The reference's Triton-tiling asserts
    (top_k % 64 == 0, top_k % compression_rate == 0, :923,1019) do not apply.
  * limits of this HIP build (AssertionError): head_dim in {32, 64, 128},
    H / H_kv <= 16, 4 <= compression_rate <= 64, top_k_per_layer <= 512 and
    top_k_per_layer * compression_rate <= 8192 candidates per level.
  * empty inputs (B == 0 or T == 0) give empty outputs (and a bwd_ctx whose
    backward gives empty gradients) without a launch.
  * the RoPE tables are built on the host with the reference's recipe
    (src/parallel.py:983-988) and copied to the device.
  * bwd_ctx carries extra keys: `packed_tree` (the MFMA operand copy of the
    tree, reused by the backward), `dims`, `parents_stacked` and
    `train_scores` (every candidate tile's scores, fp16 relative to the
    head's running max, so that the backward does not rebuild them; None
    where the configuration rebuilds them).
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch

from . import _native as N

HTREE_SCORE_NEG_INF = -1.0e10            # src/parallel.py:75
HTREE_SCORE_VALID_THRESHOLD = HTREE_SCORE_NEG_INF * 0.9  # :81

_rope_cache: Dict[Tuple, Tuple[torch.Tensor, torch.Tensor]] = {}


def rope_cache(head_dim: int, rows: int, rope_base: float, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [rows, head_dim/2] fp32 (src/parallel.py:983-988), computed on
    the host and kept per device."""
    key = (head_dim, rows, float(rope_base), str(device))
    hit = _rope_cache.get(key)
    if hit is None:
        inv_freq = 1.0 / (rope_base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
        pos = torch.arange(rows, dtype=torch.float32)
        freqs = torch.outer(pos, inv_freq)
        hit = (freqs.cos().to(device), freqs.sin().to(device))
        _rope_cache[key] = hit
    return hit


def _validate(q, k, v, compression_rate, max_top_nodes, top_k_per_layer):
    assert q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "q/k/v must be rank-4 tensors"
    B, T, H, K = q.shape
    H_kv = k.shape[2]
    assert H % H_kv == 0, f"H ({H}) must be divisible by H_kv ({H_kv})"
    assert k.shape[2] == v.shape[2], "K and V must have same number of heads"
    assert k.shape[:2] == (B, T) and v.shape[:2] == (B, T), "q/k/v batch and length must match"
    assert k.shape[3] == K and v.shape[3] == K, "this implementation needs K == V == head_dim"
    assert q.dtype == k.dtype == v.dtype, "q, k, v must share one dtype"
    assert (top_k_per_layer & (top_k_per_layer - 1)) == 0, "top_k_per_layer (TOP_K) must be a power of 2"
    assert (compression_rate & (compression_rate - 1)) == 0, "compression_rate must be a power of 2"
    assert (max_top_nodes & (max_top_nodes - 1)) == 0, "max_top_nodes must be a power of 2"
    assert max_top_nodes <= top_k_per_layer * compression_rate, (
        f"max_top_nodes ({max_top_nodes}) must be <= top_k_per_layer*compression_rate "
        f"({top_k_per_layer}*{compression_rate}={top_k_per_layer * compression_rate})")
    assert q.is_cuda and k.is_cuda and v.is_cuda, "htree_amd runs on the GPU (no CPU fallback)"
    assert q.device == k.device == v.device, "q, k, v must be on one device"


def make_dims(q, k, compression_rate, max_top_nodes, top_k_per_layer):
    B, T, H, K = q.shape
    rows = max(max_top_nodes + 1024, top_k_per_layer * compression_rate)
    return N.dims(B, T, H, k.shape[2], K, compression_rate, top_k_per_layer, max_top_nodes,
                  q.dtype, rows), rows


def build_tree(k, v, d, rows, rope_base):
    """Levels 1..L-1 (input dtype) and the packed operand tree."""
    B, T, H_kv, K = k.shape
    sizes = N.levels(d)
    layers_k, layers_v = [k], [v]
    for n in sizes[1:]:
        layers_k.append(torch.empty(B, n, H_kv, K, dtype=k.dtype, device=k.device))
        layers_v.append(torch.empty(B, n, H_kv, K, dtype=v.dtype, device=v.device))
    cos, sin = rope_cache(K, rows, rope_base, k.device)
    ws = torch.empty(N.tree_workspace_bytes(d), dtype=torch.uint8, device=k.device)
    rc = N.lib().htree_tree_build(
        d, N.ptr(k), N.ptr(v), N.ptr_array([None] + layers_k[1:]),
        N.ptr_array([None] + layers_v[1:]), N.ptr(cos), N.ptr(sin), N.ptr(ws), ws.numel(),
        N.stream_ptr(k.device))
    N.check(rc, "htree_tree_build")
    return layers_k, layers_v, ws, cos, sin


def htree_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    compression_rate: int = 16,
    max_top_nodes: int = 8192,
    top_k_per_layer: int = 512,
    scale: Optional[float] = None,
    rope_base: float = 10000.0,
    _save_for_backward: bool = False,
    _save_parents: bool = True,
):
    """htree forward.  q [B,T,H,K], k/v [B,T,H_kv,K] -> output [B,T,H,K]
    (q.dtype); with _save_for_backward also the bwd_ctx dict."""
    _validate(q, k, v, compression_rate, max_top_nodes, top_k_per_layer)
    B, T, H, K = q.shape
    H_kv = k.shape[2]
    if scale is None:
        scale = K ** -0.5
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    d, rows = make_dims(q, k, compression_rate, max_top_nodes, top_k_per_layer)
    empty = B == 0 or T == 0  # nothing to attend: no tree, no launch
    with torch.cuda.device(q.device):
        if empty:
            # the library's limits still apply: checked on one query
            N.levels(N.dims(1, 1, H, H_kv, K, compression_rate, top_k_per_layer, max_top_nodes,
                            q.dtype, rows))
            layers_k, layers_v = [k], [v]
            ws = torch.empty(0, dtype=torch.uint8, device=q.device)
            cos, sin = rope_cache(K, rows, rope_base, q.device)
        else:
            layers_k, layers_v, ws, cos, sin = build_tree(k, v, d, rows, rope_base)
        L = len(layers_k)
        out = torch.empty_like(q)
        gmax = torch.empty(B, T, H, dtype=torch.float32, device=q.device)
        gsum = torch.empty(B, T, H, dtype=torch.float32, device=q.device)
        save_par = _save_for_backward and _save_parents
        parents = (torch.empty(L, B, T, H_kv, top_k_per_layer, dtype=torch.int32, device=q.device)
                   if save_par else None)
        nsc = N.train_scores_bytes(d) if save_par and not empty else 0
        scores = torch.empty(nsc, dtype=torch.uint8, device=q.device) if nsc > 0 else None
        if empty:
            pass
        elif scores is not None:
            rc = N.lib().htree_forward_train(d, float(scale), N.ptr(q), N.ptr(ws), ws.numel(),
                                             N.ptr(cos), N.ptr(sin), N.ptr(out), N.ptr(gmax),
                                             N.ptr(gsum), N.ptr(parents), N.ptr(scores), nsc,
                                             N.stream_ptr(q.device))
            N.check(rc, "htree_forward_train")
        else:
            rc = N.lib().htree_forward(d, float(scale), N.ptr(q), N.ptr(ws), ws.numel(),
                                       N.ptr(cos), N.ptr(sin), N.ptr(out), N.ptr(gmax),
                                       N.ptr(gsum), N.ptr(parents), N.stream_ptr(q.device))
            N.check(rc, "htree_forward")
    if not _save_for_backward:
        return out
    G = H // H_kv
    bwd_ctx = dict(
        global_max=gmax,
        global_sum=gsum,
        per_layer_parents={l: parents[l] for l in range(L)} if save_par else None,
        layers_k=layers_k,
        layers_v=layers_v,
        cos_cache=cos,
        sin_cache=sin,
        num_layers=L,
        compression_rate=compression_rate,
        top_k_per_layer=top_k_per_layer,
        max_top_nodes=max_top_nodes,
        scale=scale,
        NUM_GROUPS=G,
        G_PAD=max(1 << (G - 1).bit_length(), 16),
        TILE_P=4,
        DROP_BLOCK=64,
        packed_tree=ws,
        dims=d,
        parents_stacked=parents,
        train_scores=scores,
    )
    return out, bwd_ctx


def htree_forward_parents(q, k, v, compression_rate=16, max_top_nodes=8192, top_k_per_layer=512,
                          scale=None, rope_base=10000.0):
    """Forward that also returns the per-level parent lists [L,B,T,H_kv,TK]
    (the list used at each level: the initial virtual parents at L-1, then
    each level's selection), gmax and gsum.  Used by the trace tests."""
    out, ctx = htree_forward(q, k, v, compression_rate, max_top_nodes, top_k_per_layer, scale,
                             rope_base, _save_for_backward=True, _save_parents=True)
    return out, ctx["parents_stacked"], ctx["global_max"], ctx["global_sum"], ctx
