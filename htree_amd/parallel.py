"""htree forward on MI355X: the drop-in for `htree_forward` of
/root/reference/src/parallel.py:874-1159.

Same signature, argument meaning, defaults, return values and `bwd_ctx` keys.
Differences, all deliberate:
  * `max_top_nodes <= top_k_per_layer * compression_rate` is accepted (the
    reference asserts equality, src/parallel.py:917); the algorithm never
    relies on equality.  The reference's Triton-tiling asserts
    (top_k % 64 == 0, top_k % compression_rate == 0, :923,1019) do not apply.
  * limits of this HIP build (AssertionError): max(K, V) <= 256 (K even),
    H / H_kv <= 1024, 4 <= compression_rate <= 128,
    top_k_per_layer <= 2048 and top_k_per_layer * compression_rate <= 65536
    candidates per level (top_k_per_layer <= 1024 and 16384 candidates for
    max(K, V) > 128).
  * a query group of G > 16 heads (the reference pads it to G_PAD,
    src/parallel.py:1023) runs as s = 2 (G <= 32), 4 (G <= 64) or the power
    of two s >= G / 16 (up to 64) groups of ceil(G/s) heads over s copies of
    each KV head that share one selection (the kernels' kv_share mode); each
    KV head's dk / dv is the sum of its copies'.  A group that s does not
    divide gets zero query heads appended to its last copy (the kernels'
    group_pad): the forward leaves them out of the selection, the backward
    gives them zero dO.  Shares above 4, candidate sets above 16384, lists
    of more than 1024 parents (or a pair's / quad's importances beyond one
    block's LDS) run the split selection: the parts meet through device
    memory level by level.
  * K != V (the reference carries V = v.shape[-1] apart from K,
    src/parallel.py:904), and head dims that are not a kernel head dim
    (32, 64, 128, 256; e.g. 16, or 96), run the kernels at one head dim D,
    the smallest kernel head dim >= max(K, V): V is zero-padded to D (zero
    columns add nothing to P.V and come out zero), and for K < D the query
    / key halves of each RoPE pair are placed at [0, K/2) and
    [D/2, D/2 + K/2) with zeros between, rotated by tables whose first K/2
    columns are the K-dim tables (the zero columns stay zero under any
    rotation), so every score is the K-dim score.
  * empty inputs (B == 0 or T == 0) give empty outputs (and a bwd_ctx whose
    backward gives empty gradients) without a launch.
  * the RoPE tables are built on the host with the reference's recipe
    (src/parallel.py:983-988) and copied to the device.
  * bwd_ctx carries extra keys: `rope_base`, `packed_tree` (the MFMA operand
    copy of the tree, reused by the backward), `dims`, `parents_stacked`,
    `parents_version` (the version counter of `parents_stacked` when the
    forward wrote them: lists edited in place afterwards are the caller's),
    `train_scores` (with `_save_scores=True` only: every candidate tile's
    scores, fp16 relative to the head's running max, so that the backward
    does not rebuild them; None where the configuration rebuilds them) and
    `head_frame` (how K and V map onto the kernels' head dim).
"""
from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch

from . import _native as N

HTREE_SCORE_NEG_INF = -1.0e10            # src/parallel.py:75
HTREE_SCORE_VALID_THRESHOLD = HTREE_SCORE_NEG_INF * 0.9  # :81

KERNEL_HEAD_DIMS = (32, 64, 128, 256)
MAX_GROUP = 1024              # query heads per KV head (kernel shares up to 64)
MAX_CANDIDATES = 65536        # top_k_per_layer * compression_rate
MAX_CANDIDATES_D256 = 16384   # the same at head dim 256
MAX_TOPK = 2048               # top_k_per_layer (above 1024: head dims <= 128)
MAX_TOPK_D256 = 1024

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


class HeadFrame:
    """Maps the caller's heads onto the kernels': the head dims (K for q/k, V
    for v) onto one head dim D (the smallest kernel head dim >= max(K, V)),
    and a query group of G > 16 heads onto s = 2 (G <= 32), 4 (G <= 64) or
    2^ceil(log2(G/16)) (G <= 1024) groups of Gk = ceil(G/s) over KV heads
    copied in place (KV head h becomes kernel KV heads s h .. s h + s - 1:
    query head h*G + g is then kernel group s h + g // Gk, so q keeps its
    layout; when s Gk > G, q_heads appends the gpad = s Gk - G padding heads
    to each group).  With K == V == D and G <= 16 every method returns its
    argument."""

    def __init__(self, K: int, V: int, G: int = 1):
        self.K, self.V = K, V
        # the kernels' head dim: the smallest of KERNEL_HEAD_DIMS that holds both
        self.D = next(d for d in KERNEL_HEAD_DIMS if d >= max(K, V))
        self.same = K == V == self.D
        self.G = G
        self.share = 1
        while self.share * 16 < G:
            self.share *= 2
        # kernel group size; a group that share does not divide gets gpad
        # zero heads appended (src/parallel.py:1023,428-431 pads to G_PAD)
        self.Gk = -(-G // self.share)
        self.gpad = self.share * self.Gk - G
        self.plain = self.same and self.share == 1

    def q_heads(self, x: torch.Tensor, dim: int = 2, fill: float = 0.0) -> torch.Tensor:
        """Caller heads [.., H_kv*G, ..] -> kernel heads [.., H_kv*(G+gpad), ..]
        (along `dim`): each KV head's group gets gpad heads of `fill` at its end."""
        if self.gpad == 0:
            return x
        shp = list(x.shape)
        hkv = shp[dim] // self.G
        y = x.reshape(shp[:dim] + [hkv, self.G] + shp[dim + 1:])
        pad = y.new_full(shp[:dim] + [hkv, self.gpad] + shp[dim + 1:], fill)
        return torch.cat([y, pad], dim + 1).reshape(shp[:dim] + [hkv * (self.G + self.gpad)]
                                                    + shp[dim + 1:])

    def q_heads_back(self, x: torch.Tensor, dim: int = 2) -> torch.Tensor:
        """Kernel heads -> caller heads (drops the padding heads)."""
        if self.gpad == 0:
            return x
        shp = list(x.shape)
        gs = self.G + self.gpad
        hkv = shp[dim] // gs
        y = x.reshape(shp[:dim] + [hkv, gs] + shp[dim + 1:])
        y = y.narrow(dim + 1, 0, self.G)
        return y.reshape(shp[:dim] + [hkv * self.G] + shp[dim + 1:]).contiguous()

    def kv_k(self, k: torch.Tensor) -> torch.Tensor:
        """Caller k [B,T,H_kv,K] -> kernel k [B,T,share*H_kv,D]."""
        return self.dup(self.pad_qk(k), 2)

    def kv_v(self, v: torch.Tensor) -> torch.Tensor:
        return self.dup(self.pad_v(v), 2)

    def dup(self, x: torch.Tensor, dim: int) -> torch.Tensor:
        return x if self.share == 1 else x.repeat_interleave(self.share, dim).contiguous()

    def pick(self, x: torch.Tensor, dim: int) -> torch.Tensor:
        """Kernel KV heads -> caller KV heads (the first of each copy: the
        copies agree on everything but their own dk / dv)."""
        if self.share == 1:
            return x
        idx = [slice(None)] * x.dim()
        idx[dim] = slice(0, None, self.share)
        return x[tuple(idx)]

    def pair_sum(self, x: torch.Tensor) -> torch.Tensor:
        """Kernel dk / dv [B,T,share*H_kv,D] -> caller [B,T,H_kv,D]."""
        if self.share == 1:
            return x
        B, T, Hs, D = x.shape
        return x.view(B, T, Hs // self.share, self.share, D).sum(3)

    def pad_qk(self, x: torch.Tensor) -> torch.Tensor:
        """[..., K] -> [..., D]: RoPE pair halves at [0, K/2) and [D/2, D/2 + K/2)."""
        if self.K == self.D:
            return x
        h, H = self.K // 2, self.D // 2
        y = x.new_zeros(*x.shape[:-1], self.D)
        y[..., :h] = x[..., :h]
        y[..., H:H + h] = x[..., h:]
        return y

    def unpad_qk(self, x: torch.Tensor) -> torch.Tensor:
        if self.K == self.D:
            return x
        h, H = self.K // 2, self.D // 2
        return torch.cat([x[..., :h], x[..., H:H + h]], -1)

    def pad_v(self, x: torch.Tensor) -> torch.Tensor:
        if self.V == self.D:
            return x
        return torch.nn.functional.pad(x, (0, self.D - self.V))

    def unpad_v(self, x: torch.Tensor) -> torch.Tensor:
        if self.V == self.D:
            return x
        return x[..., :self.V].contiguous()

    def tables(self, cos: torch.Tensor, sin: torch.Tensor):
        """K-dim tables [rows, K/2] -> kernel tables [rows, D/2] (identity
        rotation on the padding columns, which only ever meet zeros)."""
        if self.K == self.D:
            return cos, sin
        pad = self.D // 2 - self.K // 2
        return (torch.nn.functional.pad(cos, (0, pad), value=1.0).contiguous(),
                torch.nn.functional.pad(sin, (0, pad), value=0.0).contiguous())


def _validate(q, k, v, compression_rate, max_top_nodes, top_k_per_layer):
    assert q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "q/k/v must be rank-4 tensors"
    B, T, H, K = q.shape
    H_kv = k.shape[2]
    assert H % H_kv == 0, f"H ({H}) must be divisible by H_kv ({H_kv})"
    assert k.shape[2] == v.shape[2], "K and V must have same number of heads"
    assert k.shape[:2] == (B, T) and v.shape[:2] == (B, T), "q/k/v batch and length must match"
    assert k.shape[3] == K, f"q and k must share the head dim K ({K} vs {k.shape[3]})"
    V = v.shape[3]
    G = H // H_kv
    assert G <= MAX_GROUP, (
        f"configuration outside this HIP build: query groups of up to {MAX_GROUP} heads, "
        f"got H/H_kv = {G}")
    npos = top_k_per_layer * compression_rate
    assert npos <= MAX_CANDIDATES, (
        f"configuration outside this HIP build: top_k_per_layer * compression_rate <= "
        f"{MAX_CANDIDATES}, got {npos}")
    assert npos <= MAX_CANDIDATES_D256 or max(K, v.shape[3]) <= 128, (
        f"configuration outside this HIP build: above {MAX_CANDIDATES_D256} candidates per "
        f"level the head dim max(K, V) must be <= 128, got {max(K, v.shape[3])}")
    assert top_k_per_layer <= MAX_TOPK, (
        f"configuration outside this HIP build: top_k_per_layer <= {MAX_TOPK}, got "
        f"{top_k_per_layer}")
    assert top_k_per_layer <= MAX_TOPK_D256 or max(K, v.shape[3]) <= 128, (
        f"configuration outside this HIP build: above top_k_per_layer {MAX_TOPK_D256} the "
        f"head dim max(K, V) must be <= 128, got {max(K, v.shape[3])}")
    assert K % 2 == 0 and K > 0 and V > 0, "head dims must be positive, K even (RoPE pairs)"
    assert max(K, V) <= KERNEL_HEAD_DIMS[-1], (
        f"configuration outside this HIP build: needs max(K, V) <= {KERNEL_HEAD_DIMS[-1]}, "
        f"got K={K}, V={V}")
    assert q.dtype == k.dtype == v.dtype, "q, k, v must share one dtype"
    assert (top_k_per_layer & (top_k_per_layer - 1)) == 0, "top_k_per_layer (TOP_K) must be a power of 2"
    assert (compression_rate & (compression_rate - 1)) == 0, "compression_rate must be a power of 2"
    assert (max_top_nodes & (max_top_nodes - 1)) == 0, "max_top_nodes must be a power of 2"
    assert max_top_nodes <= top_k_per_layer * compression_rate, (
        f"max_top_nodes ({max_top_nodes}) must be <= top_k_per_layer*compression_rate "
        f"({top_k_per_layer}*{compression_rate}={top_k_per_layer * compression_rate})")
    assert q.is_cuda and k.is_cuda and v.is_cuda, "htree_amd runs on the GPU (no CPU fallback)"
    assert q.device == k.device == v.device, "q, k, v must be on one device"


def rope_rows_for(max_top_nodes: int, top_k_per_layer: int, compression_rate: int) -> int:
    """Rows of the RoPE tables: the reference's max_top_nodes + 1024
    (src/parallel.py:983), and at least every candidate position."""
    return max(max_top_nodes + 1024, top_k_per_layer * compression_rate)


def make_dims(B, T, H, H_kv, D, compression_rate, max_top_nodes, top_k_per_layer, dtype, rope_rows,
              share=1, gpad=0):
    """Kernel dims; H and H_kv count the caller's heads, the kernels see
    share * H_kv KV heads and H + gpad * H_kv query heads."""
    return N.dims(B, T, H + gpad * H_kv, H_kv * share, D, compression_rate, top_k_per_layer,
                  max_top_nodes, dtype, rope_rows, share, group_pad=gpad)


def check_tables(cos, sin, half: int, rows_min: int, device):
    """RoPE tables handed in by a caller (a bwd_ctx's cos_cache / sin_cache)
    go to the kernels as they are: fp32 [rows, half], rows >= rows_min (every
    candidate position, and the row of angle compression_rate)."""
    for name, t in (("cos_cache", cos), ("sin_cache", sin)):
        assert t.dtype == torch.float32 and t.dim() == 2 and t.shape[1] == half, \
            f"{name} must be fp32 [rows, {half}], got {t.dtype} {list(t.shape)}"
        assert t.shape[0] >= rows_min, \
            f"{name} has {t.shape[0]} rows; every candidate position needs {rows_min}"
        assert t.device == device, f"{name} must be on the inputs' device"
    assert cos.shape == sin.shape, "cos_cache and sin_cache must have one shape"


def build_tree(k, v, d, cos, sin):
    """Levels 1..L-1 (input dtype) and the packed operand tree, with K
    pre-rotated by the given kernel-frame tables.  k, v are in the kernel
    frame ([B,T,H_kv,D])."""
    B, T, H_kv, D = k.shape
    sizes = N.levels(d)
    layers_k, layers_v = [k], [v]
    for n in sizes[1:]:
        layers_k.append(torch.empty(B, n, H_kv, D, dtype=k.dtype, device=k.device))
        layers_v.append(torch.empty(B, n, H_kv, D, dtype=v.dtype, device=v.device))
    ws = torch.empty(N.tree_workspace_bytes(d), dtype=torch.uint8, device=k.device)
    rc = N.lib().htree_tree_build(
        d, N.ptr(k), N.ptr(v), N.ptr_array([None] + layers_k[1:]),
        N.ptr_array([None] + layers_v[1:]), N.ptr(cos), N.ptr(sin), N.ptr(ws), ws.numel(),
        N.stream_ptr(k.device))
    N.check(rc, "htree_tree_build")
    return layers_k, layers_v, ws


def select_frame(qf, kf, vf, d, cos_k, sin_k, scale):
    """The selection alone on kernel-frame tensors (htree_select: the lists
    of every level, no output), as the reference's backward replays it
    (src/backward.py:881-934).  Returns (parents [L,B,T,H_kv,TK], packed tree)."""
    B, T = qf.shape[:2]
    H_kv = kf.shape[2]
    dev = qf.device
    with torch.cuda.device(dev):
        layers_k, _, ws = build_tree(kf, vf, d, cos_k, sin_k)
        parents = torch.empty(len(layers_k), B, T, H_kv, d.top_k, dtype=torch.int32, device=dev)
        rc = N.lib().htree_select(d, float(scale), N.ptr(qf), N.ptr(ws), ws.numel(), N.ptr(cos_k),
                                  N.ptr(sin_k), N.ptr(parents), N.stream_ptr(dev))
        N.check(rc, "htree_select")
    return parents, ws


def forward_frame(qf, kf, vf, d, cos_k, sin_k, scale, save_parents, keep_scores):
    """The HIP forward on kernel-frame tensors.  cos_k / sin_k: the kernel
    frame's tables.  Returns (out, gmax, gsum, parents | None, layers_k,
    layers_v, packed tree, scores | None)."""
    B, T, H, D = qf.shape
    H_kv = kf.shape[2]
    dev = qf.device
    empty = B == 0 or T == 0  # nothing to attend: no tree, no launch
    with torch.cuda.device(dev):
        if empty:
            # the library's limits still apply: checked on one query
            N.levels(N.dims(1, 1, H, H_kv, D, d.compression_rate, d.top_k, d.max_top_nodes,
                            qf.dtype, d.rope_rows, d.kv_share))
            layers_k, layers_v = [kf], [vf]
            ws = torch.empty(0, dtype=torch.uint8, device=dev)
        else:
            layers_k, layers_v, ws = build_tree(kf, vf, d, cos_k, sin_k)
        L = len(layers_k)
        out = torch.empty_like(qf)
        gmax = torch.empty(B, T, H, dtype=torch.float32, device=dev)
        gsum = torch.empty(B, T, H, dtype=torch.float32, device=dev)
        parents = (torch.empty(L, B, T, H_kv, d.top_k, dtype=torch.int32, device=dev)
                   if save_parents else None)
        nsc = N.train_scores_bytes(d) if save_parents and keep_scores and not empty else 0
        scores = torch.empty(nsc, dtype=torch.uint8, device=dev) if nsc > 0 else None
        if empty:
            pass
        elif scores is not None:
            rc = N.lib().htree_forward_train(d, float(scale), N.ptr(qf), N.ptr(ws), ws.numel(),
                                             N.ptr(cos_k), N.ptr(sin_k), N.ptr(out), N.ptr(gmax),
                                             N.ptr(gsum), N.ptr(parents), N.ptr(scores), nsc,
                                             N.stream_ptr(dev))
            N.check(rc, "htree_forward_train")
        else:
            rc = N.lib().htree_forward(d, float(scale), N.ptr(qf), N.ptr(ws), ws.numel(),
                                       N.ptr(cos_k), N.ptr(sin_k), N.ptr(out), N.ptr(gmax),
                                       N.ptr(gsum), N.ptr(parents), N.stream_ptr(dev))
            N.check(rc, "htree_forward")
    return out, gmax, gsum, parents, layers_k, layers_v, ws, scores


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
    _save_scores: bool = False,
):
    """htree forward.  q [B,T,H,K], k [B,T,H_kv,K], v [B,T,H_kv,V] ->
    output [B,T,H,V] (q.dtype); with _save_for_backward also the bwd_ctx dict.
    With _save_parents (the default, as in the reference) the context holds
    every level's parent lists for the backward; without it the backward
    replays the selection (src/backward.py:881-934).  _save_scores (not in
    the reference) also keeps every candidate tile's scores, where the
    configuration allows it, so that the backward reads them instead of
    rebuilding them: faster, at 1.6 GB for a C2-sized call."""
    _validate(q, k, v, compression_rate, max_top_nodes, top_k_per_layer)
    B, T, H, K = q.shape
    H_kv = k.shape[2]
    G = H // H_kv
    hf = HeadFrame(K, v.shape[3], G)
    if scale is None:
        scale = K ** -0.5
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    rows = rope_rows_for(max_top_nodes, top_k_per_layer, compression_rate)
    d = make_dims(B, T, H, H_kv, hf.D, compression_rate, max_top_nodes, top_k_per_layer, q.dtype,
                  rows, hf.share, hf.gpad)
    cos, sin = rope_cache(K, rows, rope_base, q.device)
    cos_k, sin_k = hf.tables(cos, sin)
    save_par = _save_for_backward and _save_parents
    out_f, gmax, gsum, parents, lk, lv, ws, scores = forward_frame(
        hf.q_heads(hf.pad_qk(q)), hf.kv_k(k), hf.kv_v(v), d, cos_k, sin_k, scale, save_par,
        _save_scores)
    out = hf.unpad_v(hf.q_heads_back(out_f))
    gmax, gsum = hf.q_heads_back(gmax), hf.q_heads_back(gsum)
    if not _save_for_backward:
        return out
    L = len(lk)
    bwd_ctx = dict(
        global_max=gmax,
        global_sum=gsum,
        per_layer_parents={l: hf.pick(parents[l], 2) for l in range(L)} if save_par else None,
        # the caller's frame: layers_k[0] is k (src/parallel.py:949)
        layers_k=[k] + [hf.unpad_qk(hf.pick(x, 2)).contiguous() for x in lk[1:]]
        if not hf.plain else lk,
        layers_v=[v] + [hf.unpad_v(hf.pick(x, 2)).contiguous() for x in lv[1:]]
        if not hf.plain else lv,
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
        rope_base=rope_base,
        packed_tree=ws,
        dims=d,
        parents_stacked=parents,
        parents_version=parents._version if parents is not None else None,
        train_scores=scores,
        head_frame=hf,
    )
    return out, bwd_ctx


def htree_forward_parents(q, k, v, compression_rate=16, max_top_nodes=8192, top_k_per_layer=512,
                          scale=None, rope_base=10000.0, _save_scores=False):
    """Forward that also returns the per-level parent lists [L,B,T,H_kv,TK]
    (the list used at each level: the initial virtual parents at L-1, then
    each level's selection), gmax and gsum.  Used by the trace tests."""
    out, ctx = htree_forward(q, k, v, compression_rate, max_top_nodes, top_k_per_layer, scale,
                             rope_base, _save_for_backward=True, _save_parents=True,
                             _save_scores=_save_scores)
    par = ctx["head_frame"].pick(ctx["parents_stacked"], 3)
    return out, par, ctx["global_max"], ctx["global_sum"], ctx
