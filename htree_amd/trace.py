"""Per-level trace of the forward, for level-by-level parity checks.

Drop-in for the trace harness of the reference:
  * LayerTrace ............... /root/reference/src/naive.py:13-19
  * run_parallel_with_trace .. /root/reference/correctness_test.py:168-347
  * compare_traces ........... /root/reference/correctness_test.py:394-466

run_parallel_with_trace runs one HIP forward (htree_forward_trace of the C
ABI) that also writes each level's own softmax state; nothing is launched per
level.  The trace dict has the reference's layout:
  {"num_layers": L, "num_groups": G, "layers": {l: LayerTrace}}
with, per level l: the parent list the level selected for level l-1
([B,T,H_kv,TK] int32, ascending, -1 padded; None at the bottom), and the
level's own max / sum [B,T,H] and unnormalised output [B,T,H,V] in fp32
(-1e10 / 0 / 0 where the level accumulated nothing).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from . import _native as N
from .parallel import (HeadFrame, _validate, build_tree, make_dims, rope_cache, rope_rows_for)


@dataclass
class LayerTrace:
    layer_idx: int
    selected_parents: Optional[torch.Tensor]
    layer_max: torch.Tensor
    layer_sum: torch.Tensor
    layer_output: torch.Tensor


def run_parallel_with_trace(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    compression_rate: int,
    max_top_nodes: int,
    top_k_per_layer: int,
    scale: Optional[float],
    rope_base: float,
) -> Tuple[torch.Tensor, Dict]:
    """Forward with the per-level trace.  Returns (output [B,T,H,V] in
    q.dtype, trace dict); output, global max and sum are the merge of the
    traced level states (src/naive.py:215-231)."""
    _validate(q, k, v, compression_rate, max_top_nodes, top_k_per_layer)
    B, T, H, K = q.shape
    H_kv = k.shape[2]
    hf = HeadFrame(K, v.shape[3], H // H_kv)
    if scale is None:
        scale = K ** -0.5
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    rows = rope_rows_for(max_top_nodes, top_k_per_layer, compression_rate)
    d = make_dims(B, T, H, H_kv, hf.D, compression_rate, max_top_nodes, top_k_per_layer, q.dtype,
                  rows, hf.share, hf.gpad)
    dev = q.device
    with torch.cuda.device(dev):
        cos, sin = hf.tables(*rope_cache(K, rows, rope_base, dev))
        qf = hf.q_heads(hf.pad_qk(q))
        Hk = qf.shape[2]  # the kernels' query heads (with any group padding)
        layers_k, layers_v, ws = build_tree(hf.kv_k(k), hf.kv_v(v), d, cos, sin)
        L = len(layers_k)
        out = torch.empty_like(qf)
        gmax = torch.empty(B, T, Hk, dtype=torch.float32, device=dev)
        gsum = torch.empty(B, T, Hk, dtype=torch.float32, device=dev)
        parents = torch.empty(L, B, T, H_kv * hf.share, top_k_per_layer, dtype=torch.int32,
                              device=dev)
        lmax = torch.empty(L, B, T, Hk, dtype=torch.float32, device=dev)
        lsum = torch.empty(L, B, T, Hk, dtype=torch.float32, device=dev)
        lout = torch.empty(L, B, T, Hk, hf.D, dtype=torch.float32, device=dev)
        rc = N.lib().htree_forward_trace(d, float(scale), N.ptr(qf), N.ptr(ws), ws.numel(),
                                         N.ptr(cos), N.ptr(sin), N.ptr(out), N.ptr(gmax),
                                         N.ptr(gsum), N.ptr(parents), N.ptr(lmax), N.ptr(lsum),
                                         N.ptr(lout), N.stream_ptr(dev))
        N.check(rc, "htree_forward_trace")
        out, lout = hf.unpad_v(hf.q_heads_back(out)), hf.unpad_v(hf.q_heads_back(lout, 3))
        gmax, gsum = hf.q_heads_back(gmax), hf.q_heads_back(gsum)
        lmax, lsum = hf.q_heads_back(lmax, 3), hf.q_heads_back(lsum, 3)
        parents = hf.pick(parents, 3)
    layers = {
        l: LayerTrace(layer_idx=l,
                      selected_parents=parents[l - 1] if l > 0 else None,
                      layer_max=lmax[l], layer_sum=lsum[l], layer_output=lout[l])
        for l in range(L - 1, -1, -1)
    }
    trace = {"num_layers": L, "num_groups": H // H_kv, "layers": layers,
             "global_max": gmax, "global_sum": gsum}
    return out, trace


def _set_sizes_and_overlap(a: torch.Tensor, b: torch.Tensor):
    """|A|, |B|, |A & B| per row of two [n, TK] lists of distinct node ids
    (-1 = none)."""
    na = (a >= 0).sum(-1)
    nb = (b >= 0).sum(-1)
    inter = torch.empty_like(na)
    chunk = max(1, (1 << 24) // (a.shape[1] * a.shape[1]))
    for s in range(0, a.shape[0], chunk):
        x, y = a[s:s + chunk], b[s:s + chunk]
        eq = (x[:, :, None] == y[:, None, :]) & (x[:, :, None] >= 0)
        inter[s:s + chunk] = eq.any(-1).sum(-1)
    return na, nb, inter


def _only_with_rank(a: List[int], b: List[int]) -> List[Dict[str, int]]:
    rank: Dict[int, int] = {}
    for i, x in enumerate(a):
        rank.setdefault(x, i + 1)
    other = set(b)
    return [{"node": x, "rank": rank[x]} for x in sorted(set(rank) - other, key=lambda y: rank[y])]


def compare_traces(
    parallel_trace: Dict,
    naive_trace: Dict,
    *,
    topk_alarm_diff: int,
    layer_out_alarm_abs: float,
    max_report: int,
) -> Dict:
    """The reference's level-by-level comparison (correctness_test.py:394-466),
    evaluated with tensor operations instead of a Python loop per row.

    For every upper level, top -> down: per (b, t, h_kv) the size of the
    symmetric difference of the two selected parent sets is counted in
    `mismatch_counter`; a difference above `topk_alarm_diff` is an alarm when
    the level above matched exactly (cascade rule); where this level matched
    exactly, the per-head normalised level outputs (layer_output /
    max(layer_sum, 1e-30)) are compared and a max |diff| above
    `layer_out_alarm_abs` is an alarm.  Alarms are listed in (level desc, b,
    t, h_kv) order, at most `max_report` of each kind."""
    L = int(parallel_trace["num_layers"])
    G = int(parallel_trace["num_groups"])
    lp, ln = parallel_trace["layers"], naive_trace["layers"]
    B, T, Hkv, TK = lp[L - 1].selected_parents.shape
    prev_equal = torch.ones(B * T * Hkv, dtype=torch.bool)
    topk_alarms: List[Dict] = []
    out_alarms: List[Dict] = []
    counter: Dict[int, int] = {}
    for l in range(L - 1, 0, -1):
        ps = lp[l].selected_parents.reshape(-1, TK).cpu()
        ns = ln[l].selected_parents.reshape(-1, TK).cpu()
        na, nb, inter = _set_sizes_and_overlap(ps, ns)
        diff = na + nb - 2 * inter
        vals, cnts = torch.unique(diff, return_counts=True)
        for x, c in zip(vals.tolist(), cnts.tolist()):
            counter[x] = counter.get(x, 0) + c
        equal = diff == 0
        for r in torch.nonzero(prev_equal & (diff > topk_alarm_diff)).flatten().tolist():
            if len(topk_alarms) >= max_report:
                break
            a = [x for x in ps[r].tolist() if x >= 0]
            b_ = [x for x in ns[r].tolist() if x >= 0]
            b, rem = divmod(r, T * Hkv)
            t, h = divmod(rem, Hkv)
            topk_alarms.append({"layer": l, "b": b, "t": t, "kv_h": h, "diff_count": int(diff[r]),
                                "parallel_only": _only_with_rank(a, b_),
                                "naive_only": _only_with_rank(b_, a)})
        if len(out_alarms) < max_report and bool(equal.any()):
            def group_out(tr):
                o = tr.layer_output.float().cpu()
                s = tr.layer_sum.float().cpu().clamp_min(1e-30)
                return (o / s[..., None]).reshape(B * T * Hkv, G, -1)
            err = (group_out(lp[l]) - group_out(ln[l])).abs().amax(dim=(1, 2))
            for r in torch.nonzero(equal & (err > layer_out_alarm_abs)).flatten().tolist():
                if len(out_alarms) >= max_report:
                    break
                b, rem = divmod(r, T * Hkv)
                t, h = divmod(rem, Hkv)
                out_alarms.append({"layer": l, "b": b, "t": t, "kv_h": h, "max_abs": float(err[r])})
        prev_equal = equal
    return {"topk_alarms": topk_alarms, "layer_output_alarms": out_alarms,
            "mismatch_counter": counter}
