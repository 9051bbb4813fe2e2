"""Host logic of the trace harness: compare_traces (the methodology of
correctness_test.py:394-466) on hand-built traces with planted differences
(known answers), and against a per-row loop over random traces."""
import numpy as np
import torch

from htree_amd.trace import LayerTrace, compare_traces


def _trace(par, lmax, lsum, lout, G):
    L = len(lmax)
    return {"num_layers": L, "num_groups": G, "layers": {
        l: LayerTrace(l, None if l == 0 else torch.tensor(par[l], dtype=torch.int32),
                      torch.tensor(lmax[l]), torch.tensor(lsum[l]), torch.tensor(lout[l]))
        for l in range(L)}}


def _base(B=1, T=3, Hkv=2, TK=4, G=2, D=2, L=3):
    H = Hkv * G
    par = {l: np.tile(np.array([0, 1, 2, -1], np.int32)[:TK], (B, T, Hkv, 1)) for l in range(1, L)}
    lmax = [np.zeros((B, T, H), np.float32) for _ in range(L)]
    lsum = [np.ones((B, T, H), np.float32) for _ in range(L)]
    lout = [np.full((B, T, H, D), 0.25, np.float32) for _ in range(L)]
    return par, lmax, lsum, lout


def test_compare_traces_known_answers():
    p_par, p_max, p_sum, p_out = _base()
    n_par, n_max, n_sum, n_out = _base()
    # level 2, (t=1, h_kv=0): node 2 vs node 3 -> difference 2, alarm
    n_par[2][0, 1, 0] = [0, 1, 3, -1]
    # level 1, same row differs too ({1,2} vs {4,5}: difference 4), but
    # level 2 already differed -> no alarm
    n_par[1][0, 1, 0] = [0, 4, 5, -1]
    # level 1, (t=2, h_kv=1): one extra node on the naive side -> difference 1
    p_par[1][0, 2, 1] = [5, 6, -1, -1]
    n_par[1][0, 2, 1] = [5, 6, 7, -1]
    # level 2 output: head 1 of group (t=0, h_kv=1) = head 3, off by 0.5 -> alarm
    p_out[2][0, 0, 3, 1] += 0.5
    # differences where the selection differs, or below the bar: no alarm
    p_out[2][0, 1, 0, 0] += 5.0
    p_out[1][0, 0, 0, 0] += 1e-4
    # the bottom level is never compared
    p_out[0][0, 0, 0, 0] += 9.0
    rep = compare_traces(_trace(p_par, p_max, p_sum, p_out, 2), _trace(n_par, n_max, n_sum, n_out, 2),
                         topk_alarm_diff=0, layer_out_alarm_abs=1e-3, max_report=10)
    assert rep["topk_alarms"] == [
        {"layer": 2, "b": 0, "t": 1, "kv_h": 0, "diff_count": 2,
         "parallel_only": [{"node": 2, "rank": 3}], "naive_only": [{"node": 3, "rank": 3}]},
        {"layer": 1, "b": 0, "t": 2, "kv_h": 1, "diff_count": 1,
         "parallel_only": [], "naive_only": [{"node": 7, "rank": 3}]},
    ]
    assert len(rep["layer_output_alarms"]) == 1
    a = rep["layer_output_alarms"][0]
    assert (a["layer"], a["b"], a["t"], a["kv_h"]) == (2, 0, 0, 1)
    assert abs(a["max_abs"] - 0.5) < 1e-6
    assert rep["mismatch_counter"] == {0: 9, 2: 1, 4: 1, 1: 1}
    # threshold on the difference size and the report cap
    rep = compare_traces(_trace(p_par, p_max, p_sum, p_out, 2), _trace(n_par, n_max, n_sum, n_out, 2),
                         topk_alarm_diff=1, layer_out_alarm_abs=1e-3, max_report=1)
    assert [x["layer"] for x in rep["topk_alarms"]] == [2]


def _loop_compare(pt, nt, diff_thr, out_thr):
    """Per-row restatement with Python sets (the reference's loop structure)."""
    L, G = pt["num_layers"], pt["num_groups"]
    B, T, Hkv, TK = pt["layers"][L - 1].selected_parents.shape
    prev = np.ones((B, T, Hkv), bool)
    topk, outs, counter = [], [], {}
    for l in range(L - 1, 0, -1):
        cur = np.zeros((B, T, Hkv), bool)
        for b in range(B):
            for t in range(T):
                for h in range(Hkv):
                    A = set(x for x in pt["layers"][l].selected_parents[b, t, h].tolist() if x >= 0)
                    Bs = set(x for x in nt["layers"][l].selected_parents[b, t, h].tolist() if x >= 0)
                    d = len(A ^ Bs)
                    counter[d] = counter.get(d, 0) + 1
                    cur[b, t, h] = d == 0
                    if prev[b, t, h] and d > diff_thr:
                        topk.append((l, b, t, h, d))
                    if d == 0:
                        hs = slice(h * G, h * G + G)
                        po = pt["layers"][l].layer_output[b, t, hs] / pt["layers"][l].layer_sum[b, t, hs].clamp_min(1e-30)[:, None]
                        no = nt["layers"][l].layer_output[b, t, hs] / nt["layers"][l].layer_sum[b, t, hs].clamp_min(1e-30)[:, None]
                        m = (po - no).abs().max().item()
                        if m > out_thr:
                            outs.append((l, b, t, h))
        prev = cur
    return topk, outs, counter


def test_compare_traces_matches_row_loop():
    rng = np.random.default_rng(5)
    B, T, Hkv, TK, G, D, L = 2, 40, 2, 8, 3, 4, 4
    H = Hkv * G

    def lists():
        out = np.full((B, T, Hkv, TK), -1, np.int32)
        for idx in np.ndindex(B, T, Hkv):
            n = rng.integers(1, TK + 1)
            out[idx][:n] = np.sort(rng.choice(20, n, replace=False))
        return out

    p_par = {l: lists() for l in range(1, L)}
    n_par = {l: p_par[l].copy() for l in range(1, L)}
    for l in range(1, L):
        flip = rng.random((B, T, Hkv)) < 0.2
        n_par[l][flip] = lists()[flip]
    p_max = [rng.standard_normal((B, T, H)).astype(np.float32) for _ in range(L)]
    p_sum = [rng.uniform(1, 3, (B, T, H)).astype(np.float32) for _ in range(L)]
    p_out = [rng.standard_normal((B, T, H, D)).astype(np.float32) for _ in range(L)]
    n_out = [x + (rng.random(x.shape) < 0.05) * 0.1 for x in p_out]
    pt = _trace(p_par, p_max, p_sum, p_out, G)
    nt = _trace(n_par, p_max, p_sum, [x.astype(np.float32) for x in n_out], G)
    rep = compare_traces(pt, nt, topk_alarm_diff=1, layer_out_alarm_abs=0.01, max_report=10 ** 6)
    topk, outs, counter = _loop_compare(pt, nt, 1, 0.01)
    assert [(a["layer"], a["b"], a["t"], a["kv_h"], a["diff_count"]) for a in rep["topk_alarms"]] == topk
    assert [(a["layer"], a["b"], a["t"], a["kv_h"]) for a in rep["layer_output_alarms"]] == outs
    assert rep["mismatch_counter"] == counter
    assert len(topk) > 0 and len(outs) > 0
