"""Closed-form work model of the htree hot path (data independent).

For every query t the number of candidates, selected and evicted nodes per
level depends only on (t, CR, TK, MTN): the top level expands the virtual
parents 0..(t // CR^(L-1)) // CR (src/naive.py:108-118); each level keeps
min(TK, n_c) nodes (src/naive.py:97-101) and the rightmost child truncates
the last parent (src/naive.py:182-183).

Algorithmic bytes (the "gathered-bytes" roofline model; e = element bytes):
  fwd = sum_{b,h_kv,t} [ 2 G D e                 Q read + O write
                        + (sum_l nc_l) D e       K row of every scored candidate
                        + (nc_0 + sum_{l>=1} ev_l) D e ]   V row of every accumulated one
        + B H_kv 2 D e (T + sum_{l>=1} N_l)      tree build
  bwd = sum_{b,h_kv,t} [ 4 G D e + acc 2 D e ]   Q,O,dO read + dQ write; K,V of accumulated
        + B H_kv 2 D 4 sum_l N_l                 fp32 per-level dK/dV written once
        + B T H_kv 2 D e                         final dk, dv
MFMA flops: 2 G D per scored K row and per accumulated V row (forward);
5 x (2 G D) per accumulated candidate (backward).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List

import numpy as np


def level_sizes(T: int, CR: int, MTN: int) -> List[int]:
    sizes = [T]
    while sizes[-1] > MTN:
        sizes.append((sizes[-1] + CR - 1) // CR)
    return sizes


def counts(T: int, CR: int, TK: int, MTN: int) -> Dict[str, np.ndarray]:
    """Per-query arrays: nc[l] (scored), ev[l] (accumulated at upper levels),
    acc (accumulated over all levels)."""
    L = len(level_sizes(T, CR, MTN))
    t = np.arange(T, dtype=np.int64)
    nvp = (t // CR ** (L - 1)) // CR + 1
    nc = np.zeros((L, T), np.int64)
    ev = np.zeros((L, T), np.int64)
    for l in range(L - 1, -1, -1):
        nc[l] = (nvp - 1) * CR + (t // CR ** l) % CR + 1
        if l > 0:
            sel = np.minimum(TK, nc[l])
            ev[l] = nc[l] - sel
            nvp = sel
        else:
            ev[l] = nc[l]
    return dict(nc=nc, ev=ev, acc=ev.sum(0), L=L)


@dataclass
class Work:
    fwd_bytes: float
    fwd_kernel_bytes: float   # fwd minus the tree build
    tree_bytes: float
    bwd_bytes: float
    fwd_flops: float
    bwd_flops: float
    compulsory_fwd_bytes: float
    mean_k_rows: float
    mean_v_rows: float


def work(B: int, T: int, H: int, Hkv: int, D: int, CR: int, TK: int, MTN: int, e: int) -> Work:
    G = H // Hkv
    c = counts(T, CR, TK, MTN)
    sizes = level_sizes(T, CR, MTN)
    k_rows = c["nc"].sum(0).astype(np.float64)
    v_rows = c["acc"].astype(np.float64)
    per_group = 2 * G * D * e + (k_rows + v_rows) * D * e
    kern = B * Hkv * per_group.sum()
    tree = B * Hkv * 2 * D * e * (T + sum(sizes[1:]))
    bwd = (B * Hkv * (4 * G * D * e + v_rows * 2 * D * e).sum()
           + B * Hkv * 2 * D * 4 * sum(sizes) + B * T * Hkv * 2 * D * e)
    fwd_flops = B * Hkv * (2 * G * D * (k_rows + v_rows)).sum()
    bwd_flops = B * Hkv * (5 * 2 * G * D * v_rows).sum()
    compulsory = (2 * B * T * H * D * e) + B * Hkv * 2 * D * e * sum(sizes)
    return Work(fwd_bytes=float(kern + tree), fwd_kernel_bytes=float(kern), tree_bytes=float(tree),
                bwd_bytes=float(bwd), fwd_flops=float(fwd_flops), bwd_flops=float(bwd_flops),
                compulsory_fwd_bytes=float(compulsory), mean_k_rows=float(k_rows.mean()),
                mean_v_rows=float(v_rows.mean()))
