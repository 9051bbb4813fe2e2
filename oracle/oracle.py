"""CPU oracle for the htree hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, and only as the checker.  The product (htree_amd/) never imports it.

Python face of oracle/htree_oracle.c, a restatement of the reference's
src/naive.py (see the C file's header for the line-by-line map).  Arrays are
numpy float32 holding values exactly representable in the input dtype.

Pinning (what each function is checked against, see tests/test_oracle_*.py):
  build_tree ......... brute-force mean in float64 + dtype rounding; golden
                       fixtures from the reference's naive.py
  rope_tables ........ closed form cos/sin(p * base^(-2i/D)) in float64
  forward ............ golden fixtures (naive.py outputs, per-level parents);
                       dense float64 softmax over the union of accumulated
                       candidates; brute-force stable Top-K in float64;
                       closed-form candidate counts
  backward ........... golden fixtures (naive.py HTreeFunction grads);
                       torch float64 autograd of the dense form with the
                       selection held fixed; finite differences
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

DTYPE_CODE = {"float32": 0, "bfloat16": 1, "float16": 2}
NEG_INF = -1.0e10  # naive.py:9


def build(force: bool = False) -> str:
    """Compile liboracle.so from htree_oracle.c with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH) or (
        os.path.getmtime(_LIB_PATH) < os.path.getmtime(os.path.join(_HERE, "htree_oracle.c"))
    ):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "liboracle.so"],
                       check=True, capture_output=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int
        F = ctypes.c_float
        I64 = ctypes.c_int64
        L.orc_round_bf16.restype = F
        L.orc_round_bf16.argtypes = [F]
        L.orc_round_f16.restype = F
        L.orc_round_f16.argtypes = [F]
        L.orc_round_array.argtypes = [P, I64, I]
        L.orc_tree_build_level.argtypes = [P, I, I, I, I, I, I, P]
        L.orc_forward.restype = I
        L.orc_forward.argtypes = [P, I, I, I, I, I, P, P, P, P, I, P, P, I, I, I, F,
                                  P, I, P, P, P, P, P, P, P, P, P, P]
        L.orc_backward.restype = I
        L.orc_backward.argtypes = [P, I, I, I, I, I, P, P, P, P, I, P, P, I, I, I, F,
                                   P, P, P, P, P, P, P, P]
        L.orc_backward_dq_rows.restype = I
        L.orc_backward_dq_rows.argtypes = [P, I, I, I, I, I, P, P, P, P, I, P, P, I, I, I, F,
                                           P, I, P, P, P, P, P, P]
        L.orc_backward_dkv_nodes.restype = I
        L.orc_backward_dkv_nodes.argtypes = [P, I, I, I, I, I, P, P, P, P, I, P, P, I, I, I, F,
                                             P, P, P, P, P, I, P, I, P, P]
        L.orc_delta.argtypes = [P, P, I64, I, P]
        L.orc_tree_backward.argtypes = [P, I, I, I, P, P, I, I]
        _lib = L
    return _lib


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    if hasattr(a, "detach"):
        a = a.detach().cpu().float().numpy()
    return np.ascontiguousarray(a, dtype=np.float32)


def _check(rc: int, what: str) -> None:
    if rc == -1:
        raise RuntimeError(f"{what}: No valid parents")  # naive.py:185-186
    if rc == -2:
        raise IndexError(f"{what}: candidate node index out of range")
    if rc != 0:
        raise RuntimeError(f"{what}: oracle error {rc}")


# ---------------------------------------------------------------- structure
def level_sizes(T: int, compression_rate: int, max_top_nodes: int) -> List[int]:
    """N_0 = T; N_{l+1} = ceil(N_l / CR) while N_l > MTN (naive.py:49-50)."""
    sizes = [T]
    while sizes[-1] > max_top_nodes:
        sizes.append((sizes[-1] + compression_rate - 1) // compression_rate)
    return sizes


def candidate_counts(t: int, CR: int, TK: int, L: int) -> Dict[int, Tuple[int, int, int]]:
    """Closed-form (nc, selected, evicted) per level for query t: the counts
    depend only on t and the configuration, never on the data."""
    out = {}
    nvp = (t // CR ** (L - 1)) // CR + 1
    for l in range(L - 1, -1, -1):
        nc = (nvp - 1) * CR + (t // CR ** l) % CR + 1
        if l > 0:
            sel = min(TK, nc)
            out[l] = (nc, sel, nc - sel)
            nvp = sel
        else:
            out[l] = (nc, 0, nc)
    return out


def rope_tables(D: int, rows: int, rope_base: float) -> Tuple[np.ndarray, np.ndarray]:
    """cos/sin tables [rows, D/2] fp32, built with the reference's torch recipe
    (naive.py:63-70, parallel.py:983-988) on the CPU."""
    import torch

    inv_freq = 1.0 / (rope_base ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    pos = torch.arange(rows, dtype=torch.float32)
    freqs = torch.outer(pos, inv_freq)
    return freqs.cos().numpy().copy(), freqs.sin().numpy().copy()


def rope_rows_needed(max_top_nodes: int, top_k: int, compression_rate: int) -> int:
    return max(max_top_nodes + 1024, top_k * compression_rate)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().orc_round_array(_ptr(x), x.size, DTYPE_CODE[dtype])
    return x


def build_tree(k: np.ndarray, v: np.ndarray, compression_rate: int, max_top_nodes: int,
               dtype: str) -> Tuple[List[np.ndarray], List[np.ndarray]]:
    k = _f32(k)
    v = _f32(v)
    B, T, Hkv, D = k.shape
    sizes = level_sizes(T, compression_rate, max_top_nodes)
    lk, lv = [k], [v]
    for n in sizes[1:]:
        pk = np.empty((B, n, Hkv, D), np.float32)
        pv = np.empty((B, n, Hkv, D), np.float32)
        lib().orc_tree_build_level(_ptr(lk[-1]), B, lk[-1].shape[1], Hkv, D,
                                   compression_rate, DTYPE_CODE[dtype], _ptr(pk))
        lib().orc_tree_build_level(_ptr(lv[-1]), B, lv[-1].shape[1], Hkv, D,
                                   compression_rate, DTYPE_CODE[dtype], _ptr(pv))
        lk.append(pk)
        lv.append(pv)
    return lk, lv


def _concat_levels(levels: Sequence[np.ndarray]):
    flat = np.concatenate([np.ascontiguousarray(x, np.float32).ravel() for x in levels])
    off = np.zeros(len(levels), np.int64)
    acc = 0
    for i, x in enumerate(levels):
        off[i] = acc
        acc += x.size
    n = np.array([x.shape[1] for x in levels], np.int32)
    return flat, off, n


class Tree:
    """Tree levels + RoPE tables shared by the forward/backward calls."""

    def __init__(self, k, v, compression_rate: int, max_top_nodes: int, top_k: int,
                 dtype: str, rope_base: float = 10000.0, levels=None):
        if levels is None:
            self.lk, self.lv = build_tree(k, v, compression_rate, max_top_nodes, dtype)
        else:
            self.lk, self.lv = [_f32(x) for x in levels[0]], [_f32(x) for x in levels[1]]
        self.CR = compression_rate
        self.MTN = max_top_nodes
        self.TK = top_k
        self.dtype = dtype
        self.B, self.T, self.Hkv, self.D = self.lk[0].shape
        self.L = len(self.lk)
        self.rope_rows = rope_rows_needed(max_top_nodes, top_k, compression_rate)
        self.cos, self.sin = rope_tables(self.D, self.rope_rows, rope_base)
        self.kflat, self.off, self.n = _concat_levels(self.lk)
        self.vflat, _, _ = _concat_levels(self.lv)

    def _common(self, q):
        B, T, H, D = q.shape
        return [_ptr(q), B, T, H, self.Hkv, D, _ptr(self.kflat), _ptr(self.vflat),
                _ptr(self.off), _ptr(self.n), self.L, _ptr(self.cos), _ptr(self.sin),
                self.rope_rows, self.CR, self.TK]


def all_rows(B: int, T: int) -> np.ndarray:
    return np.stack(np.meshgrid(np.arange(B), np.arange(T), indexing="ij"), -1).reshape(-1, 2).astype(np.int32)


def forward(q, tree: Tree, scale: float, rows: Optional[np.ndarray] = None,
            forced: Optional[np.ndarray] = None, trace: bool = False) -> Dict[str, np.ndarray]:
    """htree forward for query rows `rows` ([n,2] of (b,t); default all).

    forced: [L, n, Hkv, TK] parent lists to use (teacher forcing).
    Returns out (rounded to the dtype), out_f32, gmax, gsum, parents [L,n,Hkv,TK]
    (list used per level), sel (own Top-K per level), imp, and the per-level
    trace lmax/lsum/lout when trace=True."""
    q = _f32(q)
    B, T, H, D = q.shape
    if rows is None:
        rows = all_rows(B, T)
    rows = np.ascontiguousarray(rows, np.int32)
    n = rows.shape[0]
    L, Hkv, TK, CR = tree.L, tree.Hkv, tree.TK, tree.CR
    out = np.zeros((n, H, D), np.float32)
    gmax = np.zeros((n, H), np.float32)
    gsum = np.zeros((n, H), np.float32)
    par = np.full((L, n, Hkv, TK), -1, np.int32)
    sel = np.full((L, n, Hkv, TK), -1, np.int32)
    imp = np.full((L, n, Hkv, TK * CR), -1.0, np.float32)
    lmax = lsum = lout = None
    if trace:
        lmax = np.zeros((L, n, H), np.float32)
        lsum = np.zeros((L, n, H), np.float32)
        lout = np.zeros((L, n, H, D), np.float32)
    if forced is not None:
        forced = np.ascontiguousarray(forced, np.int32)
        assert forced.shape == (L, n, Hkv, TK)
    rc = lib().orc_forward(*tree._common(q), ctypes.c_float(scale), _ptr(rows), n,
                           _ptr(forced), _ptr(out), _ptr(gmax), _ptr(gsum), _ptr(par),
                           _ptr(sel), _ptr(imp), _ptr(lmax), _ptr(lsum), _ptr(lout))
    _check(rc, "oracle forward")
    res = dict(out_f32=out, out=round_to(out, tree.dtype), gmax=gmax, gsum=gsum,
               parents=par, sel=sel, imp=imp, rows=rows)
    if trace:
        res.update(lmax=lmax, lsum=lsum, lout=lout)
    return res


def backward(q, tree: Tree, scale: float, parents: np.ndarray, gmax, gsum, out, dO):
    """Full analytical backward (naive.py:320-396) with the given per-level
    parent lists parents [L,B,T,Hkv,TK].  Returns dq, dk_levels, dv_levels
    (per level, before the mean-pool backward), dk, dv (final)."""
    q = _f32(q)
    B, T, H, D = q.shape
    parents = np.ascontiguousarray(parents, np.int32)
    gmax, gsum, out, dO = _f32(gmax), _f32(gsum), _f32(out), _f32(dO)
    dq = np.zeros_like(q)
    dk_lv = np.zeros_like(tree.kflat)
    dv_lv = np.zeros_like(tree.vflat)
    rc = lib().orc_backward(*tree._common(q), ctypes.c_float(scale), _ptr(parents),
                            _ptr(gmax), _ptr(gsum), _ptr(out), _ptr(dO), _ptr(dq),
                            _ptr(dk_lv), _ptr(dv_lv))
    _check(rc, "oracle backward")
    dk_fin = dk_lv.copy()
    dv_fin = dv_lv.copy()
    lib().orc_tree_backward(_ptr(dk_fin), B, tree.Hkv, D, _ptr(tree.off), _ptr(tree.n), tree.L, tree.CR)
    lib().orc_tree_backward(_ptr(dv_fin), B, tree.Hkv, D, _ptr(tree.off), _ptr(tree.n), tree.L, tree.CR)
    split = lambda flat: [flat[tree.off[i]:tree.off[i] + tree.lk[i].size].reshape(tree.lk[i].shape)
                          for i in range(tree.L)]
    return dict(dq=dq, dk_levels=split(dk_lv), dv_levels=split(dv_lv),
                dk=split(dk_fin)[0].copy(), dv=split(dv_fin)[0].copy())


def delta(out, dO) -> np.ndarray:
    out, dO = _f32(out), _f32(dO)
    D = out.shape[-1]
    res = np.zeros(out.shape[:-1], np.float32)
    lib().orc_delta(_ptr(out), _ptr(dO), res.size, D, _ptr(res))
    return res


def backward_dq_rows(q, tree: Tree, scale: float, rows, parents_rows, gmax_rows, gsum_rows,
                     delta_rows, dO_rows) -> np.ndarray:
    """dq for a subset of rows (needs only those rows' state)."""
    q = _f32(q)
    B, T, H, D = q.shape
    rows = np.ascontiguousarray(rows, np.int32)
    n = rows.shape[0]
    args = [np.ascontiguousarray(parents_rows, np.int32), _f32(gmax_rows), _f32(gsum_rows),
            _f32(delta_rows), _f32(dO_rows)]
    dq = np.zeros((n, H, D), np.float32)
    rc = lib().orc_backward_dq_rows(*tree._common(q), ctypes.c_float(scale), _ptr(rows), n,
                                    *[_ptr(a) for a in args], _ptr(dq))
    _check(rc, "oracle dq rows")
    return dq


def backward_dkv_nodes(q, tree: Tree, scale: float, parents, gmax, gsum, delta_, dO,
                       level: int, nodes_bhn) -> Tuple[np.ndarray, np.ndarray]:
    """Per-level dK/dV (before the mean-pool backward) for listed (b,h_kv,node)."""
    q = _f32(q)
    nodes_bhn = np.ascontiguousarray(nodes_bhn, np.int32)
    n = nodes_bhn.shape[0]
    D = q.shape[-1]
    dk = np.zeros((n, D), np.float32)
    dv = np.zeros((n, D), np.float32)
    args = [np.ascontiguousarray(parents, np.int32), _f32(gmax), _f32(gsum), _f32(delta_), _f32(dO)]
    rc = lib().orc_backward_dkv_nodes(*tree._common(q), ctypes.c_float(scale),
                                      *[_ptr(a) for a in args], level, _ptr(nodes_bhn), n,
                                      _ptr(dk), _ptr(dv))
    _check(rc, "oracle dkv nodes")
    return dk, dv


def initial_parents(B: int, T: int, Hkv: int, TK: int, CR: int, L: int) -> np.ndarray:
    """naive.py:108-118"""
    tlp = CR ** (L - 1)
    t = np.arange(T)
    nvp = t // tlp // CR + 1
    pc = np.arange(TK)[None, :]
    prev = np.where(pc < nvp[:, None], pc, -1).astype(np.int32)
    return np.ascontiguousarray(np.broadcast_to(prev[None, :, None, :], (B, T, Hkv, TK)))
