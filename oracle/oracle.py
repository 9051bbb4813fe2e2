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
                       selection held fixed
  backward_dq_rows ... the full backward's dq at the same rows
  backward_rows ...... the full backward over all rows in order, bit for bit;
                       its row chunks add up to it
  backward_dkv_nodes . the full backward's per-level dK/dV at the same nodes
  final_dkv_level0 ... the full backward's final dk/dv (after the pooling
                       backward) at the same level-0 nodes
  forward(forced=) ... dense float64 softmax over the union of the candidates
                       that perturbed (teacher-forced) lists leave accumulated
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
        # common prefix: q, B, T, H, Hkv, D, DV, levels k / v, k / v level
        # offsets, level sizes, L, cos, sin, rope_rows, CR, TK, scale
        C = [P, I, I, I, I, I, I, P, P, P, P, P, I, P, P, I, I, I, F]
        L.orc_forward.argtypes = C + [P, I, P, P, P, P, P, P, P, P, P, P, P]
        L.orc_backward.restype = I
        L.orc_backward.argtypes = C + [P, P, P, P, P, P, P, P]
        L.orc_backward_dq_rows.restype = I
        L.orc_backward_dq_rows.argtypes = C + [P, I, P, P, P, P, P, P]
        L.orc_backward_rows.restype = I
        L.orc_backward_rows.argtypes = C + [P, I, P, P, P, P, P, P, P, P]
        L.orc_backward_dkv_nodes.restype = I
        L.orc_backward_dkv_nodes.argtypes = C + [P, P, P, P, P, P, I, P, P]
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
    DV = v.shape[3]
    sizes = level_sizes(T, compression_rate, max_top_nodes)
    lk, lv = [k], [v]
    for n in sizes[1:]:
        pk = np.empty((B, n, Hkv, D), np.float32)
        pv = np.empty((B, n, Hkv, DV), np.float32)
        lib().orc_tree_build_level(_ptr(lk[-1]), B, lk[-1].shape[1], Hkv, D,
                                   compression_rate, DTYPE_CODE[dtype], _ptr(pk))
        lib().orc_tree_build_level(_ptr(lv[-1]), B, lv[-1].shape[1], Hkv, DV,
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
    """Tree levels + RoPE tables shared by the forward/backward calls.  The
    key head dim D (q, k) and the value head dim DV (v) may differ
    (naive.py:144)."""

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
        self.DV = self.lv[0].shape[3]
        self.L = len(self.lk)
        self.rope_rows = rope_rows_needed(max_top_nodes, top_k, compression_rate)
        self.cos, self.sin = rope_tables(self.D, self.rope_rows, rope_base)
        self.kflat, self.off, self.n = _concat_levels(self.lk)
        self.vflat, self.voff, _ = _concat_levels(self.lv)

    def _common(self, q):
        B, T, H, D = q.shape
        assert D == self.D, f"q head dim {D} != k head dim {self.D}"
        return [_ptr(q), B, T, H, self.Hkv, D, self.DV, _ptr(self.kflat), _ptr(self.vflat),
                _ptr(self.off), _ptr(self.voff), _ptr(self.n), self.L, _ptr(self.cos),
                _ptr(self.sin), self.rope_rows, self.CR, self.TK]


def all_rows(B: int, T: int) -> np.ndarray:
    return np.stack(np.meshgrid(np.arange(B), np.arange(T), indexing="ij"), -1).reshape(-1, 2).astype(np.int32)


def forward(q, tree: Tree, scale: float, rows: Optional[np.ndarray] = None,
            forced: Optional[np.ndarray] = None, trace: bool = False) -> Dict[str, np.ndarray]:
    """htree forward for query rows `rows` ([n,2] of (b,t); default all).

    forced: [L, n, Hkv, TK] parent lists to use (teacher forcing).
    Returns out (rounded to the dtype), out_f32, gmax, gsum, parents [L,n,Hkv,TK]
    (list used per level), sel (own Top-K per level), imp, imparg (per
    position, the largest exponent argument max_g (s_gj - m) of its
    importance), and the per-level trace lmax/lsum/lout when trace=True."""
    q = _f32(q)
    B, T, H, D = q.shape
    if rows is None:
        rows = all_rows(B, T)
    rows = np.ascontiguousarray(rows, np.int32)
    n = rows.shape[0]
    L, Hkv, TK, CR, DV = tree.L, tree.Hkv, tree.TK, tree.CR, tree.DV
    out = np.zeros((n, H, DV), np.float32)
    gmax = np.zeros((n, H), np.float32)
    gsum = np.zeros((n, H), np.float32)
    par = np.full((L, n, Hkv, TK), -1, np.int32)
    sel = np.full((L, n, Hkv, TK), -1, np.int32)
    imp = np.full((L, n, Hkv, TK * CR), -1.0, np.float32)
    imparg = np.full((L, n, Hkv, TK * CR), -1e30, np.float32)
    lmax = lsum = lout = None
    if trace:
        lmax = np.zeros((L, n, H), np.float32)
        lsum = np.zeros((L, n, H), np.float32)
        lout = np.zeros((L, n, H, DV), np.float32)
    if forced is not None:
        forced = np.ascontiguousarray(forced, np.int32)
        assert forced.shape == (L, n, Hkv, TK)
    rc = lib().orc_forward(*tree._common(q), ctypes.c_float(scale), _ptr(rows), n,
                           _ptr(forced), _ptr(out), _ptr(gmax), _ptr(gsum), _ptr(par),
                           _ptr(sel), _ptr(imp), _ptr(lmax), _ptr(lsum), _ptr(lout),
                           _ptr(imparg))
    _check(rc, "oracle forward")
    res = dict(out_f32=out, out=round_to(out, tree.dtype), gmax=gmax, gsum=gsum,
               parents=par, sel=sel, imp=imp, imparg=imparg, rows=rows)
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
    lib().orc_tree_backward(_ptr(dv_fin), B, tree.Hkv, tree.DV, _ptr(tree.voff), _ptr(tree.n), tree.L,
                            tree.CR)
    split = lambda flat, lv, off: [flat[off[i]:off[i] + lv[i].size].reshape(lv[i].shape)
                                   for i in range(tree.L)]
    return dict(dq=dq, dk_levels=split(dk_lv, tree.lk, tree.off),
                dv_levels=split(dv_lv, tree.lv, tree.voff),
                dk=split(dk_fin, tree.lk, tree.off)[0].copy(),
                dv=split(dv_fin, tree.lv, tree.voff)[0].copy())


def delta(out, dO) -> np.ndarray:
    out, dO = _f32(out), _f32(dO)
    D = out.shape[-1]  # the value head dim
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


def backward_rows(q, tree: Tree, scale: float, rows, parents_rows, gmax_rows, gsum_rows,
                  delta_rows, dO_rows, with_dkv: bool = True):
    """The full backward restricted to a subset of rows (naive.py:320-386
    for those rows): dq [n,H,D] of the rows and, with `with_dkv`, the
    per-level dK / dV (before the mean-pool backward, levels concatenated
    like the tree's) that the rows' accumulated candidates receive.  The
    scatter runs either way; without `with_dkv` its result is dropped.
    Row inputs as backward_dq_rows.  Returns (dq, dk_lv | None, dv_lv | None)."""
    q = _f32(q)
    B, T, H, D = q.shape
    rows = np.ascontiguousarray(rows, np.int32)
    n = rows.shape[0]
    args = [np.ascontiguousarray(parents_rows, np.int32), _f32(gmax_rows), _f32(gsum_rows),
            _f32(delta_rows), _f32(dO_rows)]
    dq = np.zeros((n, H, D), np.float32)
    dk = np.zeros_like(tree.kflat) if with_dkv else None
    dv = np.zeros_like(tree.vflat) if with_dkv else None
    rc = lib().orc_backward_rows(*tree._common(q), ctypes.c_float(scale), _ptr(rows), n,
                                 *[_ptr(a) for a in args], _ptr(dq), _ptr(dk), _ptr(dv))
    _check(rc, "oracle backward rows")
    return dq, dk, dv


def backward_dkv_nodes(q, tree: Tree, scale: float, parents, gmax, gsum, delta_, dO,
                       targets, threads: int = 0) -> Tuple[np.ndarray, np.ndarray]:
    """Per-level dK/dV (before the mean-pool backward) at listed nodes.

    targets [n, 4] of (level, b, h_kv, node).  Each node's contribution is
    computed from its own score in every query group that accumulates it
    (naive.py:365-386 restricted to one node), so the cost is one scan of the
    parent lists plus O(G*D) per accumulating query: usable at full workload
    sizes.  parents [L,B,T,Hkv,TK]; gmax, gsum, delta_ [B,T,H]; dO [B,T,H,D].
    The targets are split over `threads` host threads (0: all cores)."""
    from concurrent.futures import ThreadPoolExecutor

    q = _f32(q)
    D = q.shape[-1]
    targets = np.ascontiguousarray(targets, np.int32).reshape(-1, 4)
    n = targets.shape[0]
    dk = np.zeros((n, D), np.float32)
    dv = np.zeros((n, tree.DV), np.float32)
    args = [np.ascontiguousarray(parents, np.int32), _f32(gmax), _f32(gsum), _f32(delta_), _f32(dO)]
    common = tree._common(q)
    nt = max(1, min(n, threads or min(16, os.cpu_count() or 1)))
    cuts = np.linspace(0, n, nt + 1).astype(int)

    def part(i):
        a, b = cuts[i], cuts[i + 1]
        if a == b:
            return 0
        return lib().orc_backward_dkv_nodes(*common, ctypes.c_float(scale), *[_ptr(x) for x in args],
                                            _ptr(targets[a:]), int(b - a), _ptr(dk[a:]), _ptr(dv[a:]))

    lib()
    with ThreadPoolExecutor(nt) as ex:
        for rc in ex.map(part, range(nt)):
            _check(rc, "oracle dkv nodes")
    return dk, dv


def level0_ancestors(tree: Tree, node: int) -> List[Tuple[int, int, int]]:
    """(level, ancestor, children of that ancestor) for level-0 `node`, level
    1 upwards: the factors of the mean-pool backward (naive.py:388-394)."""
    out = []
    a = node
    for l in range(1, tree.L):
        a //= tree.CR
        cnt = min(tree.CR, int(tree.n[l - 1]) - a * tree.CR)
        out.append((l, a, cnt))
    return out


def final_dkv_level0(q, tree: Tree, scale: float, parents, gmax, gsum, delta_, dO, nodes_bhn,
                     threads: int = 0) -> Tuple[np.ndarray, np.ndarray]:
    """Final dk / dv (after the mean-pool backward, naive.py:388-394) at
    level-0 nodes nodes_bhn [n, 3] of (b, h_kv, node), from the per-level
    terms of every ancestor: g_0[x] = dK_0[x] + g_1[x/CR] / |Ch(x/CR)|,
    g_l[p] = dK_l[p] + g_{l+1}[p/CR] / |Ch(p/CR)|.  Returns float64 [n, D]."""
    nodes_bhn = np.asarray(nodes_bhn, np.int64).reshape(-1, 3)
    want = {}
    for b, h, x in nodes_bhn:
        want[(0, b, h, x)] = None
        for l, a, _ in level0_ancestors(tree, int(x)):
            want[(l, b, h, a)] = None
    keys = list(want)
    dk, dv = backward_dkv_nodes(q, tree, scale, parents, gmax, gsum, delta_, dO,
                                np.array(keys, np.int32), threads)
    term = {key: (dk[i].astype(np.float64), dv[i].astype(np.float64)) for i, key in enumerate(keys)}
    D, DV = dk.shape[1], dv.shape[1]
    rk = np.zeros((len(nodes_bhn), D))
    rv = np.zeros((len(nodes_bhn), DV))
    for i, (b, h, x) in enumerate(nodes_bhn):
        anc = level0_ancestors(tree, int(x))
        gk, gv = np.zeros(D), np.zeros(DV)
        for (l, a, cnt) in reversed(anc):  # top-down
            gk = (gk + term[(l, b, h, a)][0]) / cnt
            gv = (gv + term[(l, b, h, a)][1]) / cnt
        rk[i] = gk + term[(0, b, h, x)][0]
        rv[i] = gv + term[(0, b, h, x)][1]
    return rk, rv


def split_rows(rows: np.ndarray, parts: int) -> List[np.ndarray]:
    cuts = np.linspace(0, len(rows), max(1, parts) + 1).astype(int)
    return [rows[a:b] for a, b in zip(cuts[:-1], cuts[1:]) if b > a]


def forward_threaded(q, tree: Tree, scale: float, threads: int, rows: Optional[np.ndarray] = None):
    """forward() over row chunks on `threads` host threads (the C calls
    release the GIL); out, out_f32, gmax, gsum, parents for `rows` in order."""
    from concurrent.futures import ThreadPoolExecutor

    q = _f32(q)
    if rows is None:
        rows = all_rows(q.shape[0], q.shape[1])
    chunks = split_rows(np.ascontiguousarray(rows, np.int32), threads)
    with ThreadPoolExecutor(len(chunks)) as ex:
        parts = list(ex.map(lambda r: forward(q, tree, scale, rows=r), chunks))
    cat = lambda key, ax=0: np.concatenate([p[key] for p in parts], ax)
    return dict(out=cat("out"), out_f32=cat("out_f32"), gmax=cat("gmax"), gsum=cat("gsum"),
                parents=cat("parents", 1), rows=rows)


def backward_threaded(q, tree: Tree, scale: float, parents, gmax, gsum, out, dO, threads: int):
    """The full backward (as backward()) on `threads` host threads: dq by row
    chunks (backward_dq_rows), every level's dK / dV by node chunks
    (backward_dkv_nodes), then the mean-pool backward (naive.py:388-394).
    Returns dq, dk, dv (final, level 0)."""
    from concurrent.futures import ThreadPoolExecutor

    q = _f32(q)
    B, T, H, D = q.shape
    parents = np.ascontiguousarray(parents, np.int32)
    gmax, gsum, out, dO = _f32(gmax), _f32(gsum), _f32(out), _f32(dO)
    dl = delta(out, dO)
    rows = all_rows(B, T)
    chunks = split_rows(rows, threads)

    def dq_part(r):
        b, t = r[:, 0], r[:, 1]
        return backward_dq_rows(q, tree, scale, r, parents[:, b, t], gmax[b, t], gsum[b, t], dl[b, t],
                                dO[b, t])

    with ThreadPoolExecutor(len(chunks)) as ex:
        dq = np.concatenate(list(ex.map(dq_part, chunks))).reshape(B, T, H, D)
    tg = np.array([(l, b, h, x) for l in range(tree.L) for b in range(B) for h in range(tree.Hkv)
                   for x in range(int(tree.n[l]))], np.int32)
    dk_n, dv_n = backward_dkv_nodes(q, tree, scale, parents, gmax, gsum, dl, dO, tg, threads)
    dk_lv = np.zeros_like(tree.kflat)
    dv_lv = np.zeros_like(tree.vflat)
    for i, (l, b, h, x) in enumerate(tg):
        dk_lv[tree.off[l] + ((b * tree.n[l] + x) * tree.Hkv + h) * D:][:D] = dk_n[i]
        dv_lv[tree.voff[l] + ((b * tree.n[l] + x) * tree.Hkv + h) * tree.DV:][:tree.DV] = dv_n[i]
    lib().orc_tree_backward(_ptr(dk_lv), B, tree.Hkv, D, _ptr(tree.off), _ptr(tree.n), tree.L, tree.CR)
    lib().orc_tree_backward(_ptr(dv_lv), B, tree.Hkv, tree.DV, _ptr(tree.voff), _ptr(tree.n), tree.L,
                            tree.CR)
    dk = dk_lv[:tree.lk[0].size].reshape(tree.lk[0].shape)
    dv = dv_lv[:tree.lv[0].size].reshape(tree.lv[0].shape)
    return dq, dk, dv


def initial_parents(B: int, T: int, Hkv: int, TK: int, CR: int, L: int) -> np.ndarray:
    """naive.py:108-118"""
    tlp = CR ** (L - 1)
    t = np.arange(T)
    nvp = t // tlp // CR + 1
    pc = np.arange(TK)[None, :]
    prev = np.where(pc < nvp[:, None], pc, -1).astype(np.int32)
    return np.ascontiguousarray(np.broadcast_to(prev[None, :, None, :], (B, T, Hkv, TK)))
