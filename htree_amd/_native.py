"""ctypes binding of libhtree_amd.so (the C ABI declared in include/htree.h).

The library is loaded after torch so that it binds to the HIP runtime torch
already loaded (both carry the SONAME libamdhip64.so.7): device pointers and
streams from torch are then valid inside the library.  There is no fallback:
a missing library raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded first, see module docstring)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhtree_amd.so")
MAX_LEVELS = 16

HTREE_OK = 0
HTREE_ENULL = -1
HTREE_ESHAPE = -2
HTREE_ECONFIG = -3
HTREE_EUNSUPPORTED = -4
HTREE_EWORKSPACE = -5
HTREE_ESCRATCH = -6

DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

# every function the header declares; tests check the library exports them
EXPORTS = (
    "htree_strerror", "htree_levels", "htree_tree_workspace_bytes", "htree_tree_build",
    "htree_forward", "htree_backward_workspace_bytes", "htree_backward_workspace_min_bytes",
    "htree_backward",
    "htree_train_scores_bytes", "htree_forward_train", "htree_backward_train",
    "htree_forward_trace", "htree_topk_rows", "htree_backward_noalloc_bytes",
    "htree_backward_noalloc", "htree_select",
)


class HtreeDims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "B", "T", "H", "H_kv", "D", "compression_rate", "top_k", "max_top_nodes", "dtype",
        "rope_rows", "kv_share", "grad_dtype", "group_pad")]


class HtreeError(RuntimeError):
    """A HIP error reported by the library (status > 0)."""


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m htree_amd.build` "
            "(the HIP path has no CPU fallback)")
    L = ctypes.CDLL(LIB_PATH)
    P, I32, I64, F = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    DP = ctypes.POINTER(HtreeDims)
    L.htree_strerror.restype = ctypes.c_char_p
    L.htree_strerror.argtypes = [ctypes.c_int]
    L.htree_levels.restype = ctypes.c_int
    L.htree_levels.argtypes = [DP, ctypes.POINTER(I32), ctypes.POINTER(I64)]
    L.htree_tree_workspace_bytes.restype = ctypes.c_int
    L.htree_tree_workspace_bytes.argtypes = [DP, ctypes.POINTER(I64)]
    L.htree_tree_build.restype = ctypes.c_int
    L.htree_tree_build.argtypes = [DP, P, P, ctypes.POINTER(P), ctypes.POINTER(P), P, P, P, I64, P]
    L.htree_forward.restype = ctypes.c_int
    L.htree_forward.argtypes = [DP, F, P, P, I64, P, P, P, P, P, P, P]
    if hasattr(L, "htree_forward_train"):
        L.htree_train_scores_bytes.restype = ctypes.c_int
        L.htree_train_scores_bytes.argtypes = [DP, ctypes.POINTER(I64)]
        L.htree_forward_train.restype = ctypes.c_int
        L.htree_forward_train.argtypes = [DP, F, P, P, I64, P, P, P, P, P, P, P, I64, P]
    if hasattr(L, "htree_forward_trace"):
        L.htree_forward_trace.restype = ctypes.c_int
        L.htree_forward_trace.argtypes = [DP, F, P, P, I64, P, P, P, P, P, P, P, P, P, P]
    if hasattr(L, "htree_select"):
        L.htree_select.restype = ctypes.c_int
        L.htree_select.argtypes = [DP, F, P, P, I64, P, P, P, P]
    if hasattr(L, "htree_topk_rows"):
        L.htree_topk_rows.restype = ctypes.c_int
        L.htree_topk_rows.argtypes = [P, I64, I32, I32, P, I32, P, P, P, P]
    if hasattr(L, "htree_backward"):
        L.htree_backward_workspace_bytes.restype = ctypes.c_int
        L.htree_backward_workspace_bytes.argtypes = [DP, ctypes.POINTER(I64)]
        L.htree_backward_workspace_min_bytes.restype = ctypes.c_int
        L.htree_backward_workspace_min_bytes.argtypes = [DP, ctypes.POINTER(I64)]
        L.htree_backward.restype = ctypes.c_int
        L.htree_backward.argtypes = [DP, F, P, P, P, P, P, P, P, I64, P, P, P, P, P, P, I64, P]
    if hasattr(L, "htree_backward_noalloc"):
        L.htree_backward_noalloc_bytes.restype = ctypes.c_int
        L.htree_backward_noalloc_bytes.argtypes = [DP, ctypes.POINTER(I64)]
        L.htree_backward_noalloc.restype = ctypes.c_int
        L.htree_backward_noalloc.argtypes = [DP, F, P, P, P, P, P, P, P, I64, P, P, P, I64, P, P,
                                             P, P]
    if hasattr(L, "htree_backward_train"):
        L.htree_backward_train.restype = ctypes.c_int
        L.htree_backward_train.argtypes = [DP, F, P, P, P, P, P, P, P, I64, P, P, P, I64, P, P, P,
                                           P, I64, P]
    _lib = L
    return L


def strerror(rc: int) -> str:
    return lib().htree_strerror(rc).decode()


def check(rc: int, what: str) -> None:
    """Maps a status to the reference's exception classes: configuration and
    shape errors are AssertionError (the reference validates with assert,
    src/parallel.py:907-925), HIP errors are HtreeError."""
    if rc == HTREE_OK:
        return
    msg = f"{what}: {strerror(rc)}"
    if rc < 0:
        raise AssertionError(msg)
    raise HtreeError(msg)


def dims(B, T, H, H_kv, D, compression_rate, top_k, max_top_nodes, dtype, rope_rows,
         kv_share=1, grad_dtype=None, group_pad=0) -> HtreeDims:
    """grad_dtype: dtype of the backward's dq, dk, dv (None: float32).
    group_pad: padding query heads at the end of every kv_share-th KV
    head's group (the forward leaves them out of the selection)."""
    for t in (dtype, grad_dtype):
        if t is not None and t not in DTYPE_CODE:
            raise AssertionError(f"unsupported dtype {t}: expected float32, bfloat16 or float16")
    return HtreeDims(B, T, H, H_kv, D, compression_rate, top_k, max_top_nodes,
                     DTYPE_CODE[dtype], rope_rows, kv_share,
                     DTYPE_CODE[grad_dtype] if grad_dtype is not None else 0, group_pad)


def with_grad_dtype(d: HtreeDims, grad_dtype) -> HtreeDims:
    """A copy of `d` whose backward writes dq, dk, dv in grad_dtype."""
    c = HtreeDims.from_buffer_copy(d)
    c.grad_dtype = DTYPE_CODE[grad_dtype]
    return c


def levels(d: HtreeDims):
    n = ctypes.c_int32()
    arr = (ctypes.c_int64 * MAX_LEVELS)()
    check(lib().htree_levels(ctypes.byref(d), ctypes.byref(n), arr), "htree_levels")
    return [int(arr[i]) for i in range(n.value)]


def tree_workspace_bytes(d: HtreeDims) -> int:
    b = ctypes.c_int64()
    check(lib().htree_tree_workspace_bytes(ctypes.byref(d), ctypes.byref(b)),
          "htree_tree_workspace_bytes")
    return int(b.value)


def train_scores_bytes(d: HtreeDims) -> int:
    """Bytes of the score buffer the training forward keeps for the backward
    (0: this configuration rebuilds the scores in the backward)."""
    if not hasattr(lib(), "htree_train_scores_bytes"):
        return 0
    b = ctypes.c_int64()
    check(lib().htree_train_scores_bytes(ctypes.byref(d), ctypes.byref(b)),
          "htree_train_scores_bytes")
    return int(b.value)


def ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def stream_ptr(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr_array(tensors):
    arr = (ctypes.c_void_p * MAX_LEVELS)()
    for i, t in enumerate(tensors):
        arr[i] = None if t is None else t.data_ptr()
    return arr
