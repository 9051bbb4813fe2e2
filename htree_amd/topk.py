"""Row-wise Top-K on the GPU with the forward's block-wide radix select
(htree_topk_rows of the C ABI): the micro-benchmark counterpart of
/root/reference/topk_test/benchmark.py.  The k largest of each row, ties to
the lower index (a stable descending sort), returned in ascending index
order, with optional int32 payloads (1 or 8 per element) carried along."""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _native as N


def topk_rows(x: torch.Tensor, k: int, payload: Optional[torch.Tensor] = None
              ) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """x [rows, n] fp32 (n <= 8192) -> values [rows, k], index [rows, k]
    int32 and, with payload [rows, n] or [rows, n, 8] int32, the selected
    payloads [rows, k] / [rows, k, 8]."""
    assert x.is_cuda and x.dtype == torch.float32 and x.dim() == 2, "x must be a [rows, n] fp32 GPU tensor"
    x = x.contiguous()
    rows, n = x.shape
    npay = 0
    if payload is not None:
        assert payload.dtype == torch.int32 and payload.shape[:2] == (rows, n), "payload [rows, n(, 8)] int32"
        npay = 1 if payload.dim() == 2 else payload.shape[2]
        payload = payload.contiguous()
    val = torch.empty(rows, k, dtype=torch.float32, device=x.device)
    idx = torch.empty(rows, k, dtype=torch.int32, device=x.device)
    pout = None
    if npay:
        pout = torch.empty((rows, k) if npay == 1 else (rows, k, npay), dtype=torch.int32,
                           device=x.device)
    with torch.cuda.device(x.device):
        rc = N.lib().htree_topk_rows(N.ptr(x), rows, n, k, N.ptr(payload), npay, N.ptr(val),
                                     N.ptr(idx), N.ptr(pout), N.stream_ptr(x.device))
    N.check(rc, "htree_topk_rows")
    return val, idx, pout
