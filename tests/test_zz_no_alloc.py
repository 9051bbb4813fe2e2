"""htree_backward_noalloc: the backward entry point that allocates nothing
(its workspace is a file-scope device array of HTREE_NOALLOC_SCRATCH_BYTES).
No counterpart in the reference; it is for callers that cannot allocate.
Checked through the C ABI against htree_backward_train given a workspace of
the same size (the same plan: bit-identical gradients expected, held to the
parity bar), on two calls in a row, the second with a smaller input, and a
third repeating the first (the array keeps the last call's contents)."""
import ctypes

import numpy as np
import pytest
import torch

from tests.gpu_util import close, inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CASES = [
    # B, T, H, Hkv, D, CR, TK, MTN, dtype, seed
    (1, 3000, 16, 2, 128, 16, 16, 128, "bfloat16", 91),  # smallest plan (stored scores)
    (1, 1100, 8, 1, 64, 8, 16, 64, "float32", 92),       # stored-dS plan
]


def grads(cfg, noalloc, grad_dtype=None):
    import htree_amd
    from htree_amd import _native as N

    B, T, H, Hkv, D, CR, TK, MTN, dtype, seed = cfg
    q, k, v, dO = (x.to(DEV) for x in inputs(B, T, H, Hkv, D, dtype, seed, dO=True))
    out, par, gmax, gsum, ctx = htree_amd.htree_forward_parents(q, k, v, CR, MTN, TK,
                                                                _save_scores=True)
    d = ctx["dims"] if grad_dtype is None else N.with_grad_dtype(ctx["dims"], grad_dtype)
    need = ctypes.c_int64()
    N.check(N.lib().htree_backward_noalloc_bytes(ctypes.byref(d), ctypes.byref(need)), "bytes")
    ws, cos, sin, sc = ctx["packed_tree"], ctx["cos_cache"], ctx["sin_cache"], ctx["train_scores"]
    gdt = grad_dtype or torch.float32
    dq = torch.empty(B, T, H, D, dtype=gdt, device=DEV)
    dk = torch.empty(B, T, Hkv, D, dtype=gdt, device=DEV)
    dv = torch.empty_like(dk)
    common = (ctypes.byref(d), float(ctx["scale"]), N.ptr(q), N.ptr(out), N.ptr(dO), N.ptr(gmax),
              N.ptr(gsum), N.ptr(par), N.ptr(ws), ws.numel(), N.ptr(cos), N.ptr(sin), N.ptr(sc),
              0 if sc is None else sc.numel(), N.ptr(dq), N.ptr(dk), N.ptr(dv))
    if noalloc:
        rc = N.lib().htree_backward_noalloc(*common, N.stream_ptr(q.device))
        N.check(rc, "htree_backward_noalloc")
    else:
        bws = torch.empty(need.value, dtype=torch.uint8, device=DEV)
        rc = N.lib().htree_backward_train(*common, N.ptr(bws), bws.numel(), N.stream_ptr(q.device))
        N.check(rc, "htree_backward_train")
    torch.cuda.synchronize()
    return [x.float().cpu().numpy() for x in (dq, dk, dv)]


def test_noalloc_matches_workspace_entry():
    for cfg in (CASES[0], CASES[1], CASES[0]):
        print(f"case {cfg}", flush=True)
        ref = grads(cfg, False)
        got = grads(cfg, True)
        for name, a, b in zip(("dq", "dk", "dv"), got, ref):
            assert np.all(np.isfinite(a)), name
            ok, worst = close(a, b, cfg[8])
            assert ok, f"{name}: worst {worst:.3f} of the bar"
            assert np.array_equal(a, b), f"{name}: not bit-identical to the workspace entry"


def test_noalloc_rejects_large_problems():
    """A backward that needs more than the array holds is refused before any
    launch (the pointers are never read)."""
    from htree_amd import _native as N

    d = N.dims(1, 32768, 32, 2, 128, 16, 16, 128, torch.bfloat16, 1152)
    need = ctypes.c_int64()
    assert N.lib().htree_backward_noalloc_bytes(ctypes.byref(d), ctypes.byref(need)) == N.HTREE_ESCRATCH
    assert need.value > 128 << 20
    rc = N.lib().htree_backward_noalloc(ctypes.byref(d), 1.0, *([None] * 7), 0, None, None, None, 0,
                                        None, None, None, None)
    assert rc == N.HTREE_ESCRATCH
    assert "htree_backward_noalloc" in N.strerror(rc)


def test_noalloc_gradients_in_input_dtype():
    """With grad_dtype bf16 the entry point stores the gradients rounded to
    bf16: the fp32 call's values cast, bit for bit."""
    cfg = CASES[0]
    ref = grads(cfg, True)
    got = grads(cfg, True, torch.bfloat16)
    for name, a, b in zip(("dq", "dk", "dv"), got, ref):
        assert np.array_equal(a, torch.from_numpy(b).bfloat16().float().numpy()), name
