"""Write golden fixtures from the reference's own CPU oracle (src/naive.py).

Run in the build container only (the reference is not present on GPU boxes):
    python tests/golden/make_golden.py [--ref /root/reference]

Each fixture is data only: the configuration, the seed and SHA-256 of the
inputs (inputs are regenerated from the seed by golden_inputs() below, a CPU
torch.Generator recipe), and the reference's outputs:
  out, dq, dk, dv          in the input dtype (uint16 bit patterns for bf16/fp16)
  parents_l{l}             LayerTrace.selected_parents per upper level
                           (naive.py:225-227), int16
  lmax/lsum                per-level online-softmax state, fp32
The configurations satisfy the reference's own asserts (naive.py:141-151:
max_top_nodes == top_k * compression_rate), so naive.py runs unmodified.
"""
from __future__ import annotations

import argparse
import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

# name: (B, T, H, Hkv, D, CR, TK, MTN, dtype, seed)
CONFIGS = {
    "cr4_d16_fp32": (1, 300, 4, 1, 16, 4, 8, 32, "float32", 11),
    "cr16_tk4_bf16": (1, 1100, 4, 1, 64, 16, 4, 64, "bfloat16", 12),
    "cr8_tk16_fp32_g8": (1, 300, 8, 1, 64, 8, 16, 128, "float32", 13),
    "cr16_tk4_fp16_b2": (2, 700, 4, 2, 64, 16, 4, 64, "float16", 14),
}

DT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


def golden_inputs(B, T, H, Hkv, D, dtype: str, seed: int):
    """q, k, v, dO iid N(0,1) drawn in fp32 on the CPU from one generator,
    then cast to the dtype."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g).to(DT[dtype])
    k = torch.randn(B, T, Hkv, D, generator=g).to(DT[dtype])
    v = torch.randn(B, T, Hkv, D, generator=g).to(DT[dtype])
    dO = torch.randn(B, T, H, D, generator=g).to(DT[dtype])
    return q, k, v, dO


def inputs_sha(*ts) -> str:
    h = hashlib.sha256()
    for t in ts:
        t = t.contiguous()
        raw = t.numpy() if t.dtype == torch.float32 else t.view(torch.int16).numpy()
        h.update(raw.tobytes())
    return h.hexdigest()


def native(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().astype(np.float32)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--only", default=None)
    args = ap.parse_args()
    sys.path.insert(0, args.ref)
    from src import naive  # the reference's CPU semantic oracle

    torch.set_num_threads(8)
    for name, (B, T, H, Hkv, D, CR, TK, MTN, dtype, seed) in CONFIGS.items():
        if args.only and name != args.only:
            continue
        q, k, v, dO = golden_inputs(B, T, H, Hkv, D, dtype, seed)
        scale = D ** -0.5
        with torch.no_grad():
            out_t, trace = naive.htree_forward_naive(q, k, v, compression_rate=CR, max_top_nodes=MTN,
                                                     top_k_per_layer=TK, scale=scale, return_trace=True)
        qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
        out_a = naive.htree_forward_naive_autograd(qg, kg, vg, compression_rate=CR, max_top_nodes=MTN,
                                                   top_k_per_layer=TK, scale=scale)
        out_a.backward(dO)
        L = trace["num_layers"]
        rec = dict(
            config=np.array([B, T, H, Hkv, D, CR, TK, MTN, seed], np.int64),
            dtype=np.array(dtype),
            inputs_sha256=np.array(inputs_sha(q, k, v, dO)),
            num_layers=np.array(L),
            out=native(out_t),
            out_autograd=native(out_a),
            dq=native(qg.grad), dk=native(kg.grad), dv=native(vg.grad),
        )
        for l in range(L):
            tr = trace["layers"][l]
            rec[f"lmax_l{l}"] = tr.layer_max.numpy().astype(np.float32)
            rec[f"lsum_l{l}"] = tr.layer_sum.numpy().astype(np.float32)
            if tr.selected_parents is not None:
                rec[f"parents_l{l}"] = tr.selected_parents.numpy().astype(np.int16)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **rec)
        print(f"wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB), levels={L}")


if __name__ == "__main__":
    main()
