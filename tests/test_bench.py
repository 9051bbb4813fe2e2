"""CPU checks of bench.py's contract (no GPU): one GPU only, the fused
forward kernel each workload's roofline names, and the committed PMC traffic
summaries it reads agree with the work model's algorithmic bytes."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from htree_amd.workmodel import work  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one MI355X" in r.stderr


def test_unknown_extra_workload_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--also", "C9"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "unknown workload" in r.stderr


@pytest.mark.parametrize("workload,kernel", [("C2", "fwd_reg_kernel"), ("C3", "fwd_reg_kernel"),
                                             ("C4", "fwd_kernel"), ("C5", "fwd_reg_kernel"),
                                             ("REF_FWD", "fwd_wide_kernel"),
                                             ("REF_BWD", "fwd_wide_kernel")])
def test_forward_kernel_of_each_workload(workload, kernel):
    # one-wave forms up to 16 / 64 candidate tiles of 16 per level, the
    # block-per-group form beyond (or top_k > 64)
    assert bench.forward_kernel(workload) == kernel


@pytest.mark.parametrize("workload", ["C2", "C4", "C5"])
def test_committed_traffic_matches_work_model(workload):
    path = os.path.join(ROOT, "profiles", f"{bench.forward_kernel(workload)}_{workload.lower()}_traffic.json")
    rec = json.load(open(path))
    (B, T, H, Hkv, D, CR, TK, MTN), dtype, _ = bench.WORKLOADS[workload]
    w = work(B, T, H, Hkv, D, CR, TK, MTN, 2 if dtype != "float32" else 4)
    assert rec["algorithmic_bytes_per_launch"] == pytest.approx(w.fwd_kernel_bytes, rel=1e-9)
    assert rec["traffic_bytes_per_launch"] == rec["fetch_bytes_per_launch"] + rec["write_bytes_per_launch"]
    # the counters are scaled by what they read for a copy of known size
    cal = rec["calibration"]
    assert cal["fetch_factor"] == pytest.approx(cal["bytes_read"] / (cal["fetch_size_kib"] * 1024), rel=1e-3)
    assert rec["fetch_bytes_per_launch"] == pytest.approx(
        rec["fetch_size_kib_per_dispatch"] * 1024 * cal["fetch_factor"], rel=1e-3)
    assert bench.measured_traffic(workload)["bytes"] == rec["traffic_bytes_per_launch"]
