"""The tree build's stores and reads replayed on the host through the index
functions the kernels call (htree_amd/csrc/htree_tree_index.h,
tests/build_replay_check.cpp): every store in bounds and every packed and
pooled element written exactly once, every child read and LDS row inside its
array, for CR 4..128, 1..7 levels and every split between the span launch and
the per-level launches (including level 1 pooled from the leaves at CR 128)."""
import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_tree_build_stores_in_bounds_and_once():
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "build_replay_check")
        subprocess.run([hipcc, "-x", "hip", "--offload-arch=gfx950", "-O2", "-std=c++17",
                        f"-I{ROOT}/include", f"-I{ROOT}/htree_amd/csrc",
                        os.path.join(ROOT, "tests", "build_replay_check.cpp"), "-o", exe],
                       check=True, capture_output=True)
        r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert " 0 failures" in r.stdout
    assert int(r.stdout.split()[0]) > 500
