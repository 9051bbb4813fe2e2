"""fwd_wide_kernel's LDS addressing replayed on the host against the layout
its launch allocates (tests/wide_lds_check.cpp, built with the same header
the kernel uses): every index in bounds, regions disjoint, for every wide
configuration the library accepts."""
import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_wide_kernel_lds_indices_in_bounds():
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "wide_lds_check")
        subprocess.run([hipcc, "-x", "hip", "--offload-arch=gfx950", "-O1", "-std=c++17",
                        f"-I{ROOT}/include", f"-I{ROOT}/htree_amd/csrc",
                        os.path.join(ROOT, "tests", "wide_lds_check.cpp"), "-o", exe],
                       check=True, capture_output=True)
        r = subprocess.run([exe], capture_output=True, text=True)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert "0 failures" in r.stdout
