"""Host check (no GPU) of the index helpers every prefill kernel uses to place
its workgroup: the multiply-high division constants (FastDiv) and the
XCD-aware workgroup map (GridMap) of voxtral.cpp_amd/csrc/fa_common.h, built
from the header itself by tests/host/grid_map_check.cpp and compared with the
/ and % operators."""
import os
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_fastdiv_and_grid_map_match_integer_division():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "grid_map_check")
        r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-x", "hip",
                            os.path.join(ROOT, "tests", "host", "grid_map_check.cpp"), "-o", exe],
                           capture_output=True, text=True, timeout=600)
        assert r.returncode == 0, r.stderr[-3000:]
        r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
        assert r.returncode == 0 and r.stdout.startswith("ok"), (r.stdout + r.stderr)[-3000:]
