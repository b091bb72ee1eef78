"""Host check (no GPU) of the rotary embedding's cos / sin helper that every
kernel with a fused rotation uses (rope_cs / rope_cs_of_angle in
voxtral.cpp_amd/csrc/fa_common.h: the angle reduced by multiples of pi/2 in
double precision, Taylor series on the remainder, quadrant swap and signs),
built from the header itself by tests/host/rope_cs_check.cpp and compared
with libm's double-precision cos / sin of the same float angles: ggml's
running-product angles at positions up to 2^20 for three bases and two head
sizes, and a sweep of plain angles over [-1000, 1000]. A wrong quadrant,
sign, swap or series term shows as an error of order 1e-3 or more; the bar
is 1e-6."""
import os
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_rope_cos_sin_match_libm():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "rope_cs_check")
        r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-x", "hip",
                            os.path.join(ROOT, "tests", "host", "rope_cs_check.cpp"), "-o", exe],
                           capture_output=True, text=True, timeout=600)
        assert r.returncode == 0, r.stderr[-3000:]
        r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
        assert r.returncode == 0 and r.stdout.startswith("ok"), (r.stdout + r.stderr)[-3000:]
