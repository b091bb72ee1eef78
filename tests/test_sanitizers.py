"""Host-side sanitizer runs (no GPU):

  * AddressSanitizer + UndefinedBehaviorSanitizer over the C ABI's contract
    validation (voxtral.cpp_amd/csrc/vxfa_api.cpp: vxfa_supports,
    vxfa_check_mask_desc, vxfa_status_str), fuzzed with random descriptors by
    tests/sanitize/abi_fuzz.cpp, with the kernel launchers stubbed; the
    sanitizers instrument host code only (each -fsanitize= follows
    -Xarch_host), no kernel runs;
  * the same sanitizers over every entry point's run path (routing, split
    choice, workspace and scratch placement, F32 staging, implicit masks,
    ring, append, rope, no-alloc) by tests/sanitize/run_fuzz.cpp: the HIP
    runtime calls replaced by host stand-ins and the launchers by stubs that
    check the kernels' argument assumptions (records and staging inside one
    workspace allocation, the mask interval table clear of staged K/V);
  * ThreadSanitizer over the oracle's threaded routines (the scalar
    restatement and the vectorised baseline's thread pool) by
    tests/sanitize/oracle_threads.c.

Each builds into a temporary directory; a toolchain without the sanitizer
runtime skips the test."""
import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"


def _run(cmd, **kw):
    return subprocess.run(cmd, capture_output=True, text=True, timeout=600, **kw)


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_abi_validation_under_asan_ubsan():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "abi_fuzz")
        r = _run([HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17",
                  "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                  "-Xarch_host", "-fno-sanitize-recover=all",
                  "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                  "-x", "hip", os.path.join(ROOT, "tests", "sanitize", "abi_fuzz.cpp"),
                  os.path.join(ROOT, "voxtral.cpp_amd", "csrc", "vxfa_api.cpp"), "-o", exe])
        if r.returncode != 0 and "sanitizer" in (r.stderr or "").lower() and "not" in r.stderr.lower():
            pytest.skip("sanitizer runtime unavailable: " + r.stderr[-300:])
        assert r.returncode == 0, r.stderr[-3000:]
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="halt_on_error=1")
        r = _run([exe, "100000"], env=env)
        assert r.returncode == 0, (r.stdout + r.stderr)[-3000:]
        assert r.stdout.startswith("ok"), r.stdout


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_run_paths_under_asan_ubsan():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "run_fuzz")
        r = _run([HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17",
                  "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                  "-Xarch_host", "-fno-sanitize-recover=all",
                  "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                  "-x", "hip", os.path.join(ROOT, "tests", "sanitize", "run_fuzz.cpp"),
                  os.path.join(ROOT, "voxtral.cpp_amd", "csrc", "vxfa_api.cpp"), "-o", exe])
        if r.returncode != 0 and "sanitizer" in (r.stderr or "").lower() and "not" in r.stderr.lower():
            pytest.skip("sanitizer runtime unavailable: " + r.stderr[-300:])
        assert r.returncode == 0, r.stderr[-3000:]
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="halt_on_error=1")
        r = _run([exe, "200000"], env=env)
        assert r.returncode == 0, (r.stdout + r.stderr)[-3000:]
        assert r.stdout.startswith("ok"), r.stdout
        ok_calls, launches = int(r.stdout.split()[1]), int(r.stdout.split()[-1])
        assert ok_calls > 50000 and launches > 50000, r.stdout   # most calls reach the launchers


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")
def test_oracle_threads_under_tsan():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "oracle_threads")
        r = _run(["gcc", "-O1", "-g", "-std=c11", "-D_GNU_SOURCE", "-march=x86-64-v3", "-fsanitize=thread",
                  os.path.join(ROOT, "tests", "sanitize", "oracle_threads.c"),
                  os.path.join(ROOT, "oracle", "fa_oracle.c"), os.path.join(ROOT, "oracle", "fa_cpu_simd.c"),
                  "-o", exe, "-lm", "-pthread"])
        if r.returncode != 0 and "tsan" in (r.stderr or "").lower():
            pytest.skip("ThreadSanitizer runtime unavailable: " + r.stderr[-300:])
        assert r.returncode == 0, r.stderr[-3000:]
        r = _run([exe], env=dict(os.environ, TSAN_OPTIONS="halt_on_error=1:second_deadlock_stack=1"))
        assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
        assert r.stdout.strip() == "ok"
