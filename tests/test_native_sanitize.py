"""CPU builds under AddressSanitizer + UndefinedBehaviorSanitizer (no GPU):
the host-only runtime of liborca_hip.so (orcaml_amd/csrc/runtime_host.cpp)
against a HIP API stand-in, and the oracle's C sources.  Each program checks
its own results and exits non-zero on the first sanitizer report."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NATIVE = os.path.join(ROOT, "tests", "native")
SAN = ["-g", "-O1", "-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-fno-sanitize-recover=all"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
           OMP_NUM_THREADS="4")


def _build_and_run(cmd, exe):
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    r = subprocess.run([exe], capture_output=True, text=True, env=ENV, timeout=300)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-4000:])
    return r.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_runtime_host_under_asan_ubsan(tmp_path):
    exe = str(tmp_path / "runtime_host_test")
    out = _build_and_run(["g++", "-std=c++17", *SAN, "-I", os.path.join(NATIVE, "hip_stub"), "-I",
                          os.path.join(ROOT, "orcaml_amd", "csrc"), os.path.join(ROOT, "orcaml_amd", "csrc",
                                                                                  "runtime_host.cpp"),
                          os.path.join(NATIVE, "runtime_host_test.cpp"), "-o", exe], exe)
    assert "all checks passed" in out


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_oracle_under_asan_ubsan(tmp_path):
    exe = str(tmp_path / "oracle_sanitize")
    src = [os.path.join(ROOT, "oracle", f) for f in ("orca_ops.c", "orca_mlp.c", "orca_gemm.c")]
    out = _build_and_run(["gcc", "-std=gnu11", *SAN, "-fopenmp", "-ffp-contract=off", "-I", os.path.join(ROOT, "oracle"),
                          *src, os.path.join(NATIVE, "oracle_sanitize.c"), "-lm", "-o", exe], exe)
    assert "all checks passed" in out
