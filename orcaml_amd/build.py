"""Builds liborca_hip.so (the HIP backend) for gfx950 with hipcc, in-tree.

Every translation unit is compiled with
  * --offload-arch=gfx950 (MI355X, CDNA4) only;
  * -ffp-contract=off, so elementwise / optimizer arithmetic keeps the
    reference's separate f32 multiply and add;
  * -Xclang -target-feature -Xclang -packed-fp32-ops, so the compiler emits
    no packed-FP32 VALU instructions.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "liborca_hip.so")
SOURCES = ["runtime_host.cpp", "storage.cpp", "runtime.hip", "ops.hip", "gemm.hip", "fused.hip", "head.hip", "mlp.hip", "ewprog.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def _embed_ew_ops() -> None:
    """ew_ops.hpp's text as a C++ raw string literal (_build/ew_ops_text.inc): ewprog.hip
    hands it to hipRTC, so run-time compiled programs use the same functors."""
    with open(os.path.join(CSRC, "ew_ops.hpp")) as fh:
        text = fh.read()
    if ")EWOPS\"" in text:
        raise RuntimeError("ew_ops.hpp contains the raw-string delimiter")
    inc = 'R"EWOPS(' + text + ')EWOPS"\n'
    path = os.path.join(BUILD_DIR, "ew_ops_text.inc")
    if not os.path.exists(path) or open(path).read() != inc:
        with open(path, "w") as fh:
            fh.write(inc)


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, src.replace(".", "_") + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-I", BUILD_DIR, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compiles every HIP source and links the shared library; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    _embed_ew_ops()
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-ldl"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
