"""The storage layer (orcaml_amd/csrc/storage.cpp) built for the CPU against a host stand-in
of liborca_hip.so's buffer-level entry points (tests/native/fake_device.cpp, which computes
with the oracle's C ops), and the helpers that point the Python binding at it.  Test
infrastructure: the planner's decisions can then be checked without a GPU, through the same
binding and ABI the GPU runs use."""
from __future__ import annotations

import ctypes
import os
import subprocess
from concurrent.futures import ThreadPoolExecutor

from orcaml_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NATIVE = os.path.join(ROOT, "tests", "native")
CSRC = os.path.join(ROOT, "orcaml_amd", "csrc")
ORACLE = os.path.join(ROOT, "oracle")


def build(out_dir: str, extra_flags=()) -> str:
    """Compiles the CPU library into out_dir and returns its path."""
    os.makedirs(out_dir, exist_ok=True)
    jobs = []
    # the oracle's files as oracle/Makefile builds them (the same summation bits as its library)
    for src, contract in (("orca_ops.c", "off"), ("orca_mlp.c", "off"), ("orca_gemm.c", "fast")):
        jobs.append(["gcc", "-std=gnu11", "-O3", "-fPIC", "-fopenmp", "-fno-fast-math", f"-ffp-contract={contract}",
                     *extra_flags, "-I", ORACLE, "-c", os.path.join(ORACLE, src), "-o",
                     os.path.join(out_dir, src + ".o")])
    for src in (os.path.join(CSRC, "storage.cpp"), os.path.join(CSRC, "runtime_host.cpp"),
                os.path.join(NATIVE, "fake_device.cpp")):
        jobs.append(["g++", "-std=c++17", "-O1", "-fPIC", "-ffp-contract=off", *extra_flags, "-I",
                     os.path.join(NATIVE, "hip_stub"), "-I", CSRC, "-I", ORACLE, "-c", src, "-o",
                     os.path.join(out_dir, os.path.basename(src) + ".o")])

    def run(cmd):
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"{' '.join(cmd)}\n{r.stderr[-4000:]}")

    with ThreadPoolExecutor(max_workers=6) as ex:
        list(ex.map(run, jobs))
    path = os.path.join(out_dir, "liborca_fake.so")
    objs = [os.path.join(out_dir, f) for f in os.listdir(out_dir) if f.endswith(".o")]
    run(["g++", "-shared", "-fopenmp", *extra_flags, "-o", path, *objs, "-lm"])
    return path


def load(path: str) -> ctypes.CDLL:
    """The CPU library with the binding's signatures on the entry points it has."""
    lib = ctypes.CDLL(path)
    for name, argtypes in _lib.SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            continue
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    lib.orca_hip_last_error.argtypes = []
    lib.orca_hip_last_error.restype = ctypes.c_char_p
    lib.fake_log_text.argtypes = [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    lib.fake_race_count.argtypes = []
    lib.fake_race_count.restype = ctypes.c_uint64
    return lib


def install(monkeypatch, lib) -> None:
    """Routes the binding's calls to `lib` for one test."""
    monkeypatch.setattr(_lib, "_lib", lib)
    monkeypatch.setattr(_lib, "_FNS", {})


def log(lib) -> list:
    """The stand-in's launch log since the last clear, one entry per launch."""
    need = ctypes.c_size_t()
    lib.fake_log_text(None, 0, ctypes.byref(need))
    buf = ctypes.create_string_buffer(need.value)
    lib.fake_log_text(buf, need.value, ctypes.byref(need))
    return [line for line in buf.value.decode().splitlines() if line]


def clear(lib) -> None:
    lib.fake_log_clear()


def races(lib) -> int:
    """Accesses of one stream to memory the other stream touched after the last point it
    waited for (the stand-in's happens-before check), since the library was loaded."""
    return int(lib.fake_race_count())
