"""CPU checks of the C ABI: liborca_hip.so loads (no GPU needed to load it)
and exports every function include/orca_hip.h declares, and the Python
binding declares exactly those."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from orcaml_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "orca_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(orca_hip_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from orcaml_amd import build

        build.build()
    return ctypes.CDLL(_lib.LIB_PATH)


def test_header_declares_the_trait_ops():
    names = declared_functions()
    for op in ["matmul", "transpose", "add", "sub", "mul", "div", "mul_scalar", "relu", "relu_backward", "expand",
               "sum_to_shape", "reshape", "exp", "log", "exp_backward", "log_backward", "sqrt", "accumulate_grad",
               "max_to_shape", "max_to_shape_backward", "zeros", "from_f32_slice", "to_f32_vec", "has_nan_or_inf",
               "from_bytes", "to_bytes", "sigmoid", "sigmoid_backward", "div_backward_lhs", "div_backward_rhs",
               "sqrt_backward"]:
        assert f"orca_hip_{op}" in names, op


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_the_header():
    names = set(declared_functions())
    bound = set(_lib.SIGNATURES) | {"orca_hip_last_error"}
    assert names == bound, (names - bound, bound - names)


def test_errors_without_a_context_are_status_codes(lib):
    """Every entry point reports failure as an OrcaError status + message, never a crash."""
    lib.orca_hip_last_error.restype = ctypes.c_char_p
    out = ctypes.c_void_p()
    rc = lib.orca_hip_zeros(None, None, ctypes.c_size_t(0), 0, ctypes.byref(out))
    assert rc == _lib.ERR_INTERNAL
    assert b"null" in lib.orca_hip_last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError):
        _lib.load()
