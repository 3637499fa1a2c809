"""CPU checks of the Rust crate orca-backend-hip (no Rust toolchain in this image, so the crate
is checked as source): its `extern "C"` block declares each entry point exactly as
include/orca_hip.h does, its #[repr(C)] structs match the header's field for field, its
`impl Backend for HipBackend` has the trait's 42 methods (orca-tensor/src/backend.rs:19-315),
each calling its own `orca_hip_trait_*` entry point once, and build.rs compiles the same
sources as orcaml_amd/build.py."""
from __future__ import annotations

import os
import re

import pytest

from orcaml_amd import build as hip_build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CRATE = os.path.join(ROOT, "orca-backend-hip")
HEADER = os.path.join(ROOT, "include", "orca_hip.h")

# The trait's methods in declaration order (orca-tensor/src/backend.rs:19-315).
TRAIT_METHODS = [
    "device", "zeros", "from_f32_slice", "to_f32_vec", "matmul", "transpose", "add", "sub", "mul_scalar", "mul",
    "relu", "sigmoid", "relu_backward", "sigmoid_backward", "expand", "sum_to_shape", "reshape", "exp", "log",
    "exp_backward", "log_backward", "div", "sqrt", "div_backward_lhs", "div_backward_rhs", "sqrt_backward",
    "accumulate_grad", "conv2d", "conv2d_backward_input", "conv2d_backward_weight", "conv2d_backward_bias", "cast",
    "scatter", "gather", "scatter_backward_src", "scatter_backward_base", "gather_backward", "from_bytes", "to_bytes",
    "has_nan_or_inf", "max_to_shape", "max_to_shape_backward"]

C_BASE = {"size_t": "usize", "int": "c_int", "float": "f32", "double": "f64", "int64_t": "i64", "uint8_t": "u8",
          "uint32_t": "u32", "uint64_t": "u64", "char": "c_char", "void": "c_void", "orca_hip_ctx": "OrcaHipCtx",
          "orca_hip_backend": "OrcaHipBackend", "orca_hip_storage": "OrcaHipStorage",
          "orca_hip_backend_options": "BackendOptions", "orca_hip_error_info": "ErrorInfo", "orca_hip_opt_row": "OptRow"}


def _strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def c_type(decl: str) -> str:
    """A C parameter or return type in the Rust spelling: `const size_t*` -> `*const usize`,
    `orca_hip_storage**` -> `*mut *mut OrcaHipStorage`, `float` -> `f32`."""
    decl = decl.strip()
    m = re.fullmatch(r"(const\s+)?([A-Za-z_][A-Za-z0-9_]*)\s*((?:\*\s*(?:const\s*)?)*)", decl)
    assert m, decl
    const_base, base, stars = m.group(1), m.group(2), m.group(3)
    # types the crate does not bind keep a CamelCase name (they only need to parse)
    t = C_BASE.get(base) or "".join(w.capitalize() for w in base.split("_"))
    levels = re.findall(r"\*\s*(const)?", stars)
    for i, trailing_const in enumerate(levels):
        # the first * points to the base (const if the base is const); a `* const` makes the next level const
        is_const = bool(const_base) if i == 0 else bool(levels[i - 1])
        t = f"*{'const' if is_const else 'mut'} {t}"
    return t


def header_functions():
    text = _strip_comments(open(HEADER).read())
    out = {}
    for ret, name, params in re.findall(r"\b(int|const char\s*\*)\s+(orca_hip_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        types = []
        params = " ".join(params.split())
        if params and params != "void":
            for p in params.split(","):
                p = p.strip()
                m = re.fullmatch(r"(.*?)([A-Za-z_][A-Za-z0-9_]*)?", p)
                typ = p
                # drop the parameter name (the last identifier after the type)
                mm = re.fullmatch(r"(.*[\s\*])([A-Za-z_][A-Za-z0-9_]*)", p)
                if mm and mm.group(2) not in C_BASE and mm.group(2) != "const":
                    typ = mm.group(1)
                types.append(c_type(typ))
        out[name] = (c_type(ret), types)
    return out


def rust_functions():
    text = _strip_comments(open(os.path.join(CRATE, "src", "ffi.rs")).read())
    block = text[text.index('extern "C" {'):]
    out = {}
    for name, params, ret in re.findall(r"pub fn (orca_hip_[a-z0-9_]+)\s*\(([^)]*)\)\s*->\s*([^;]+);", block):
        types = []
        for p in [q for q in (x.strip() for x in params.split(",")) if q]:
            _, typ = p.split(":", 1)
            types.append(" ".join(typ.replace("std::os::raw::", "").split()))
        out[name] = (" ".join(ret.split()), types)
    return out


def test_every_extern_declaration_matches_the_header():
    hdr, rs = header_functions(), rust_functions()
    assert len(rs) > 60
    for name, (ret, params) in rs.items():
        assert name in hdr, name
        assert (ret, params) == hdr[name], (name, (ret, params), hdr[name])


def test_the_storage_api_is_declared_in_full():
    hdr, rs = header_functions(), rust_functions()
    for name in hdr:
        if name.startswith(("orca_hip_trait_", "orca_hip_be_", "orca_hip_storage_", "orca_hip_backend_")):
            assert name in rs, name
    assert sorted(n[len("orca_hip_trait_"):] for n in rs if n.startswith("orca_hip_trait_")) == sorted(TRAIT_METHODS)


def _c_struct(name):
    text = _strip_comments(open(HEADER).read())
    body = re.search(r"typedef struct\s*\{([^}]*)\}\s*" + name + r"\s*;", text).group(1)
    fields = []
    for decl in body.split(";"):
        decl = " ".join(decl.split())
        if not decl:
            continue
        m = re.fullmatch(r"(.*?)\s*([A-Za-z_][A-Za-z0-9_]*)(\[(\d+)\])?", decl)
        typ, fname, arr = m.group(1), m.group(2), m.group(4)
        t = c_type(typ)
        fields.append((fname, f"[{t}; {arr}]" if arr else t))
    return fields


def _rust_struct(name):
    text = _strip_comments(open(os.path.join(CRATE, "src", "ffi.rs")).read())
    body = re.search(r"pub struct " + name + r"\s*\{([^}]*)\}", text).group(1)
    return [(f.strip().split(":", 1)[0].replace("pub ", "").strip(), " ".join(f.split(":", 1)[1].split()))
            for f in body.split(",") if f.strip()]


@pytest.mark.parametrize("c_name,rust_name", [("orca_hip_backend_options", "BackendOptions"),
                                              ("orca_hip_error_info", "ErrorInfo"), ("orca_hip_opt_row", "OptRow")])
def test_repr_c_structs_match_the_header(c_name, rust_name):
    assert _rust_struct(rust_name) == _c_struct(c_name)


def test_the_trait_impl_has_42_methods_each_one_call():
    text = _strip_comments(open(os.path.join(CRATE, "src", "backend.rs")).read())
    impl = text[text.index("impl Backend for HipBackend"):]
    methods = re.findall(r"\n    fn ([a-z0-9_]+)\s*\(", impl)
    assert methods == TRAIT_METHODS
    bodies = re.split(r"\n    fn ", impl)[1:]
    for name, body in zip(methods, bodies):
        calls = re.findall(r"ffi::(orca_hip_[a-z0-9_]+)", body)
        if name == "device":
            assert calls == []  # the ordinal the backend was created on
        else:
            assert calls == [f"orca_hip_trait_{name}"], (name, calls)


def test_build_script_compiles_the_library_sources():
    text = open(os.path.join(CRATE, "build.rs")).read()
    block = re.search(r"const SOURCES: \[&str; (\d+)\] = \[(.*?)\];", text, re.S)
    names = re.findall(r'"([^"]+)"', block.group(2))
    assert int(block.group(1)) == len(names) and names == hip_build.SOURCES
    for flag in ("--offload-arch=gfx950", "-ffp-contract=off", "-packed-fp32-ops"):
        assert flag in text
