"""CPU checks of the run-time compiled elementwise programs (no GPU): the HIP
source the library generates for a program compiles under hipRTC with the
library's own flags for every opcode and every input access, has one value per
instruction and one store per output, and malformed programs are refused
before anything is generated or launched.  Bit-identity with the interpreter
is checked on the GPU (tests/test_gpu_lazy_ew.py)."""
from __future__ import annotations

import ctypes
import os
import re
import struct

import pytest

from orcaml_amd import _lib
from orcaml_amd import backend as B

HIPRTC_OPTS = [b"--offload-arch=gfx950", b"-O3", b"-ffp-contract=off", b"-Xclang", b"-target-feature", b"-Xclang",
               b"-packed-fp32-ops"]


def program(instrs, n_in, out_regs):
    """(instruction array, output-register array) in the C ABI layout (orca_hip_ew_instr:
    five bytes, three of padding, the f32 scalar)."""
    raw = b"".join(struct.pack("<BBBBBxxxf", *ins) for ins in instrs)
    return ctypes.create_string_buffer(raw, max(1, len(raw))), (ctypes.c_uint8 * len(out_regs))(*out_regs)


def source(n, inputs, instrs, out_regs, n_regs):
    ins = (B.EwInput * max(1, len(inputs)))(*[(None, d, m) for d, m in inputs])
    arr, oregs = program(instrs, len(inputs), out_regs)
    needed = ctypes.c_size_t()
    _lib.call("orca_hip_ew_jit_source", n, ins, len(inputs), oregs, len(out_regs), arr, len(instrs), n_regs, None, 0,
              ctypes.byref(needed))
    buf = ctypes.create_string_buffer(needed.value)
    _lib.call("orca_hip_ew_jit_source", n, ins, len(inputs), oregs, len(out_regs), arr, len(instrs), n_regs, buf,
              needed.value, None)
    return buf.value.decode()


# Every opcode once, over inputs read in each access the launcher picks for n = 4096:
# plain, one value, a row broadcast (mod % 4 == 0), a column broadcast per group of 4
# (div % 4 == 0), the general index (div 3), and again the general index (mod 5).
N = 4096
INPUTS = [(1, N), (1, 1), (1, 64), (8, 512), (3, 1365), (1, 5)]
ALL_OPS = [
    (B.EW_ADD, 6, 0, 1, 0, 0.0), (B.EW_SUB, 7, 6, 2, 0, 0.0), (B.EW_MUL, 8, 7, 3, 0, 0.0), (B.EW_DIV, 9, 8, 4, 0, 0.0),
    (B.EW_MUL_SCALAR, 10, 9, 9, 9, 0.5), (B.EW_RELU, 11, 10, 10, 10, 0.0), (B.EW_RELU_BW, 12, 11, 5, 0, 0.0),
    (B.EW_EXP, 13, 12, 12, 12, 0.0), (B.EW_LOG, 14, 13, 13, 13, 0.0), (B.EW_SQRT, 15, 14, 14, 14, 0.0),
    (B.EW_SIGMOID, 6, 15, 15, 15, 0.0), (B.EW_EXP_BW, 7, 6, 0, 0, 0.0), (B.EW_LOG_BW, 8, 7, 1, 0, 0.0),
    (B.EW_SQRT_BW, 9, 8, 2, 0, 0.0), (B.EW_SIGMOID_BW, 10, 9, 3, 0, 0.0), (B.EW_DIV_BW_RHS, 11, 10, 4, 5, 0.0),
    (B.EW_SUM_VISIT, 12, 11, 11, 11, 0.0), (B.EW_MAX_VISIT, 13, 12, 12, 12, 0.0), (B.EW_COPY, 14, 13, 13, 13, 0.0),
    (B.EW_ADD_SCALAR, 15, 14, 14, 14, 0.25),
]


def hiprtc():
    for name in ("libhiprtc.so.7", "libhiprtc.so", "/opt/rocm/lib/libhiprtc.so"):
        try:
            return ctypes.CDLL(name)
        except OSError:
            continue
    return None


def test_source_has_one_value_per_instruction_and_one_store_per_output():
    src = source(N, INPUTS, ALL_OPS, [14, 6, 0], 16)
    vec = src[src.index("ew_fused_vec"):src.index("ew_fused_scalar")]
    loop = vec[:vec.index("if (blockIdx.x == 0")]
    assert len(re.findall(r"const floatx4 t\d+ = ", loop)) == len(ALL_OPS)
    assert len(re.findall(r"const floatx4 x\d+ = ", loop)) == len(INPUTS)
    stores = re.findall(r"reinterpret_cast<floatx4\*>\(p\.out\[(\d)\]\)\[q\] = (\w+);", loop)
    assert [int(o) for o, _ in stores] == [0, 1, 2]
    assert stores[0][1] == "t18"      # register 14 last written by the COPY
    assert stores[1][1] == "t10"      # register 6 last written by SIGMOID (instruction 10)
    assert stores[2][1] == "x0"       # register 0 is never overwritten: the input itself
    # the scalar is a kernel argument, not a constant: programs that differ only in scalars share a kernel
    assert "OpScale{p.sc[4]}" in src and "0.5" not in src
    assert "OpAddScalar{p.sc[19]}" in src and "0.25" not in src
    # each input is read with the access its (div, mod) selects
    assert "reinterpret_cast<const floatx4*>(p.in[0])[q]" in loop
    assert "bc4(p.in[1][0])" in loop
    assert "*reinterpret_cast<const floatx4*>(p.in[2] + ix32(p, 2" in loop
    assert "bc4(p.in[3][ix32(p, 3" in loop
    assert loop.count("ix32(p, 4,") == 4 and loop.count("ix32(p, 5,") == 4


def test_indices_past_2_31_elements_take_64_bit_division():
    src = source(2 ** 31 + 8, [(1, 2 ** 31 + 8), (3, 7)], [(B.EW_ADD, 2, 0, 1, 0, 0.0)], [2], 3)
    assert "ix64(p, 1," in src and "ix32(p, 1," not in src


@pytest.mark.parametrize("out_regs", [[14, 6, 0], [13]])
def test_generated_source_compiles_with_the_library_flags(out_regs):
    rtc = hiprtc()
    if rtc is None:
        pytest.skip("libhiprtc not present")
    src = source(N, INPUTS, ALL_OPS, out_regs, 16).encode()
    ops_text = ctypes.c_char_p()
    _lib.call("orca_hip_ew_jit_headers", ctypes.byref(ops_text))
    headers = (ctypes.c_char_p * 3)(ops_text.value, b"#pragma once\n#define FLT_MAX 3.40282347e+38F\n",
                                    b"#pragma once\n")
    names = (ctypes.c_char_p * 3)(b"ew_ops.hpp", b"cfloat", b"cmath")
    prog = ctypes.c_void_p()
    assert rtc.hiprtcCreateProgram(ctypes.byref(prog), src, b"ew_fused.hip", 3, headers, names) == 0
    opts = (ctypes.c_char_p * len(HIPRTC_OPTS))(*HIPRTC_OPTS)
    rc = rtc.hiprtcCompileProgram(prog, len(HIPRTC_OPTS), opts)
    log = b""
    if rc != 0:
        size = ctypes.c_size_t()
        rtc.hiprtcGetProgramLogSize(prog, ctypes.byref(size))
        buf = ctypes.create_string_buffer(size.value + 1)
        rtc.hiprtcGetProgramLog(prog, buf)
        log = buf.value
    code = ctypes.c_size_t()
    rtc.hiprtcGetCodeSize(prog, ctypes.byref(code))
    rtc.hiprtcDestroyProgram(ctypes.byref(prog))
    assert rc == 0, log.decode(errors="replace")[-3000:]
    assert code.value > 0


def test_functor_header_is_the_one_the_build_compiled():
    ops_text = ctypes.c_char_p()
    _lib.call("orca_hip_ew_jit_headers", ctypes.byref(ops_text))
    here = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "orcaml_amd", "csrc",
                        "ew_ops.hpp")
    assert ops_text.value.decode() == open(here).read()


@pytest.mark.parametrize("instrs,out_regs,n_regs,what", [
    ([(B.EW_ADD, 2, 0, 3, 0, 0.0)], [2], 4, "reads register 3 before any write"),
    ([(B.EW_RELU, 2, 0, 0, 0, 0.0)], [3], 4, "outputs register 3, never written"),
    ([(B.EW_DIV_BW_RHS, 2, 0, 1, 3, 0.0)], [2], 4, "third operand not written"),
    ([(20, 2, 0, 1, 0, 0.0)], [2], 3, "unknown opcode"),
    ([(B.EW_ADD, 5, 0, 1, 0, 0.0)], [5], 4, "destination past the registers"),
])
def test_malformed_programs_are_refused(instrs, out_regs, n_regs, what):
    with pytest.raises(_lib.OrcaHipError, match="invalid|out of range"):
        source(64, [(1, 64), (1, 64)], instrs, out_regs, n_regs)
