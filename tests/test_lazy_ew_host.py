"""CPU checks of HipBackend's lazy elementwise chains (no GPU): the compiled
programs are run by a numpy interpreter of the instruction bytes in place of
orca_hip_ew_program, against the oracle's ops (orca-backend-cpu semantics) run
one by one.  Pins the program compiler (register reuse, shared subexpressions,
operand order), the choice of outputs (values referenced from outside the
chain), the split of chains past the interpreter's limits, and the program
cache."""
from __future__ import annotations

import ctypes
import itertools
import struct

import numpy as np
import pytest

from oracle import oracle as O
from orcaml_amd import backend as B
from orcaml_amd import device

_OPS = {
    B.EW_ADD: lambda a, b, c, s: O.add(a, b), B.EW_SUB: lambda a, b, c, s: O.sub(a, b),
    B.EW_MUL: lambda a, b, c, s: O.mul(a, b), B.EW_DIV: lambda a, b, c, s: O.div(a, b),
    B.EW_MUL_SCALAR: lambda a, b, c, s: O.mul_scalar(a, s), B.EW_RELU: lambda a, b, c, s: O.relu(a),
    B.EW_RELU_BW: lambda a, b, c, s: O.relu_backward(a, b), B.EW_EXP: lambda a, b, c, s: O.exp(a),
    B.EW_LOG: lambda a, b, c, s: O.log(a), B.EW_SQRT: lambda a, b, c, s: O.sqrt(a),
    B.EW_SIGMOID: lambda a, b, c, s: O.sigmoid(a), B.EW_EXP_BW: lambda a, b, c, s: O.exp_backward(a, b),
    B.EW_LOG_BW: lambda a, b, c, s: O.log_backward(a, b), B.EW_SQRT_BW: lambda a, b, c, s: O.sqrt_backward(a, b),
    B.EW_SIGMOID_BW: lambda a, b, c, s: O.sigmoid_backward(a, b),
    B.EW_DIV_BW_RHS: lambda a, b, c, s: O.div_backward_rhs(a, b, c), B.EW_COPY: lambda a, b, c, s: a.copy(),
    B.EW_ADD_SCALAR: lambda a, b, c, s: O.add(a, np.full_like(a, s)),
}


class FakeDevice:
    """Host memory behind fake device pointers, and the C calls the lazy path makes."""

    def __init__(self):
        self.mem = {}
        self.ids = itertools.count(1)
        self.programs = []

    def call(self, name, *args):
        if name == "orca_hip_from_f32_slice":
            _, dims, rank, data, n, out = args
            ptr = next(self.ids) << 8
            self.mem[ptr] = np.ctypeslib.as_array(ctypes.cast(data, ctypes.POINTER(ctypes.c_float)), (n,)).copy()
            out._obj.value = ptr
        elif name == "orca_hip_alloc":
            _, nbytes, out = args
            ptr = next(self.ids) << 8
            self.mem[ptr] = np.zeros(max(1, nbytes // 4), np.float32)
            out._obj.value = ptr
        elif name == "orca_hip_to_f32_vec":
            _, ptr, n, host = args
            np.ctypeslib.as_array(ctypes.cast(host, ctypes.POINTER(ctypes.c_float)), (n,))[:] = self.mem[ptr][:n]
        elif name == "orca_hip_free":
            pass
        elif name == "orca_hip_ew_program":
            _, n, ins, n_in, outs, oregs, n_out, instrs, n_ops, n_regs = args
            raw = ctypes.string_at(instrs, 12 * n_ops)
            regs = [None] * n_regs
            e = np.arange(n)
            for i in range(n_in):
                regs[i] = self.mem[ins[i].ptr][(e // ins[i].div) % ins[i].mod].copy()
            for k in range(n_ops):
                op, dst, a, b, c, s = struct.unpack_from("<BBBBBxxxf", raw, 12 * k)
                regs[dst] = _OPS[op](regs[a], regs[b], regs[c], s).astype(np.float32)
            for o in range(n_out):
                self.mem[outs[o]][:n] = regs[oregs[o]]
            self.programs.append((n_in, n_out, n_ops, n_regs))
        else:
            raise AssertionError(f"unexpected call {name}")


class FakeContext:
    device = 0
    handle = None  # Buffer.free skips the C call (buffers may outlive the patched binding)

    def __init__(self, dev):
        self.dev = dev

    def alloc(self, nbytes):
        out = ctypes.c_void_p()
        self.dev.call("orca_hip_alloc", None, nbytes, ctypes.byref(out))
        return device.Buffer(self, out.value, nbytes)


@pytest.fixture()
def fake(monkeypatch):
    dev = FakeDevice()
    monkeypatch.setattr(B._lib, "call", dev.call)
    monkeypatch.setattr(device._lib, "call", dev.call)
    return dev, B.HipBackend(FakeContext(dev))


def up(hb, a):
    a = np.ascontiguousarray(a, np.float32)
    return hb.from_f32_slice(a.shape, a)


def down(hb, s):
    return hb.to_f32_vec(s)


def test_adamw_chain_is_one_program_with_three_outputs(fake):
    """The composed AdamW update of one parameter (python/orca/optim/adamw.py:66-99): the new
    parameter, m and v come from one program; the temporaries are not written."""
    dev, hb = fake
    rng = np.random.default_rng(1)
    n = 1001
    p, g = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    m, v = rng.standard_normal(n).astype(np.float32), np.abs(rng.standard_normal(n)).astype(np.float32)
    eps = np.full(n, 1e-8, np.float32)
    P, G, M, V, E = (up(hb, a) for a in (p, g, m, v, eps))
    sh = (n,)
    decayed = hb.mul_scalar(P, 1.0 - 1e-3 * 0.01, sh)
    m_new = hb.add(hb.mul_scalar(M, 0.9, sh), hb.mul_scalar(G, 1.0 - 0.9, sh), sh)
    v_new = hb.add(hb.mul_scalar(V, 0.999, sh), hb.mul_scalar(hb.mul(G, G, sh), 1.0 - 0.999, sh), sh)
    m_hat = hb.mul_scalar(m_new, 1.0 / (1.0 - 0.9 ** 3), sh)
    v_hat = hb.mul_scalar(v_new, 1.0 / (1.0 - 0.999 ** 3), sh)
    new_p = hb.sub(decayed, hb.mul_scalar(hb.div(m_hat, hb.add(hb.sqrt(v_hat, sh), E, sh), sh), 1e-3, sh), sh)
    del decayed, m_hat, v_hat
    got_p = down(hb, new_p)
    assert dev.programs == [(5, 3, 15, dev.programs[0][3])] and dev.programs[0][3] <= B.EW_MAX_REGS
    f = np.float32
    want_m = O.add(O.mul_scalar(m, f(0.9)), O.mul_scalar(g, f(1.0 - 0.9)))
    want_v = O.add(O.mul_scalar(v, f(0.999)), O.mul_scalar(O.mul(g, g), f(1.0 - 0.999)))
    denom = O.add(O.sqrt(O.mul_scalar(want_v, f(1.0 / (1.0 - 0.999 ** 3)))), eps)
    want_p = O.sub(O.mul_scalar(p, f(1.0 - 1e-3 * 0.01)),
                   O.mul_scalar(O.div(O.mul_scalar(want_m, f(1.0 / (1.0 - 0.9 ** 3))), denom), f(1e-3)))
    np.testing.assert_array_equal(got_p, want_p)
    np.testing.assert_array_equal(down(hb, m_new), want_m)
    np.testing.assert_array_equal(down(hb, v_new), want_v)
    assert len(dev.programs) == 1  # m_new and v_new were written by the same launch


@pytest.mark.parametrize("seed,n_leaves,n_ops,hold_every", [(1, 2, 6, 0), (2, 4, 25, 3), (3, 8, 70, 2), (4, 3, 150, 1)])
def test_random_chains_match_ops_run_one_by_one(fake, seed, n_leaves, n_ops, hold_every):
    dev, hb = fake
    rng = np.random.default_rng(seed)
    n = 37
    host = [rng.standard_normal(n).astype(np.float32) for _ in range(n_leaves)]
    dvals, hvals, held = [up(hb, a) for a in host], list(host), []
    sh = (n,)
    for k in range(n_ops):
        i, j, c = (int(rng.integers(0, len(dvals))) for _ in range(3))
        kind = int(rng.integers(0, 7))
        if kind == 0:
            d, h = hb.add(dvals[i], dvals[j], sh), O.add(hvals[i], hvals[j])
        elif kind == 1:
            d, h = hb.mul(dvals[i], dvals[j], sh), O.mul(hvals[i], hvals[j])
        elif kind == 2:
            s = float(rng.standard_normal())
            d, h = hb.mul_scalar(dvals[i], s, sh), O.mul_scalar(hvals[i], s)
        elif kind == 3:
            d, h = hb.sub(dvals[i], dvals[j], sh), O.sub(hvals[i], hvals[j])
        elif kind == 4:
            d, h = hb.relu_backward(dvals[i], dvals[j], sh), O.relu_backward(hvals[i], hvals[j])
        elif kind == 5:
            d, h = hb.div_backward_rhs(dvals[i], dvals[j], dvals[c], sh), O.div_backward_rhs(hvals[i], hvals[j],
                                                                                              hvals[c])
        else:
            d, h = hb.sqrt(hb.exp(dvals[i], sh), sh), O.sqrt(O.exp(hvals[i]))
        dvals.append(d)
        hvals.append(h)
        if hold_every and k % hold_every == 0:
            held.append((d, h))
    np.testing.assert_array_equal(down(hb, dvals[-1]), hvals[-1])
    for d, h in held:
        np.testing.assert_array_equal(down(hb, d), h)
    for n_in, n_out, n_ops_, n_regs in dev.programs:
        assert n_in <= B.EW_MAX_INPUTS and n_out <= B.EW_MAX_OUTPUTS and n_ops_ <= B.EW_MAX_OPS
        assert n_regs <= B.EW_MAX_REGS


def test_programs_are_reused_across_steps(fake):
    """One compiled program per chain structure; the scalars of each step (AdamW's bias
    corrections change every step) are written into it and each step computes with its own."""
    dev, hb = fake
    rng = np.random.default_rng(5)
    x0 = rng.standard_normal(64).astype(np.float32)
    x, want = up(hb, x0), x0
    for step in range(5):
        c = 0.5 + 0.25 * step
        y = hb.relu(hb.add(hb.mul_scalar(x, c, (64,)), x, (64,)), (64,))
        got = down(hb, y)
        want = O.relu(O.add(O.mul_scalar(want, c), want))
        np.testing.assert_array_equal(got, want)
        x = up(hb, got)
    assert len(hb._programs) == 1 and len(dev.programs) == 5


@pytest.mark.parametrize("in_shape,out_shape", [((1, 6), (5, 6)), ((5, 1), (5, 6)), ((1,), (4, 3)), ((6,), (2, 5, 6)),
                                                ((5, 1), (3, 5, 4)), ((1, 1), (1, 7)), ((2, 1, 3), (2, 4, 3))])
def test_broadcast_inputs_match_expand(fake, in_shape, out_shape):
    """Backend::expand of a contiguous block of dims is a program input read through
    (e / div) % mod; the result equals the oracle's expand (orca-backend-cpu/src/backend.rs:466-497)."""
    dev, hb = fake
    rng = np.random.default_rng(len(in_shape) * 10 + len(out_shape))
    a = rng.standard_normal(in_shape).astype(np.float32)
    d = up(hb, a.reshape(-1))
    want = O.expand(a, out_shape).reshape(-1)
    if B._broadcast_map(in_shape, out_shape) is None:
        pytest.skip("not a contiguous-block broadcast")
    got = hb.expand(d, in_shape, out_shape)
    assert got.pending
    np.testing.assert_array_equal(down(hb, hb.add(got, got, (want.size,))), O.add(want, want))


def test_one_element_constants_become_instruction_scalars(fake):
    """A one-element upload (the backward seed, Tensor::scalar) stays on the host: mul_scalar of
    it is computed there, and add / mul with its expand take it as an instruction's scalar,
    with either operand order, so the program reads only the other input and the constant is
    never uploaded.  Every value equals the ops run one by one."""
    dev, hb = fake
    rng = np.random.default_rng(8)
    n = 50
    f = np.float32
    x0 = np.abs(rng.standard_normal(n)).astype(np.float32)
    x = up(hb, x0)
    eps = hb.from_f32_slice((1,), np.array([1e-8], np.float32))
    seed = hb.from_f32_slice((1,), np.array([1.0], np.float32))
    assert eps.pending and eps._const == f(1e-8) and seed._const == 1.0
    g = hb.mul_scalar(seed, 1.0 / 7.0, (1,))
    assert g._const == f(1.0) * f(1.0 / 7.0)
    ge = hb.expand(g, (1,), (n,))
    denom = hb.add(hb.sqrt(x, (n,)), hb.expand(eps, (1,), (n,)), (n,))
    z = hb.accumulate_grad(hb.mul(ge, denom, (n,)), hb.expand(eps, (1,), (n,)))
    got = down(hb, z)
    want_denom = O.add(O.sqrt(x0), O.expand(np.array([1e-8], np.float32), (n,)))
    want_g = O.expand(O.mul_scalar(np.array([1.0], np.float32), f(1.0 / 7.0)), (n,))
    want = O.accumulate_grad(O.mul(want_g, want_denom), O.expand(np.array([1e-8], np.float32), (n,)))
    np.testing.assert_array_equal(got, want)
    assert dev.programs[-1][0] == 1  # one input: x
    assert eps._buf is None and seed._buf is None and g._buf is None  # never uploaded
    # a constant the device needs (here the input of exp) is uploaded at that use
    e = down(hb, hb.exp(hb.expand(eps, (1,), (n,)), (n,)))
    np.testing.assert_array_equal(e, O.exp(O.expand(np.array([1e-8], np.float32), (n,))))
    assert eps._buf is not None


def test_broadcast_map_rejects_split_blocks():
    assert B._broadcast_map((2, 1, 3), (2, 4, 3)) is None  # kept dims 0 and 2 around a broadcast one
    assert B._broadcast_map((1, 6), (5, 6)) == (1, 6)
    assert B._broadcast_map((5, 1), (5, 6)) == (6, 5)
    assert B._broadcast_map((1,), (4, 3)) == (1, 1)


def test_flushed_chains_leave_no_reference_cycles(fake):
    """Running a chain must not leave its storages in a reference cycle: their device
    buffers go back to the caching allocator as soon as the last reference drops, not
    at the next cyclic garbage collection (which would make the allocator's hipMalloc
    count grow step after step)."""
    import gc
    import weakref
    dev, hb = fake
    rng = np.random.default_rng(9)
    x = up(hb, rng.standard_normal(32).astype(np.float32))
    gc.disable()
    try:
        a = hb.mul_scalar(x, 2.0, (32,))
        b = hb.add(a, x, (32,))
        c = hb.relu(b, (32,))
        down(hb, c)
        watch = [weakref.ref(v) for v in (a, b, c)]
        del a, b, c
        assert all(w() is None for w in watch)
    finally:
        gc.enable()


@pytest.mark.parametrize("frac", [0.0, 0.3, 0.7, 0.999, 1.0])
def test_side_update_split_keeps_every_element_once(frac):
    """_split_rows (the fused optimizer's update on the second stream, split between a bounded
    and a full grid): every element of every segment lands in exactly one part, in order; a
    split segment is cut at a multiple of 64 elements with all its pointers advanced by the
    same bytes (so the halves stay 256-byte aligned); absent moment pointers stay absent."""
    sizes = [4096 * 4096, 4096, 40960, 10, 1, 64, 127]
    ptrs, base = [], 1 << 20
    for n in sizes:
        ptrs.append((base, base + (1 << 32), base + (2 << 32), None if n == 10 else base + (3 << 32),
                     None if n == 10 else base + (4 << 32), n))
        base += 4 * n + 256
    a, b = B._split_rows(ptrs, frac)
    cut = int(sum(sizes) * frac) // 64 * 64
    assert cut - 64 < sum(p[5] for p in a) <= cut or not b
    covered = {}
    for p in a + b:
        for k in range(5):
            if p[k] is not None:
                covered.setdefault(k, []).append((p[k], p[k] + 4 * p[5]))
    for k in range(5):
        spans = sorted(covered[k])
        want = sorted((q[k], q[k] + 4 * q[5]) for q in ptrs if q[k] is not None)
        merged = []
        for lo, hi in spans:
            if merged and merged[-1][1] == lo:
                merged[-1] = (merged[-1][0], hi)
            else:
                merged.append((lo, hi))
        assert merged == want, k
    for p in a + b:
        assert p[5] > 0
        src = next(q for q in ptrs if q[0] <= p[0] < q[0] + 4 * q[5])
        off = p[0] - src[0]
        assert off % 256 == 0
        assert all((p[k] is None) == (src[k] is None) for k in range(5))
        assert all(p[k] - src[k] == off for k in range(5) if p[k] is not None)
