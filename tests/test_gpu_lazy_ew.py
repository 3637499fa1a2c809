"""Lazy elementwise ops of HipBackend run as fused programs (orca_hip_ew_program):
bit-identical to the same trait ops run one kernel at a time
(orca-backend-cpu/src/backend.rs elementwise semantics), for single ops on
special values, for random chains with shared subexpressions and values
referenced from outside the chain, for chains larger than the interpreter's
registers, across in-place updates of an input, and for whole composed
training steps."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from orcaml_amd import _lib, synth
from orcaml_amd import autodiff as A
from orcaml_amd.backend import HipBackend

pytestmark = pytest.mark.gpu


def up(hb, a):
    a = np.ascontiguousarray(a, np.float32)
    return hb.from_f32_slice(a.shape, a.reshape(-1))


def special(rng, n):
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    x[::17] = 0.0
    x[1::19] = -0.0
    x[2::23] = np.nan
    x[3::29] = np.inf
    x[4::31] = -np.inf
    x[5::37] = 1e-40
    return x


UNARY = ["relu", "sigmoid", "exp", "log", "sqrt"]
BINARY = ["add", "sub", "mul", "div", "relu_backward", "sigmoid_backward", "exp_backward", "log_backward",
          "sqrt_backward", "div_backward_lhs"]


@pytest.fixture(scope="module")
def pair(ctx):
    return HipBackend(ctx), HipBackend(ctx, lazy=False)


@pytest.fixture(params=[0, 2], ids=["interpreted", "compiled"])
def jit(request, ctx):
    """Runs the test with every program interpreted, then with every program compiled at
    its first use (orca_hip_ew_set_jit); the compiled run must not fall back.  (A test whose
    ops leave no chain to run -- the fused loss and update -- launches no program at all.)"""
    before = ctx.ew_jit_stats()
    ctx.set_ew_jit(request.param)
    yield request.param
    ctx.set_ew_jit(1)
    after = ctx.ew_jit_stats()
    assert after["failures"] == before["failures"]
    if request.param == 2:
        none_expected = request.node.callspec.params.get("fused", False)
        assert (after["compiled_launches"] > before["compiled_launches"]) != none_expected
        assert after["interpreted"] == before["interpreted"]
    else:
        assert after["compiled_launches"] == before["compiled_launches"]


@pytest.mark.parametrize("n", [1, 7, 4096, 1000003])
def test_each_op_bit_identical(pair, jit, n):
    lazy, eager = pair
    rng = np.random.default_rng(n)
    a, b, c = special(rng, n), special(rng, n), special(rng, n)
    shape = (n,)
    for be in pair:
        be._a, be._b, be._c = up(be, a), up(be, b), up(be, c)
    got, want = {}, {}
    for be, res in ((lazy, got), (eager, want)):
        for op in UNARY:
            res[op] = getattr(be, op)(be._a, shape)
        for op in BINARY:
            res[op] = getattr(be, op)(be._a, be._b, shape)
        res["mul_scalar"] = be.mul_scalar(be._a, -0.37, shape)
        res["div_backward_rhs"] = be.div_backward_rhs(be._a, be._b, be._c, shape)
        res["accumulate_grad"] = be.accumulate_grad(be._a, be._b)
        res["sum_ident"] = be.sum_to_shape(be._b, shape, shape)
        res["max_ident"] = be.max_to_shape(be._c, shape, shape)
    assert got["relu"].pending and not want["relu"].pending
    for k in want:
        np.testing.assert_array_equal(lazy.to_f32_vec(got[k]), eager.to_f32_vec(want[k]), err_msg=k)


def _random_chain(be, leaves, rng, n_ops, keep):
    """A random DAG of elementwise ops over `leaves`; every `keep`-th value is also
    returned (held from outside the chain)."""
    vals = list(leaves)
    held = []
    shape = (leaves[0].n,)
    for k in range(n_ops):
        pick = lambda: vals[int(rng.integers(0, len(vals)))]  # noqa: E731
        kind = int(rng.integers(0, 6))
        if kind == 0:
            v = be.add(pick(), pick(), shape)
        elif kind == 1:
            v = be.mul(pick(), pick(), shape)
        elif kind == 2:
            v = be.mul_scalar(pick(), float(rng.standard_normal()), shape)
        elif kind == 3:
            v = be.sub(pick(), pick(), shape)
        elif kind == 4:
            v = be.relu_backward(pick(), pick(), shape)
        else:
            v = be.sqrt(be.add(be.mul(pick(), pick(), shape), pick(), shape), shape)
        vals.append(v)
        if keep and k % keep == 0:
            held.append(v)
    return vals[-1], held


@pytest.mark.parametrize("seed,n_leaves,n_ops,keep", [(1, 2, 5, 0), (2, 4, 20, 3), (3, 8, 40, 2), (4, 3, 60, 1),
                                                      (5, 6, 120, 7)])
def test_random_chains_bit_identical(pair, jit, seed, n_leaves, n_ops, keep):
    """Shared subexpressions, values held from outside (written by the same launch), chains
    past the interpreter's 16 registers and 64 instructions (run in parts)."""
    n = 10007
    out = []
    for be in pair:
        rng = np.random.default_rng(seed)
        leaves = [up(be, rng.standard_normal(n).astype(np.float32)) for _ in range(n_leaves)]
        root, held = _random_chain(be, leaves, rng, n_ops, keep)
        out.append([be.to_f32_vec(root)] + [be.to_f32_vec(h) for h in held])
    for g, w in zip(*out):
        np.testing.assert_array_equal(g, w)


def test_pending_value_survives_in_place_update_of_its_input(pair):
    """adamw_step_ updates p, m, v in place: a pending op reading p is run first, on the old p."""
    lazy, _ = pair
    rng = np.random.default_rng(9)
    n = 5000
    p0 = rng.standard_normal(n).astype(np.float32)
    p, g = up(lazy, p0), up(lazy, rng.standard_normal(n).astype(np.float32))
    m, v = up(lazy, np.zeros(n, np.float32)), up(lazy, np.zeros(n, np.float32))
    twice = lazy.mul_scalar(p, 2.0, (n,))
    assert twice.pending
    lazy.adamw_step_(p, g, m, v, n, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1)
    np.testing.assert_array_equal(lazy.to_f32_vec(twice), p0 * np.float32(2.0))


def test_constant_updated_in_place_is_read_from_the_device_afterwards(pair):
    """A one-element upload folded into a pending chain as an instruction's scalar keeps its
    value there; once an in-place update changes it, later ops read the new value."""
    lazy, eager = pair
    rng = np.random.default_rng(12)
    n = 4096
    x0 = rng.standard_normal(n).astype(np.float32)
    x = up(lazy, x0)
    c = lazy.from_f32_slice((1,), np.array([0.75], np.float32))
    g = lazy.from_f32_slice((1,), np.array([0.5], np.float32))
    before = lazy.add(x, lazy.expand(c, (1,), (n,)), (n,))
    assert before.pending
    lazy.sgd_step_(c, g, 1, 0.5)  # c = 0.75 - 0.5 * 0.5
    after = lazy.mul(lazy.expand(c, (1,), (n,)), x, (n,))
    np.testing.assert_array_equal(lazy.to_f32_vec(before), O.add(x0, np.full(n, 0.75, np.float32)))
    np.testing.assert_array_equal(lazy.to_f32_vec(after), O.mul(np.full(n, 0.5, np.float32), x0))
    np.testing.assert_array_equal(lazy.to_f32_vec(c), np.array([0.5], np.float32))


def test_one_launch_for_a_chain(pair, ctx):
    lazy, _ = pair
    rng = np.random.default_rng(3)
    n = 1 << 20
    a, b = up(lazy, rng.standard_normal(n).astype(np.float32)), up(lazy, rng.standard_normal(n).astype(np.float32))
    ctx.sync()
    ctx.prof_reset()
    ctx.prof_enable(True)
    r = lazy.relu(lazy.add(lazy.mul_scalar(a, 0.5, (n,)), b, (n,)), (n,))
    lazy.to_f32_vec(r)
    ctx.prof_enable(False)
    names = {k["name"]: k["launches"] for k in ctx.prof_report()["kernels"]}
    assert names == {"ew_program": 1}, names


def test_structures_compile_at_their_second_use_and_share_kernels_across_scalars(pair, ctx):
    """Default mode: a chain's first run is interpreted, its second compiles the structure and
    runs the compiled kernel; a third run with other scalars and another length reuses it.
    Every run equals the ops run one by one."""
    lazy, eager = pair
    ctx.set_ew_jit(1)
    rng = np.random.default_rng(21)
    runs = [(4099, 0.5, -1.25), (4099, 0.75, 2.0), (1 << 16, -3.0, 0.125)]
    deltas = []
    for n, s1, s2 in runs:
        a, b = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
        out = []
        before = ctx.ew_jit_stats()
        for be in pair:
            # a structure no other test builds: sigmoid_backward of a scaled sum, then relu
            x, y = up(be, a), up(be, b)
            r = be.relu(be.sigmoid_backward(be.mul_scalar(be.add(x, y, (n,)), s1, (n,)), be.mul_scalar(y, s2, (n,)),
                                            (n,)), (n,))
            out.append(be.to_f32_vec(r))
        after = ctx.ew_jit_stats()
        deltas.append({k: after[k] - before[k] for k in after})
        np.testing.assert_array_equal(out[0], out[1])
    assert deltas[0] == {"interpreted": 1, "compiled_launches": 0, "compiles": 0, "failures": 0}
    assert deltas[1] == {"interpreted": 0, "compiled_launches": 1, "compiles": 1, "failures": 0}
    assert deltas[2] == {"interpreted": 0, "compiled_launches": 1, "compiles": 0, "failures": 0}


def _composed(hb, dims, params, x, onehot, kind, fused, steps):
    ad = A.Autodiff(hb)
    model = A.build_mlp(ad, params)
    opt = (A.SGD(model.parameters(), lr=0.1, fused=fused) if kind == "sgd" else
           A.AdamW(model.parameters(), lr=1e-3, weight_decay=0.01, fused=fused))
    xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
    losses, grads = [], None
    for _ in range(steps):
        opt.zero_grad()
        loss = A.CrossEntropyLoss(fused=fused)(model(xt), tt)
        loss.backward()
        losses.append(loss.to_list()[0])
        grads = [p.tensor.grad().numpy() for p in model.parameters()]
        opt.step()
    return losses, grads, [p.tensor.numpy() for p in model.parameters()]


@pytest.mark.parametrize("kind,fused", [("sgd", False), ("adamw", False), ("adamw", True)])
@pytest.mark.parametrize("dims,batch", [((784, 128, 128, 10), 64), ((784, 1024, 1024, 10), 256)])
def test_composed_steps_bit_identical(pair, jit, kind, fused, dims, batch):
    """Three steps of the reference frontend through the tape: lazy fused programs change no bit
    of the losses, gradients or parameters."""
    params, x, labels, onehot = synth.mlp_problem(7, dims, batch)
    runs = [_composed(be, dims, params, x, onehot, kind, fused, 3) for be in pair]
    (l1, g1, p1), (l2, g2, p2) = runs
    assert l1 == l2
    for a, b in zip(g1 + p1, g2 + p2):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("in_shape,out_shape", [
    ((1, 4096), (1024, 4096)),  # row broadcast, float4 loads
    ((1, 1048576), (4, 1048576)),
    ((1024, 1), (1024, 10)),  # column broadcast, index per element
    ((1000, 1), (1000, 12)),  # column broadcast, one value per group of 4
    ((3, 1), (3, 1048579)),  # a large divisor
    ((1, 1000003), (3, 1000003)),  # a large odd modulus
    ((1,), (333, 7)), ((1, 1), (4097, 1)),  # one value
    ((6,), (2, 5, 6)), ((5, 1), (3, 5, 4)), ((1, 10), (64, 10)),
    ((7, 1, 3), (7, 4, 3))])
def test_broadcast_expand_bit_identical(pair, jit, in_shape, out_shape):
    """expand as a program input read through (e / div) % mod (row, column and single-value
    broadcasts, a middle block, large divisors and moduli, a rank-3 case the map does not
    cover) equals the expand kernel's result, also when combined with other ops."""
    lazy, eager = pair
    rng = np.random.default_rng(sum(out_shape))
    a = rng.standard_normal(in_shape).astype(np.float32)
    b = rng.standard_normal(out_shape).astype(np.float32)
    n = int(np.prod(out_shape))
    out = []
    for be in pair:
        da, db = up(be, a.reshape(-1)), up(be, b.reshape(-1))
        e = be.expand(da, in_shape, out_shape)
        out.append((be.to_f32_vec(be.mul(be.add(e, db, out_shape), e, out_shape)), be.to_f32_vec(e)))
    np.testing.assert_array_equal(out[0][0], out[1][0])
    np.testing.assert_array_equal(out[0][1], out[1][1])
    np.testing.assert_array_equal(out[1][1], O.expand(a, out_shape).reshape(n))


def test_broadcast_beyond_2_31_elements(pair, jit):
    """Past 2^31 output elements the program input's index takes the 64-bit division; the
    expanded sum equals that of the expand kernel (its column-broadcast kernel, another
    implementation), compared on the device: the sum of squared differences of the
    2^31 + 10 elements is zero only when every element agrees."""
    lazy, eager = pair
    rows = (2 ** 31 + 10) // 3
    in_shape, out_shape = (rows, 1), (rows, 3)
    n = rows * 3
    assert n >= 2 ** 31
    a = np.random.default_rng(77).standard_normal(rows).astype(np.float32)
    da = up(lazy, a)
    got = lazy.add(lazy.expand(da, in_shape, out_shape), lazy.expand(da, in_shape, out_shape), out_shape)
    want = eager.add(eager.expand(da, in_shape, out_shape), eager.expand(da, in_shape, out_shape), out_shape)
    d = eager.sub(got, want, out_shape)
    ss = eager.sum_to_shape(eager.mul(d, d, out_shape), out_shape, (1,))
    assert eager.to_f32_vec(ss)[0] == 0.0


@pytest.mark.parametrize("n", [1, 6, 4099])
def test_unaligned_inputs_take_the_element_kernel(ctx, pair, jit, n):
    """Inputs that are not 16-byte aligned (slices one float into an arena) run the
    element-at-a-time kernel, interpreted and compiled; it equals the ops run one by one."""
    lazy, eager = pair
    rng = np.random.default_rng(n + 40)
    a, b = special(rng, n), special(rng, n)
    arena = lazy.arena(2 * n + 8)
    _lib.call("orca_hip_h2d", ctx.handle, arena.ptr + 4, a.ctypes.data_as(ctypes.c_void_p), a.nbytes)
    _lib.call("orca_hip_h2d", ctx.handle, arena.ptr + 4 * (n + 5), b.ctypes.data_as(ctypes.c_void_p), b.nbytes)
    va, vb = lazy.view(arena, 1, n), lazy.view(arena, n + 5, n)
    sh = (n,)
    got = lazy.sqrt(lazy.add(lazy.mul(va, vb, sh), lazy.relu(va, sh), sh), sh)
    want = eager.sqrt(eager.add(eager.mul(va, vb, sh), eager.relu(va, sh), sh), sh)
    np.testing.assert_array_equal(lazy.to_f32_vec(got), eager.to_f32_vec(want))


@pytest.mark.parametrize("rows,cols", [(1024, 10), (1, 64), (1000, 64), (4097, 3), (255, 2), (100003, 7),
                                       (33, 4)])
@pytest.mark.parametrize("is_max", [False, True], ids=["sum", "max"])
def test_row_reductions_with_their_chain_bit_identical(pair, ctx, rows, cols, is_max):
    """sum_to_shape / max_to_shape([R, C] -> [R, 1]) of a pending chain runs in the chain's
    launch (orca_hip_ew_program_rows) and equals the eager backend's chain and reduction
    kernels bit for bit, over special values (NaN, +-inf, -0, subnormals, whole rows of -inf,
    f32::MIN), with a per-row and a per-column broadcast input.  Against the oracle: the
    reduction and every op but exp bit for bit on the device's values; exp within the device
    library's ulp of glibc's."""
    lazy, eager = pair
    rng = np.random.default_rng(rows + 7 * cols)
    n = rows * cols
    a = special(rng, n).reshape(rows, cols)
    a[min(1, rows - 1), :] = -np.inf
    a[min(2, rows - 1), 0] = np.finfo(np.float32).min
    m = rng.standard_normal((rows, 1)).astype(np.float32)
    t = special(rng, n).reshape(rows, cols)
    bias = rng.standard_normal((1, cols)).astype(np.float32)
    sh, rs, cs = (rows, cols), (rows, 1), (1, cols)
    got = {}
    ctx.prof_enable(True)
    ctx.prof_reset()
    for be in pair:
        A_, M_, T_, B_ = up(be, a), up(be, m), up(be, t), up(be, bias)
        e = be.exp(be.sub(A_, be.expand(M_, rs, sh), sh), sh)
        y = be.mul_scalar(be.mul(be.add(T_, be.expand(B_, cs, sh), sh), e, sh), -1.0, sh)
        r = (be.max_to_shape if is_max else be.sum_to_shape)(y, sh, rs)
        got[be is lazy] = (be.to_f32_vec(r), be.to_f32_vec(e), be.to_f32_vec(y))
    names = {k["name"] for k in ctx.prof_report()["kernels"]}
    ctx.prof_enable(False)
    assert "ew_program_rows" in names, names
    for g, w in zip(got[True], got[False]):
        np.testing.assert_array_equal(g, w)
    e, y = got[True][1].reshape(sh), got[True][2].reshape(sh)
    np.testing.assert_allclose(e, O.exp(O.sub(a, O.expand(m, sh))), rtol=4e-7, atol=0)
    np.testing.assert_array_equal(y, O.mul_scalar(O.mul(O.add(t, O.expand(bias, sh)), e), np.float32(-1.0)))
    want = (O.max_to_shape if is_max else O.sum_to_shape)(y, rs)
    np.testing.assert_array_equal(got[True][0], np.asarray(want).reshape(-1))
