"""CPU checks of the storage layer (orcaml_amd/csrc/storage.cpp) through the Python binding,
with the library's buffer-level entry points replaced by a host stand-in that computes with
the oracle's ops (tests/native/fake_device.cpp) and logs every launch.

Because each stand-in kernel is the oracle's own op (its matmul included), a composed
training step through the storage layer must equal the oracle's training loop bit for bit:
that pins which values every fused program, folded epilogue, deferred column sum and
second-stream update computes.  The launch log pins the decisions themselves: one program
per chain with the values held outside it as its outputs, folds taken only on products
nobody else holds, constants never uploaded, the optimizer pass split between the streams.
"""
from __future__ import annotations

import gc
import re

import numpy as np
import pytest

from oracle import oracle as O
from orcaml_amd import _lib, synth
from orcaml_amd import autodiff as A
from tests import fake_lib

N_REGS_MAX = _lib.EW_MAX_REGS


@pytest.fixture(scope="session")
def fake_path(tmp_path_factory):
    return fake_lib.build(str(tmp_path_factory.mktemp("fake_device")))


@pytest.fixture()
def lib(fake_path, monkeypatch):
    lib = fake_lib.load(fake_path)
    fake_lib.install(monkeypatch, lib)
    fake_lib.clear(lib)
    before = fake_lib.races(lib)
    yield lib
    gc.collect()
    # every access the two streams make is ordered by the events and joins the library placed
    assert fake_lib.races(lib) == before, [line for line in fake_lib.log(lib) if line.startswith("RACE")]


@pytest.fixture()
def ctx(lib):
    from orcaml_amd.device import Context

    c = Context(0)
    yield c
    gc.collect()
    c.close()


@pytest.fixture()
def hb(ctx):
    from orcaml_amd.backend import HipBackend

    return HipBackend(ctx)


def up(hb, a):
    a = np.ascontiguousarray(a, np.float32)
    return hb.from_f32_slice(a.shape, a)


def down(hb, s):
    return hb.to_f32_vec(s)


def programs(lib):
    """(inputs, outputs, ops, registers) of every program launched since the last clear."""
    return [tuple(int(v) for v in line.split()[1:5]) for line in fake_lib.log(lib) if line.startswith("program ")]


def test_adamw_chain_is_one_program_with_three_outputs(lib, hb):
    """The composed AdamW update of one parameter (python/orca/optim/adamw.py:66-99): the new
    parameter, m and v come from one program; the temporaries are not written."""
    rng = np.random.default_rng(1)
    n = 1001
    p, g = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    m, v = rng.standard_normal(n).astype(np.float32), np.abs(rng.standard_normal(n)).astype(np.float32)
    eps = np.full(n, 1e-8, np.float32)
    P, G, M, V, E = (up(hb, a) for a in (p, g, m, v, eps))
    fake_lib.clear(lib)
    sh = (n,)
    decayed = hb.mul_scalar(P, 1.0 - 1e-3 * 0.01, sh)
    m_new = hb.add(hb.mul_scalar(M, 0.9, sh), hb.mul_scalar(G, 1.0 - 0.9, sh), sh)
    v_new = hb.add(hb.mul_scalar(V, 0.999, sh), hb.mul_scalar(hb.mul(G, G, sh), 1.0 - 0.999, sh), sh)
    m_hat = hb.mul_scalar(m_new, 1.0 / (1.0 - 0.9 ** 3), sh)
    v_hat = hb.mul_scalar(v_new, 1.0 / (1.0 - 0.999 ** 3), sh)
    new_p = hb.sub(decayed, hb.mul_scalar(hb.div(m_hat, hb.add(hb.sqrt(v_hat, sh), E, sh), sh), 1e-3, sh), sh)
    del decayed, m_hat, v_hat
    got_p = down(hb, new_p)
    progs = programs(lib)
    assert len(progs) == 1 and progs[0][:3] == (5, 3, 15) and progs[0][3] <= N_REGS_MAX, progs
    f = np.float32
    want_m = O.add(O.mul_scalar(m, f(0.9)), O.mul_scalar(g, f(1.0 - 0.9)))
    want_v = O.add(O.mul_scalar(v, f(0.999)), O.mul_scalar(O.mul(g, g), f(1.0 - 0.999)))
    denom = O.add(O.sqrt(O.mul_scalar(want_v, f(1.0 / (1.0 - 0.999 ** 3)))), eps)
    want_p = O.sub(O.mul_scalar(p, f(1.0 - 1e-3 * 0.01)),
                   O.mul_scalar(O.div(O.mul_scalar(want_m, f(1.0 / (1.0 - 0.9 ** 3))), denom), f(1e-3)))
    np.testing.assert_array_equal(got_p, want_p)
    np.testing.assert_array_equal(down(hb, m_new), want_m)
    np.testing.assert_array_equal(down(hb, v_new), want_v)
    assert len(programs(lib)) == 1  # m_new and v_new were written by the same launch


@pytest.mark.parametrize("seed,n_leaves,n_ops,hold_every", [(1, 2, 6, 0), (2, 4, 25, 3), (3, 8, 70, 2), (4, 3, 150, 1)])
def test_random_chains_match_ops_run_one_by_one(lib, hb, seed, n_leaves, n_ops, hold_every):
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
    for n_in, n_out, n_ops_, n_regs in programs(lib):
        assert n_in <= _lib.EW_MAX_INPUTS and n_out <= _lib.EW_MAX_OUTPUTS and n_ops_ <= _lib.EW_MAX_OPS
        assert n_regs <= N_REGS_MAX


@pytest.mark.parametrize("rows,cols,is_max", [(16, 10, False), (16, 10, True), (37, 1, False), (5, 64, True),
                                               (300, 3, False), (9, 65, False), (9, 65, True)])
def test_row_reductions_run_with_their_chain(lib, ctx, rows, cols, is_max):
    """sum_to_shape / max_to_shape([R, C] -> [R, 1]) of a pending chain runs in the chain's own
    launch (C <= 64) and gives the bits of the chain's values reduced one op at a time: the
    eager backend's kernels and the oracle.  The chain's values held elsewhere are written by
    the same launch.  Rows with NaN, -inf and f32::MIN keep max_to_shape's strict `>` from
    f32::MIN (orca-backend-cpu/src/backend.rs:1336-1381)."""
    from orcaml_amd.backend import HipBackend

    rng = np.random.default_rng(rows * 100 + cols)
    a = rng.standard_normal((rows, cols)).astype(np.float32) * 4
    if cols > 1:
        a[0, 1] = np.nan
        a[min(1, rows - 1), :] = -np.inf
        a[min(2, rows - 1), 0] = np.finfo(np.float32).min
    m = rng.standard_normal((rows, 1)).astype(np.float32)
    t = rng.standard_normal((rows, cols)).astype(np.float32)
    sh, rs = (rows, cols), (rows, 1)
    got = {}
    for lazy in (True, False):
        hb = HipBackend(ctx, lazy=lazy)
        A_, M_, T_ = (up(hb, v.reshape(-1)) for v in (a, m, t))
        fake_lib.clear(lib)
        e = hb.exp(hb.sub(A_, hb.expand(M_, rs, sh), sh), sh)  # held: written by the reducing launch
        y = hb.mul_scalar(hb.mul(T_, e, sh), -1.0, sh)
        r = (hb.max_to_shape if is_max else hb.sum_to_shape)(y, sh, rs)
        got[lazy] = (down(hb, r), down(hb, e), down(hb, y))
        rows_launches = [line for line in fake_lib.log(lib) if line.startswith("program_rows ")]
        if lazy:  # (one column: the identity reduction, an instruction of the chain)
            fused = 1 < cols <= 64
            assert len(rows_launches) == int(fused) and len(programs(lib)) == 1 - int(fused), fake_lib.log(lib)
        del A_, M_, T_, e, y, r, hb
        gc.collect()
    for g, w in zip(got[True], got[False]):
        np.testing.assert_array_equal(g, w)
    e = O.exp(O.sub(a, O.expand(m, sh)))
    y = O.mul_scalar(O.mul(t, e), np.float32(-1.0))
    want = (O.max_to_shape if is_max else O.sum_to_shape)(y, rs)
    np.testing.assert_array_equal(got[True][0], np.asarray(want).reshape(-1))
    np.testing.assert_array_equal(got[True][1], np.asarray(e).reshape(-1))


def test_programs_are_reused_across_steps(lib, hb):
    """Each step's chain has the same structure and its own scalar (AdamW's bias corrections
    change every step); every step computes with its own."""
    rng = np.random.default_rng(5)
    x0 = rng.standard_normal(64).astype(np.float32)
    x, want = up(hb, x0), x0
    fake_lib.clear(lib)
    for step in range(5):
        c = 0.5 + 0.25 * step
        y = hb.relu(hb.add(hb.mul_scalar(x, c, (64,)), x, (64,)), (64,))
        got = down(hb, y)
        want = O.relu(O.add(O.mul_scalar(want, c), want))
        np.testing.assert_array_equal(got, want)
        x = up(hb, got)
    assert programs(lib) == [programs(lib)[0]] * 5


@pytest.mark.parametrize("in_shape,out_shape,lazy", [((1, 6), (5, 6), True), ((5, 1), (5, 6), True),
                                                     ((1,), (4, 3), True), ((6,), (2, 5, 6), True),
                                                     ((5, 1), (3, 5, 4), True), ((1, 1), (1, 7), True),
                                                     ((2, 1, 3), (2, 4, 3), False)])
def test_broadcast_inputs_match_expand(lib, hb, in_shape, out_shape, lazy):
    """Backend::expand of a contiguous block of dims is a program input read through
    (e / div) % mod; any other broadcast runs the expand kernel.  Both equal the oracle's
    expand (orca-backend-cpu/src/backend.rs:466-497)."""
    rng = np.random.default_rng(len(in_shape) * 10 + len(out_shape))
    a = rng.standard_normal(in_shape).astype(np.float32)
    d = up(hb, a.reshape(-1))
    want = O.expand(a, out_shape).reshape(-1)
    got = hb.expand(d, in_shape, out_shape)
    assert got.pending == lazy
    np.testing.assert_array_equal(down(hb, hb.add(got, got, (want.size,))), O.add(want, want))


def test_one_element_constants_become_instruction_scalars(lib, hb):
    """A one-element upload (the backward seed, Tensor::scalar) stays on the host: mul_scalar of
    it is computed there, and add / mul with its expand take it as an instruction's scalar,
    with either operand order, so the program reads only the other input and the constant is
    never uploaded.  Every value equals the ops run one by one."""
    rng = np.random.default_rng(8)
    n = 50
    f = np.float32
    x0 = np.abs(rng.standard_normal(n)).astype(np.float32)
    x = up(hb, x0)
    fake_lib.clear(lib)
    eps = hb.from_f32_slice((1,), np.array([1e-8], np.float32))
    seed = hb.from_f32_slice((1,), np.array([1.0], np.float32))
    const = 8  # ORCA_HIP_STORAGE_CONSTANT
    assert eps.pending and eps.flags() & const and seed.flags() & const
    g = hb.mul_scalar(seed, 1.0 / 7.0, (1,))
    assert g.flags() & const
    ge = hb.expand(g, (1,), (n,))
    denom = hb.add(hb.sqrt(x, (n,)), hb.expand(eps, (1,), (n,)), (n,))
    z = hb.accumulate_grad(hb.mul(ge, denom, (n,)), hb.expand(eps, (1,), (n,)))
    got = down(hb, z)
    want_denom = O.add(O.sqrt(x0), O.expand(np.array([1e-8], np.float32), (n,)))
    want_g = O.expand(O.mul_scalar(np.array([1.0], np.float32), f(1.0 / 7.0)), (n,))
    want = O.accumulate_grad(O.mul(want_g, want_denom), O.expand(np.array([1e-8], np.float32), (n,)))
    np.testing.assert_array_equal(got, want)
    assert programs(lib)[-1][0] == 1  # one input: x
    assert not any(line.startswith("upload") for line in fake_lib.log(lib))  # never uploaded
    assert eps.pending and seed.pending and g.pending
    # a constant the device needs (here the input of exp) is uploaded at that use
    e = down(hb, hb.exp(hb.expand(eps, (1,), (n,)), (n,)))
    np.testing.assert_array_equal(e, O.exp(O.expand(np.array([1e-8], np.float32), (n,))))
    assert "upload 1" in fake_lib.log(lib) and not eps.pending


def test_storages_are_freed_when_dropped(ctx, hb):
    """A run chain leaves nothing referenced: the blocks of its values go back to the caching
    allocator as soon as the last handle drops (no cycle waits for a collection)."""
    rng = np.random.default_rng(9)
    x = up(hb, rng.standard_normal(4096).astype(np.float32))
    base = ctx.mem_stats()["live"]
    gc.disable()
    try:
        for _ in range(3):
            a = hb.mul_scalar(x, 2.0, (4096,))
            b = hb.add(a, x, (4096,))
            c = hb.relu(b, (4096,))
            s = hb.sum_to_shape(c, (4096,), (4096,))
            down(hb, s)
            del a, b, c, s
            assert ctx.mem_stats()["live"] == base
    finally:
        gc.enable()


def test_identity_ops_give_back_the_same_storage(hb):
    """An identity expand, the identity sum_to_shape memo and reshape return the storage the
    binding already holds (the trait allows it: orca-backend-cpu/src/backend.rs:546)."""
    x = up(hb, np.arange(12, dtype=np.float32))
    assert hb.expand(x, (3, 4), (3, 4)) is x
    assert hb.reshape(x, (12,), (3, 4)) is x
    s = hb.sum_to_shape(x, (3, 4), (3, 4))
    assert hb.sum_to_shape(x, (3, 4), (3, 4)) is s


def test_times_one_gives_back_a_computed_value(lib, hb):
    """x * 1 is x bit for bit unless x is a signaling NaN: the gradient of a loss (computed
    by arithmetic) times the backward seed is that gradient, with no program; an upload (which
    may hold a signaling NaN) times one is still a multiply."""
    logits = up(hb, np.random.default_rng(3).standard_normal((4, 5)).astype(np.float32))
    onehot = up(hb, np.eye(5, dtype=np.float32)[[0, 2, 4, 1]])
    _, dl = hb.softmax_ce(logits, onehot, 4, 5)
    one = hb.from_f32_slice((1,), np.ones(1, np.float32))
    fake_lib.clear(lib)
    assert hb.mul(hb.expand(one, (1,), (4, 5)), dl, (4, 5)) is dl
    up_x = up(hb, np.arange(20, dtype=np.float32))
    y = hb.mul(hb.expand(one, (1,), (20,)), up_x, (20,))
    assert y is not up_x
    np.testing.assert_array_equal(down(hb, y), np.arange(20, dtype=np.float32))
    assert len(programs(lib)) == 1  # the multiply of the upload, run when read


def test_errors_carry_the_variant_fields(lib, hb, ctx):
    """Each failure maps to its OrcaError variant with the variant's fields
    (orca-core/src/error.rs:5-31), through orca_hip_last_error_info."""
    x = up(hb, np.zeros(12, np.float32))
    with pytest.raises(_lib.OrcaHipError) as e:
        hb.reshape(x, (12,), (5,))
    assert e.value.code == _lib.ERR_SHAPE
    assert e.value.fields["op"] == "reshape" and e.value.fields["expected"] == "12 elements"
    assert e.value.fields["got"] == "5 elements"
    with pytest.raises(_lib.OrcaHipError) as e:
        hb.cast(x, (12,), _lib.F32, _lib.BF16)
    assert e.value.code == _lib.ERR_UNSUPPORTED_DTYPE and e.value.fields["dtype"] == _lib.BF16
    assert "bfloat16" in str(e.value)
    assert hb.cast(x, (12,), _lib.F32, _lib.F32) is x
    with pytest.raises(_lib.OrcaHipError) as e:
        hb.relu(x, (12,), _lib.F64) if not hb.lazy else hb.zeros((3,), _lib.I32)
    assert e.value.code == _lib.ERR_UNSUPPORTED_DTYPE and e.value.fields["dtype"] == _lib.I32
    # a storage of another device
    from orcaml_amd.backend import HipBackend
    from orcaml_amd.device import Context

    other_ctx = Context(1)
    other = HipBackend(other_ctx)
    y = up(other, np.zeros(12, np.float32))
    with pytest.raises(_lib.OrcaHipError) as e:
        hb.add(x, y, (12,))
    assert e.value.code == _lib.ERR_DEVICE_MISMATCH
    assert e.value.fields["devices"] == [(2, 0), (2, 1)]
    del y, other
    gc.collect()
    other_ctx.close()


def test_lazy_and_eager_backends_share_storages(ctx):
    """Backends with other switches on one context take each other's storages (one planner
    per context); the eager one computes a pending value it is handed."""
    from orcaml_amd.backend import HipBackend

    lazy, eager = HipBackend(ctx), HipBackend(ctx, lazy=False)
    a = np.linspace(-2, 2, 10).astype(np.float32)
    x = up(lazy, a)
    r = lazy.relu(lazy.mul_scalar(x, 3.0, (10,)), (10,))
    assert r.pending
    y = eager.add(r, x, (10,))
    assert not y.pending
    np.testing.assert_array_equal(down(eager, y), O.add(O.relu(O.mul_scalar(a, np.float32(3.0))), a))


def composed(ad, params, x, onehot, kind, steps, fused=False, **opt):
    model = A.build_mlp(ad, params)
    if kind == "sgd":
        optim = A.SGD(model.parameters(), lr=opt["lr"], fused=fused)
    else:
        optim = A.AdamW(model.parameters(), lr=opt["lr"], weight_decay=opt.get("weight_decay", 0.01), fused=fused)
    xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
    loss_fn = A.CrossEntropyLoss(fused=fused)
    losses, grads, logits = [], None, None
    for _ in range(steps):
        optim.zero_grad()
        out = model(xt)
        loss = loss_fn(out, tt)
        losses.append(loss.to_list()[0])
        loss.backward()
        grads = [p.tensor.grad().numpy() for p in model.parameters()]
        logits = out.numpy()
        optim.step()
    return np.array(losses, np.float32), grads, logits, [p.tensor.numpy() for p in model.parameters()]


@pytest.mark.parametrize("kind,steps,switches", [
    ("sgd", 2, {}), ("adamw", 3, {}), ("adamw", 2, dict(lazy=False)), ("adamw", 2, dict(deferred=False)),
    ("adamw", 2, dict(fold=False)), ("sgd", 2, dict(lazy=False, deferred=False))])
def test_composed_steps_equal_the_oracle_loop_bit_for_bit(ctx, kind, steps, switches):
    """The reference frontend + tape (unchanged) over the storage layer: every fused program,
    folded epilogue and deferred column sum computes the ops' own f32 operations, so the
    losses, logits, gradients and parameters equal the oracle's training loop exactly."""
    from orcaml_amd.backend import HipBackend

    dims, B = (784, 48, 40, 10), 16
    params, x, labels, onehot = synth.mlp_problem(12, dims, B)
    opt = dict(lr=0.1) if kind == "sgd" else dict(lr=1e-3, weight_decay=0.01)
    ad = A.Autodiff(HipBackend(ctx, **switches))
    losses, grads, logits, new_params = composed(ad, params, x, onehot, kind, steps, **opt)
    ref = O.mlp_train(dims, params, x, onehot, O.make_opt(kind, **opt), steps=steps)
    np.testing.assert_array_equal(losses, ref["losses"])
    np.testing.assert_array_equal(logits, ref["logits"])
    for g, r in zip(grads, ref["grads"]):
        np.testing.assert_array_equal(g.reshape(r.shape), r)
    for p, r in zip(new_params, ref["params"]):
        np.testing.assert_array_equal(p.reshape(r.shape), r)


def test_composed_step_folds_and_fuses(lib, ctx):
    """What one steady-state composed step launches: the Linear forwards as products with the
    bias (+ ReLU) epilogue, each ReluBackward as the next product's mask epilogue, the weight
    gradients with their bias column sums in one launch, the head's weight, bias and masked
    input gradients from one grid, the loss's row sums in the launches of the chains they
    reduce, and no single elementwise op (only the logits' row maximum, its backward and the
    batch sum run as kernels of their own)."""
    from orcaml_amd.backend import HipBackend

    dims, B = (784, 48, 40, 10), 16
    params, x, labels, onehot = synth.mlp_problem(13, dims, B)
    ad = A.Autodiff(HipBackend(ctx))
    composed(ad, params, x, onehot, "adamw", 1, lr=1e-3)
    model = A.build_mlp(ad, params)
    optim = A.AdamW(model.parameters(), lr=1e-3, weight_decay=0.01)
    xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
    fake_lib.clear(lib)
    optim.zero_grad()
    loss = A.CrossEntropyLoss()(model(xt), tt)
    loss.backward()
    optim.step()
    log = fake_lib.log(lib)
    gemms = [line for line in log if line.startswith("gemm ")]
    epis = sorted(int(line.split()[line.split().index("epi") + 1]) for line in gemms)
    # forward: two hidden layers with bias + ReLU (pre-activation kept for ReluBackward) and the
    # head with its bias; backward: dX through the two ReLUs with the mask epilogue
    assert epis.count(_lib.EPI_BIAS_RELU_PRE) == 2 and epis.count(_lib.EPI_BIAS) == 1, gemms
    assert epis.count(_lib.EPI_RELU_MASK) + epis.count(_lib.EPI_RELU_MASK_PRE) == 1, gemms
    # the hidden layers' dW with its db; the head's dW, db and masked dX from one grid
    assert sum(line.startswith("matmul_colsum ") for line in log) == 2, log
    assert sum(line.startswith("narrow_linear_backward 16x40x10 mask") for line in log) == 1, log
    # the softmax's and its backward's row sums run with the chains before them
    assert sum(line.startswith("program_rows ") for line in log) == 4, log
    reductions = ("op max_to_shape", "op sum_to_shape", "op max_to_shape_backward")
    assert not [line for line in log if line.startswith("op ") and line not in reductions], log


def test_fused_step_hands_the_loss_gradient_on_unchanged(lib, ctx):
    """With the fused loss, the loss gradient times the seed of one and the identity
    sum_to_shape of the head's bias add are the gradient itself (it holds no -0 and no
    signaling NaN): the head's backward grid reads softmax_ce's output, and a steady-state
    step runs no elementwise program at all."""
    from orcaml_amd.backend import HipBackend

    dims, B = (784, 48, 40, 10), 16
    params, x, labels, onehot = synth.mlp_problem(16, dims, B)
    ad = A.Autodiff(HipBackend(ctx))
    composed(ad, params, x, onehot, "adamw", 1, fused=True, lr=1e-3)
    model = A.build_mlp(ad, params)
    optim = A.AdamW(model.parameters(), lr=1e-3, weight_decay=0.01, fused=True)
    xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
    fake_lib.clear(lib)
    optim.zero_grad()
    A.CrossEntropyLoss(fused=True)(model(xt), tt).backward()
    optim.step()
    log = fake_lib.log(lib)
    assert not [line for line in log if line.startswith("program")], log
    i = next(k for k, line in enumerate(log) if line.startswith("softmax_ce"))
    assert log[i + 1].startswith("narrow_linear_backward 16x40x10 mask"), log


@pytest.mark.parametrize("kind", ["adamw", "sgd"])
def test_composed_update_runs_beside_the_backward_products(lib, ctx, kind):
    """The reference's own composed optimizer (unchanged user code): an update program whose
    inputs were all computed before the backward's last product runs on the second stream,
    after the mark of the product its gradient came from, with every output written there
    (the program's launch is the only thing between the switch to the second stream, its
    wait and its mark), and every later access to what it read or wrote is ordered after it
    (the stand-in's happens-before check).  The values equal the same steps without overlap
    and the oracle's loop."""
    from orcaml_amd.backend import HipBackend

    dims, B = (784, 48, 40, 10), 16
    params, x, labels, onehot = synth.mlp_problem(15, dims, B)
    opt = dict(lr=0.1) if kind == "sgd" else dict(lr=1e-3, weight_decay=0.01)
    out = {}
    for overlap in (True, False):
        fake_lib.clear(lib)
        ad = A.Autodiff(HipBackend(ctx, overlap=overlap))
        out[overlap] = composed(ad, params, x, onehot, kind, 3, **opt)
        log = fake_lib.log(lib)
        side = [i for i, line in enumerate(log) if line.startswith("program ") and line.endswith(" side")]
        if overlap:
            # the updates of layers 1 and 2 (flushed when the next step or the final read needs them)
            assert len(side) >= 4, log
            for i in side:
                # a bounded part first (beside the product after its mark), or the rest on the full grid
                assert re.match(r"side (-1|[1-9])", log[i - 2]) and log[i - 1].startswith("wait ") and \
                    log[i - 1].endswith(" side"), log[i - 3:i + 3]
                if re.match(r"side [1-9]", log[i - 2]) and log[i + 1] == "main":
                    assert log[i + 2] == "side -1", log[i:i + 4]  # its remainder follows
                else:
                    assert log[i + 1].startswith("record ") and log[i + 1].endswith(" side") and log[i + 2] == "main"
            # and whatever reads what they wrote waits for them: the stand-in's order check
            assert not [line for line in log if line.startswith("RACE")], log
        else:
            assert not side and not any(line.startswith("side ") for line in log)
    for a, b in zip(out[True][3], out[False][3]):
        np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(out[True][0], out[False][0])
    ref = O.mlp_train(dims, params, x, onehot, O.make_opt(kind, **opt), steps=3)
    for p, r in zip(out[True][3], ref["params"]):
        np.testing.assert_array_equal(p.reshape(r.shape), r)


@pytest.mark.parametrize("kind", ["adamw", "sgd"])
def test_fused_update_on_the_second_stream_changes_no_bit(lib, ctx, kind):
    """The fused optimizer's pass with overlap: the parameters whose gradients came from an
    earlier weight-gradient product are updated on the second stream (split between a bounded
    and a full grid: every element exactly once), the rest on the context stream.  The values
    equal the pass without overlap and the composed oracle loop."""
    from orcaml_amd.backend import HipBackend

    dims, B = (784, 64, 48, 10), 16
    params, x, labels, onehot = synth.mlp_problem(14, dims, B)
    opt = dict(lr=0.1) if kind == "sgd" else dict(lr=1e-3, weight_decay=0.01)
    out = {}
    for overlap in (True, False):
        fake_lib.clear(lib)
        ad = A.Autodiff(HipBackend(ctx, overlap=overlap, side_frac=0.6))
        out[overlap] = composed(ad, params, x, onehot, kind, 3, fused=True, **opt)
        log = fake_lib.log(lib)
        side = [line for line in log if line.startswith(f"{kind}_multi") and line.endswith(" side")]
        if overlap:
            # in every step (the backward products leave marks whenever overlap is allowed), layers
            # >= 1 (W, b of layers 1 and 2) go to the second stream
            n_side = sum(int(line.split()[2]) for line in side)
            per_step = sum(int(np.prod(p.shape)) for p in params[2:])
            assert n_side == 3 * per_step, (side, per_step)
            assert any(re.match(r"side [1-9]", line) for line in log) and "side -1" in log
        else:
            assert not side
    for a, b in zip(out[True][3], out[False][3]):
        np.testing.assert_array_equal(a, b)
    ref = O.mlp_train(dims, params, x, onehot, O.make_opt(kind, **opt), steps=3)
    for p, r in zip(out[True][3], ref["params"]):
        np.testing.assert_array_equal(p.reshape(r.shape), r)
