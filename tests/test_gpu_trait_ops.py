"""GPU parity of every Backend trait op of HipBackend against the CPU oracle,
and of the unchanged composed training step (reference frontend replayed
through the tape) on HipBackend."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from orcaml_amd import autodiff as A
from orcaml_amd import _lib, synth
from orcaml_amd._lib import OrcaHipError
from tests.util import assert_close, assert_close_scaled

pytestmark = pytest.mark.gpu


def up(hb, a):
    a = np.ascontiguousarray(a, np.float32)
    return hb.from_f32_slice(a.shape, a.reshape(-1))


def down(hb, s, shape):
    return hb.to_f32_vec(s).reshape(shape)


def special_values(rng, shape):
    x = rng.standard_normal(shape).astype(np.float32) * 3
    flat = x.reshape(-1)
    flat[::17] = 0.0
    flat[1::19] = -0.0
    flat[2::23] = np.nan
    flat[3::29] = np.inf
    flat[4::31] = -np.inf
    flat[5::37] = 1e-40  # denormal
    return x


BIT_EXACT_BINARY = ["add", "sub", "mul", "div", "relu_backward", "exp_backward", "log_backward", "sqrt_backward",
                    "div_backward_lhs"]


@pytest.mark.parametrize("op", BIT_EXACT_BINARY)
@pytest.mark.parametrize("shape", [(1,), (3, 5), (64, 131), (1024, 4096)])
def test_binary_ops_bit_exact(hb, op, shape):
    rng = np.random.default_rng(len(shape) * 100 + shape[-1])
    a, b = special_values(rng, shape), special_values(rng, shape)
    got = down(hb, getattr(hb, op)(up(hb, a), up(hb, b), shape), shape)
    want = getattr(O, op)(a, b)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("shape", [(7,), (256, 333)])
def test_unary_and_scalar_ops(hb, shape):
    rng = np.random.default_rng(shape[-1])
    a = special_values(rng, shape)
    for op in ("relu", "sqrt"):  # correctly rounded / exact: bit-identical
        np.testing.assert_array_equal(down(hb, getattr(hb, op)(up(hb, a), shape), shape), getattr(O, op)(a))
    for s in (-1.0, 0.1, 1.0 / 1024):
        np.testing.assert_array_equal(down(hb, hb.mul_scalar(up(hb, a), s, shape), shape), O.mul_scalar(a, s))
    finite = rng.uniform(-20, 20, shape).astype(np.float32)
    pos = rng.uniform(1e-8, 50, shape).astype(np.float32)
    for op, x in (("exp", finite), ("log", pos), ("sigmoid", finite)):  # libm vs device math: ulp-level
        got, want = down(hb, getattr(hb, op)(up(hb, x), shape), shape), getattr(O, op)(x)
        np.testing.assert_allclose(got, want, rtol=4e-7, atol=0)
    clamp = np.array([0.0, -1.0, 1e-9, np.nan], np.float32)  # log clamps at 1e-7 (backend.rs:577)
    got = down(hb, hb.log(up(hb, clamp), (4,)), (4,))
    np.testing.assert_allclose(got, O.log(clamp), rtol=4e-7, atol=0)
    assert len(set(got.tolist())) == 1  # every clamped input gives ln(1e-7)
    g, l, r = (rng.standard_normal(shape).astype(np.float32) for _ in range(3))
    np.testing.assert_array_equal(down(hb, hb.div_backward_rhs(up(hb, g), up(hb, l), up(hb, r), shape), shape),
                                  O.div_backward_rhs(g, l, r))
    y = rng.uniform(0, 1, shape).astype(np.float32)
    np.testing.assert_array_equal(down(hb, hb.sigmoid_backward(up(hb, g), up(hb, y), shape), shape),
                                  O.sigmoid_backward(g, y))
    np.testing.assert_array_equal(down(hb, hb.accumulate_grad(up(hb, g), up(hb, l)), shape),
                                  O.accumulate_grad(g, l))


@pytest.mark.parametrize("in_shape,out_shape", [((1, 7), (5, 7)), ((5, 1), (5, 9)), ((1,), (3, 4)),
                                                ((2, 1, 3), (4, 2, 5, 3)), ((1, 4096), (1024, 4096)),
                                                ((2, 3, 1), (2, 3, 5)), ((1, 1, 8), (3, 2, 8)), ((7,), (7,)),
                                                ((1024, 1), (1024, 10)), ((1,), (33, 65)), ((1, 1), (4096, 16)),
                                                ((1, 100), (1000, 100)), ((70,), (3, 300, 70)),
                                                ((1, 1, 33), (2, 129, 33)), ((1, 10), (1024, 10)),
                                                ((1, 4100), (300, 4100)), ((1, 64), (127, 64)), ((1, 5), (128, 5)),
                                                # at most 16 columns: 1024-row slabs, ragged last slab
                                                ((1, 16), (8192, 16)), ((1, 3), (2049, 3)), ((1, 10), (3000, 10))])
def test_expand_and_sum_to_shape_bit_exact(hb, in_shape, out_shape):
    rng = np.random.default_rng(sum(out_shape))
    a = rng.standard_normal(in_shape).astype(np.float32)
    np.testing.assert_array_equal(down(hb, hb.expand(up(hb, a), in_shape, out_shape), out_shape),
                                  O.expand(a, out_shape))
    big = rng.standard_normal(out_shape).astype(np.float32)
    np.testing.assert_array_equal(down(hb, hb.sum_to_shape(up(hb, big), out_shape, in_shape), in_shape),
                                  O.sum_to_shape(big, in_shape))


def test_sum_to_scalar_and_rank_padding(hb):
    rng = np.random.default_rng(1)
    a = rng.standard_normal((1024, 1)).astype(np.float32)
    np.testing.assert_array_equal(down(hb, hb.sum_to_shape(up(hb, a), (1024, 1), (1,)), (1,)),
                                  O.sum_to_shape(a, (1,)))
    with pytest.raises(OrcaHipError):
        hb.expand(up(hb, a), (1024, 1), (3, 7))


@pytest.mark.parametrize("shape", [(64, 10), (8192, 10), (3, 4, 5)])
def test_max_to_shape_and_backward_bit_exact(hb, shape):
    rng = np.random.default_rng(shape[0])
    x = rng.integers(-3, 3, shape).astype(np.float32)  # many ties
    x.reshape(-1)[::11] = np.nan
    out_shape = shape[:-1] + (1,)
    y = O.max_to_shape(x, out_shape)
    np.testing.assert_array_equal(down(hb, hb.max_to_shape(up(hb, x), shape, out_shape), out_shape), y)
    g = rng.standard_normal(out_shape).astype(np.float32)
    np.testing.assert_array_equal(
        down(hb, hb.max_to_shape_backward(up(hb, g), up(hb, x), up(hb, y), shape, out_shape), shape),
        O.max_to_shape_backward(g, x, y))


@pytest.mark.parametrize("shape", [(1024, 4096), (7, 33), (3, 5, 8)])
def test_reductions_that_reduce_nothing_bit_exact(hb, shape):
    """sum_to_shape / max_to_shape onto the input's own shape still take the reduction's first
    step (0 + x; max(-FLT_MAX, x) with a strict >): -0 becomes +0, NaN and -inf become -FLT_MAX
    for max, as the reference's loops give."""
    from orcaml_amd.backend import HipBackend

    plain = HipBackend(hb.ctx, deferred=False)  # no memo: the kernel runs on every call
    x = special_values(np.random.default_rng(shape[-1]), shape)
    got = down(plain, plain.sum_to_shape(up(plain, x), shape, shape), shape)
    want = O.sum_to_shape(x, shape)
    np.testing.assert_array_equal(got, want)
    assert not np.signbit(got[x == 0]).any()
    np.testing.assert_array_equal(down(plain, plain.max_to_shape(up(plain, x), shape, shape), shape),
                                  O.max_to_shape(x, shape))


@pytest.mark.parametrize("shape,out_shape", [((1000, 70), (1, 70)), ((3, 300, 33), (33,)), ((129, 4096), (1, 4096)),
                                             ((5000, 10), (1, 10)), ((1030, 16), (1, 16)), ((128, 1), (1, 1))])
def test_column_max_to_shape_bit_exact(hb, shape, out_shape):
    rng = np.random.default_rng(shape[-1])
    x = rng.integers(-3, 3, shape).astype(np.float32)  # many ties
    x.reshape(-1)[::13] = np.nan
    x.reshape(-1)[5::17] = -np.inf
    np.testing.assert_array_equal(down(hb, hb.max_to_shape(up(hb, x), shape, out_shape), out_shape),
                                  O.max_to_shape(x, out_shape))


@pytest.mark.parametrize("shape,d0,d1", [((5, 7), 0, 1), ((3, 130, 70), 1, 2), ((2, 3, 4, 5), 0, 2),
                                         ((4096, 1024), 1, 0)])
def test_transpose_bit_exact(hb, shape, d0, d1):
    rng = np.random.default_rng(shape[-1])
    a = rng.standard_normal(shape).astype(np.float32)
    s = hb.transpose(up(hb, a), shape, d0, d1)
    out_shape = list(shape)
    out_shape[d0], out_shape[d1] = out_shape[d1], out_shape[d0]
    np.testing.assert_array_equal(down(hb, s, out_shape), O.transpose(a, d0, d1))


def test_matmul_with_lazy_transpose_views(hb):
    """MatMulBackward's transpose(W) / transpose(X) are views folded into the GEMM."""
    rng = np.random.default_rng(2)
    X = rng.integers(-5, 5, (96, 40)).astype(np.float32)
    W = rng.integers(-5, 5, (40, 24)).astype(np.float32)
    G = rng.integers(-5, 5, (96, 24)).astype(np.float32)
    Wt = hb.transpose(up(hb, W), (40, 24), 0, 1)
    Xt = hb.transpose(up(hb, X), (96, 40), 0, 1)
    dX = down(hb, hb.matmul(up(hb, G), Wt, (96, 24), (24, 40)), (96, 40))
    dW = down(hb, hb.matmul(Xt, up(hb, G), (40, 96), (96, 24)), (40, 24))
    np.testing.assert_array_equal(dX, O.matmul(G, O.transpose(W, 0, 1)))
    np.testing.assert_array_equal(dW, O.matmul(O.transpose(X, 0, 1), G))
    np.testing.assert_array_equal(down(hb, Wt, (24, 40)), W.T)  # a view read back materialises
    a = rng.integers(-4, 4, (3, 6, 5)).astype(np.float32)
    b = rng.integers(-4, 4, (3, 5, 7)).astype(np.float32)
    np.testing.assert_array_equal(down(hb, hb.matmul(up(hb, a), up(hb, b), a.shape, b.shape), (3, 6, 7)),
                                  O.matmul(a, b))


def test_errors_map_to_orca_error_variants(hb):
    a = up(hb, np.ones((2, 3), np.float32))
    with pytest.raises(OrcaHipError) as e:
        hb.matmul(a, a, (2, 3), (2, 3))
    assert e.value.code == -1  # ShapeMismatch
    with pytest.raises(OrcaHipError) as e:
        hb.relu(a, (2, 3), dtype=2)  # F16
    assert e.value.code == -2  # UnsupportedDType
    with pytest.raises(OrcaHipError):
        hb.transpose(a, (2, 3), 0, 5)


def test_has_nan_or_inf_and_bytes_roundtrip(hb):
    a = np.arange(10, dtype=np.float32)
    s = up(hb, a)
    assert not hb.has_nan_or_inf(s)
    a[7] = np.inf
    assert hb.has_nan_or_inf(up(hb, a))
    b = hb.from_bytes((10,), a.tobytes())
    assert hb.to_bytes(b) == a.tobytes()
    z = hb.zeros((3, 3))
    assert down(hb, z, (9,)).tolist() == [0.0] * 9


def composed(ad, dims, params, x, onehot, kind, steps, **opt):
    model = A.build_mlp(ad, params)
    optim = A.SGD(model.parameters(), lr=opt["lr"]) if kind == "sgd" else A.AdamW(
        model.parameters(), lr=opt["lr"], weight_decay=opt.get("weight_decay", 0.01))
    xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
    losses, grads, logits = [], None, None
    for _ in range(steps):
        optim.zero_grad()
        out = model(xt)
        loss = A.CrossEntropyLoss()(out, tt)
        losses.append(loss.to_list()[0])
        loss.backward()
        grads = [p.tensor.grad().numpy() for p in model.parameters()]
        logits = out.numpy()
        optim.step()
    return np.array(losses, np.float32), grads, logits, [p.tensor.numpy() for p in model.parameters()]


@pytest.mark.parametrize("kind,steps", [("sgd", 1), ("adamw", 3)])
def test_composed_step_mlp784_128_on_hip(hb, kind, steps):
    """The reference's unchanged frontend + tape driving HipBackend's trait ops."""
    w = synth.WORKLOADS[synth.MLP_SMALL]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    opt = dict(lr=0.1) if kind == "sgd" else dict(lr=1e-3, weight_decay=0.01)
    ad = A.Autodiff(hb)
    losses, grads, logits, new_params = composed(ad, w["dims"], params, x, onehot, kind, steps, **opt)
    ref = O.mlp_train(w["dims"], params, x, onehot, O.make_opt(kind, **opt), steps=steps)
    assert_close(losses, ref["losses"], what="loss")
    assert_close(logits, ref["logits"], what="logits")
    for i, (g, r) in enumerate(zip(grads, ref["grads"])):
        assert_close(g.reshape(r.shape), r, what=f"grad {i}")
        assert_close_scaled(g.reshape(r.shape), r, rtol=1e-3, what=f"grad {i} (scaled)")
    for i, (p, r) in enumerate(zip(new_params, ref["params"])):
        assert_close(p.reshape(r.shape), r, what=f"param {i}")
    np.testing.assert_array_equal(A.argmax_rows(logits), ref["preds"])


@pytest.mark.parametrize("M,K,N,view", [(784, 1024, 4096, True), (128, 64, 128, True), (64, 2048, 64, True),
                                        (33, 300, 70, True), (1000, 100, 1030, True), (96, 256, 160, False),
                                        (784, 64, 128, False), (64, 64, 128, False), (130, 72, 70, False),
                                        (0, 16, 8, True), (8, 0, 12, True)])
def test_matmul_colsum_equals_matmul_and_sum_to_shape(hb, M, K, N, view):
    """orca_hip_matmul_colsum (via a pending sum_to_shape consumed by matmul): the product bit
    for bit as matmul, the column sum bit for bit as the oracle's sum_to_shape loop -- folded
    into the product (pipelined or generic kernel) or, when K is split, in its own pass."""
    from orcaml_amd.backend import HipBackend

    rng = np.random.default_rng(M + 7 * K + N)
    g = rng.standard_normal((K, N)).astype(np.float32)
    if view:
        lhs = hb.transpose(up(hb, rng.standard_normal((K, M)).astype(np.float32)), (K, M), 0, 1)
    else:
        lhs = up(hb, rng.standard_normal((M, K)).astype(np.float32))
    plain = HipBackend(hb.ctx, deferred=False)
    want = down(hb, plain.matmul(lhs, up(hb, g), (M, K), (K, N)), (M, N))
    G = up(hb, g)
    pend = hb.sum_to_shape(G, (K, N), (1, N))
    assert pend.pending
    got = hb.matmul(lhs, G, (M, K), (K, N))
    assert not pend.pending
    np.testing.assert_array_equal(down(hb, got, (M, N)), want)
    np.testing.assert_array_equal(down(hb, pend, (1, N)), O.sum_to_shape(g, (1, N)))


def test_pending_column_sum_used_first_and_identity_memo(hb):
    """A pending column sum read before any matmul is computed by the sum_to_shape kernel, and
    the matmul that follows leaves it alone; an identity sum_to_shape of one storage is one
    storage; an in-place update drops what was derived from the old values."""
    rng = np.random.default_rng(5)
    g = rng.standard_normal((300, 70)).astype(np.float32)
    G = up(hb, g)
    pend = hb.sum_to_shape(G, (300, 70), (70,))
    first = down(hb, pend, (70,))
    np.testing.assert_array_equal(first, O.sum_to_shape(g, (70,)))
    x = up(hb, rng.standard_normal((300, 40)).astype(np.float32))
    hb.matmul(hb.transpose(x, (300, 40), 0, 1), G, (40, 300), (300, 70))
    np.testing.assert_array_equal(down(hb, pend, (70,)), first)
    a = hb.sum_to_shape(G, (300, 70), (300, 70))
    assert hb.sum_to_shape(G, (300, 70), (300, 70)) is a
    np.testing.assert_array_equal(down(hb, a, (300, 70)), O.sum_to_shape(g, (300, 70)))
    p = up(hb, rng.standard_normal((300, 70)).astype(np.float32))
    m, v = (up(hb, np.zeros((300, 70), np.float32)) for _ in range(2))
    before = hb.sum_to_shape(p, (300, 70), (1, 70))
    ident = hb.sum_to_shape(p, (300, 70), (300, 70))
    p_old = down(hb, p, (300, 70))
    hb.adamw_step_(p, G, m, v, 300 * 70, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1)
    np.testing.assert_array_equal(down(hb, before, (1, 70)), O.sum_to_shape(p_old, (1, 70)))
    assert hb.sum_to_shape(p, (300, 70), (300, 70)) is not ident


@pytest.mark.parametrize("name,kind", [(synth.MLP_SMALL, "sgd"), (synth.MLP_SMALL, "adamw"),
                                       (synth.MLP_MEDIUM, "adamw")])
def test_composed_step_deferred_reductions_change_no_bit(hb, name, kind):
    """The composed step with the identity memo and the deferred bias column sums equals the
    same step with every sum_to_shape run at once, bit for bit (the 784-1024-1024-10 case
    splits dW1's K, so its column sum takes the separate pass)."""
    from orcaml_amd.backend import HipBackend

    w = synth.WORKLOADS[name]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    opt = dict(lr=0.1) if kind == "sgd" else dict(lr=1e-3, weight_decay=0.01)
    runs = [composed(A.Autodiff(HipBackend(hb.ctx, deferred=d)), w["dims"], params, x, onehot, kind, 2, **opt)
            for d in (True, False)]
    (l1, g1, o1, p1), (l2, g2, o2, p2) = runs
    np.testing.assert_array_equal(l1, l2)
    np.testing.assert_array_equal(o1, o2)
    for a, b in zip(g1 + p1, g2 + p2):
        np.testing.assert_array_equal(a, b)


def test_composed_step_allocates_nothing_in_steady_state(hb, ctx):
    """After warm-up the caching allocator serves every buffer of a step."""
    w = synth.WORKLOADS[synth.MLP_SMALL]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    ad = A.Autodiff(hb)
    composed(ad, w["dims"], params, x, onehot, "sgd", 2, lr=0.1)
    composed(ad, w["dims"], params, x, onehot, "sgd", 2, lr=0.1)
    before = ctx.mem_stats()["device_allocs"]
    composed(ad, w["dims"], params, x, onehot, "sgd", 3, lr=0.1)
    assert ctx.mem_stats()["device_allocs"] == before


def test_extent_guard_rejects_overruns_before_any_launch(ctx):
    """A size that runs past the end of a context allocation is a
    ShapeMismatch raised on the host.  Only copies are used here: even
    unguarded, the runtime bounds-checks them, so nothing can reach the GPU
    out of bounds."""
    buf = ctx.alloc(4096)
    host = np.empty(2048, np.float32)
    hp = host.ctypes.data_as(ctypes.c_void_p)
    for ptr, nbytes in ((buf.ptr, 8192), (buf.ptr + 1024, 4096)):
        with pytest.raises(_lib.OrcaHipError) as e:
            _lib.call("orca_hip_d2h", ctx.handle, hp, ptr, nbytes)
        assert e.value.code == _lib.ERR_SHAPE
        with pytest.raises(_lib.OrcaHipError) as e:
            _lib.call("orca_hip_h2d", ctx.handle, ptr, hp, nbytes)
        assert e.value.code == _lib.ERR_SHAPE
    _lib.call("orca_hip_d2h", ctx.handle, hp, buf.ptr + 1024, 3072)  # fits exactly
