"""GPU parity of the GEMM epilogues that the drop-in storage folds products into:
the two-output bias + ReLU epilogue (pre-activation and activation) on every
GEMM kernel path, and a composed training step whose Linear layers run as one
product each (no elementwise program for `x @ W + b` and its ReLU), bit-identical
to the same step with products and programs run one by one."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from orcaml_amd import _lib, synth
from orcaml_amd import autodiff as A
from orcaml_amd.backend import HipBackend
from tests.test_gpu_fused import run_gemm

pytestmark = pytest.mark.gpu


def gemm_pre(ctx, A_, B_, bias):
    """(C, pre) of orca_hip_gemm with EPI_BIAS_RELU_PRE, A and B row-major."""
    M, K = A_.shape
    N = B_.shape[1]
    dA, dB, db = ctx.upload(A_), ctx.upload(B_), ctx.upload(bias)
    dC, dP = ctx.alloc(4 * M * N), ctx.alloc(4 * M * N)
    e = _lib.Epilogue(_lib.EPI_BIAS_RELU_PRE, db.ptr, None, 0, None)
    e.pre = dP.ptr
    _lib.call("orca_hip_gemm", ctx.handle, 0, 0, M, N, K, dA.ptr, K, dB.ptr, N, dC.ptr, N, ctypes.byref(e))
    return dC.download(count=M * N).reshape(M, N), dP.download(count=M * N).reshape(M, N)


@pytest.mark.parametrize("M,N,K", [
    (256, 384, 160),    # pipelined 128 x 128 kernel
    (260, 196, 164),    # pipelined, edge tiles
    (256, 1024, 784),   # skinny kernel
    (1024, 1024, 256),  # 64 x 64 tiles
    (128, 256, 3076),   # split K: the epilogue runs in the float4 reduce
    (130, 70, 33),      # generic kernel, unaligned
    (129, 1029, 1021),  # skinny, ragged
    (64, 13, 2050),     # N <= 16 stays on the tiles (split K, scalar reduce)
])
def test_bias_relu_pre_epilogue_matches_composed_ops(ctx, M, N, K):
    rng = np.random.default_rng(M + N + K)
    A_ = rng.standard_normal((M, K)).astype(np.float32)
    B_ = rng.standard_normal((K, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    bias[::7] = -bias[::7] * 1e3  # columns that are mostly negative: ReLU zeros
    C, pre = gemm_pre(ctx, A_, B_, bias)
    np.testing.assert_array_equal(C, O.relu(pre))
    np.testing.assert_array_equal(C, run_gemm(ctx, False, False, A_, B_, _lib.EPI_BIAS_RELU, bias=bias))
    if N > 16:  # the plain product runs on the same kernel: the epilogue's bits are the composed ops'
        prod = run_gemm(ctx, False, False, A_, B_)
        np.testing.assert_array_equal(pre, O.add(prod, O.expand(bias.reshape(1, N), (M, N))))
    else:  # the plain product takes the narrow kernel (another order): within the dot-product bound
        exact = A_.astype(np.float64) @ B_.astype(np.float64) + bias
        bound = K * 2.0 ** -24 * (np.abs(A_.astype(np.float64)) @ np.abs(B_.astype(np.float64))) + 2.0 ** -23 * np.abs(exact)
        assert (np.abs(pre - exact) <= bound).all()


@pytest.mark.parametrize("M,N,K", [
    (256, 384, 160),    # pipelined 128 x 128 kernel (B^T)
    (256, 1024, 1024),  # skinny kernel (B^T)
    (128, 256, 3076),   # split K: the float4 reduce
    (130, 70, 33),      # generic kernel, unaligned: the scalar reduce or the tile store
    (1024, 4096, 10),   # narrow K against B^T
    (33, 1001, 3),
])
def test_relu_mask_pre_epilogue_keeps_the_product(ctx, M, N, K):
    """dY W^T with the ReLU mask applied, writing the unmasked product as well: both equal
    the plain product and relu_backward of it, bit for bit."""
    rng = np.random.default_rng(M * 3 + N + K)
    A_ = rng.standard_normal((M, K)).astype(np.float32)
    Bt = rng.standard_normal((N, K)).astype(np.float32)
    mask = rng.standard_normal((M, N)).astype(np.float32)
    mask[::3, ::5] = 0.0
    prod = run_gemm(ctx, False, True, A_, Bt)
    dA, dB, dm = ctx.upload(A_), ctx.upload(Bt), ctx.upload(mask)
    dC, dP = ctx.alloc(4 * M * N), ctx.alloc(4 * M * N)
    e = _lib.Epilogue(_lib.EPI_RELU_MASK_PRE, None, dm.ptr, N, None)
    e.pre = dP.ptr
    _lib.call("orca_hip_gemm", ctx.handle, 0, 1, M, N, K, dA.ptr, K, dB.ptr, K, dC.ptr, N, ctypes.byref(e))
    np.testing.assert_array_equal(dP.download(count=M * N).reshape(M, N), prod)
    np.testing.assert_array_equal(dC.download(count=M * N).reshape(M, N), O.relu_backward(prod, mask))


def test_bias_relu_pre_epilogue_requires_its_output(ctx):
    M = N = K = 64
    dA, dC = ctx.alloc(4 * M * K), ctx.alloc(4 * M * N)
    db = ctx.alloc(4 * N)
    e = _lib.Epilogue(_lib.EPI_BIAS_RELU_PRE, db.ptr, None, 0, None)
    with pytest.raises(_lib.OrcaHipError, match="pre"):
        _lib.call("orca_hip_gemm", ctx.handle, 0, 0, M, N, K, dA.ptr, K, dA.ptr, N, dC.ptr, N, ctypes.byref(e))
    e.kind = 6
    with pytest.raises(_lib.OrcaHipError, match="unknown gemm epilogue"):
        _lib.call("orca_hip_gemm", ctx.handle, 0, 0, M, N, K, dA.ptr, K, dA.ptr, N, dC.ptr, N, ctypes.byref(e))


def _step_run(hb, ctx, dims, params, x, onehot, kind, fused, steps):
    """Losses, final gradients and parameters of `steps` composed steps, and the elementwise
    programs launched per step (interpreted + compiled)."""
    ad = A.Autodiff(hb)
    model = A.build_mlp(ad, params)
    opt = (A.SGD(model.parameters(), lr=0.1, fused=fused) if kind == "sgd" else
           A.AdamW(model.parameters(), lr=1e-3, weight_decay=0.01, fused=fused))
    xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
    losses, grads, programs = [], None, []
    for _ in range(steps):
        before = ctx.ew_jit_stats()
        opt.zero_grad()
        loss = A.CrossEntropyLoss(fused=fused)(model(xt), tt)
        loss.backward()
        losses.append(loss.to_list()[0])
        grads = [p.tensor.grad().numpy() for p in model.parameters()]
        opt.step()
        ctx.sync()
        after = ctx.ew_jit_stats()
        programs.append(after["interpreted"] + after["compiled_launches"] - before["interpreted"] -
                        before["compiled_launches"])
    return losses, grads, [p.tensor.numpy() for p in model.parameters()], programs


@pytest.mark.parametrize("kind,fused", [("sgd", False), ("adamw", False), ("adamw", True)])
@pytest.mark.parametrize("dims,batch", [((784, 128, 128, 10), 64), ((784, 1024, 1024, 10), 256)])
def test_composed_step_with_folded_epilogues_bit_identical(ctx, kind, fused, dims, batch):
    """Each Linear's `x @ W + b` (and the ReLU after it) runs as one product with its
    epilogue, and so does each ReLU backward on the product that brings its gradient: 2L - 1
    fewer elementwise programs per step (L Linear layers) than with folding off, and not one
    bit of the losses, gradients or parameters changes.  (2L - 2 with the composed loss: with
    folding off the head's bias add runs in the launch of the logits' row maximum, a
    row-reducing program not counted here.  The count is taken without the second stream,
    whose updates split a program in two wherever a product runs beside it.)"""
    params, x, labels, onehot = synth.mlp_problem(11, dims, batch)
    l1, g1, p1, _ = _step_run(HipBackend(ctx), ctx, dims, params, x, onehot, kind, fused, 3)
    l2, g2, p2, _ = _step_run(HipBackend(ctx, fold=False), ctx, dims, params, x, onehot, kind, fused, 3)
    assert l1 == l2
    for a, b in zip(g1 + p1, g2 + p2):
        np.testing.assert_array_equal(a, b)
    _, _, p3, n1 = _step_run(HipBackend(ctx, overlap=False), ctx, dims, params, x, onehot, kind, fused, 3)
    _, _, _, n2 = _step_run(HipBackend(ctx, fold=False, overlap=False), ctx, dims, params, x, onehot, kind, fused, 3)
    for a, b in zip(p1, p3):
        np.testing.assert_array_equal(a, b)
    layers = len(dims) - 1
    assert [b - a for a, b in zip(n1, n2)] == [2 * layers - (1 if fused else 2)] * 3, (n1, n2)


def test_folded_product_leaves_other_users_unchanged(ctx):
    """A product that something else still holds is not folded (it runs by itself, then the
    program): both values are the composed ops'."""
    hb = HipBackend(ctx)
    rng = np.random.default_rng(2)
    M, K, N = 96, 80, 160
    a, w = rng.standard_normal((M, K)).astype(np.float32), rng.standard_normal((K, N)).astype(np.float32)
    b = rng.standard_normal((1, N)).astype(np.float32)
    da, dw = hb.from_f32_slice((M, K), a), hb.from_f32_slice((K, N), w)
    db = hb.from_f32_slice((1, N), b)
    prod = hb.matmul(da, dw, (M, K), (K, N))
    assert prod.pending
    h = hb.relu(hb.add(prod, hb.expand(db, (1, N), (M, N)), (M, N)), (M, N))
    got_h = hb.to_f32_vec(h).reshape(M, N)
    got_p = hb.to_f32_vec(prod).reshape(M, N)
    np.testing.assert_array_equal(got_h, O.relu(O.add(got_p, O.expand(b, (M, N)))))
    # the same chain with nothing else holding the product: folded, same bits
    h2 = hb.relu(hb.add(hb.matmul(da, dw, (M, K), (K, N)), hb.expand(db, (1, N), (M, N)), (M, N)), (M, N))
    before = ctx.ew_jit_stats()
    got_h2 = hb.to_f32_vec(h2).reshape(M, N)
    after = ctx.ew_jit_stats()
    assert after["interpreted"] + after["compiled_launches"] == before["interpreted"] + before["compiled_launches"]
    np.testing.assert_array_equal(got_h2, got_h)


def test_relu_backward_on_a_held_product(ctx):
    """relu_backward(g @ W^T, z) while the product is held elsewhere (as the tape holds a
    gradient): one product launch writes both, no program, and both equal the ops'."""
    hb = HipBackend(ctx)
    rng = np.random.default_rng(6)
    M, K, N = 200, 96, 300
    g, w = rng.standard_normal((M, K)).astype(np.float32), rng.standard_normal((N, K)).astype(np.float32)
    z = rng.standard_normal((M, N)).astype(np.float32)
    dg, dw, dz = hb.from_f32_slice((M, K), g), hb.from_f32_slice((N, K), w), hb.from_f32_slice((M, N), z)
    prod = hb.matmul(dg, hb.transpose(dw, (N, K), 0, 1), (M, K), (K, N))
    held = [prod]
    r = hb.relu_backward(prod, dz, (M, N))
    before = ctx.ew_jit_stats()
    got_r = hb.to_f32_vec(r).reshape(M, N)
    after = ctx.ew_jit_stats()
    assert after["interpreted"] + after["compiled_launches"] == before["interpreted"] + before["compiled_launches"]
    assert not held[0].pending
    got_p = hb.to_f32_vec(held[0]).reshape(M, N)
    eager = HipBackend(ctx, lazy=False)
    want_p = eager.to_f32_vec(eager.matmul(dg, eager.transpose(dw, (N, K), 0, 1), (M, K), (K, N))).reshape(M, N)
    np.testing.assert_array_equal(got_p, want_p)
    np.testing.assert_array_equal(got_r, O.relu_backward(want_p, z))


@pytest.mark.parametrize("M,N,K", [(256, 384, 160), (256, 1024, 1024), (128, 256, 3076), (130, 70, 33),
                                   (1024, 10, 4096), (1024, 4096, 10), (64, 13, 2050)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False)])
def test_products_never_hold_negative_zero(ctx, M, N, K, ta, tb):
    """Every GEMM path (pipelined, skinny, split K, generic, narrow) returns +0 where all
    products are -0 (negative x +0), where a row is all -0, and where terms cancel: the
    property that lets a masked product share its buffer with its identity sum (0 + x)."""
    rng = np.random.default_rng(M + N + K + 2 * ta + tb)
    A_ = -np.abs(rng.standard_normal((M, K))).astype(np.float32) - 1.0
    B_ = np.zeros((K, N), np.float32)
    B_[:, ::2] = rng.integers(-3, 3, (K, (N + 1) // 2)).astype(np.float32)
    A_[1::4] = -0.0  # rows of -0: every product -0 or +0
    A_[2::4, : K // 2] = 1.0  # rows whose terms cancel against the next half
    A_[2::4, K // 2: 2 * (K // 2)] = -1.0
    B_[K // 2: 2 * (K // 2)] = B_[: K // 2]
    got = run_gemm(ctx, ta, tb, np.ascontiguousarray(A_.T) if ta else A_, np.ascontiguousarray(B_.T) if tb else B_)
    zeros = got == 0
    assert zeros.any()
    assert not np.signbit(got[zeros]).any()


def test_identity_sum_keeps_nan_bits(ctx):
    """0 + x returns x's bits for quiet NaNs of any payload and sign (and +0 for -0): the
    identity sum of a masked product may share its buffer."""
    hb = HipBackend(ctx, lazy=False)
    bits = np.array([0x7FC00000, 0xFFC00000, 0x7FC00001, 0xFFD23456, 0x7FFFFFFF, 0x3F800000, 0x80000000], np.uint32)
    x = bits.view(np.float32)
    got = hb.to_f32_vec(hb.sum_to_shape(hb.from_f32_slice((7,), x), (7,), (7,))).view(np.uint32)
    np.testing.assert_array_equal(got[:6], bits[:6])
    assert got[6] == 0  # -0 -> +0


@pytest.mark.parametrize("form,lt,rt,M,K,N,folds", [
    ("bias", False, False, 96, 200, 10, True),      # narrow X W takes the bias itself
    ("bias", False, True, 96, 10, 300, False),      # narrow dY W^T has no bias epilogue: not folded
    ("bias", True, False, 300, 96, 10, False),      # nor narrow X^T dY
    ("relu", False, False, 96, 200, 10, False),     # bias + ReLU never runs narrow
    ("relu", False, True, 96, 10, 300, False),
    ("relu", False, False, 96, 200, 40, True),
    ("mask", False, True, 96, 10, 300, True),       # narrow dY W^T takes the mask itself
    ("mask", False, False, 96, 200, 10, False),     # narrow X W has no mask epilogue: not folded
    ("mask", True, False, 300, 96, 10, False),
    ("mask", True, False, 300, 96, 40, True),
])
def test_fold_only_where_the_product_keeps_its_kernel(ctx, form, lt, rt, M, K, N, folds):
    """A chain over a pending product folds only where the product with the epilogue runs on
    the same kernel as the plain product, so folding never changes a bit."""
    rng = np.random.default_rng(M + K + N + 2 * lt + rt)
    a = rng.standard_normal((K, M) if lt else (M, K)).astype(np.float32)
    w = rng.standard_normal((N, K) if rt else (K, N)).astype(np.float32)
    b = rng.standard_normal((1, N)).astype(np.float32)
    z = rng.standard_normal((M, N)).astype(np.float32)
    out = []
    for fold in (True, False):
        hb = HipBackend(ctx, fold=fold)
        da, dw = hb.from_f32_slice(a.shape, a), hb.from_f32_slice(w.shape, w)
        lhs = hb.transpose(da, a.shape, 0, 1) if lt else da
        rhs = hb.transpose(dw, w.shape, 0, 1) if rt else dw
        prod = hb.matmul(lhs, rhs, (M, K), (K, N))
        if form == "mask":
            r = hb.relu_backward(prod, hb.from_f32_slice((M, N), z), (M, N))
        else:
            r = hb.add(prod, hb.expand(hb.from_f32_slice((1, N), b), (1, N), (M, N)), (M, N))
            if form == "relu":
                r = hb.relu(r, (M, N))
        del prod
        before = ctx.ew_jit_stats()
        out.append(hb.to_f32_vec(r))
        after = ctx.ew_jit_stats()
        launched = after["interpreted"] + after["compiled_launches"] - before["interpreted"] - before["compiled_launches"]
        if fold:
            assert (launched == 0) == folds, launched
    np.testing.assert_array_equal(out[0], out[1])


def test_pending_product_runs_before_its_input_is_updated(ctx):
    """An in-place optimizer update of a product's input first runs the pending product on
    the old values."""
    hb = HipBackend(ctx)
    rng = np.random.default_rng(4)
    n = 64
    a = rng.standard_normal((n, n)).astype(np.float32)
    p0 = rng.standard_normal((n, n)).astype(np.float32)
    da = hb.from_f32_slice((n, n), a)
    p = hb.from_f32_slice((n, n), p0)
    g = hb.from_f32_slice((n, n), rng.standard_normal((n, n)).astype(np.float32))
    prod = hb.matmul(da, p, (n, n), (n, n))
    assert prod.pending
    hb.sgd_step_(p, g, n * n, 0.5)
    want = hb.to_f32_vec(HipBackend(ctx, lazy=False).matmul(da, hb.from_f32_slice((n, n), p0), (n, n), (n, n)))
    np.testing.assert_array_equal(hb.to_f32_vec(prod), want)
