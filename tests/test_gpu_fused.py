"""GPU parity of the fused kernels (GEMM, softmax-CE, AdamW/SGD) and of the
device-resident MLP training step against the CPU oracle, through the C ABI."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as O
from orcaml_amd import _lib, synth
from orcaml_amd.mlp import MLPTrainer
from tests.util import assert_close, assert_close_scaled, int_matrix

pytestmark = pytest.mark.gpu


def run_gemm(ctx, ta, tb, A, B, epi_kind=_lib.EPI_NONE, bias=None, mask=None, colsum=False):
    """C = op(A) op(B) on the GPU; A/B are passed in their stored layout."""
    M = A.shape[1] if ta else A.shape[0]
    K = A.shape[0] if ta else A.shape[1]
    N = B.shape[0] if tb else B.shape[1]
    dA, dB = ctx.upload(A), ctx.upload(B)
    dC = ctx.alloc(4 * M * N)
    keep = []
    e = _lib.Epilogue(epi_kind, None, None, 0, None)
    if bias is not None:
        keep.append(ctx.upload(bias))
        e.bias = keep[-1].ptr
    if mask is not None:
        keep.append(ctx.upload(mask))
        e.mask = keep[-1].ptr
        e.ldmask = N
    dcs = None
    if colsum:
        dcs = ctx.alloc(4 * N)
        e.colsum = dcs.ptr
    _lib.call("orca_hip_gemm", ctx.handle, int(ta), int(tb), M, N, K, dA.ptr, A.shape[1], dB.ptr, B.shape[1],
              dC.ptr, N, ctypes.byref(e))
    C = dC.download(count=M * N).reshape(M, N)
    return (C, dcs.download(count=N)) if colsum else C


def assert_gemm_error_bound(got, A, B):
    """Forward error of an f32 dot product of length K is at most
    gamma_K * sum_k |a_k b_k| with gamma_K ~ K * 2^-24 (any summation order);
    checked against the fp64 product."""
    A64, B64 = A.astype(np.float64), B.astype(np.float64)
    exact = A64 @ B64
    bound = A.shape[1] * 2.0 ** -24 * (np.abs(A64) @ np.abs(B64)) + 1e-30
    err = np.abs(got.astype(np.float64) - exact)
    assert (err <= bound).all(), f"max err/bound {float((err / bound).max()):.3f}"


GEMM_SHAPES = [
    # generic kernel (a dimension not a multiple of 4, or N / K = 10 as in the output layer)
    (1, 1, 1), (130, 70, 33), (257, 129, 1000), (1024, 10, 4096), (1024, 4096, 10),
    # pipelined kernel, edge tiles and partial K slabs (K = 784 as in the input layer)
    (64, 128, 784), (784, 384, 1024), (96, 16, 4), (4, 8, 12), (132, 260, 36), (200, 300, 152),
    # pipelined kernel, tile-aligned: 1..5 and 32 slabs, and split-K launches
    (128, 128, 32), (256, 128, 64), (128, 256, 96), (256, 256, 128), (384, 128, 160), (256, 384, 1024),
    (128, 128, 4096), (128, 256, 3076),
    # 128 tiles of 128 x 128: half of MI355X's 256 CUs, so K splits in two
    (1024, 2048, 128)]


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_gemm_exact_on_integers(ctx, ta, tb, M, N, K):
    rng = np.random.default_rng(M * 7 + N * 13 + K)
    A = int_matrix(rng, (M, K))
    B = int_matrix(rng, (K, N))
    want = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)
    got = run_gemm(ctx, ta, tb, np.ascontiguousarray(A.T) if ta else A, np.ascontiguousarray(B.T) if tb else B)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("ta,tb,colsum", [(False, False, False), (False, False, True), (False, True, False),
                                          (True, False, True), (True, False, False), (True, True, False)])
def test_gemm_aligned_shapes_take_pipelined_kernel(ctx, ta, tb, colsum):
    """Products whose M, N, K are multiples of 4 run on the pipelined 128 x 128
    kernel (profiler name *_pipe), the rest on the generic kernel; both exact
    on integers."""
    rng = np.random.default_rng(3)
    name = "gemm_" + ("t" if ta else "n") + ("t" if tb else "n")
    for (M, N, K), pipe in (((256, 384, 160), True), ((260, 196, 164), True), ((256, 384, 161), False),
                            ((256, 202, 160), False)):
        A = int_matrix(rng, (M, K))
        B = int_matrix(rng, (K, N))
        ctx.prof_reset()
        ctx.prof_enable(True)
        out = run_gemm(ctx, ta, tb, np.ascontiguousarray(A.T) if ta else A, np.ascontiguousarray(B.T) if tb else B,
                       colsum=colsum and not tb)
        ctx.prof_enable(False)
        names = {k["name"] for k in ctx.prof_report()["kernels"]}
        want = f"{name}_pipe {M}x{N}x{K}" if pipe else f"{name} {M}x{N}x{K}"
        assert want in names, names
        C, cs = out if colsum else (out, None)
        np.testing.assert_array_equal(C, (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32))
        if cs is not None:
            np.testing.assert_array_equal(cs, O.sum_to_shape(B, (1, N)).reshape(N))


SKINNY_SHAPES = [(256, 1024, 784), (256, 1024, 1024), (200, 1000, 1000), (256, 1024, 30), (130, 1030, 777),
                 (129, 1029, 1021)]


@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("M,N,K", SKINNY_SHAPES)
def test_gemm_skinny_exact_on_integers(ctx, tb, M, N, K):
    """Few-row, short-K products with row-major A (the 784-1024-1024-10 / B = 256 forward and
    dX products; ragged M, N, K; K shorter than a wave's 8-k group) run whole on the skinny
    32 x 32 kernel (no K split, no reduce launch); exact on integers, with the column sum of
    a row-major B taken by its own pass."""
    cus = ctx.prof_report()["num_cus"]
    if cus != 256:
        pytest.skip("tile counts chosen for 256 compute units")
    rng = np.random.default_rng(M + N + K + tb)
    A = int_matrix(rng, (M, K))
    B = int_matrix(rng, (K, N))
    ctx.prof_reset()
    ctx.prof_enable(True)
    out = run_gemm(ctx, False, tb, A, np.ascontiguousarray(B.T) if tb else B, colsum=not tb)
    ctx.prof_enable(False)
    names = {k["name"] for k in ctx.prof_report()["kernels"]}
    assert ("gemm_nt_skinny" if tb else "gemm_nn_skinny") + f" {M}x{N}x{K}" in names, names
    assert "gemm_splitk_reduce" not in names
    C, cs = out if not tb else (out, None)
    np.testing.assert_array_equal(C, (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))
    if cs is not None:
        np.testing.assert_array_equal(cs, B.astype(np.float64).sum(0).astype(np.float32))


@pytest.mark.parametrize("M,N,K", [(256, 1024, 1024), (130, 1030, 777)])
def test_gemm_skinny_epilogues_match_composed_ops(ctx, M, N, K):
    """The skinny kernel's bias, bias + ReLU and ReLU-mask epilogues equal the composed ops
    applied to its own product, bit for bit; the product is within the f32 dot-product bound."""
    rng = np.random.default_rng(M + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    prod = run_gemm(ctx, False, False, A, B)
    assert_gemm_error_bound(prod, A, B)
    np.testing.assert_array_equal(run_gemm(ctx, False, False, A, B, _lib.EPI_BIAS, bias=bias),
                                  O.add(prod, O.expand(bias.reshape(1, N), (M, N))))
    np.testing.assert_array_equal(run_gemm(ctx, False, False, A, B, _lib.EPI_BIAS_RELU, bias=bias),
                                  O.relu(O.add(prod, O.expand(bias.reshape(1, N), (M, N)))))
    mask = rng.standard_normal((M, N)).astype(np.float32)
    mask[::7, ::3] = 0.0
    np.testing.assert_array_equal(run_gemm(ctx, False, False, A, B, _lib.EPI_RELU_MASK, mask=mask),
                                  O.relu_backward(prod, mask))
    # the transposed-B form on the same data: same product bits
    np.testing.assert_array_equal(run_gemm(ctx, False, True, A, np.ascontiguousarray(B.T)), prod)


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(1024, 1024, 256), (784, 1024, 256), (1000, 1030, 250), (1024, 1024, 33)])
def test_gemm_small_tiles_exact_on_integers(ctx, ta, tb, M, N, K):
    """Short products (K <= 512) whose 128 x 128 grid leaves half the CUs idle but whose
    64 x 64 grid covers three quarters of them run unsplit on 64 x 64 tiles (profiler name
    without _pipe, no reduce launch): the 784-1024-1024-10 / B = 256 weight gradients,
    ragged edges and a K that is not a multiple of the slab.  Exact on integers, with the
    folded column sum."""
    cus = ctx.prof_report()["num_cus"]
    if cus != 256:
        pytest.skip("tile counts chosen for 256 compute units")
    rng = np.random.default_rng(M + N + K)
    A = int_matrix(rng, (M, K))
    B = int_matrix(rng, (K, N))
    ctx.prof_reset()
    ctx.prof_enable(True)
    out = run_gemm(ctx, ta, tb, np.ascontiguousarray(A.T) if ta else A, np.ascontiguousarray(B.T) if tb else B,
                   colsum=not tb)
    ctx.prof_enable(False)
    names = {k["name"] for k in ctx.prof_report()["kernels"]}
    name = "gemm_" + ("t" if ta else "n") + ("t" if tb else "n") + f" {M}x{N}x{K}"
    assert name in names and "gemm_splitk_reduce" not in names, names
    C, cs = out if not tb else (out, None)
    np.testing.assert_array_equal(C, (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))
    if cs is not None:
        np.testing.assert_array_equal(cs, B.astype(np.float64).sum(0).astype(np.float32))


@pytest.mark.parametrize("M,N,K", [(200, 300, 150), (200, 300, 152), (256, 384, 128), (128, 256, 1024),
                                   (130, 70, 1000), (1024, 2048, 128)])
def test_gemm_epilogues_match_composed_ops(ctx, M, N, K):
    """Generic kernel (K = 150), pipelined kernel with edge tiles (152) and aligned (128); split-K
    launches whose epilogue runs in the float4 reduce (N = 256, 2048) or the scalar one (N = 70)."""
    rng = np.random.default_rng(5)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    prod = run_gemm(ctx, False, False, A, B)
    assert_gemm_error_bound(prod, A, B)
    # bias: the reference adds the expanded bias in f32 after the product
    got = run_gemm(ctx, False, False, A, B, _lib.EPI_BIAS, bias=bias)
    np.testing.assert_array_equal(got, O.add(prod, O.expand(bias.reshape(1, N), (M, N))))
    got = run_gemm(ctx, False, False, A, B, _lib.EPI_BIAS_RELU, bias=bias)
    np.testing.assert_array_equal(got, O.relu(O.add(prod, O.expand(bias.reshape(1, N), (M, N)))))
    mask = rng.standard_normal((M, N)).astype(np.float32)
    mask[::7, ::3] = 0.0
    got = run_gemm(ctx, False, False, A, B, _lib.EPI_RELU_MASK, mask=mask)
    np.testing.assert_array_equal(got, O.relu_backward(prod, mask))


def test_gemm_grid_of_half_the_cus_splits_k(ctx):
    """A 128 x 128 tile grid that covers exactly half the CUs runs as two K chunks (every CU busy,
    then the in-order chunk sum); the product stays exact on integers."""
    cus = ctx.prof_report()["num_cus"]
    M, N, K = 128, 128 * (cus // 2), 2048  # K > 1024: neither 64 x 64 tiles nor the skinny kernel
    rng = np.random.default_rng(11)
    A = int_matrix(rng, (M, K))
    B = int_matrix(rng, (K, N))
    ctx.prof_reset()
    ctx.prof_enable(True)
    got = run_gemm(ctx, False, False, A, B)
    ctx.prof_enable(False)
    names = {k["name"] for k in ctx.prof_report()["kernels"]}
    assert "gemm_splitk_reduce" in names, names
    np.testing.assert_array_equal(got, (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("M,N,K", [(128, 256, 64), (784, 4096, 1024), (4096, 10, 1024), (33, 70, 5), (512, 384, 96),
                                   (128, 128, 4096), (784, 4092, 1020), (132, 260, 36)])
def test_gemm_colsum_is_bias_gradient(ctx, M, N, K):
    """dW = X^T dY with the bias column sum fused.  The column sum equals
    sum_to_shape(dY, [1, N]) bit for bit (ascending row order): folded into the
    product's loads of dY with one K-chunk per tile, else (a split K, a narrow
    product) taken in a pass of its own."""
    rng = np.random.default_rng(M + N + K)
    X = rng.standard_normal((K, M)).astype(np.float32)  # stored [B][in]
    dY = rng.standard_normal((K, N)).astype(np.float32)
    dW, cs = run_gemm(ctx, True, False, X, dY, colsum=True)
    np.testing.assert_array_equal(cs, O.sum_to_shape(dY, (1, N)).reshape(N))
    assert_gemm_error_bound(dW, X.T, dY)


# Banded weight gradients X^T dY (N = 128 j, one round of blocks between half and all of a
# 256-CU GPU's CUs): the 112-row tiles (M = 112 R, R <= 7) and the eight-band grid
# (M = 768 + E, E = 4 .. 16); 784 takes either, as the context prefers.  Whole and partial
# K slabs, K from one slab to 32, every leftover-row count.
BAND_SHAPES = [(2, 784, 4096, 1024), (2, 784, 4096, 1020), (2, 784, 4096, 36), (2, 784, 4096, 4),
               (2, 672, 4096, 64), (2, 784, 2432, 96), (1, 784, 4096, 1024), (1, 784, 4096, 1020),
               (1, 784, 4096, 512), (1, 784, 4096, 36), (1, 784, 4096, 4), (1, 772, 4096, 64), (1, 776, 2304, 128),
               (1, 780, 3968, 100), (1, 784, 2176, 32)]


@pytest.fixture(scope="module")
def band_ctx(request):
    """A context preferring the eight-band grid (1) or the 112-row tiles (2) for 784 rows."""
    from orcaml_amd.device import Context

    old = os.environ.get("ORCA_HIP_GEMM_BAND")
    os.environ["ORCA_HIP_GEMM_BAND"] = str(request.param)
    try:
        c = Context(0)
    finally:
        if old is None:
            del os.environ["ORCA_HIP_GEMM_BAND"]
        else:
            os.environ["ORCA_HIP_GEMM_BAND"] = old
    c.band_mode = request.param
    yield c
    c.close()


def _band_kernel(M, N, mode, cus):
    """The banded kernel a product takes (None when neither form's grid fits one round)."""
    cols = N // 128
    r112 = M // 112
    rows112 = M % 112 == 0 and 1 <= r112 <= 7 and r112 * cols <= cus < 2 * r112 * cols
    eight = 768 < M <= 784 and 8 * cols <= cus < 16 * cols
    if eight and (not rows112 or mode == 1):
        return "gemm_tn_band8"
    return "gemm_tn_band112" if rows112 else None


@pytest.mark.parametrize("band_ctx,M,N,K", BAND_SHAPES, indirect=["band_ctx"])
def test_gemm_band_exact_on_integers_with_exact_colsum(band_ctx, M, N, K):
    """The banded weight gradient (32 x 32 blocks for 96 rows, 16 x 16 blocks for 16 more):
    exact on integers, and its bias column sum equals sum_to_shape bit for bit, with and
    without the column sum; every element of C is written."""
    ctx = band_ctx
    cus = ctx.prof_report()["num_cus"]
    kernel = _band_kernel(M, N, ctx.band_mode, cus)
    if kernel is None:
        pytest.skip(f"no banded grid is one round of {cus} CUs for {M} x {N}")
    rng = np.random.default_rng(M + 3 * N + 5 * K)
    X, dY = int_matrix(rng, (K, M)), int_matrix(rng, (K, N))
    want = (X.T.astype(np.int64) @ dY.astype(np.int64)).astype(np.float32)
    for colsum in (False, True):
        ctx.prof_reset()
        ctx.prof_enable(True)
        out = run_gemm(ctx, True, False, X, dY, colsum=colsum)
        ctx.prof_enable(False)
        names = {k["name"] for k in ctx.prof_report()["kernels"]}
        assert f"{kernel} {M}x{N}x{K}" in names, names
        C, cs = out if colsum else (out, None)
        np.testing.assert_array_equal(C, want)
        if colsum:
            np.testing.assert_array_equal(cs, O.sum_to_shape(dY, (1, N)).reshape(N))


@pytest.mark.parametrize("band_ctx", [1, 2], indirect=True, ids=["band8", "band112"])
@pytest.mark.parametrize("K", [1024, 256, 60])
def test_gemm_band_error_bound_and_bias_gradient_bits(band_ctx, K):
    """Real-valued X^T dY on either banded kernel: within the f32 dot-product bound of the
    fp64 product, and the folded bias gradient bit-identical to sum_to_shape (NaN,
    infinities, signed zeros and subnormals in dY pass through its adds as in the loop)."""
    ctx = band_ctx
    rng = np.random.default_rng(K)
    X = rng.standard_normal((K, 784)).astype(np.float32)
    dY = rng.standard_normal((K, 4096)).astype(np.float32)
    dW, cs = run_gemm(ctx, True, False, X, dY, colsum=True)
    assert_gemm_error_bound(dW, X.T, dY)
    np.testing.assert_array_equal(cs, O.sum_to_shape(dY, (1, 4096)).reshape(4096))
    dY[:, 7] = -0.0
    dY[3, 100] = np.inf
    dY[5, 200] = np.nan
    dY[:, 300] = np.float32(1e-40)
    _, cs = run_gemm(ctx, True, False, X, dY, colsum=True)
    np.testing.assert_array_equal(cs, O.sum_to_shape(dY, (1, 4096)).reshape(4096))


def _relu_bw_colsum_order(g, pre):
    """The column sums in the kernels' own f32 order: rows summed in ascending order
    within chunks of 64, then for each column four threads add a contiguous quarter of
    the chunk partials each (in chunk order) and the quarters are added in order."""
    rows, cols = g.shape
    d = np.where(pre > 0, g, np.float32(0)).astype(np.float32)
    chunks = -(-rows // 64)
    part = np.zeros((chunks, cols), np.float32)
    for c in range(chunks):
        s = np.zeros(cols, np.float32)
        for r in range(c * 64, min(rows, c * 64 + 64)):
            s = (s + d[r]).astype(np.float32)
        part[c] = s
    per = -(-chunks // 4)
    quarters = []
    for q in range(4):
        s = np.zeros(cols, np.float32)
        for c in range(q * per, min(chunks, q * per + per)):
            s = (s + part[c]).astype(np.float32)
        quarters.append(s)
    t = quarters[0]
    for q in quarters[1:]:
        t = (t + q).astype(np.float32)
    return d, t


@pytest.mark.parametrize("rows,cols", [(8192, 4096), (1000, 1032), (3, 8), (130, 260), (4099, 256), (77, 5)])
def test_relu_bw_colsum_order_and_bound(ctx, rows, cols):
    """ReLU backward + bias column sum: the mask exact; the column sums equal the kernels'
    own summation order reproduced in f32 bit for bit (shapes up to 2^20 elements), and
    the exact sum within the f32 bound n * 2^-24 * sum|x| (N(0, 1) data cancels, so a
    relative check against the sequential order would test the data)."""
    rng = np.random.default_rng(rows + cols)
    g = rng.standard_normal((rows, cols)).astype(np.float32)
    pre = rng.standard_normal((rows, cols)).astype(np.float32)
    pre.reshape(-1)[::11] = 0.0
    dg, dp = ctx.upload(g), ctx.upload(pre)
    dpre, cs = ctx.alloc(4 * rows * cols), ctx.alloc(4 * cols)
    _lib.call("orca_hip_relu_bw_colsum", ctx.handle, dg.ptr, dp.ptr, rows, cols, dpre.ptr, cs.ptr)
    got = cs.download(count=cols)
    d_ref = O.relu_backward(g, pre)
    np.testing.assert_array_equal(dpre.download(count=rows * cols).reshape(rows, cols), d_ref)
    if rows * cols <= 1 << 20:
        np.testing.assert_array_equal(got, _relu_bw_colsum_order(g, pre)[1])
    d64 = d_ref.astype(np.float64)
    bound = rows * 2.0 ** -24 * np.abs(d64).sum(0) + 1e-30
    assert (np.abs(got.astype(np.float64) - d64.sum(0)) <= bound).all()


def run_ce(ctx, logits, onehot=None, labels=None, want_grad=True):
    B, C = logits.shape
    dl = ctx.upload(logits)
    doh = ctx.upload(onehot) if onehot is not None else None
    dlb = ctx.upload(labels.astype(np.int32)) if labels is not None else None
    loss = ctx.alloc(4)
    grad = ctx.alloc(4 * B * C) if want_grad else None
    preds = ctx.alloc(4 * B)
    correct = ctx.alloc(8)
    _lib.call("orca_hip_softmax_ce", ctx.handle, dl.ptr, B, C, doh.ptr if doh else None, dlb.ptr if dlb else None,
              loss.ptr, grad.ptr if grad else None, preds.ptr, correct.ptr)
    return (float(loss.download(count=1)[0]), grad.download(count=B * C).reshape(B, C) if grad else None,
            preds.download(np.int32, B), int(correct.download(np.int64, 1)[0]))


@pytest.mark.parametrize("B,C", [(64, 10), (1024, 10), (37, 300), (16, 4096), (3, 1)])
def test_softmax_ce_matches_composed_reference(ctx, B, C):
    rng = np.random.default_rng(B * C)
    logits = (2.0 * rng.standard_normal((B, C))).astype(np.float32)
    labels = rng.integers(0, C, B)
    onehot = synth.one_hot(labels, C)
    loss_ref, grad_ref = O.cross_entropy(logits, onehot)
    for kw in (dict(onehot=onehot), dict(labels=labels)):
        loss, grad, preds, correct = run_ce(ctx, logits, **kw)
        assert_close(loss, loss_ref, what="loss")
        assert_close(grad, grad_ref, what="dlogits")
        assert_close_scaled(grad, grad_ref, what="dlogits (scaled)")
        np.testing.assert_array_equal(preds, O.argmax_rows(logits))
        assert correct == int((O.argmax_rows(logits) == labels).sum())


@pytest.mark.parametrize("B,C", [(5, 2000), (7, 1027), (300, 4096), (4, 1025)])
def test_softmax_ce_wide_rows_match_composed_reference(ctx, B, C):
    """Rows of 1025..4096 logits (a block per row): float4 and element-wise
    column layouts, full and partial rows."""
    test_softmax_ce_matches_composed_reference(ctx, B, C)


@pytest.mark.parametrize("C", [1, 10, 64, 300, 1025, 2048, 4096])
def test_softmax_ce_labels_equal_onehot_bit_exact(ctx, C):
    """Class-index targets and their one-hot rows give the same bits (loss,
    gradient, argmax, count), also for rows with infinite or NaN logits,
    whose loss term the class-index path forms in full as the reference does."""
    B = 12
    rng = np.random.default_rng(C + 5)
    logits = (3.0 * rng.standard_normal((B, C))).astype(np.float32)
    logits[1, C // 2] = np.inf
    logits[2, 0] = np.nan
    logits[3, :] = -np.inf
    logits[3, C - 1] = 2.0
    logits[4, :] = 7.0                      # equal logits
    logits[5, C // 3] = 300.0               # every other exp underflows: se == 1
    labels = rng.integers(0, C, B)
    labels[5] = C // 3                      # the label is the only non-underflowing column
    labels[6] = C // 3 if C > 1 else 0
    onehot = synth.one_hot(labels, C)
    a = run_ce(ctx, logits, labels=labels)
    b = run_ce(ctx, logits, onehot=onehot)
    np.testing.assert_array_equal(np.float32(a[0]), np.float32(b[0]))
    np.testing.assert_array_equal(a[1], b[1])
    np.testing.assert_array_equal(a[2], b[2])
    assert a[3] == b[3]


def test_softmax_ce_ties_nan_and_equal_logits(ctx):
    B, C = 6, 10
    logits = np.zeros((B, C), np.float32)  # equal logits: loss = ln C, ties everywhere
    logits[1, 3] = logits[1, 7] = 5.0      # tie at the max: first index wins
    logits[2, 0] = np.nan                  # NaN first: argmax 0 (nothing is > NaN)
    logits[3, 4] = np.nan                  # NaN later: ignored by the max
    logits[4, :] = -np.inf
    logits[4, 9] = 1.0
    logits[5, :] = np.float32(-3.0e38)
    labels = np.array([1, 7, 0, 4, 9, 2])
    onehot = synth.one_hot(labels, C)
    _, grad_ref = O.cross_entropy(logits, onehot)
    _, grad, preds, _ = run_ce(ctx, logits, onehot=onehot)
    np.testing.assert_array_equal(preds, O.argmax_rows(logits))
    rows = [0, 1, 4, 5]  # rows without NaN have finite gradients to compare
    assert_close(grad[rows], grad_ref[rows], what="dlogits")


@pytest.mark.parametrize("B,C", [(1024, 10), (64, 64), (37, 300), (6, 4096)])
def test_softmax_ce_onehot_gradient_holds_no_negative_zero(ctx, B, C):
    """With one-hot targets every element of dL/dlogits is (0 + a) + (0 + b), plus (0 + c) at a
    row's maximum: never -0 and never a signaling NaN, so 0 + d is d bit for bit.  The storage
    layer relies on it to hand the loss gradient on as its own identity sum_to_shape.  Rows of
    zeros, ties, +-inf, NaN, huge and tiny logits, labels on and off the maximum."""
    rng = np.random.default_rng(B + C)
    logits = (3.0 * rng.standard_normal((B, C))).astype(np.float32)
    logits[0, :] = 0.0
    logits[1, :] = -np.inf
    logits[1, C // 2] = 0.0
    logits[2, 0] = np.nan
    logits[3, C - 1] = np.inf
    logits[4, :] = np.float32(-3.0e38)
    logits[5, :] = 1e-30
    if B > 6:
        logits[6, C // 3] = 300.0
        logits[7, :] = np.float32(3.0e38)
    labels = rng.integers(0, C, B)
    labels[0] = 0
    labels[1] = C // 2
    onehot = synth.one_hot(labels, C)
    _, grad, _, _ = run_ce(ctx, logits, onehot=onehot)
    bits = grad.view(np.uint32)
    assert not (bits == 0x80000000).any(), np.argwhere(bits == 0x80000000)[:5]
    nan = np.isnan(grad)
    assert ((bits[nan] & 0x00400000) != 0).all()  # quiet NaNs only
    np.testing.assert_array_equal((np.float32(0.0) + grad).view(np.uint32), bits)


def test_adamw_and_sgd_bit_exact(ctx):
    rng = np.random.default_rng(11)
    n = 100003  # odd length exercises the scalar tail
    p = (0.02 * rng.standard_normal(n)).astype(np.float32)
    g = (1e-3 * rng.standard_normal(n)).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    dp, dg, dm, dv = (ctx.upload(a) for a in (p, g, m, v))
    ref = (p, m, v)
    for t in range(1, 4):
        _lib.call("orca_hip_adamw_step", ctx.handle, dp.ptr, dg.ptr, dm.ptr, dv.ptr, n, 1e-3, 0.9, 0.999, 1e-8,
                  0.01, t)
        ref = O.adamw_update(ref[0], g, ref[1], ref[2], t)
    np.testing.assert_array_equal(dp.download(count=n), ref[0])
    np.testing.assert_array_equal(dm.download(count=n), ref[1])
    np.testing.assert_array_equal(dv.download(count=n), ref[2])
    ds = ctx.upload(p)
    _lib.call("orca_hip_sgd_step", ctx.handle, ds.ptr, dg.ptr, n, 0.1)
    np.testing.assert_array_equal(ds.download(count=n), O.sgd_update(p, g, 0.1))


def _trainer_run(ctx, w, steps, use_labels=False):
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    o = w["opt"]
    tr = MLPTrainer(ctx, w["dims"], w["batch"], kind=o["kind"], lr=o["lr"], weight_decay=o.get("weight_decay", 0.0),
                    betas=o.get("betas", (0.9, 0.999)), eps=o.get("eps", 1e-8))
    tr.set_params(params)
    if use_labels:
        tr.set_batch(x, labels=labels)
    else:
        tr.set_batch(x, onehot=onehot)
    losses = []
    for _ in range(steps):
        tr.step()
        losses.append(tr.metrics()[0])
    ref = O.mlp_train(w["dims"], params, x, onehot, O.make_opt(o["kind"], o["lr"], o.get("weight_decay", 0.0),
                                                            o.get("betas", (0.9, 0.999)), o.get("eps", 1e-8)),
                      steps=steps)
    return tr, ref, np.array(losses, np.float32)


@pytest.mark.parametrize("use_labels", [False, True])
def test_mlp_step_784_128_128_10_sgd(ctx, use_labels):
    tr, ref, losses = _trainer_run(ctx, synth.WORKLOADS[synth.MLP_SMALL], 1, use_labels)
    assert_close(losses, ref["losses"], what="loss")
    for i, (g, gr) in enumerate(zip(tr.grads(), ref["grads"])):
        assert_close(g, gr, what=f"grad {i}")
        assert_close_scaled(g, gr, rtol=1e-3, what=f"grad {i} (scaled)")
    for i, (p, pr) in enumerate(zip(tr.params(), ref["params"])):
        assert_close(p, pr, what=f"param {i}")
    np.testing.assert_array_equal(tr.preds(), ref["preds"])
    assert tr.metrics()[1] == ref["correct"]


@pytest.mark.parametrize("dims,batch,kind", [
    ((20, 7), 33, "sgd"),              # one layer: the fused head reads the input, no ReLU below it
    ((37, 50, 19), 33, "adamw"),       # 19 classes (GEMM head), widths not multiples of 4 (generic GEMM)
    ((784, 128, 128, 10), 1, "adamw"), # batch of one
    ((64, 96, 64, 32, 16), 70, "sgd"), # four layers, 16 classes (widest fused head), ragged batch
    ((33, 41, 5), 129, "adamw"),       # head input width 41 (not a multiple of 4: GEMM head path)
])
def test_mlp_step_odd_shapes(ctx, dims, batch, kind):
    """The trainer on shapes other than the three benchmark MLPs, two steps against the oracle."""
    params, x, labels, onehot = synth.mlp_problem(7, dims, batch)
    opt = dict(kind=kind, lr=0.05 if kind == "sgd" else 1e-3, weight_decay=0.0 if kind == "sgd" else 0.01)
    tr = MLPTrainer(ctx, dims, batch, kind=kind, lr=opt["lr"], weight_decay=opt["weight_decay"])
    tr.set_params(params)
    tr.set_batch(x, onehot=onehot)
    losses = []
    for _ in range(2):
        tr.step()
        losses.append(tr.metrics()[0])
    ref = O.mlp_train(dims, params, x, onehot, O.make_opt(kind, opt["lr"], opt["weight_decay"]), steps=2)
    assert_close(np.array(losses, np.float32), ref["losses"], what="loss")
    for i, (g, gr) in enumerate(zip(tr.grads(), ref["grads"])):
        assert_close(g, gr, what=f"grad {i}")
    for i, (p, pr) in enumerate(zip(tr.params(), ref["params"])):
        assert_close(p, pr, what=f"param {i}")
    np.testing.assert_array_equal(tr.preds(), ref["preds"])
    tr.close()


@pytest.mark.parametrize("kind", ["adamw", "sgd"])
def test_multi_segment_optimizer_equals_one_tensor_kernels(ctx, kind):
    """orca_hip_adamw_multi / orca_hip_sgd_multi over many parameters (more than one launch's
    table; sizes not multiples of 4; slices at unaligned offsets, which take the element path;
    p_dst apart from p_src and equal to it) give the bits of orca_hip_adamw_step /
    orca_hip_sgd_step run parameter by parameter."""
    from orcaml_amd.backend import HipBackend

    be = HipBackend(ctx, lazy=False)
    rng = np.random.default_rng(17)
    sizes = [1, 5, 4, 1023, 4096, 3, 100001] + [7 + i for i in range(30)]
    assert len(sizes) > _lib.OPT_MAX_SEGMENTS
    offs, total = [], 0
    for k, n in enumerate(sizes):
        offs.append(total + (k % 3 == 1))  # every third slice one float off 16-byte alignment
        total = offs[-1] + n + 8
    p0 = rng.standard_normal(total).astype(np.float32)
    g0 = (rng.standard_normal(total) * 1e-2).astype(np.float32)
    m0 = (rng.standard_normal(total) * 1e-3).astype(np.float32)
    v0 = np.abs(rng.standard_normal(total) * 1e-4).astype(np.float32)
    arenas = {}
    for name, a in (("p", p0), ("g", g0), ("m", m0), ("v", v0), ("q", np.zeros(total, np.float32))):
        arenas[name] = be.arena(total)
        _lib.call("orca_hip_h2d", ctx.handle, arenas[name].ptr, a.ctypes.data_as(ctypes.c_void_p), a.nbytes)
    views = {k: [be.view(arenas[k], o, n) for o, n in zip(offs, sizes)] for k in arenas}
    in_place = [k % 2 == 0 for k in range(len(sizes))]  # p_dst = p_src for every other parameter
    dst = [views["p"][k] if in_place[k] else views["q"][k] for k in range(len(sizes))]
    want_p, want_m, want_v = [], [], []
    for k, n in enumerate(sizes):
        o = offs[k]
        p, g = be.from_f32_slice((n,), p0[o:o + n]), be.from_f32_slice((n,), g0[o:o + n])
        m, v = be.from_f32_slice((n,), m0[o:o + n]), be.from_f32_slice((n,), v0[o:o + n])
        if kind == "adamw":
            be.adamw_step_(p, g, m, v, n, 1e-3, 0.9, 0.999, 1e-8, 0.01, 3)
            want_m.append(be.to_f32_vec(m))
            want_v.append(be.to_f32_vec(v))
        else:
            be.sgd_step_(p, g, n, 0.1)
        want_p.append(be.to_f32_vec(p))
    if kind == "adamw":
        be.adamw_multi_([(views["p"][k], dst[k], views["g"][k], views["m"][k], views["v"][k], n)
                         for k, n in enumerate(sizes)], 1e-3, 0.9, 0.999, 1e-8, 0.01, 3)
    else:
        be.sgd_multi_([(views["p"][k], dst[k], views["g"][k], n) for k, n in enumerate(sizes)], 0.1)
    for k, n in enumerate(sizes):
        np.testing.assert_array_equal(be.to_f32_vec(dst[k]), want_p[k], err_msg=f"p of segment {k}")
        if kind == "adamw":
            np.testing.assert_array_equal(be.to_f32_vec(views["m"][k]), want_m[k], err_msg=f"m of segment {k}")
            np.testing.assert_array_equal(be.to_f32_vec(views["v"][k]), want_v[k], err_msg=f"v of segment {k}")
    # the bytes between slices are untouched
    q = np.empty(total, np.float32)
    _lib.call("orca_hip_d2h", ctx.handle, q.ctypes.data_as(ctypes.c_void_p), arenas["q"].ptr, q.nbytes)
    written = np.zeros(total, bool)
    for k, (o, n) in enumerate(zip(offs, sizes)):
        if not in_place[k]:
            written[o:o + n] = True
    assert not q[~written].any()


@pytest.mark.parametrize("band_ctx", [1, 2], indirect=True, ids=["band8", "band112"])
def test_gemm_band_padded_leading_dimensions(band_ctx):
    """The banded kernels read A, B and write C through their leading dimensions: X stored
    [K][lda] with lda = 800 > 784, dY [K][ldb] with ldb = 4100, C [784][ldc] with ldc = 4104;
    exact on integers, the padding of C untouched, the column sum bit-identical."""
    ctx = band_ctx
    M, N, K, lda, ldb, ldc = 784, 4096, 96, 800, 4100, 4104
    rng = np.random.default_rng(8)
    X = int_matrix(rng, (K, lda))
    dY = int_matrix(rng, (K, ldb))
    dA, dB = ctx.upload(X), ctx.upload(dY)
    C0 = np.full((M, ldc), 7.0, np.float32)
    dC, dcs = ctx.upload(C0), ctx.alloc(4 * N)
    e = _lib.Epilogue(_lib.EPI_NONE, None, None, 0, None)
    e.colsum = dcs.ptr
    ctx.prof_reset()
    ctx.prof_enable(True)
    _lib.call("orca_hip_gemm", ctx.handle, 1, 0, M, N, K, dA.ptr, lda, dB.ptr, ldb, dC.ptr, ldc, ctypes.byref(e))
    ctx.prof_enable(False)
    names = {k["name"] for k in ctx.prof_report()["kernels"]}
    assert f"{'gemm_tn_band8' if ctx.band_mode == 1 else 'gemm_tn_band112'} {M}x{N}x{K}" in names, names
    C = dC.download(count=M * ldc).reshape(M, ldc)
    want = (X[:, :M].T.astype(np.int64) @ dY[:, :N].astype(np.int64)).astype(np.float32)
    np.testing.assert_array_equal(C[:, :N], want)
    np.testing.assert_array_equal(C[:, N:], C0[:, N:])
    np.testing.assert_array_equal(dcs.download(count=N), O.sum_to_shape(np.ascontiguousarray(dY[:, :N]), (1, N)).reshape(N))
