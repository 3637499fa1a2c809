"""GPU parity of the narrow products (N <= 16 with a row-major B, K <= 16 against
B^T), which run on vector-unit kernels instead of matrix-core tiles: X W and
X^T dY of a 10-class head, dY W^T back through it.  Exact on integers (any
summation order), within the f32 dot-product bound on real data, and the
column sum of a narrow X^T dY equals sum_to_shape bit for bit."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from orcaml_amd import _lib
from tests.test_gpu_fused import assert_gemm_error_bound, run_gemm
from tests.util import int_matrix

pytestmark = pytest.mark.gpu

NARROW_N = [(1024, 10, 4096), (1024, 10, 784), (1, 1, 1), (5, 3, 7), (1023, 16, 1001), (4099, 1, 4096), (64, 13, 2)]
SMALL_K = [(1024, 4096, 10), (1, 1, 1), (7, 1001, 3), (1000, 4099, 16), (256, 784, 10), (3, 12, 13)]
NARROW_TN = [(4096, 10, 1024), (4096, 10, 256), (784, 10, 1024), (1, 1, 1), (1001, 7, 300), (260, 16, 4099),
             (4099, 1, 63), (33, 10, 64)]


def kernel_names(ctx, fn):
    ctx.prof_reset()
    ctx.prof_enable(True)
    try:
        out = fn()
    finally:
        ctx.prof_enable(False)
    return out, {k["name"] for k in ctx.prof_report()["kernels"]}


@pytest.mark.parametrize("M,N,K", NARROW_N)
def test_nn_narrow_exact_on_integers(ctx, M, N, K):
    rng = np.random.default_rng(M + 3 * N + 7 * K)
    A, B = int_matrix(rng, (M, K)), int_matrix(rng, (K, N))
    got, names = kernel_names(ctx, lambda: run_gemm(ctx, False, False, A, B))
    assert f"gemm_nn_narrow {M}x{N}x{K}" in names, names
    np.testing.assert_array_equal(got, (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("M,N,K", SMALL_K)
def test_nt_small_k_exact_on_integers(ctx, M, N, K):
    rng = np.random.default_rng(M + 5 * N + 11 * K)
    A, B = int_matrix(rng, (M, K)), int_matrix(rng, (K, N))
    got, names = kernel_names(ctx, lambda: run_gemm(ctx, False, True, A, np.ascontiguousarray(B.T)))
    assert f"gemm_nt_smallk {M}x{N}x{K}" in names, names
    np.testing.assert_array_equal(got, (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("M,N,K", NARROW_TN)
def test_tn_narrow_exact_on_integers_with_exact_colsum(ctx, M, N, K):
    """X^T dY (X stored [K][M]) in K slices summed in slice order, and the bias gradient
    (column sum of dY) in ascending row order: bit-identical to sum_to_shape."""
    rng = np.random.default_rng(M + 17 * N + K)
    X, dY = int_matrix(rng, (K, M)), int_matrix(rng, (K, N))
    (got, cs), names = kernel_names(ctx, lambda: run_gemm(ctx, True, False, X, dY, colsum=True))
    assert f"gemm_tn_narrow {M}x{N}x{K}" in names, names
    assert ("gemm_narrow_reduce" in names) == (K > 64), names  # one slice up to one 64-row chunk
    np.testing.assert_array_equal(got, (X.T.astype(np.int64) @ dY.astype(np.int64)).astype(np.float32))
    np.testing.assert_array_equal(cs, O.sum_to_shape(dY, (1, N)).reshape(N))


@pytest.mark.parametrize("ta,tb,M,N,K", [(False, False, 1024, 10, 4096), (False, True, 1024, 4096, 10),
                                         (True, False, 4096, 10, 1024), (False, False, 130, 16, 1000),
                                         (True, False, 1000, 13, 777)])
def test_narrow_within_dot_product_bound(ctx, ta, tb, M, N, K):
    rng = np.random.default_rng(M * N + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    got = run_gemm(ctx, ta, tb, np.ascontiguousarray(A.T) if ta else A, np.ascontiguousarray(B.T) if tb else B)
    assert_gemm_error_bound(got, A, B)


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False)])
def test_narrow_unaligned_operands(ctx, ta, tb):
    """Operands at an odd float offset with an odd leading dimension (the scalar-load
    paths) give the same integers as the aligned call."""
    M, N, K = (1023, 9, 517) if not tb else (1023, 517, 9)
    rng = np.random.default_rng(5)
    A, B = int_matrix(rng, (M, K)), int_matrix(rng, (K, N))
    a_st = np.ascontiguousarray(A.T) if ta else A
    b_st = np.ascontiguousarray(B.T) if tb else B
    want = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)
    # stored operands padded by one column and shifted by one float
    a_pad = np.zeros((a_st.shape[0], a_st.shape[1] + 1), np.float32)
    a_pad[:, 1:] = a_st
    b_pad = np.zeros((b_st.shape[0], b_st.shape[1] + 1), np.float32)
    b_pad[:, 1:] = b_st
    dA, dB = ctx.upload(a_pad), ctx.upload(b_pad)
    dC = ctx.alloc(4 * M * N)
    e = _lib.Epilogue(_lib.EPI_NONE, None, None, 0, None)
    _lib.call("orca_hip_gemm", ctx.handle, int(ta), int(tb), M, N, K, dA.ptr + 4, a_pad.shape[1], dB.ptr + 4,
              b_pad.shape[1], dC.ptr, N, ctypes.byref(e))
    np.testing.assert_array_equal(dC.download(count=M * N).reshape(M, N), want)
    np.testing.assert_array_equal(run_gemm(ctx, ta, tb, a_st, b_st), want)


def test_narrow_epilogues_match_composed_ops(ctx):
    """A bias on a narrow X W and a ReLU mask on a narrow dY W^T run inside the narrow kernels
    (sliced or not), bit-identical to the composed ops on their own product; bias + ReLU keeps
    a narrow product on the tiled kernels."""
    rng = np.random.default_rng(9)
    for M, N, K in ((256, 10, 512), (1024, 10, 4096), (7, 3, 5)):  # one slice, 8 slices, one tiny block
        A, B = rng.standard_normal((M, K)).astype(np.float32), rng.standard_normal((K, N)).astype(np.float32)
        bias = rng.standard_normal(N).astype(np.float32)
        prod = run_gemm(ctx, False, False, A, B)
        got, names = kernel_names(ctx, lambda: run_gemm(ctx, False, False, A, B, _lib.EPI_BIAS, bias=bias))
        assert f"gemm_nn_narrow {M}x{N}x{K}" in names, names
        np.testing.assert_array_equal(got, O.add(prod, O.expand(bias.reshape(1, N), (M, N))))
        _, names = kernel_names(ctx, lambda: run_gemm(ctx, False, False, A, B, _lib.EPI_BIAS_RELU, bias=bias))
        assert not any("narrow" in n for n in names), names
    for M, N, K in ((1024, 4096, 10), (33, 1001, 3)):
        A, B = rng.standard_normal((M, K)).astype(np.float32), rng.standard_normal((K, N)).astype(np.float32)
        Bt = np.ascontiguousarray(B.T)
        mask = rng.standard_normal((M, N)).astype(np.float32)
        mask[::5, ::3] = 0.0
        prod = run_gemm(ctx, False, True, A, Bt)
        got, names = kernel_names(ctx, lambda: run_gemm(ctx, False, True, A, Bt, _lib.EPI_RELU_MASK, mask=mask))
        assert f"gemm_nt_smallk {M}x{N}x{K}" in names, names
        np.testing.assert_array_equal(got, O.relu_backward(prod, mask))
