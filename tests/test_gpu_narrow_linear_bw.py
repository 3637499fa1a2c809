"""orca_hip_narrow_linear_backward -- a classifier head's backward (dW = H^T G, db = the column
sums of G, dH = G W^T through a ReLU mask) from one grid -- against the same products computed
one by one through the C ABI (orca_hip_matmul_colsum for dW and db, orca_hip_gemm with the mask
epilogue for dH): bit for bit, since each block role runs its own kernel's code with the plan
that product would take; and db against the oracle's sum_to_shape (ascending rows) bit for bit."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from orcaml_amd import _lib
from tests.test_gpu_narrow_gemm import kernel_names

pytestmark = pytest.mark.gpu

SHAPES = [(1024, 4096, 10), (256, 1024, 10), (64, 128, 10), (1000, 4092, 7), (1, 1, 1), (300, 1030, 16),
          (4099, 260, 3), (33, 64, 5), (512, 784, 12)]


def _one_by_one(ctx, dH_, dG, dWt, dmask, B, K, C, variant):
    """dW, db, dH (and dH_pre) from the separate entry points."""
    db = ctx.alloc(4 * C)
    out = ctypes.c_void_p()
    _lib.call("orca_hip_matmul_colsum", ctx.handle, dH_.ptr, dG.ptr, K, B, C, _lib.VIEW_TRANSPOSED, _lib.F32, db.ptr,
              ctypes.byref(out))
    dW_host = np.empty(K * C, np.float32)
    _lib.call("orca_hip_d2h", ctx.handle, dW_host.ctypes.data_as(ctypes.c_void_p), out, 4 * K * C)
    _lib.call("orca_hip_free", ctx.handle, out)
    dH = ctx.alloc(4 * B * K)
    pre = ctx.alloc(4 * B * K) if variant == "mask_pre_db" else None
    e = _lib.Epilogue()
    e.kind = {"mask_pre_db": _lib.EPI_RELU_MASK_PRE, "mask": _lib.EPI_RELU_MASK, "plain": _lib.EPI_NONE}[variant]
    if variant != "plain":
        e.mask = dmask.ptr
        e.ldmask = K
    if pre is not None:
        e.pre = pre.ptr
    _lib.call("orca_hip_gemm", ctx.handle, 0, 1, B, K, C, dG.ptr, C, dWt.ptr, C, dH.ptr, K, ctypes.byref(e))
    return (dW_host, db.download(count=C), dH.download(count=B * K),
            pre.download(count=B * K) if pre is not None else None)


@pytest.mark.parametrize("variant", ["mask_pre_db", "mask", "plain"])
@pytest.mark.parametrize("B,K,C", SHAPES)
def test_narrow_linear_backward_equals_products_one_by_one(ctx, B, K, C, variant):
    print(f"narrow_linear_backward B={B} K={K} C={C} {variant}", flush=True)
    rng = np.random.default_rng(B + 7 * K + 31 * C)
    H = rng.standard_normal((B, K)).astype(np.float32)
    G = rng.standard_normal((B, C)).astype(np.float32)
    W = rng.standard_normal((K, C)).astype(np.float32)
    z = rng.standard_normal((B, K)).astype(np.float32)
    z.reshape(-1)[::7] = 0.0
    dH_, dG, dWt, dz = ctx.upload(H), ctx.upload(G), ctx.upload(W), ctx.upload(z)
    want_dW, want_db, want_dH, want_pre = _one_by_one(ctx, dH_, dG, dWt, dz, B, K, C, variant)
    dW, dH = ctx.alloc(4 * K * C), ctx.alloc(4 * B * K)
    db = ctx.alloc(4 * C) if variant == "mask_pre_db" else None
    pre = ctx.alloc(4 * B * K) if variant == "mask_pre_db" else None
    _, names = kernel_names(ctx, lambda: _lib.call(
        "orca_hip_narrow_linear_backward", ctx.handle, dH_.ptr, B, K, dG.ptr, C, dWt.ptr,
        dz.ptr if variant != "plain" else None, dH.ptr, pre.ptr if pre is not None else None, dW.ptr,
        db.ptr if db is not None else None, None))
    assert "narrow_linear_bw" in names, names
    np.testing.assert_array_equal(dW.download(count=K * C), want_dW)
    np.testing.assert_array_equal(dH.download(count=B * K), want_dH)
    if db is not None:
        got_db = db.download(count=C)
        np.testing.assert_array_equal(got_db, want_db)
        np.testing.assert_array_equal(got_db, O.sum_to_shape(G, (1, C)).reshape(C))
    if pre is not None:
        np.testing.assert_array_equal(pre.download(count=B * K), want_pre)


def test_narrow_linear_backward_rejects_wide_outputs(ctx):
    d = ctx.alloc(4 * 64 * 32)
    rc = _lib.load().orca_hip_narrow_linear_backward(ctx.handle, d.ptr, 8, 8, d.ptr, 17, d.ptr, None, d.ptr, None,
                                                      d.ptr, None, None)
    assert rc == _lib.ERR_INTERNAL
    assert b"C <= 16" in _lib.load().orca_hip_last_error()
