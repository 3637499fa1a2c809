"""orca_hip_relu_bw_colsum_noalloc (no device allocation; fixed per-GPU scratch)
against orca_hip_relu_bw_colsum (ReluBackward + the bias ExpandBackward's
sum_to_shape, orca-autograd/src/backend.rs:1633-1645, 1684-1697): both run the
same kernels in the same order, so dpre and the column sums must agree bit for
bit.  Two calls in a row, the second smaller, with no allocator call between."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from orcaml_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(ctx, rng, rows, cols):
    g = rng.standard_normal((rows, cols)).astype(np.float32)
    pre = rng.standard_normal((rows, cols)).astype(np.float32)
    pre.reshape(-1)[::13] = 0.0
    pre.reshape(-1)[5::17] = -0.0
    return ctx.upload(g), ctx.upload(pre)


def _run(ctx, fn, dg, dpre_in, rows, cols):
    dpre = ctx.alloc(4 * max(rows * cols, 1))
    cs = ctx.alloc(4 * max(cols, 1))
    _lib.call(fn, ctx.handle, dg.ptr, dpre_in.ptr, rows, cols, dpre.ptr, cs.ptr)
    return dpre, cs


@pytest.mark.parametrize("shapes", [((8192, 4096), (1000, 1030)), ((4096, 256), (64, 4096)), ((777, 130), (3, 5))])
def test_noalloc_matches_allocating_entry_point(ctx, shapes):
    rng = np.random.default_rng(sum(shapes[0]) + sum(shapes[1]))
    for rows, cols in shapes:
        print(f"relu_bw_colsum_noalloc rows={rows} cols={cols}", flush=True)
        dg, dp = _inputs(ctx, rng, rows, cols)
        want_d, want_cs = _run(ctx, "orca_hip_relu_bw_colsum", dg, dp, rows, cols)
        out_d, out_cs = ctx.alloc(4 * rows * cols), ctx.alloc(4 * cols)
        before = ctx.mem_stats()
        _lib.call("orca_hip_relu_bw_colsum_noalloc", ctx.handle, dg.ptr, dp.ptr, rows, cols, out_d.ptr, out_cs.ptr)
        after = ctx.mem_stats()
        assert after == before  # no block taken from the cache, no device allocation
        np.testing.assert_array_equal(out_d.download(count=rows * cols), want_d.download(count=rows * cols))
        np.testing.assert_array_equal(out_cs.download(count=cols), want_cs.download(count=cols))


def test_noalloc_rejects_sizes_beyond_its_scratch(ctx):
    rows, cols = 64 * 257, 4096  # 257 * 4096 partials > 2^20
    out = ctx.alloc(4 * cols)
    rc = _lib.load().orca_hip_relu_bw_colsum_noalloc(ctx.handle, None, None, ctypes.c_size_t(rows),
                                                      ctypes.c_size_t(cols), None, ctypes.c_void_p(out.ptr))
    assert rc == _lib.ERR_INTERNAL
    assert b"scratch" in _lib.load().orca_hip_last_error()
    # without a column sum no scratch is used: any size goes, still without allocating
    dg, dp = _inputs(ctx, np.random.default_rng(1), 128, 64)
    d = ctx.alloc(4 * 128 * 64)
    before = ctx.mem_stats()
    _lib.call("orca_hip_relu_bw_colsum_noalloc", ctx.handle, dg.ptr, dp.ptr, 128, 64, d.ptr, None)
    assert ctx.mem_stats() == before
    want_d, _ = _run(ctx, "orca_hip_relu_bw_colsum", dg, dp, 128, 64)
    np.testing.assert_array_equal(d.download(count=128 * 64), want_d.download(count=128 * 64))


def test_noalloc_calls_from_two_contexts_take_the_scratch_in_turn(ctx):
    """Two contexts on one GPU (two streams) share its one scratch array: each call's stream first
    waits on the device for the last call that used it, so calls issued back to back from both,
    with no host wait between, each equal the allocating entry point bit for bit."""
    from orcaml_amd.device import Context

    other = Context(ctx.device)
    try:
        rng = np.random.default_rng(21)
        jobs = []
        for c, (rows, cols) in [(ctx, (8192, 4096)), (other, (4096, 2048)), (ctx, (1000, 1030)),
                                (other, (8192, 4096)), (ctx, (64, 4096)), (other, (777, 130))]:
            print(f"two contexts: rows={rows} cols={cols}", flush=True)
            dg, dp = _inputs(c, rng, rows, cols)
            want_d, want_cs = _run(c, "orca_hip_relu_bw_colsum", dg, dp, rows, cols)
            out_d, out_cs = c.alloc(4 * rows * cols), c.alloc(4 * cols)
            jobs.append((c, dg, dp, rows, cols, want_d, want_cs, out_d, out_cs))
        ctx.sync()
        other.sync()
        for c, dg, dp, rows, cols, _, _, out_d, out_cs in jobs:  # back to back, alternating contexts
            _lib.call("orca_hip_relu_bw_colsum_noalloc", c.handle, dg.ptr, dp.ptr, rows, cols, out_d.ptr, out_cs.ptr)
        for c, dg, dp, rows, cols, want_d, want_cs, out_d, out_cs in jobs:
            np.testing.assert_array_equal(out_d.download(count=rows * cols), want_d.download(count=rows * cols))
            np.testing.assert_array_equal(out_cs.download(count=cols), want_cs.download(count=cols))
        del jobs
    finally:
        other.close()
