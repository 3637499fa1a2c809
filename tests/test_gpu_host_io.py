"""GPU checks of the host boundary: uploads are stream-ordered without a host
wait (the trait's from_f32_slice / from_bytes, orca-backend-cpu/src/backend.rs:87-89
and 296-297), the composed backward pass and optimizer step never wait for the
device (orca-autograd/src/tensor.rs:47-56 uploads the seed and walks the tape;
python/orca/optim/adamw.py:48-99), and a pointer into a freed buffer is refused."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from orcaml_amd import _lib, synth
from orcaml_amd import autodiff as A

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 7, 256, 257, 1000, 300_000, 1_500_000, 9_000_001])
def test_upload_without_host_wait_round_trips(hb, n):
    """Payloads up to 1 KiB go as a kernel argument, larger ones through the pinned
    staging ring in 4 MiB regions (9M floats = 36 MB wraps the 16 MiB ring twice,
    so later regions wait for earlier copies).  The host array is overwritten
    right after each call: the device must hold the values at call time."""
    rng = np.random.default_rng(n)
    a = rng.standard_normal(n).astype(np.float32)
    keep = a.copy()
    before = hb.ctx.sync_count()
    s = hb.from_f32_slice((n,), a)
    a[:] = -1.0
    b = hb.from_bytes((n,), keep.tobytes())
    syncs = hb.ctx.sync_count() - before
    ring_waits_allowed = (2 * 4 * n) // (16 << 20)  # back-pressure only when more than the ring is queued
    assert syncs <= ring_waits_allowed, syncs
    np.testing.assert_array_equal(hb.to_f32_vec(s), keep)
    np.testing.assert_array_equal(hb.to_f32_vec(b), keep)


def test_many_small_and_large_uploads_interleaved(hb):
    """Regions are recycled by events in ring order: 200 uploads of mixed sizes, every
    result checked after one final host read."""
    rng = np.random.default_rng(3)
    arrays, stores = [], []
    for i in range(200):
        n = int(rng.choice([3, 250, 5000, 400_000]))
        a = rng.standard_normal(n).astype(np.float32)
        arrays.append(a.copy())
        stores.append(hb.from_f32_slice((n,), a))
        a[:] = np.nan
    for a, s in zip(arrays, stores):
        np.testing.assert_array_equal(hb.to_f32_vec(s), a)


@pytest.mark.parametrize("fused", [False, True])
def test_backward_and_optimizer_step_never_wait_for_the_device(hb, fused):
    """Between loss.backward() and the end of AdamW.step() the composed path performs no
    host wait: the seed and the optimizer's eps scalar are stream-ordered uploads."""
    w = synth.WORKLOADS[synth.MLP_SMALL]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    ad = A.Autodiff(hb)
    model = A.build_mlp(ad, params)
    opt = A.AdamW(model.parameters(), lr=1e-3, weight_decay=0.01, fused=fused)
    xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
    loss_fn = A.CrossEntropyLoss(fused=fused)
    for _ in range(2):
        opt.zero_grad()
        loss = loss_fn(model(xt), tt)
        before = hb.ctx.sync_count()
        loss.backward()
        opt.step()
        assert hb.ctx.sync_count() == before
        assert np.isfinite(loss.to_list()[0])
        assert hb.ctx.sync_count() == before + 1  # the loss read is the one host wait


def test_pointer_into_a_freed_buffer_is_refused(hb):
    """check_extent knows the blocks the allocator holds after a free: an op given such a
    pointer fails with InternalError before anything is launched."""
    ctx = hb.ctx
    buf = ctx.alloc(4096)
    ptr = buf.ptr
    buf.free()
    out = ctypes.c_void_p()
    d, r = _lib.dims((16,))
    live_before = ctx.mem_stats()["live"]
    rc = _lib.load().orca_hip_relu(ctx.handle, ctypes.c_void_p(ptr + 64), d, r, _lib.F32, ctypes.byref(out))
    assert rc == _lib.ERR_INTERNAL
    assert b"freed" in _lib.load().orca_hip_last_error()
    assert ctx.mem_stats()["live"] == live_before  # the op's output went back to the allocator
    live = ctx.alloc(4096)  # the same size class: the cached block is handed out again and is live
    _lib.call("orca_hip_relu", ctx.handle, ctypes.c_void_p(live.ptr), d, r, _lib.F32, ctypes.byref(out))
    _lib.call("orca_hip_free", ctx.handle, out)
