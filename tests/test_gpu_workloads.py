"""Full-size workloads of the MLP hot path on the GPU against the CPU oracle:
100 AdamW steps at H=1024 / B=256, one AdamW step of the 784-4096-4096-10 MLP
at B=1024, the fused backward epilogue on [8192, 4096], and AdamW over 2^28
parameters."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from orcaml_amd import _lib, synth
from orcaml_amd.mlp import MLPTrainer
from tests.parity import check_one_adamw_step, check_teacher_forced_adamw_step, oracle_hidden
from tests.util import assert_close, assert_close_scaled

pytestmark = pytest.mark.gpu


def make_trainer(ctx, w, params):
    o = w["opt"]
    tr = MLPTrainer(ctx, w["dims"], w["batch"], kind=o["kind"], lr=o["lr"], weight_decay=o.get("weight_decay", 0.0),
                    betas=o.get("betas", (0.9, 0.999)), eps=o.get("eps", 1e-8))
    tr.set_params(params)
    return tr


def ref_opt(w):
    o = w["opt"]
    return O.make_opt(o["kind"], o["lr"], o.get("weight_decay", 0.0), o.get("betas", (0.9, 0.999)), o.get("eps", 1e-8))


def test_mlp784_1024_b256_hundred_adamw_steps_teacher_forced(ctx):
    """784-1024-1024-10, batch 256, 100 AdamW(1e-3, wd 0.01) steps on one fixed
    batch.  At every step the oracle takes one step from the GPU's own state
    (parameters, moments, t):
      * the loss agrees to the path's tolerance (1e-5 abs + 1e-4 rel);
      * every gradient agrees to that tolerance, except entries attributed to
        counted ReLU mask flips between the two forward passes;
      * the new parameters and both moments are bit-identical to the oracle's
        AdamW applied to the GPU's own gradients from the same state (AdamW
        normalises gradients, so near-cancelling moments would turn rounding-
        level gradient differences into parameter differences of order lr;
        the update itself has no rounding freedom)."""
    w = synth.WORKLOADS[synth.MLP_MEDIUM]
    dims = w["dims"]
    o = w["opt"]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], dims, w["batch"])
    tr = make_trainer(ctx, w, params)
    tr.set_batch(x, onehot=onehot)
    zeros = [np.zeros_like(p) for p in params]
    state = dict(params=params, m=zeros, v=zeros, t=0)
    total_flips = 0
    for step in range(w["steps"]):
        tr.step()
        loss, _ = tr.metrics()
        ref = O.mlp_train(dims, state["params"], x, onehot, ref_opt(w), steps=1, m=state["m"], v=state["v"],
                          t=state["t"], want_grads=True)
        ref["hidden"] = oracle_hidden(state["params"], x, dims)
        hidden = [tr.activation(l) for l in range(len(dims) - 2)]
        got_g, got_p, got_m, got_v = tr.grads(), tr.params(), tr.moments(0), tr.moments(1)
        flips = check_teacher_forced_adamw_step(dims, o, state, ref, loss, hidden, got_g, got_p, got_m, got_v,
                                                what=f"step {step}")
        total_flips += sum(flips)
        t = state["t"] + 1
        state = dict(params=got_p, m=got_m, v=got_v, t=t)
    print(f"784-1024-1024-10 teacher-forced: {total_flips} ReLU mask flips over {w['steps']} steps")
    assert tr.step_count() == state["t"] == 100


def test_side_stream_update_at_ragged_widths_teacher_forced(ctx):
    """100-2100-2002-10 at batch 129: more than 2^22 parameters above layer 0, so the update of
    layers 1-2 runs on the second stream beside the dZ and dW products, reading one parameter
    arena and writing the other, split at a ragged offset; partial GEMM tiles everywhere.
    Three steps, each from the GPU's own state (parameters, moments, t): loss and gradients to
    the path's tolerance (modulo counted ReLU mask flips), new parameters and moments
    bit-identical to the oracle's AdamW on the GPU's gradients."""
    dims, batch = (100, 2100, 2002, 10), 129
    o = dict(kind="adamw", lr=1e-3, weight_decay=0.01)
    w = dict(dims=dims, batch=batch, opt=o)
    assert sum(a * b + b for a, b in zip(dims[1:-1], dims[2:])) > 1 << 22
    params, x, labels, onehot = synth.mlp_problem(11, dims, batch)
    tr = make_trainer(ctx, w, params)
    tr.set_batch(x, onehot=onehot)
    zeros = [np.zeros_like(p) for p in params]
    state = dict(params=params, m=zeros, v=zeros, t=0)
    for step in range(3):
        tr.step()
        loss, _ = tr.metrics()
        ref = O.mlp_train(dims, state["params"], x, onehot, ref_opt(w), steps=1, m=state["m"], v=state["v"],
                          t=state["t"], want_grads=True)
        ref["hidden"] = oracle_hidden(state["params"], x, dims)
        hidden = [tr.activation(l) for l in range(len(dims) - 2)]
        got_g, got_p, got_m, got_v = tr.grads(), tr.params(), tr.moments(0), tr.moments(1)
        check_teacher_forced_adamw_step(dims, o, state, ref, loss, hidden, got_g, got_p, got_m, got_v,
                                        what=f"step {step}")
        state = dict(params=got_p, m=got_m, v=got_v, t=state["t"] + 1)
    tr.close()


def _fraction_outside(got, want):
    bad = sum(int((np.abs(g.astype(np.float64) - w) > 1e-5 + 1e-4 * np.abs(w.astype(np.float64))).sum())
              for g, w in zip(got, want))
    return bad / sum(w.size for w in want)


def test_mlp784_1024_b256_free_running_within_natural_spread(ctx):
    """Free-running, 100 AdamW steps amplify rounding (near-zero gradients get +-lr
    updates while t is small), so trajectories from different valid f32 summation
    orders drift apart; per-step parity is the teacher-forced test above.  The natural
    envelope is measured here, on the same box, from three more valid GEMM orders of the
    oracle (f64-accumulated, ascending f32, descending f32 with FMA) against its default
    blocked order: the GPU's loss drift (max over steps of |L - L_oracle| / L0) must stay
    within twice the largest drift among them, and its fraction of final parameters
    outside 1e-5 + 1e-4|x| within 1.25 times theirs.  Measured on one box: loss drift
    f64-acc 0.16 %, ascending f32 0.94 %, descending FMA 0.02 %, GPU 0.55 % of L0; final
    parameters outside tolerance 53 %, 56 %, 30 %, GPU 54 %.  The first steps agree to
    1e-4 relative, and the fixed batch is memorised."""
    w = synth.WORKLOADS[synth.MLP_MEDIUM]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    tr = make_trainer(ctx, w, params)
    tr.set_batch(x, onehot=onehot)
    losses = []
    for _ in range(w["steps"]):
        tr.step()
        losses.append(tr.metrics()[0])
    gpu = np.array(losses, np.float64)
    gpu_params = tr.params()
    runs = []
    try:
        for variant in range(4):
            O.lib().orc_set_gemm_variant(variant)
            runs.append(O.mlp_train(w["dims"], params, x, onehot, ref_opt(w), steps=w["steps"], want_grads=False))
    finally:
        O.lib().orc_set_gemm_variant(0)
    ref = runs[0]["losses"].astype(np.float64)
    l0 = ref[0]
    loss_env = max(float((np.abs(r["losses"] - ref) / l0).max()) for r in runs[1:])
    param_env = max(_fraction_outside(r["params"], runs[0]["params"]) for r in runs[1:])
    dev = float((np.abs(gpu - ref) / l0).max())
    frac = _fraction_outside(gpu_params, runs[0]["params"])
    print(f"784-1024-1024-10 free-running: loss drift / L0 GPU {dev:.2e}, envelope of valid orders {loss_env:.2e}; "
          f"final parameters outside tolerance GPU {frac:.3f}, envelope {param_env:.3f}; "
          f"final loss gpu {gpu[-1]:.6f} oracle {ref[-1]:.6f}")
    assert np.isfinite(gpu).all()
    assert (np.abs(gpu[:5] - ref[:5]) <= 1e-4 * ref[:5]).all()  # identical until rounding differences can act
    assert dev <= 2.0 * loss_env
    assert frac <= 1.25 * param_env
    assert gpu[-1] < 0.05 * gpu[0]  # the fixed batch is memorised


@pytest.mark.parametrize("batch", [1024, 512, 256, 128])
def test_mlp784_4096_b1024_one_adamw_step(ctx, batch):
    """784-4096-4096-10, batch 1024, one AdamW step against the oracle, end to end
    (and the 512 / 256 / 128-row shares of 2-, 4- and 8-way data parallelism: F2 and dX2
    split K in two, four and eight chunks and sum them in their reduce pass, which also
    applies the epilogue; at 128 rows F1 runs whole on the skinny kernel; dW1 stays on the
    banded kernel with K = 512, 256, 128):
    loss and logits to the path's tolerance (1e-5 abs + 1e-4 rel); gradients and
    updated parameters to that tolerance except for a reported fraction <= 1e-5
    of elements.  Those outliers come from ReLU masks that differ between the
    two forward passes (pre-activations within rounding of zero: a flipped
    dZ[b, j] moves a whole column of dW by H[b, :] * dZ[b, j]); the flip count is
    printed, and the shared-input layer-wise test below shows the kernels agree
    when the masks are the same.  Argmax / accuracy are exact outside rows whose
    top-2 margin is within rounding."""
    w = dict(synth.WORKLOADS[synth.MLP_LARGE], batch=batch)
    dims = w["dims"]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], dims, w["batch"])
    tr = make_trainer(ctx, w, params)
    tr.set_batch(x, onehot=onehot)
    tr.step()
    loss, correct = tr.metrics()
    ref = O.mlp_train(dims, params, x, onehot, ref_opt(w), steps=1)
    ref["hidden"] = oracle_hidden(params, x, dims)
    hidden = [tr.activation(l) for l in range(len(dims) - 2)]
    check_one_adamw_step(dims, w["opt"], ref, loss, tr.logits(), hidden, tr.grads(), tr.params(), tr.preds(), correct,
                         what=f"784-4096-4096-10 b{batch} end-to-end")


@pytest.mark.parametrize("batch,count", [(128, 8), (512, 2), (256, 3)])
def test_update_shards_partition_the_whole_update(ctx, batch, count):
    """784-4096-4096-10 at a data-parallel share, one AdamW step with the optimizer state
    sharded over `count` ranks (set_update_shard), each rank's share run in turn from the
    same state: at 2 ranks the slices of layers 1-2 update on the second stream beside dX2 and
    dW1; at 3 and 8 ranks every slice updates after the backward on the context stream.  Every parameter, m and v element either takes the whole step's bits or keeps
    its value (the parameters read back come from the second arena, which the update wrote);
    each element the whole step changes is taken by exactly one share; the shares are
    balanced (every update pass is cut at multiples of 64 floats); loss and logits are the
    whole step's."""
    w = dict(synth.WORKLOADS[synth.MLP_LARGE], batch=batch)
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], batch)
    full = make_trainer(ctx, w, params)
    full.set_batch(x, onehot=onehot)
    full.step()
    loss_full, logits_full = full.metrics()[0], full.logits()
    want = [np.concatenate([a.ravel() for a in arrs]) for arrs in (full.params(), full.moments(0), full.moments(1))]
    full.close()
    p0 = np.concatenate([p.ravel() for p in params])
    changed = (want[0] != p0) | (want[1] != 0) | (want[2] != 0)
    takers = np.zeros(p0.size, np.int32)
    for s in range(count):
        tr = make_trainer(ctx, w, params)
        tr.set_update_shard(s, count)
        tr.set_batch(x, onehot=onehot)
        tr.step()
        assert tr.metrics()[0] == loss_full
        np.testing.assert_array_equal(tr.logits(), logits_full)
        got = [np.concatenate([a.ravel() for a in arrs]) for arrs in (tr.params(), tr.moments(0), tr.moments(1))]
        tr.close()
        took = (got[0] == want[0]) & (got[1] == want[1]) & (got[2] == want[2])
        kept = (got[0] == p0) & (got[1] == 0) & (got[2] == 0)
        assert np.all(took | kept), f"share {s}: {np.count_nonzero(~(took | kept))} elements neither updated nor kept"
        mine = took & ~kept
        takers += mine
        share = np.count_nonzero(mine) / np.count_nonzero(changed)
        assert abs(share - 1.0 / count) < 0.01, (s, share)
    assert np.all(takers[changed] == 1), np.bincount(takers[changed])


@pytest.mark.parametrize("switch", ["ORCA_HIP_DOUBLE_ARENA", "ORCA_HIP_BIND_EVENTS"])
def test_mlp784_4096_b1024_schedule_changes_no_bit(ctx, monkeypatch, switch):
    """784-4096-4096-10, batch 1024, three AdamW steps, each schedule switch on and off: every
    parameter, moment-driven update and gradient is the same bit for bit. ORCA_HIP_DOUBLE_ARENA:
    the second parameter arena (the update of layers >= 1 beside layer 1's dZ product, P and
    P_next swapping every step) against the single-arena schedule. ORCA_HIP_BIND_EVENTS: the
    events that start the update on the second stream completing with the GEMM launches
    before them, against event records of their own."""
    w = synth.WORKLOADS[synth.MLP_LARGE]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    out = []
    for on in ("1", "0"):
        monkeypatch.setenv(switch, on)
        tr = make_trainer(ctx, w, params)
        tr.set_batch(x, onehot=onehot)
        losses = []
        for _ in range(3):
            tr.step()
            losses.append(tr.metrics()[0])
        out.append((losses, tr.params(), tr.grads()))
        tr.close()
    (l1, p1, g1), (l2, p2, g2) = out
    assert l1 == l2
    for a, b in zip(p1 + g1, p2 + g2):
        np.testing.assert_array_equal(a, b)


def test_mlp784_4096_b1024_layerwise_on_shared_inputs(ctx):
    """Each layer of the fused step against the oracle's ops fed the GPU's own
    inputs to that layer (so ReLU masks are identical): forward activations,
    the CE gradient, every dZ-driven gradient -- tight, scale-relative
    tolerance.  End-to-end ReLU mask flips (pre-activations within rounding of
    zero) are counted and must be rare."""
    w = synth.WORKLOADS[synth.MLP_LARGE]
    dims = w["dims"]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], dims, w["batch"])
    tr = make_trainer(ctx, w, params)
    tr.set_batch(x, onehot=onehot)
    tr.step()
    W = [params[0], params[2], params[4]]
    b = [params[1], params[3], params[5]]
    H1, H2, logits = tr.activation(0), tr.activation(1), tr.activation(2)
    grads = tr.grads()
    B = w["batch"]

    def lin(a, l):
        return O.add(O.matmul(a, W[l]), O.expand(b[l], (B, dims[l + 1])))

    # forward, layer by layer from the GPU's own input to that layer
    for name, got, want in (("H1", H1, O.relu(lin(x, 0))), ("H2", H2, O.relu(lin(H1, 1))),
                            ("logits", logits, lin(H2, 2))):
        assert_close_scaled(got, want, rtol=1e-5, what=name)
    flips = [int(((O.relu(lin(x, 0)) > 0) != (H1 > 0)).sum()), int(((O.relu(lin(H1, 1)) > 0) != (H2 > 0)).sum())]
    print(f"784-4096-4096-10 ReLU mask flips vs the oracle's own pre-activations: layer1 {flips[0]}, layer2 {flips[1]} "
          f"of {H1.size} each")
    assert max(flips) <= 1e-5 * H1.size
    # backward from the GPU's logits and activations
    _, dlog = O.cross_entropy(logits, onehot)
    dZ2 = O.relu_backward(O.matmul(dlog, O.transpose(W[2], 0, 1)), H2)
    dZ1 = O.relu_backward(O.matmul(dZ2, O.transpose(W[1], 0, 1)), H1)
    want = [O.matmul(O.transpose(x, 0, 1), dZ1), O.sum_to_shape(dZ1, (1, dims[1])),
            O.matmul(O.transpose(H1, 0, 1), dZ2), O.sum_to_shape(dZ2, (1, dims[2])),
            O.matmul(O.transpose(H2, 0, 1), dlog), O.sum_to_shape(dlog, (1, dims[3]))]
    for i, (g, r) in enumerate(zip(grads, want)):
        assert_close_scaled(g, r, rtol=1e-4, what=f"grad {i}")


def test_ce_and_relu_backward_8192x4096(ctx):
    """Logits [8192, 4096] ~ N(0, 2^2) with int targets -> softmax-CE gradient;
    then ReLU-mask backward on a N(0,1) pre-activation and the bias column sum."""
    B, C = 8192, 4096
    logits = synth.normal(4, 1, (B, C), 0.0, 2.0)
    labels = synth.integers(4, 2, B, C)
    pre = synth.normal(4, 3, (B, C))
    dl, dlab, dpre_in = ctx.upload(logits), ctx.upload(labels), ctx.upload(pre)
    loss, grad = ctx.alloc(4), ctx.alloc(4 * B * C)
    _lib.call("orca_hip_softmax_ce", ctx.handle, dl.ptr, B, C, None, dlab.ptr, loss.ptr, grad.ptr, None, None)
    dpre, colsum = ctx.alloc(4 * B * C), ctx.alloc(4 * C)
    _lib.call("orca_hip_relu_bw_colsum", ctx.handle, grad.ptr, dpre_in.ptr, B, C, dpre.ptr, colsum.ptr)
    g_gpu = grad.download(count=B * C).reshape(B, C)
    d_gpu = dpre.download(count=B * C).reshape(B, C)
    cs_gpu = colsum.download(count=C)

    loss_ref, g_ref = O.cross_entropy(logits, synth.one_hot(labels, C))
    assert_close(float(loss.download(count=1)[0]), loss_ref, what="loss")
    assert_close(g_gpu, g_ref, what="CE grad")
    assert_close_scaled(g_gpu, g_ref, what="CE grad (scaled)")
    # ReLU mask on identical inputs is exact: apply it to the GPU's own gradient.
    d_ref = O.relu_backward(g_gpu, pre)
    np.testing.assert_array_equal(d_gpu, d_ref)
    assert ((d_gpu != 0) <= (pre > 0)).all()
    cs_ref = O.sum_to_shape(d_ref, (1, C)).reshape(C)
    assert_close(cs_gpu, cs_ref, what="bias colsum")
    # Each CE-gradient row sums to ~0 (softmax - onehot); column sums of the masked gradient are the bias grad.
    np.testing.assert_allclose(g_gpu.astype(np.float64).sum(1), 0.0, atol=1e-9)


@pytest.mark.timeout(600)
def test_adamw_2pow28(ctx):
    """AdamW over one flat buffer of 2^28 f32 params, 10 steps from zero moments:
    bit-exact against the oracle on a sample of 2^20 positions (the update is
    elementwise), and finite everywhere."""
    n = 1 << 28
    chunk = 1 << 24
    p_dev, g_dev = ctx.alloc(4 * n), ctx.alloc(4 * n)
    m_dev, v_dev = ctx.alloc(4 * n), ctx.alloc(4 * n)
    _lib.call("orca_hip_fill", ctx.handle, m_dev.ptr, ctypes.c_float(0.0), n)
    _lib.call("orca_hip_fill", ctx.handle, v_dev.ptr, ctypes.c_float(0.0), n)
    rng = np.random.default_rng(5)
    idx = np.sort(rng.choice(n, size=1 << 20, replace=False))
    p_s = np.empty(idx.size, np.float32)
    g_s = np.empty(idx.size, np.float32)
    for off in range(0, n, chunk):
        pc = synth.normal_range(5, 1, off, chunk, 0.0, 0.02)
        gc = synth.normal_range(5, 2, off, chunk, 0.0, 1e-3)
        _upload_at(ctx, p_dev, off, pc)
        _upload_at(ctx, g_dev, off, gc)
        sel = (idx >= off) & (idx < off + chunk)
        p_s[sel] = pc[idx[sel] - off]
        g_s[sel] = gc[idx[sel] - off]
    for t in range(1, 11):
        _lib.call("orca_hip_adamw_step", ctx.handle, p_dev.ptr, g_dev.ptr, m_dev.ptr, v_dev.ptr, n, 1e-3, 0.9, 0.999,
                  1e-8, 0.01, t)
    ctx.sync()
    ref_p, ref_m, ref_v = p_s, np.zeros_like(p_s), np.zeros_like(p_s)
    for t in range(1, 11):
        ref_p, ref_m, ref_v = O.adamw_update(ref_p, g_s, ref_m, ref_v, t)
    got_p = _gather(ctx, p_dev, idx, n)
    got_m = _gather(ctx, m_dev, idx, n)
    np.testing.assert_array_equal(got_p, ref_p)
    np.testing.assert_array_equal(got_m, ref_m)
    assert np.isfinite(got_p).all()


def _upload_at(ctx, buf, off, arr):
    arr = np.ascontiguousarray(arr, np.float32)
    _lib.call("orca_hip_h2d", ctx.handle, buf.ptr + 4 * off, arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes)


def _gather(ctx, buf, idx, n, chunk=1 << 24):
    out = np.empty(idx.size, np.float32)
    host = np.empty(chunk, np.float32)
    for off in range(0, n, chunk):
        sel = (idx >= off) & (idx < off + chunk)
        if not sel.any():
            continue
        _lib.call("orca_hip_d2h", ctx.handle, host.ctypes.data_as(ctypes.c_void_p), buf.ptr + 4 * off, 4 * chunk)
        out[sel] = host[idx[sel] - off]
    return out
