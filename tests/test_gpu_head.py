"""GPU parity of the fused classifier head (orca_hip_head_forward_ce,
orca_hip_head_backward) against the CPU oracle's composed ops, and of the MLP
trainer with and without it."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from orcaml_amd import _lib, synth
from orcaml_amd.mlp import MLPTrainer
from tests.util import assert_close, assert_close_scaled, int_matrix

pytestmark = pytest.mark.gpu

# (B, K, C): the output layers of the three benchmark MLPs, ragged rows (B not a multiple of
# the 4-row forward block), one float4 of K, K not a multiple of the 32-column
# backward panel, the 1- and 16-class extremes, and row-split backward grids.
HEAD_SHAPES = [(1024, 4096, 10), (64, 128, 10), (256, 1024, 10), (37, 20, 3), (5, 4, 1), (1000, 36, 16),
               (33, 4100, 7), (4096, 64, 10)]


def run_head(ctx, H, W, bias, onehot=None, labels=None, relu_mask=True, with_dh=True):
    B, K = H.shape
    C = W.shape[1]
    dH_, dW_, db_ = ctx.upload(H), ctx.upload(W), ctx.upload(bias)
    doh = ctx.upload(onehot) if onehot is not None else None
    dlb = ctx.upload(labels.astype(np.int32)) if labels is not None else None
    logits, dlogits = ctx.alloc(4 * B * C), ctx.alloc(4 * B * C)
    loss, preds, correct = ctx.alloc(4), ctx.alloc(4 * B), ctx.alloc(8)
    _lib.call("orca_hip_head_forward_ce", ctx.handle, dH_.ptr, B, K, dW_.ptr, db_.ptr, C,
              doh.ptr if doh else None, dlb.ptr if dlb else None, logits.ptr, loss.ptr, dlogits.ptr, preds.ptr,
              correct.ptr)
    gH = ctx.alloc(4 * B * K) if with_dh else None
    gW, gb = ctx.alloc(4 * K * C), ctx.alloc(4 * C)
    _lib.call("orca_hip_head_backward", ctx.handle, dH_.ptr, B, K, dW_.ptr, C, dlogits.ptr, int(relu_mask),
              gH.ptr if gH else None, gW.ptr, gb.ptr)
    return dict(logits=logits.download(count=B * C).reshape(B, C), loss=float(loss.download(count=1)[0]),
                dlogits=dlogits.download(count=B * C).reshape(B, C), preds=preds.download(np.int32, B),
                correct=int(correct.download(np.int64, 1)[0]),
                dH=gH.download(count=B * K).reshape(B, K) if gH else None,
                dW=gW.download(count=K * C).reshape(K, C), db=gb.download(count=C))


def reference_head(H, W, bias, onehot, relu_mask=True):
    """The reference's op sequence on the oracle: Linear (matmul, expand the
    bias, add), composed CE, MatMulBackward, the bias ExpandBackward's
    sum_to_shape and ReluBackward."""
    B, C = H.shape[0], W.shape[1]
    z = O.matmul(H, W)
    logits = O.add(z, O.expand(bias.reshape(1, C), (B, C)))
    loss, dl = O.cross_entropy(logits, onehot)
    dx = O.matmul(dl, O.transpose(W, 0, 1))
    dH = O.relu_backward(dx, H) if relu_mask else dx
    dW = O.matmul(O.transpose(H, 0, 1), dl)
    db = O.sum_to_shape(dl, (1, C)).reshape(C)
    return dict(logits=logits, loss=loss, dlogits=dl, dH=dH, dW=dW, db=db, preds=O.argmax_rows(logits))


def relu_like(rng, shape):
    """A ReLU output: about half the entries exactly zero."""
    return np.maximum(rng.standard_normal(shape), 0.0).astype(np.float32)


@pytest.mark.parametrize("B,K,C", HEAD_SHAPES)
def test_head_exact_on_integers(ctx, B, K, C):
    """Small-integer H, W, bias make every product and sum exact in f32 (any
    order), so logits, the argmax, dW, db and the masked dH are bit-exact;
    the loss and dlogits then go through exp/log (within tolerance)."""
    rng = np.random.default_rng(B + K + C)
    H = np.maximum(int_matrix(rng, (B, K), -3, 4), 0.0).astype(np.float32)
    W = int_matrix(rng, (K, C), -3, 4)
    bias = int_matrix(rng, (C,), -4, 5)
    labels = rng.integers(0, C, B)
    onehot = synth.one_hot(labels, C)
    got = run_head(ctx, H, W, bias, onehot=onehot)
    ref = reference_head(H, W, bias, onehot)
    np.testing.assert_array_equal(got["logits"], ref["logits"])
    np.testing.assert_array_equal(got["preds"], ref["preds"])
    assert got["correct"] == int((ref["preds"] == labels).sum())
    assert_close(got["loss"], ref["loss"], what="loss")
    assert_close(got["dlogits"], ref["dlogits"], what="dlogits")
    assert_close_scaled(got["dlogits"], ref["dlogits"], what="dlogits (scaled)")
    # The backward on the oracle's own dlogits scaled to integers: exact.
    dl = int_matrix(rng, (B, C), -5, 6)
    dlp = ctx.upload(dl)
    dHp, dWp = ctx.upload(H), ctx.upload(W)
    gH, gW, gb = ctx.alloc(4 * B * K), ctx.alloc(4 * K * C), ctx.alloc(4 * C)
    _lib.call("orca_hip_head_backward", ctx.handle, dHp.ptr, B, K, dWp.ptr, C, dlp.ptr, 1, gH.ptr, gW.ptr, gb.ptr)
    np.testing.assert_array_equal(gW.download(count=K * C).reshape(K, C), O.matmul(O.transpose(H, 0, 1), dl))
    np.testing.assert_array_equal(gb.download(count=C), O.sum_to_shape(dl, (1, C)).reshape(C))
    np.testing.assert_array_equal(gH.download(count=B * K).reshape(B, K),
                                  O.relu_backward(O.matmul(dl, O.transpose(W, 0, 1)), H))


@pytest.mark.parametrize("B,K,C", [(1024, 4096, 10), (1000, 36, 16), (37, 20, 3), (4096, 64, 7)])
def test_head_backward_unaligned_dlogits(ctx, B, K, C):
    """dlogits, dW and db one float past a 16-byte boundary: dlogits is then
    staged element by element instead of as float4s; the results are the
    same bits as with aligned buffers (integer data: exact against the oracle)."""
    rng = np.random.default_rng(11 * B + C)
    H = int_matrix(rng, (B, K), -3, 4)
    W = int_matrix(rng, (K, C), -3, 4)
    dl = int_matrix(rng, (B, C), -5, 6)
    dHp, dWp = ctx.upload(H), ctx.upload(W)
    outs = []
    for off in (0, 1):
        pad = np.zeros(off, np.float32)
        dlp = ctx.upload(np.concatenate([pad, dl.ravel()]))
        gW, gb = ctx.upload(np.zeros(off + K * C, np.float32)), ctx.upload(np.zeros(off + C, np.float32))
        gH = ctx.alloc(4 * B * K)
        _lib.call("orca_hip_head_backward", ctx.handle, dHp.ptr, B, K, dWp.ptr, C, dlp.ptr + 4 * off, 1, gH.ptr,
                  gW.ptr + 4 * off, gb.ptr + 4 * off)
        outs.append((gH.download(count=B * K).reshape(B, K), gW.download(count=off + K * C)[off:].reshape(K, C),
                     gb.download(count=off + C)[off:]))
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
    gH, gW, gb = outs[1]
    np.testing.assert_array_equal(gW, O.matmul(O.transpose(H, 0, 1), dl))
    np.testing.assert_array_equal(gb, O.sum_to_shape(dl, (1, C)).reshape(C))
    np.testing.assert_array_equal(gH, O.relu_backward(O.matmul(dl, O.transpose(W, 0, 1)), H))


@pytest.mark.parametrize("B,K,C", HEAD_SHAPES)
def test_head_matches_composed_reference(ctx, B, K, C):
    rng = np.random.default_rng(7 * B + K + C)
    H = relu_like(rng, (B, K))
    bound = 1.0 / np.sqrt(K)
    W = rng.uniform(-bound, bound, (K, C)).astype(np.float32)
    bias = rng.uniform(-bound, bound, C).astype(np.float32)
    labels = rng.integers(0, C, B)
    onehot = synth.one_hot(labels, C)
    ref = reference_head(H, W, bias, onehot)
    for kw in (dict(onehot=onehot), dict(labels=labels)):
        got = run_head(ctx, H, W, bias, **kw)
        assert_close(got["logits"], ref["logits"], what="logits")
        assert_close(got["loss"], ref["loss"], what="loss")
        assert_close(got["dlogits"], ref["dlogits"], what="dlogits")
        assert_close_scaled(got["dlogits"], ref["dlogits"], what="dlogits (scaled)")
        # argmax is exact wherever the top two logits are further apart than rounding
        top2 = np.sort(ref["logits"], axis=1)[:, -2:] if C > 1 else None
        clear = np.ones(B, bool) if C == 1 else (top2[:, 1] - top2[:, 0]) > 1e-5 * (1 + np.abs(top2[:, 1]))
        np.testing.assert_array_equal(got["preds"][clear], ref["preds"][clear])
        assert_close(got["dW"], ref["dW"], what="dW")
        assert_close_scaled(got["dW"], ref["dW"], rtol=1e-4, what="dW (scaled)")
        assert_close(got["db"], ref["db"], what="db")
        assert_close(got["dH"], ref["dH"], what="dH")
        assert_close_scaled(got["dH"], ref["dH"], rtol=1e-4, what="dH (scaled)")
        # the mask is exact: dH is zero exactly where H is not positive
        assert not got["dH"][H <= 0].any()


def test_head_repeated_calls_and_unmasked_input_layer(ctx):
    """Counters reset between launches (the second, smaller call must not see
    the first one's state); relu_mask = 0 gives the plain product (a head that
    is also the input layer has no ReLU below it)."""
    rng = np.random.default_rng(3)
    for B, K in ((1024, 4096), (100, 512)):
        H = rng.standard_normal((B, K)).astype(np.float32)
        W = (0.05 * rng.standard_normal((K, 10))).astype(np.float32)
        bias = np.zeros(10, np.float32)
        labels = rng.integers(0, 10, B)
        onehot = synth.one_hot(labels, 10)
        got = run_head(ctx, H, W, bias, onehot=onehot, relu_mask=False)
        ref = reference_head(H, W, bias, onehot, relu_mask=False)
        assert_close(got["loss"], ref["loss"], what="loss")
        assert_close(got["dW"], ref["dW"], what="dW")
        assert_close(got["db"], ref["db"], what="db")
        assert_close(got["dH"], ref["dH"], what="dH")


def test_head_rejects_unsupported_shapes(ctx):
    buf = ctx.alloc(4 * 64 * 64)
    for K, C in ((6, 10), (8, 17), (8, 0)):
        with pytest.raises(_lib.OrcaHipError) as e:
            _lib.call("orca_hip_head_forward_ce", ctx.handle, buf.ptr, 4, K, buf.ptr, buf.ptr, C, buf.ptr, None,
                      buf.ptr, None, None, None, None)
        assert e.value.code == _lib.ERR_SHAPE
        with pytest.raises(_lib.OrcaHipError) as e:
            _lib.call("orca_hip_head_backward", ctx.handle, buf.ptr, 4, K, buf.ptr, C, buf.ptr, 1, None, buf.ptr,
                      None)
        assert e.value.code == _lib.ERR_SHAPE


@pytest.mark.parametrize("workload", [synth.MLP_SMALL, synth.MLP_LARGE])
def test_trainer_fused_head_equals_gemm_head(ctx, monkeypatch, workload):
    """The trainer's fused head and its GEMM + softmax-CE path agree on one
    step (both are checked against the oracle elsewhere)."""
    w = synth.WORKLOADS[workload]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    out = {}
    for fused in ("1", "0"):
        monkeypatch.setenv("ORCA_HIP_FUSED_HEAD", fused)
        tr = MLPTrainer(ctx, w["dims"], w["batch"], kind="sgd", lr=0.1)
        tr.set_params(params)
        tr.set_batch(x, labels=labels)
        tr.step()
        out[fused] = (tr.metrics(), tr.grads(), tr.params(), tr.preds())
        tr.close()
    (l1, c1), g1, p1, pr1 = out["1"]
    (l0, c0), g0, p0, pr0 = out["0"]
    assert_close(l1, l0, what="loss")
    assert c1 == c0
    np.testing.assert_array_equal(pr1, pr0)
    for i, (a, b) in enumerate(zip(g1, g0)):
        assert_close_scaled(a, b, rtol=1e-3, what=f"grad {i}")
    for i, (a, b) in enumerate(zip(p1, p0)):
        assert_close(a, b, what=f"param {i}")
