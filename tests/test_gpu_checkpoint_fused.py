"""On the GPU: checkpoints of HIP tensors and of the device-resident trainer
(safetensors through to_bytes / from_bytes), and the opt-in fused loss and
optimizer paths of the composed model against the composed path and the
oracle."""
from __future__ import annotations

import numpy as np
import pytest
from safetensors.numpy import load_file

from oracle import oracle as O
from orcaml_amd import autodiff as A
from orcaml_amd import serialize, synth
from orcaml_amd.mlp import MLPTrainer
from tests.cpu_backend import OracleBackend
from tests.test_checkpoint_fused import make_optim, run
from tests.util import assert_close, assert_close_scaled

pytestmark = pytest.mark.gpu

W1 = synth.WORKLOADS[synth.MLP_SMALL]


def problem():
    params, x, labels, onehot = synth.mlp_problem(W1["seed"], W1["dims"], W1["batch"])
    return params, x, labels, onehot


def test_module_checkpoint_round_trip_across_backends(hb, tmp_path):
    """HIP model -> file -> fresh HIP model and oracle-backend model: the same bits."""
    params, x, _, onehot = problem()
    ad = A.Autodiff(hb)
    model = A.build_mlp(ad, params)
    run(ad, model, make_optim(model, "adamw"), x, onehot, 2)  # weights that differ from the initial ones
    trained = [p.tensor.numpy() for p in model.parameters()]
    f = str(tmp_path / "w.safetensors")
    model.save_weights(f)
    arrays = load_file(f)
    for (n, _), t in zip(model.named_parameters(), trained):
        np.testing.assert_array_equal(arrays[n], t)
    for backend in (hb, OracleBackend()):
        other = A.build_mlp(A.Autodiff(backend), [np.zeros_like(p) for p in params])
        other.load_weights(f)
        for q, t in zip(other.parameters(), trained):
            np.testing.assert_array_equal(q.tensor.numpy(), t)
            assert q.tensor.requires_grad


@pytest.mark.parametrize("kind", ["sgd", "adamw"])
def test_fused_optimizers_equal_composed_on_hip(hb, kind):
    """The fused update kernels on HIP against the composed update on HIP
    (same loss path): the same bits after 3 steps."""
    params, x, _, onehot = problem()
    out = []
    for fused in (False, True):
        ad = A.Autodiff(hb)
        model = A.build_mlp(ad, params)
        out.append(run(ad, model, make_optim(model, kind, fused), x, onehot, 3))
    np.testing.assert_array_equal(out[0][0], out[1][0])
    for a, b in zip(out[0][2], out[1][2]):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("kind", ["sgd", "adamw"])
def test_fused_loss_and_optimizer_match_oracle_teacher_forced(hb, kind):
    """nn.CrossEntropyLoss(fused=True) + the fused optimizer on HIP, 3 steps,
    each checked against the oracle's reference step from the GPU's own
    parameters and moments: loss and gradients within tolerance (the fused
    loss adds its rows in another order), and the update bit-exact as the
    oracle's SGD / AdamW applied to the GPU's own gradient.  (AdamW divides
    by sqrt(v) + eps, so a last-bit difference in a gradient near eps moves
    the parameter by a visible fraction of lr; that is why the parameters
    are not compared across independent 3-step runs.)"""
    params, x, _, onehot = problem()
    opt = dict(lr=0.1) if kind == "sgd" else dict(lr=1e-3, weight_decay=0.01)
    ad = A.Autodiff(hb)
    model = A.build_mlp(ad, params)
    optim = make_optim(model, kind, True)
    xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
    for step in range(3):
        before = [p.tensor.numpy() for p in model.parameters()]
        if kind == "adamw":
            m0 = [t.numpy() for t in optim.m]
            v0 = [t.numpy() for t in optim.v]
        ref = O.mlp_train(W1["dims"], before, x, onehot, O.make_opt(kind, **opt), steps=1,
                          m=m0 if kind == "adamw" else None, v=v0 if kind == "adamw" else None, t=step)
        optim.zero_grad()
        loss = A.CrossEntropyLoss(fused=True)(model(xt), tt)
        loss.backward()
        grads = [p.tensor.grad().numpy() for p in model.parameters()]
        optim.step()
        assert_close(loss.to_list()[0], ref["losses"][0], what=f"step {step} loss")
        for i, (g, r) in enumerate(zip(grads, ref["grads"])):
            assert_close(g, r.reshape(g.shape), what=f"step {step} grad {i}")
            assert_close_scaled(g, r.reshape(g.shape), rtol=1e-3, what=f"step {step} grad {i} (scaled)")
        after = [p.tensor.numpy() for p in model.parameters()]
        for i, (p0, g, p1) in enumerate(zip(before, grads, after)):
            if kind == "sgd":
                np.testing.assert_array_equal(p1.reshape(-1), O.sgd_update(p0, g, opt["lr"]).reshape(-1))
            else:
                pe, me, ve = O.adamw_update(p0, g, m0[i], v0[i], step + 1, **opt)
                np.testing.assert_array_equal(p1, pe, err_msg=f"step {step} param {i}")
                np.testing.assert_array_equal(optim.m[i].numpy(), me)
                np.testing.assert_array_equal(optim.v[i].numpy(), ve)


def make_trainer(ctx, wl):
    w = synth.WORKLOADS[wl]
    o = w["opt"]
    return MLPTrainer(ctx, w["dims"], w["batch"], kind=o["kind"], lr=o["lr"], weight_decay=o.get("weight_decay", 0.0))


@pytest.mark.parametrize("workload", [synth.MLP_SMALL, synth.MLP_MEDIUM, synth.MLP_LARGE])
def test_trainer_checkpoint_resume_matches_uninterrupted(ctx, tmp_path, workload):
    """3 steps, save, load into a fresh trainer, 2 more steps: the same
    parameters, moments, step count and metrics as 5 uninterrupted steps
    (784-4096-4096-10 runs with two parameter arenas that swap each step).  The restore
    and the batch upload are stream-ordered through the context's 16 MiB pinned staging ring:
    they wait for the device only when the ring is full (at most once per 4 MiB region it
    moves), never once per tensor, and not at all when everything fits in the ring."""
    w = synth.WORKLOADS[workload]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    a = make_trainer(ctx, workload)
    a.set_params(params)
    a.set_batch(x, labels=labels)
    for _ in range(5):
        a.step()
    b = make_trainer(ctx, workload)
    b.set_params(params)
    b.set_batch(x, labels=labels)
    for _ in range(3):
        b.step()
    f = str(tmp_path / "trainer.safetensors")
    b.save(f)
    b.close()
    c = make_trainer(ctx, workload)
    waits = ctx.sync_count()
    c.load(f)
    c.set_batch(x, labels=labels)
    waits = ctx.sync_count() - waits
    n_params = sum(int(np.prod(p.shape)) for p in params)
    moved = 4 * n_params * (3 if w["opt"]["kind"] == "adamw" else 1) + x.nbytes + labels.nbytes
    assert waits <= -(-moved // (4 << 20)), (waits, moved)
    if moved <= 16 << 20:
        assert waits == 0
    for _ in range(2):
        c.step()
    assert c.step_count() == a.step_count()
    assert c.metrics() == a.metrics()
    for p, q in zip(c.params(), a.params()):
        np.testing.assert_array_equal(p, q)
    if w["opt"]["kind"] == "adamw":
        for which in (0, 1):
            for p, q in zip(c.moments(which), a.moments(which)):
                np.testing.assert_array_equal(p, q)
    a.close()
    c.close()


def test_trainer_file_loads_into_the_composed_model(ctx, hb, tmp_path):
    """The trainer's checkpoint names its parameters as nn.Sequential does, so
    the composed model's load_weights reads it; a weights-only file resets
    the trainer's AdamW state."""
    w = synth.WORKLOADS[synth.MLP_MEDIUM]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    tr = make_trainer(ctx, synth.MLP_MEDIUM)
    tr.set_params(params)
    tr.set_batch(x, labels=labels)
    tr.step()
    f = str(tmp_path / "trainer.safetensors")
    tr.save(f)
    model = A.build_mlp(A.Autodiff(hb), [np.zeros_like(p) for p in params])
    model.load_weights(f)
    for q, p in zip(model.parameters(), tr.params()):
        np.testing.assert_array_equal(q.tensor.numpy(), p)
    fw = str(tmp_path / "weights.safetensors")
    model.save_weights(fw)
    fresh = make_trainer(ctx, synth.MLP_MEDIUM)
    fresh.load(fw)
    assert fresh.step_count() == 0
    for p, q in zip(fresh.params(), tr.params()):
        np.testing.assert_array_equal(p, q)
    for m in fresh.moments(0):
        assert not m.any()
    tr.close()
    fresh.close()


def test_trainer_load_rejects_other_dims(ctx, tmp_path):
    tr = make_trainer(ctx, synth.MLP_SMALL)
    f = str(tmp_path / "t.safetensors")
    tr.save(f)
    other = make_trainer(ctx, synth.MLP_MEDIUM)
    with pytest.raises(A.OrcaError):
        other.load(f)
    tr.close()
    other.close()
