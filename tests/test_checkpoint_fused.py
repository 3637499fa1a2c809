"""Checkpoints (safetensors through to_bytes / from_bytes) and the opt-in
fused loss / optimizer paths, on the CPU oracle backend: the host logic of
both, with the reference's parameter names, and the composed path as the
reference for the fused one."""
from __future__ import annotations

import numpy as np
import pytest
from safetensors.numpy import load_file, save_file

from orcaml_amd import autodiff as A
from orcaml_amd import serialize, synth
from tests.cpu_backend import OracleBackend
from tests.util import assert_close

W1 = synth.WORKLOADS[synth.MLP_SMALL]


def problem():
    params, x, labels, onehot = synth.mlp_problem(W1["seed"], W1["dims"], W1["batch"])
    return params, x, onehot


def make_optim(model, kind, fused=False):
    if kind == "sgd":
        return A.SGD(model.parameters(), lr=0.1, fused=fused)
    return A.AdamW(model.parameters(), lr=1e-3, weight_decay=0.01, fused=fused)


def run(ad, model, optim, x, onehot, steps, fused_loss=False):
    xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
    losses, grads = [], None
    for _ in range(steps):
        optim.zero_grad()
        loss = A.CrossEntropyLoss(fused=fused_loss)(model(xt), tt)
        losses.append(loss.to_list()[0])
        loss.backward()
        grads = [p.tensor.grad().numpy() for p in model.parameters()]
        optim.step()
    return np.array(losses, np.float32), grads, [p.tensor.numpy() for p in model.parameters()]


def test_trainer_param_names_follow_sequential():
    assert serialize.trainer_param_names(3) == ["0.weight", "0.bias", "2.weight", "2.bias", "4.weight", "4.bias"]


def test_save_weights_names_shapes_and_round_trip(tmp_path):
    params, _, _ = problem()
    ad = A.Autodiff(OracleBackend())
    model = A.build_mlp(ad, params)
    f = str(tmp_path / "w.safetensors")
    model.save_weights(f)
    arrays = load_file(f)
    names = serialize.trainer_param_names(3)
    assert sorted(arrays) == sorted(names)
    for n, p in zip(names, params):
        a = arrays[n]
        assert a.dtype == np.float32
        assert a.shape == (p.shape if n.endswith("weight") else (1, p.size))  # bias [1, out] (linear.py:34)
        np.testing.assert_array_equal(a.reshape(-1), p.reshape(-1))
    other = A.build_mlp(ad, [np.zeros_like(p) for p in params])
    other.load_weights(f)
    for p, (n, q) in zip(params, other.named_parameters()):
        np.testing.assert_array_equal(q.tensor.numpy().reshape(-1), p.reshape(-1))
        assert q.tensor.requires_grad


def test_load_weights_leaves_parameters_not_in_the_file(tmp_path):
    params, _, _ = problem()
    ad = A.Autodiff(OracleBackend())
    f = str(tmp_path / "partial.safetensors")
    save_file({"2.weight": np.full(params[2].shape, 3.0, np.float32)}, f)
    model = A.build_mlp(ad, params)
    model.load_weights(f)
    got = [p.tensor.numpy() for p in model.parameters()]
    np.testing.assert_array_equal(got[2], np.full(params[2].shape, 3.0, np.float32))
    for i in (0, 1, 3, 4, 5):
        np.testing.assert_array_equal(got[i].reshape(-1), params[i].reshape(-1))


def test_load_rejects_non_f32(tmp_path):
    f = str(tmp_path / "int.safetensors")
    save_file({"0.weight": np.zeros((2, 2), np.int32)}, f)
    with pytest.raises(A.OrcaError):
        serialize.load_tensors(f, A.Autodiff(OracleBackend()))


def test_optimizer_state_resume_matches_uninterrupted(tmp_path):
    """2 steps, save model + AdamW state, restore into fresh objects, 1 more
    step: the same bits as 3 uninterrupted steps."""
    params, x, onehot = problem()
    ad = A.Autodiff(OracleBackend())
    model = A.build_mlp(ad, params)
    straight = run(ad, model, make_optim(model, "adamw"), x, onehot, 3)

    ad2 = A.Autodiff(OracleBackend())
    m2 = A.build_mlp(ad2, params)
    o2 = make_optim(m2, "adamw")
    run(ad2, m2, o2, x, onehot, 2)
    fw, fo = str(tmp_path / "m.safetensors"), str(tmp_path / "o.safetensors")
    m2.save_weights(fw)
    serialize.save_optimizer(fo, o2)
    assert serialize.read_metadata(fo)["t"] == "2"

    ad3 = A.Autodiff(OracleBackend())
    m3 = A.build_mlp(ad3, [np.zeros_like(p) for p in params])
    o3 = make_optim(m3, "adamw")
    m3.load_weights(fw)
    serialize.load_optimizer(fo, o3)
    assert o3.t == 2
    resumed = run(ad3, m3, o3, x, onehot, 1)
    np.testing.assert_array_equal(resumed[0][-1], straight[0][-1])
    for a, b in zip(resumed[2], straight[2]):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("kind", ["sgd", "adamw"])
def test_fused_optimizer_equals_composed(kind):
    """The fused update is the composed update's f32 arithmetic: same bits."""
    params, x, onehot = problem()
    out = []
    for fused in (False, True):
        ad = A.Autodiff(OracleBackend())
        model = A.build_mlp(ad, params)
        out.append(run(ad, model, make_optim(model, kind, fused), x, onehot, 3))
    np.testing.assert_array_equal(out[0][0], out[1][0])
    for a, b in zip(out[0][2], out[1][2]):
        np.testing.assert_array_equal(a, b)


def test_fused_loss_records_one_node_and_matches_composed():
    params, x, onehot = problem()
    res = []
    for fused in (False, True):
        ad = A.Autodiff(OracleBackend())
        model = A.build_mlp(ad, params)
        xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
        out = model(xt)
        n_before = len(ad.tape.nodes)
        loss = A.CrossEntropyLoss(fused=fused)(out, tt)
        n_loss_nodes = len(ad.tape.nodes) - n_before
        loss.backward()
        res.append((loss.to_list()[0], [p.tensor.grad().numpy() for p in model.parameters()], n_loss_nodes))
    assert res[1][2] == 1 and res[0][2] > 10
    assert_close(res[1][0], res[0][0], what="loss")
    for a, b in zip(res[1][1], res[0][1]):
        assert_close(a, b, what="grad")


def test_fused_loss_scales_by_the_incoming_gradient():
    """backward of (2 * loss) through the fused node = 2 * the seed-1 gradient."""
    params, x, onehot = problem()
    grads = []
    for scale in (1.0, 2.0):
        ad = A.Autodiff(OracleBackend())
        model = A.build_mlp(ad, params)
        loss = A.CrossEntropyLoss(fused=True)(model(A.Tensor.from_numpy(ad, x)), A.Tensor.from_numpy(ad, onehot))
        (loss * scale).backward()
        grads.append(model.parameters().__next__().tensor.grad().numpy())
    np.testing.assert_array_equal(grads[1], grads[0] * np.float32(2.0))


def test_fused_loss_under_no_grad_records_nothing():
    params, x, onehot = problem()
    ad = A.Autodiff(OracleBackend())
    model = A.build_mlp(ad, params)
    with A.no_grad(ad):
        n = len(ad.tape.nodes)
        loss = A.CrossEntropyLoss(fused=True)(model(A.Tensor.from_numpy(ad, x)), A.Tensor.from_numpy(ad, onehot))
        assert len(ad.tape.nodes) == n and not loss.requires_grad


@pytest.mark.parametrize("kind", ["sgd", "adamw"])
def test_flat_arenas_alternate_and_keep_held_values(kind):
    """The fused optimizers keep parameters in flat arenas and write each step into the other
    one: with no reader left, two arenas alternate; a parameter storage held from an earlier
    step (a caller, a tape) keeps its values, because the arena it lives in is not written
    again while it is referenced (a fresh one is taken instead)."""
    params, x, onehot = problem()
    ad = A.Autodiff(OracleBackend())
    model = A.build_mlp(ad, params)
    optim = make_optim(model, kind, fused=True)
    flat = optim._flat
    assert flat is not None
    ids = []
    for _ in range(4):
        run(ad, model, optim, x, onehot, 1)
        ids.append(id(flat.cur))
    assert len(set(ids)) == 2 and ids[0] == ids[2] and ids[1] == ids[3]
    held = list(model.parameters())[0].tensor.storage.primal
    snapshot = held.copy()
    run(ad, model, optim, x, onehot, 3)
    np.testing.assert_array_equal(held, snapshot)
    assert id(flat.cur) not in ids or id(flat.spare) not in ids  # the held arena was not reused


@pytest.mark.parametrize("kind", ["sgd", "adamw"])
def test_fused_optimizer_made_after_backward_keeps_the_gradients(kind):
    """Moving the parameters into the arena keeps each tensor and its recorded gradient: an
    optimizer built between backward and step applies that step."""
    params, x, onehot = problem()
    out = []
    for fused in (False, True):
        ad = A.Autodiff(OracleBackend())
        model = A.build_mlp(ad, params)
        xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
        A.CrossEntropyLoss()(model(xt), tt).backward()
        make_optim(model, kind, fused).step()
        out.append([p.tensor.numpy() for p in model.parameters()])
    for a, b in zip(*out):
        np.testing.assert_array_equal(a, b)
