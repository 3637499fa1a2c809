"""The trainer's captured step (a HIP graph replayed every step) against the
same step launched kernel by kernel: bit-identical losses, gradients,
parameters and moments after every step, with host reads, synchronisations
and batch changes between the replays."""
from __future__ import annotations

import numpy as np
import pytest

from orcaml_amd import synth
from orcaml_amd.mlp import MLPTrainer

pytestmark = pytest.mark.gpu


def make(ctx, monkeypatch, w, graph: bool):
    monkeypatch.setenv("ORCA_HIP_GRAPH", "1" if graph else "0")
    o = w["opt"]
    return MLPTrainer(ctx, w["dims"], w["batch"], kind=o["kind"], lr=o["lr"], weight_decay=o.get("weight_decay", 0.0),
                      betas=o.get("betas", (0.9, 0.999)), eps=o.get("eps", 1e-8))


def state(tr):
    out = {"params": tr.params(), "grads": tr.grads(), "preds": tr.preds()}
    if tr.step_count() > 0:
        out["m"], out["v"] = tr.moments(0), tr.moments(1)
    return out


def assert_same(a, b, what):
    for key in a:
        for i, (x, y) in enumerate(zip(a[key], b[key]) if isinstance(a[key], list) else [(a[key], b[key])]):
            np.testing.assert_array_equal(x, y, err_msg=f"{what}: {key} {i}")


@pytest.mark.parametrize("workload,steps", [(synth.MLP_SMALL, 6), (synth.MLP_MEDIUM, 6), (synth.MLP_LARGE, 3)])
def test_graph_replays_match_eager_steps(ctx, monkeypatch, workload, steps):
    w = dict(synth.WORKLOADS[workload])
    if workload == synth.MLP_SMALL:  # SGD in the workload; also run AdamW so both update paths replay
        w["opt"] = dict(kind="adamw", lr=1e-3, weight_decay=0.01)
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    trs = [make(ctx, monkeypatch, w, graph) for graph in (True, False)]
    for tr in trs:
        tr.set_params(params)
        tr.set_batch(x, onehot=onehot)
    for step in range(steps):
        if step == steps // 2:  # switch to class-index targets: the captured step must be rebuilt
            for tr in trs:
                tr.set_batch(x, labels=labels)
        results = []
        for tr in trs:
            tr.step()
            results.append((tr.metrics(), state(tr)))
        (m_g, s_g), (m_e, s_e) = results
        assert m_g == m_e, f"step {step}: loss / correct differ between replay and eager"
        assert_same(s_g, s_e, f"step {step}")
    for tr in trs:
        tr.close()


def test_graph_replays_back_to_back_sgd(ctx, monkeypatch):
    """Several replays enqueued without a host read in between, then compared."""
    w = synth.WORKLOADS[synth.MLP_SMALL]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    trs = [make(ctx, monkeypatch, w, graph) for graph in (True, False)]
    for tr in trs:
        tr.set_params(params)
        tr.set_batch(x, labels=labels)
        for _ in range(10):
            tr.step()
    assert trs[0].metrics() == trs[1].metrics()
    assert_same(state(trs[0]), state(trs[1]), "after 10 steps")
    for tr in trs:
        tr.close()


@pytest.mark.parametrize("batch,count", [(512, 2), (128, 8)])
def test_graph_replays_with_an_update_shard(ctx, monkeypatch, batch, count):
    """784-4096-4096-10 at a data-parallel share: after one step, the optimizer update is
    sharded (rank count - 1 of count), which must rebuild the captured step; every later
    replay matches the eager trainer with the same shard bit for bit (the eager one keeps two
    parameter arenas, the captured one updates in place)."""
    w = dict(synth.WORKLOADS[synth.MLP_LARGE], batch=batch)
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], batch)
    trs = [make(ctx, monkeypatch, w, graph) for graph in (True, False)]
    for tr in trs:
        tr.set_params(params)
        tr.set_batch(x, onehot=onehot)
    for step in range(3):
        if step == 1:
            for tr in trs:
                tr.set_update_shard(count - 1, count)
        results = []
        for tr in trs:
            tr.step()
            results.append((tr.metrics(), state(tr)))
        (m_g, s_g), (m_e, s_e) = results
        assert m_g == m_e, f"step {step}: loss / correct differ between replay and eager"
        assert_same(s_g, s_e, f"step {step}")
    for tr in trs:
        tr.close()
