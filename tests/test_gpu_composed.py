"""The unchanged composed drop-in path at full size -- the reference frontend
(python/orca/nn/{linear,activation,container,loss}.py, python/orca/optim/adamw.py)
replayed through the tape (orca-autograd/src/tape.rs:107-118) onto HipBackend's
trait ops -- against the oracle, as it runs in the bench: plain, and with the
opt-in fused loss and AdamW (CrossEntropyLoss(fused=True), AdamW(fused=True))."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from orcaml_amd import autodiff as A
from orcaml_amd import synth
from tests.parity import check_one_adamw_step, check_teacher_forced_adamw_step, oracle_hidden

pytestmark = pytest.mark.gpu


class Composed:
    """nn.Sequential + CrossEntropyLoss + AdamW on HipBackend, stepping like a user
    script, keeping the ReLU outputs of the forward pass for the mask-flip count."""

    def __init__(self, hb, dims, params, x, onehot, opt, fused):
        self.ad = A.Autodiff(hb)
        self.model = A.build_mlp(self.ad, params)
        self.opt = A.AdamW(self.model.parameters(), lr=opt["lr"], betas=opt.get("betas", (0.9, 0.999)),
                           eps=opt.get("eps", 1e-8), weight_decay=opt["weight_decay"], fused=fused)
        self.loss_fn = A.CrossEntropyLoss(fused=fused)
        self.xt = A.Tensor.from_numpy(self.ad, x)
        self.tt = A.Tensor.from_numpy(self.ad, onehot)

    def step(self):
        self.opt.zero_grad()
        a, hidden = self.xt, []
        for m in self.model._modules.values():  # Sequential.forward, keeping the ReLU outputs
            a = m(a)
            if isinstance(m, A.ReLU):
                hidden.append(a)
        loss = self.loss_fn(a, self.tt)
        loss.backward()
        grads = [p.tensor.grad().numpy() for p in self.model.parameters()]
        logits = a.numpy()
        self.opt.step()
        return dict(loss=loss.to_list()[0], logits=logits, hidden=[h.numpy() for h in hidden], grads=grads)

    def params(self):
        return [p.tensor.numpy() for p in self.model.parameters()]

    def moments(self):
        return [m.numpy() for m in self.opt.m], [v.numpy() for v in self.opt.v]


def ref_opt(o):
    return O.make_opt(o["kind"], o["lr"], o.get("weight_decay", 0.0), o.get("betas", (0.9, 0.999)), o.get("eps", 1e-8))


@pytest.mark.parametrize("jit", [1, 2], ids=["programs_interpreted", "programs_compiled"])
@pytest.mark.parametrize("fused", [False, True], ids=["unchanged", "fused_loss_adamw"])
def test_composed_mlp784_4096_b1024_one_adamw_step(ctx, hb, fused, jit):
    """784-4096-4096-10, batch 1024, one fwd + bwd + AdamW step through the drop-in path,
    with the same attribution of outliers as the fused trainer's one-step test.  A single
    step runs its fused elementwise programs on the interpreter by default (each structure's
    first use); the second case compiles them at their first use.  With the fused loss and
    update there is no program to run."""
    w = synth.WORKLOADS[synth.MLP_LARGE]
    dims, o = w["dims"], w["opt"]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], dims, w["batch"])
    run = Composed(hb, dims, params, x, onehot, o, fused)
    ctx.set_ew_jit(jit)
    try:
        before = ctx.ew_jit_stats()
        out = run.step()
        new_params = run.params()  # runs the pending update programs under the same setting
        after = ctx.ew_jit_stats()
    finally:
        ctx.set_ew_jit(1)
    launched = after["compiled_launches"] + after["interpreted"] - before["compiled_launches"] - before["interpreted"]
    assert after["failures"] == before["failures"]
    if fused:  # the fused loss and update leave no elementwise chain to run
        assert launched == 0, launched
    elif jit == 2:
        assert after["compiled_launches"] > before["compiled_launches"]
    ref = O.mlp_train(dims, params, x, onehot, ref_opt(o), steps=1)
    ref["hidden"] = oracle_hidden(params, x, dims)
    preds = A.argmax_rows(out["logits"])
    correct = int((preds == labels).sum())
    check_one_adamw_step(dims, o, ref, out["loss"], out["logits"], out["hidden"], out["grads"], new_params, preds,
                         correct, what=f"composed 784-4096-4096-10 ({'fused' if fused else 'unchanged'})")


@pytest.mark.parametrize("fused", [False, True], ids=["unchanged", "fused_loss_adamw"])
def test_composed_mlp784_1024_b256_teacher_forced(hb, fused):
    """784-1024-1024-10, batch 256, 12 AdamW steps on one fixed batch through the drop-in
    path; at every step the oracle steps from the GPU's own parameters, moments and t
    (loss and gradients to tolerance with counted mask flips, the update bit-exact)."""
    w = synth.WORKLOADS[synth.MLP_MEDIUM]
    dims, o = w["dims"], w["opt"]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], dims, w["batch"])
    run = Composed(hb, dims, params, x, onehot, o, fused)
    zeros = [np.zeros_like(p) for p in params]
    state = dict(params=params, m=zeros, v=zeros, t=0)
    total = 0
    for step in range(12):
        out = run.step()
        ref = O.mlp_train(dims, state["params"], x, onehot, ref_opt(o), steps=1, m=state["m"], v=state["v"],
                          t=state["t"], want_grads=True)
        ref["hidden"] = oracle_hidden(state["params"], x, dims)
        new_p = run.params()
        new_m, new_v = run.moments()
        flips = check_teacher_forced_adamw_step(dims, o, state, ref, out["loss"], out["hidden"], out["grads"], new_p,
                                                new_m, new_v, what=f"step {step}")
        total += sum(flips)
        state = dict(params=[p.reshape(s.shape) for p, s in zip(new_p, params)],
                     m=[m.reshape(s.shape) for m, s in zip(new_m, params)],
                     v=[v.reshape(s.shape) for v, s in zip(new_v, params)], t=state["t"] + 1)
    print(f"composed 784-1024-1024-10 ({'fused' if fused else 'unchanged'}) teacher-forced: {total} mask flips")
    assert run.opt.t == 12


@pytest.mark.parametrize("wl", [synth.MLP_LARGE, synth.MLP_SMALL])
def test_composed_update_on_second_stream_changes_no_bit(ctx, wl):
    """The unchanged drop-in step (the reference's composed optimizer): an update program whose
    gradient came from an earlier weight-gradient product runs on the context's second stream,
    beside the backward's remaining products, into blocks released before that product.  Four
    steps and the next forward with and without that, from the same start, no host read in
    between: logits, parameters and moments bit-identical, and the second stream wrote moments
    when it was allowed."""
    from orcaml_amd.backend import HipBackend

    w = synth.WORKLOADS[wl]
    o = w["opt"]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    out = {}
    for overlap in (True, False):
        print(f"composed update, {wl}, overlap={overlap}", flush=True)
        ad = A.Autodiff(HipBackend(ctx, overlap=overlap))
        model = A.build_mlp(ad, params)
        if o["kind"] == "adamw":
            opt = A.AdamW(model.parameters(), lr=o["lr"], weight_decay=o["weight_decay"])
        else:
            opt = A.SGD(model.parameters(), lr=o["lr"])
        loss_fn = A.CrossEntropyLoss()
        xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
        for _ in range(4):
            opt.zero_grad()
            loss_fn(model(xt), tt).backward()
            opt.step()
        logits = model(xt).numpy()  # runs the last update's programs, then the forward
        if o["kind"] == "adamw":
            marked = sum(m.storage.primal.marked for m in opt.m)  # written there, not yet read here
            assert (marked > 0) == overlap, marked
        out[overlap] = [logits] + [p.tensor.numpy() for p in model.parameters()]
        if o["kind"] == "adamw":
            out[overlap] += [m.numpy() for m in opt.m] + [v.numpy() for v in opt.v]
    for i, (a, b) in enumerate(zip(out[True], out[False])):
        np.testing.assert_array_equal(a, b, err_msg=f"array {i}")


@pytest.mark.parametrize("wl,bias", [(synth.MLP_LARGE, True), (synth.MLP_SMALL, True), (synth.MLP_MEDIUM, False)])
def test_fused_update_on_second_stream_changes_no_bit(ctx, wl, bias):
    """The fused optimizer pass (AdamW at 784-4096-4096-10 / B 1024, SGD at 784-128-128-10 /
    B 64) updates the parameters whose gradients an earlier weight-gradient product made on the
    context's second stream, beside the backward's remaining products.  Four steps of the
    drop-in path with the fused loss and optimizer, with and without that, from the same start,
    and no host read in between: parameters and moments bit-identical, and the second stream
    took part from the second step on.  Without biases (784-1024-1024-10 / B 256) the weight
    gradients are still pending products when the pass starts: it runs them first, the last
    layer's first, and splits the update at their marks."""
    from orcaml_amd.backend import HipBackend

    w = synth.WORKLOADS[wl]
    o = w["opt"]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    if not bias:
        params = [q if k % 2 == 0 else None for k, q in enumerate(params)]
    out = {}
    for overlap in (True, False):
        ad = A.Autodiff(HipBackend(ctx, overlap=overlap))
        model = A.build_mlp(ad, params)
        if o["kind"] == "adamw":
            opt = A.AdamW(model.parameters(), lr=o["lr"], weight_decay=o["weight_decay"], fused=True)
        else:
            opt = A.SGD(model.parameters(), lr=o["lr"], fused=True)
        loss_fn = A.CrossEntropyLoss(fused=True)
        xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)
        for _ in range(4):
            opt.zero_grad()
            loss_fn(model(xt), tt).backward()
            opt.step()
        marked = sum(p.tensor.storage.primal.marked for p in model.parameters())
        assert (marked > 0) == overlap, marked
        # a snapshot of the moments first: device copies on the context stream, taken right
        # after the step, while the second stream may still be writing them
        snap = opt.state_dict() if o["kind"] == "adamw" else {}
        out[overlap] = [p.tensor.numpy() for p in model.parameters()]
        if o["kind"] == "adamw":
            out[overlap] += [m.numpy() for m in opt.m] + [v.numpy() for v in opt.v]
            out[overlap] += [snap[k].numpy() for k in sorted(k for k in snap if k != "t")]
    for i, (a, b) in enumerate(zip(out[True], out[False])):
        np.testing.assert_array_equal(a, b, err_msg=f"array {i}")
