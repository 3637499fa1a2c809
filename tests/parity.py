"""End-to-end parity checks shared by the GPU tests of the fused trainer and of
the composed drop-in path: one step of an MLP against the oracle with the
ReLU-mask-flip and AdamW-amplification attribution, and one teacher-forced step."""
from __future__ import annotations

import numpy as np

from oracle import oracle as O
from tests.util import assert_close, outside_tolerance


def oracle_hidden(params, x, dims):
    """The oracle's ReLU outputs of layers 0..L-2 (its own forward pass)."""
    B = x.shape[0]
    hs, a = [], x
    for l in range(len(dims) - 2):
        a = O.relu(O.add(O.matmul(a, params[2 * l]), O.expand(params[2 * l + 1], (B, dims[l + 1]))))
        hs.append(a)
    return hs


def mask_flips(gpu_hidden, ref_hidden):
    """Per layer, entries whose ReLU mask differs between the GPU's forward and the
    oracle's (pre-activations within rounding of zero); 0 for the last layer."""
    return [int(((h > 0) != (g > 0)).sum()) for g, h in zip(gpu_hidden, ref_hidden)] + [0]


def allowed_outliers(i, size, flips, dims):
    """A flip at (b, j) of layer l's mask changes dZ_l[b, j]: column j of dW_l
    (dims[l] entries) and entry j of db_l; plus a 1e-5 fraction of slack."""
    l = i // 2
    return int(np.ceil(1e-5 * size)) + flips[l] * (dims[l] if i % 2 == 0 else 1)


def near_tie_rows(logits_ref: np.ndarray, tol: float) -> np.ndarray:
    """Rows whose top-2 margin is within rounding: their argmax may legitimately
    differ when the logits come from differently-rounded GEMMs."""
    s = np.sort(logits_ref, axis=1)
    return (s[:, -1] - s[:, -2]) <= tol * np.maximum(1.0, np.abs(s[:, -1]))


def check_one_adamw_step(dims, opt, ref, loss, logits, hidden, grads, new_params, preds, correct, what=""):
    """One AdamW step from the same state, end to end: loss and logits to the path's
    tolerance (1e-5 abs + 1e-4 rel); gradients and updated parameters to that tolerance
    except for elements explained by counted ReLU mask flips between the two forward
    passes, or (parameters) by AdamW's first-step normalisation g / (|g| + eps), which
    turns a gradient difference well inside the tolerance into a parameter difference of
    up to 2 lr where |g| is within a few orders of eps.  Argmax / accuracy are exact
    outside rows whose top-2 margin is within rounding.  `ref` is O.mlp_train's result
    for one step from the same parameters plus ref["hidden"] = oracle_hidden(...);
    returns the report line."""
    assert_close(loss, ref["losses"][0], what=f"{what} loss")
    assert_close(logits, ref["logits"], what=f"{what} logits")
    flips = mask_flips(hidden, ref["hidden"])
    report, over = [], []
    for kind, got_all, ref_all in (("grad", grads, ref["grads"]), ("param", new_params, ref["params"])):
        for i, (g, r) in enumerate(zip(got_all, ref_all)):
            g = np.asarray(g).reshape(r.shape)
            bad = np.abs(g.astype(np.float64) - r) > 1e-5 + 1e-4 * np.abs(r.astype(np.float64))
            if kind == "param":
                gg = np.asarray(grads[i]).reshape(r.shape).astype(np.float64)
                gr = ref["grads"][i].astype(np.float64)
                predicted = opt["lr"] * np.abs(gg / (np.abs(gg) + opt["eps"]) - gr / (np.abs(gr) + opt["eps"]))
                amplified = predicted >= 0.5 * (1e-5 + 1e-4 * np.abs(r.astype(np.float64)))
                report.append(f"param{i}-from-grad:{int((bad & amplified).sum())}")
                bad = bad & ~amplified
            n_out = int(bad.sum())
            allowed = allowed_outliers(i, g.size, flips, dims)
            report.append(f"{kind}{i}:{n_out}/{allowed}")
            if n_out > allowed:
                over.append(f"{kind} {i}: {n_out} of {g.size} outside tolerance (allowed {allowed})")
    line = f"{what}: ReLU mask flips {flips[:-1]}; outside 1e-5+1e-4|x| / allowed: {' '.join(report)}"
    print(line)
    assert not over, over
    for i, (gg, gr) in enumerate(zip(grads, ref["grads"])):  # sign noise itself is rare
        gg = np.asarray(gg).reshape(gr.shape)
        assert (np.sign(gg) != np.sign(gr)).mean() <= 2e-3, f"{what} grad {i}: too many sign disagreements"
    ties = near_tie_rows(ref["logits"], 1e-5)
    np.testing.assert_array_equal(np.asarray(preds)[~ties], ref["preds"][~ties])
    assert abs(int(correct) - int(ref["correct"])) <= int(ties.sum())
    return line


def check_teacher_forced_adamw_step(dims, opt, state, ref, loss, hidden, grads, new_params, new_m, new_v, what=""):
    """One step from the GPU's own state (`state`: params, m, v, t before the step; `ref`:
    O.mlp_train's one step from that state): the loss to the path's tolerance, every gradient
    to that tolerance except entries attributed to counted ReLU mask flips, and the new
    parameters and moments bit-identical to the oracle's AdamW applied to the GPU's own
    gradients (the update has no rounding freedom).  Returns the mask flips."""
    assert_close(loss, ref["losses"][0], what=f"{what} loss")
    flips = mask_flips(hidden, ref["hidden"])
    t = state["t"] + 1
    for i in range(len(new_params)):
        shape = state["params"][i].shape
        g = np.asarray(grads[i]).reshape(shape)
        n_out = outside_tolerance(g, ref["grads"][i])
        allowed = allowed_outliers(i, g.size, flips, dims)
        assert n_out <= allowed, (f"{what} grad {i}: {n_out} of {g.size} outside tolerance "
                                  f"(ReLU mask flips {flips}, allowed {allowed})")
        p1, m1, v1 = O.adamw_update(state["params"][i], g, state["m"][i], state["v"][i], t, lr=opt["lr"],
                                    weight_decay=opt["weight_decay"], betas=opt.get("betas", (0.9, 0.999)),
                                    eps=opt.get("eps", 1e-8))
        np.testing.assert_array_equal(np.asarray(new_params[i]).reshape(shape), p1, err_msg=f"{what} param {i}")
        np.testing.assert_array_equal(np.asarray(new_m[i]).reshape(shape), m1, err_msg=f"{what} m {i}")
        np.testing.assert_array_equal(np.asarray(new_v[i]).reshape(shape), v1, err_msg=f"{what} v {i}")
    return flips
