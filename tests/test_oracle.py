"""CPU tests that pin the oracle (no GPU): the explicit step sequence against
the reference frontend replayed through the tape, closed forms, exact
integer arithmetic, fp64 brute force and the committed golden fixtures."""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import oracle as O
from orcaml_amd import autodiff as A
from orcaml_amd import synth
from tests.cpu_backend import OracleBackend

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def composed_train(dims, params, x, onehot, kind, steps, **opt):
    """The reference frontend (nn.Sequential + CrossEntropyLoss + SGD/AdamW)
    through the tape on the oracle backend."""
    ad = A.Autodiff(OracleBackend())
    model = A.build_mlp(ad, params)
    optim = A.SGD(model.parameters(), lr=opt["lr"]) if kind == "sgd" else A.AdamW(
        model.parameters(), lr=opt["lr"], betas=opt.get("betas", (0.9, 0.999)), eps=opt.get("eps", 1e-8),
        weight_decay=opt.get("weight_decay", 0.01))
    xt = A.Tensor.from_numpy(ad, x)
    tt = A.Tensor.from_numpy(ad, onehot)
    loss_fn = A.CrossEntropyLoss()
    losses, grads, logits = [], None, None
    for _ in range(steps):
        optim.zero_grad()
        out = model(xt)
        loss = loss_fn(out, tt)
        losses.append(loss.to_list()[0])
        loss.backward()
        grads = [p.tensor.grad().numpy() for p in model.parameters()]
        logits = out.numpy()
        optim.step()
    return dict(losses=np.array(losses, np.float32), grads=grads, logits=logits,
                params=[p.tensor.numpy() for p in model.parameters()])


@pytest.mark.parametrize("kind,steps", [("sgd", 2), ("adamw", 3)])
def test_explicit_sequence_equals_tape_replay(kind, steps):
    """orc_mlp_train writes the tape order out by hand; replaying the
    reference's Python frontend through the tape on the same ops must give
    bit-identical losses, gradients and parameters."""
    dims, B = (784, 48, 40, 10), 32
    params, x, labels, onehot = synth.mlp_problem(9, dims, B)
    opt = dict(lr=0.1) if kind == "sgd" else dict(lr=1e-3, weight_decay=0.01)
    ref = composed_train(dims, params, x, onehot, kind, steps, **opt)
    got = O.mlp_train(dims, params, x, onehot, O.make_opt(kind, **opt), steps=steps)
    np.testing.assert_array_equal(got["losses"], ref["losses"])
    np.testing.assert_array_equal(got["logits"], ref["logits"])
    for g, r in zip(got["grads"], ref["grads"]):
        np.testing.assert_array_equal(g, r.reshape(g.shape))
    for p, r in zip(got["params"], ref["params"]):
        np.testing.assert_array_equal(p, r.reshape(p.shape))
    np.testing.assert_array_equal(got["preds"], A.argmax_rows(ref["logits"]))


def test_ce_equal_logits_closed_form():
    B, C = 8, 10
    labels = np.arange(B) % C
    loss, g = O.cross_entropy(np.zeros((B, C), np.float32), synth.one_hot(labels, C))
    assert abs(loss - np.log(C)) < 1e-6
    np.testing.assert_allclose(g, (1.0 / C - synth.one_hot(labels, C)) / B, rtol=1e-6, atol=1e-9)


def test_ce_matches_fp64_softmax():
    rng = np.random.default_rng(1)
    z = (3 * rng.standard_normal((128, 37))).astype(np.float32)
    t = synth.one_hot(rng.integers(0, 37, 128), 37)
    loss, g = O.cross_entropy(z, t)
    z64 = z.astype(np.float64)
    sm = np.exp(z64 - z64.max(1, keepdims=True))
    sm /= sm.sum(1, keepdims=True)
    assert abs(loss - (-(t * np.log(sm)).sum(1).mean())) < 1e-5
    np.testing.assert_allclose(g, (sm - t) / 128, rtol=1e-4, atol=1e-8)
    np.testing.assert_allclose(g.sum(1), 0.0, atol=1e-8)  # each row's gradient sums to zero


def test_adamw_first_step_closed_form():
    rng = np.random.default_rng(2)
    p = rng.standard_normal(1000).astype(np.float32)
    g = rng.standard_normal(1000).astype(np.float32)
    lr, wd, eps = 1e-3, 0.01, 1e-8
    p1, m1, v1 = O.adamw_update(p, g, np.zeros_like(p), np.zeros_like(p), 1, lr=lr, weight_decay=wd, eps=eps)
    p64, g64 = p.astype(np.float64), g.astype(np.float64)
    np.testing.assert_allclose(p1, p64 * (1 - lr * wd) - lr * g64 / (np.abs(g64) + eps), rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(m1, 0.1 * g64, rtol=1e-6)
    np.testing.assert_allclose(v1, 0.001 * g64 * g64, rtol=1e-5)


def test_adamw_constant_gradient_closed_form_over_ten_steps():
    """With a fixed gradient g and m = v = 0 at the start, m_t = (1 - b1^t) g and
    v_t = (1 - b2^t) g^2 exactly, so the bias-corrected m_hat = g and v_hat = g^2 at every t
    (python/orca/optim/adamw.py:82-94) and each step is p <- p * f32(1 - lr*wd) - lr * g / (|g| + eps).
    t = 1 alone cannot tell the correction 1 - b^t from 1 - b*t or 1 - b^(t-1); steps 2..10 can."""
    rng = np.random.default_rng(4)
    n = 2048
    p0 = rng.standard_normal(n).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    g[:64] *= np.float32(1e-8)  # |g| comparable to eps: the eps term matters here
    lr, wd, eps, b1, b2 = 1e-3, 0.01, 1e-8, 0.9, 0.999
    decay = float(np.float32(1.0 - lr * wd))  # the f32 factor PyO3 hands the multiply
    g64 = g.astype(np.float64)
    p, m, v = p0, np.zeros(n, np.float32), np.zeros(n, np.float32)
    want = p0.astype(np.float64)
    for t in range(1, 11):
        p, m, v = O.adamw_update(p, g, m, v, t, lr=lr, weight_decay=wd, betas=(b1, b2), eps=eps)
        want = want * decay - lr * g64 / (np.abs(g64) + eps)
        np.testing.assert_allclose(m, (1.0 - b1 ** t) * g64, rtol=4e-6 * t, atol=0)
        np.testing.assert_allclose(v, (1.0 - b2 ** t) * g64 * g64, rtol=4e-6 * t, atol=0)
        np.testing.assert_allclose(p, want, rtol=2e-7 * t, atol=lr * 1e-6 * t)  # update rounding: ulps of lr
        if t >= 2:
            # what the two wrong corrections would make of m_hat: far outside the tolerance above
            for wrong in (1.0 - b1 * t, 1.0 - b1 ** (t - 1)):
                m_hat_wrong = (1.0 - b1 ** t) / wrong if wrong else np.inf
                assert abs(m_hat_wrong - 1.0) > 0.05


def test_sgd_closed_form():
    rng = np.random.default_rng(3)
    p = rng.standard_normal(999).astype(np.float32)
    g = rng.standard_normal(999).astype(np.float32)
    np.testing.assert_array_equal(O.sgd_update(p, g, 0.1), p - g * np.float32(0.1))


@pytest.mark.parametrize("variant", [0, 1, 2, 3])
def test_gemm_integer_exact_and_fp64_bound(variant):
    """Every summation-order variant (blocked f32 with FMA, f64-accumulated, ascending f32,
    descending f32 with FMA) is exact on small integers and within the gamma_K bound."""
    O.lib().orc_set_gemm_variant(variant)
    try:
        _gemm_checks()
    finally:
        O.lib().orc_set_gemm_variant(0)


def _gemm_checks():
    rng = np.random.default_rng(4)
    for (m, k, n) in [(1, 1, 1), (5, 3, 2), (130, 257, 67), (64, 784, 128)]:
        a = rng.integers(-8, 8, (m, k)).astype(np.float32)
        b = rng.integers(-8, 8, (k, n)).astype(np.float32)
        np.testing.assert_array_equal(O.matmul(a, b), (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        exact = a.astype(np.float64) @ b.astype(np.float64)
        bound = k * 2.0 ** -24 * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)))
        assert (np.abs(O.matmul(a, b) - exact) <= bound + 1e-30).all()
    # batched (..., M, K) x (..., K, N)
    a = rng.integers(-4, 4, (3, 5, 7)).astype(np.float32)
    b = rng.integers(-4, 4, (3, 7, 2)).astype(np.float32)
    np.testing.assert_array_equal(O.matmul(a, b), np.matmul(a, b))


def test_shape_ops_against_numpy():
    rng = np.random.default_rng(5)
    x = rng.integers(-9, 9, (4, 1, 3)).astype(np.float32)
    np.testing.assert_array_equal(O.expand(x, (2, 4, 5, 3)), np.broadcast_to(x, (2, 4, 5, 3)))
    y = rng.integers(-9, 9, (6, 5)).astype(np.float32)
    np.testing.assert_array_equal(O.sum_to_shape(y, (1, 5)), y.sum(0, keepdims=True))
    np.testing.assert_array_equal(O.sum_to_shape(y, (6, 1)), y.sum(1, keepdims=True))
    np.testing.assert_array_equal(O.sum_to_shape(y, (1,)), np.array([y.sum()], np.float32))
    np.testing.assert_array_equal(O.max_to_shape(y, (6, 1)), y.max(1, keepdims=True))
    z = rng.standard_normal((2, 3, 4)).astype(np.float32)
    np.testing.assert_array_equal(O.transpose(z, 0, 2), np.ascontiguousarray(np.swapaxes(z, 0, 2)))
    np.testing.assert_array_equal(O.transpose(z, 1, 2), np.ascontiguousarray(np.swapaxes(z, 1, 2)))


def test_elementwise_semantics():
    """relu(NaN) = 0 and relu(-0) = +0 (backend.rs:386); log clamps at 1e-7
    (backend.rs:577); max_to_shape starts at f32::MIN and ignores NaN; its
    backward gives every tie the full gradient (backend.rs:1421)."""
    x = np.array([np.nan, -0.0, 2.0, -1.0], np.float32)
    r = O.relu(x)
    assert r.tolist() == [0.0, 0.0, 2.0, 0.0] and not np.signbit(r[1])
    assert O.log(np.array([0.0, -5.0], np.float32)).tolist() == [np.float32(np.log(np.float32(1e-7)))] * 2
    m = O.max_to_shape(np.array([[np.nan, 1.0, 3.0, 3.0]], np.float32), (1, 1))
    assert m.tolist() == [[3.0]]
    g = O.max_to_shape_backward(np.array([[2.0]], np.float32), np.array([[1.0, 3.0, 3.0]], np.float32),
                                np.array([[3.0]], np.float32))
    assert g.tolist() == [[0.0, 2.0, 2.0]]
    assert O.max_to_shape(np.full((1, 2), -np.inf, np.float32), (1, 1)).tolist() == [[np.finfo(np.float32).min]]


def test_bias_gradient_is_column_sum_and_mask_from_preactivation():
    """Closed forms of one Linear+ReLU backward: db = column sums of dZ and
    dpre = g * [pre > 0]."""
    rng = np.random.default_rng(6)
    dims, B = (16, 12, 5), 7
    params, x, labels, onehot = synth.mlp_problem(3, dims, B)
    r = O.mlp_train(dims, params, x, onehot, O.make_opt("sgd", 0.0), steps=1)
    W1, W2 = params[0], params[2]
    h = x @ W1
    a = np.where(h > 0, h, 0)
    _, dlog = O.cross_entropy(a.astype(np.float32) @ W2 + params[3], onehot)
    np.testing.assert_allclose(r["grads"][3].reshape(-1), dlog.sum(0), rtol=1e-5, atol=1e-9)
    dz1 = (dlog @ W2.T) * (h > 0)
    np.testing.assert_allclose(r["grads"][1].reshape(-1), dz1.sum(0), rtol=1e-4, atol=1e-8)
    np.testing.assert_allclose(r["grads"][0], x.T @ dz1, rtol=1e-4, atol=1e-8)


def test_golden_mlp784_128_128_10_b64_sgd():
    """The committed fixture of the 784-128-128-10 / batch 64 / SGD(0.1) step
    (tests/golden/make_golden.py) reproduces bit for bit."""
    path = os.path.join(GOLDEN, "mlp784-128-128-10_b64_sgd.npz")
    gold = np.load(path, allow_pickle=False)
    w = synth.WORKLOADS[synth.MLP_SMALL]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    np.testing.assert_array_equal(labels, gold["labels"])
    assert float(x.astype(np.float64).sum()) == float(gold["x_sum"])
    r = O.mlp_train(w["dims"], params, x, onehot, O.make_opt("sgd", 0.1), steps=1)
    np.testing.assert_array_equal(r["losses"], gold["loss"])
    np.testing.assert_array_equal(r["logits"], gold["logits"])
    np.testing.assert_array_equal(r["preds"], gold["preds"])
    for i in range(6):
        np.testing.assert_allclose(r["grads"][i], gold[f"grad{i}"], rtol=1e-6, atol=1e-9)
        np.testing.assert_allclose(r["params"][i], gold[f"param{i}"], rtol=1e-6, atol=1e-9)


def test_synth_generator_fixed_values():
    """SplitMix64 reference values (first outputs of seed 0) and the uniform map."""
    z = synth.stream(0, 0, 3)
    assert [int(v) for v in z] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    u = synth.uniform(1, 1, (4,))
    assert u.dtype == np.float32 and (u >= 0).all() and (u < 1).all()
    n = synth.normal(5, 1, (200000,))
    assert abs(float(n.mean())) < 0.01 and abs(float(n.std()) - 1.0) < 0.01
    # chunked generation (used for 2^28-element buffers) reproduces the flat stream
    np.testing.assert_array_equal(synth.normal_range(5, 1, 1024, 2048, 0.0, 0.02),
                                  synth.normal(5, 1, (4096,), 0.0, 0.02)[1024:3072])


# ---- independent pins of the functions the MLP step does not exercise ----------
# Each check below is chosen so that a plausible slip in the restatement (a sign,
# a dropped factor, a swapped operand, a wrong comparison) fails it; none of them
# re-types the oracle's own expression.

def _ulps(got: np.ndarray, want64: np.ndarray) -> np.ndarray:
    """|got - want| in units of the f32 spacing at want."""
    want32 = want64.astype(np.float32)
    spacing = np.spacing(np.abs(want32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - want64) / spacing


def test_argmax_rows_first_maximum_and_nan():
    """python/orca/nn/model.py:65-75: first maximum on strict `>`.  NaN-free rows with planted
    ties agree with np.argmax (which also returns the first maximum); a NaN in column 0 wins
    (nothing compares greater than it); a NaN later is never taken (np.nanargmax)."""
    rng = np.random.default_rng(21)
    x = rng.integers(-3, 4, (400, 10)).astype(np.float32)  # many ties among 7 values
    x[5] = 2.0                                              # all equal -> 0
    x[6] = -np.inf                                          # all -inf -> 0
    x[7, 9] = np.inf
    np.testing.assert_array_equal(O.argmax_rows(x), np.argmax(x, axis=1))
    y = rng.standard_normal((300, 7)).astype(np.float32)
    y[:100, 0] = np.nan
    np.testing.assert_array_equal(O.argmax_rows(y[:100]), np.zeros(100, np.int32))
    cols = rng.integers(1, 7, 200)
    y[100 + np.arange(200), cols] = np.nan
    np.testing.assert_array_equal(O.argmax_rows(y[100:]), np.nanargmax(y[100:], axis=1))
    assert O.argmax_rows(np.array([[3.0]], np.float32)).tolist() == [0]


def test_sigmoid_against_fp64_and_limits():
    """backend.rs:392-412 in f32: sigmoid(0) = 0.5 exactly, within 3 ulp of the fp64 logistic
    over [-30, 30] (expf's error below 1 ulp, then one rounding each for the add and the
    division; measured 2.2 ulp at worst), monotone, sigmoid(x) + sigmoid(-x) = 1 to rounding, and the f32 limits
    (exp overflows to inf below -88.7, so the result is exactly 0; above 17 it rounds to 1)."""
    assert O.sigmoid(np.zeros(3, np.float32)).tolist() == [0.5, 0.5, 0.5]
    x = np.linspace(-30, 30, 200001, dtype=np.float32)
    got = O.sigmoid(x)
    want = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert _ulps(got, want).max() <= 3.0
    assert (np.diff(got) >= 0).all()
    np.testing.assert_allclose(got.astype(np.float64) + O.sigmoid(-x), 1.0, atol=2 ** -23)
    assert (O.sigmoid(np.array([-89.0, -1e4, -np.inf], np.float32)) == 0.0).all()
    assert (O.sigmoid(np.array([17.0, 1e4, np.inf], np.float32)) == 1.0).all()
    assert np.isnan(O.sigmoid(np.array([np.nan], np.float32))[0])


def test_sigmoid_backward_exact_on_dyadic_values():
    """backend.rs:440-464: g * y * (1 - y).  With y = k/64 and g a small integer over 8 every
    intermediate fits in f32 exactly, so the result must equal the fp64 value bit for bit."""
    k = np.arange(0, 65, dtype=np.float64)
    y = np.tile(k / 64.0, 31)
    g = np.repeat(np.arange(-15, 16, dtype=np.float64) / 8.0, 65)
    got = O.sigmoid_backward(g.astype(np.float32), y.astype(np.float32))
    np.testing.assert_array_equal(got, (g * y * (1.0 - y)).astype(np.float32))
    # the derivative of the logistic at x is s(x)(1 - s(x)): a central difference in fp64
    x = np.linspace(-6, 6, 97)
    s = lambda t: 1.0 / (1.0 + np.exp(-t))  # noqa: E731
    h = 1e-6
    fd = (s(x + h) - s(x - h)) / (2 * h)
    got = O.sigmoid_backward(np.ones_like(x, np.float32), s(x).astype(np.float32))
    # y is rounded to f32 first (absolute error up to 6e-8 near 1, which 1 - y keeps)
    np.testing.assert_allclose(got, fd, rtol=2e-6, atol=1e-7)


def test_sqrt_backward_is_the_derivative_of_sqrt():
    """backend.rs:734-759: with y = sqrt(x) stored, d sqrt(x)/dx = 1 / (2 y); checked against an
    fp64 central difference of sqrt, scaled by the incoming gradient."""
    rng = np.random.default_rng(22)
    x = rng.uniform(0.01, 100.0, 5000)
    g = rng.standard_normal(5000)
    y = np.sqrt(x).astype(np.float32)
    h = 1e-6 * x
    fd = (np.sqrt(x + h) - np.sqrt(x - h)) / (2 * h)
    got = O.sqrt_backward(g.astype(np.float32), y)
    np.testing.assert_allclose(got, g * fd, rtol=1e-5, atol=1e-12)


def test_div_backward_are_the_partial_derivatives_of_a_quotient():
    """backend.rs:678-732: d(l/r)/dl = 1/r and d(l/r)/dr = -l/r^2, each times the incoming
    gradient; checked against fp64 central differences of l/r in each operand."""
    rng = np.random.default_rng(23)
    l = rng.uniform(-10, 10, 5000)
    r = rng.uniform(0.5, 10, 5000) * rng.choice([-1.0, 1.0], 5000)
    g = rng.standard_normal(5000)
    l32, r32, g32 = (v.astype(np.float32) for v in (l, r, g))
    l, r, g = (v.astype(np.float64) for v in (l32, r32, g32))
    h = 1e-6
    fd_l = ((l + h) / r - (l - h) / r) / (2 * h)
    fd_r = (l / (r + h) - l / (r - h)) / (2 * h)
    np.testing.assert_allclose(O.div_backward_lhs(g32, r32), g * fd_l, rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(O.div_backward_rhs(g32, l32, r32), g * fd_r, rtol=1e-4, atol=1e-8)


def test_has_nan_or_inf_matches_isfinite():
    """backend.rs:1319-1334: true exactly when some element is NaN or +-inf.  FLT_MAX,
    denormals and -0 are finite; a single bad value at the first or last position counts."""
    rng = np.random.default_rng(24)
    fmax = np.finfo(np.float32).max
    finite_specials = np.array([fmax, -fmax, 1e-45, -1e-45, -0.0, 0.0], np.float32)
    assert not O.has_nan_or_inf(finite_specials)
    assert not O.has_nan_or_inf(np.zeros(0, np.float32))
    for bad in (np.nan, np.inf, -np.inf):
        for pos in (0, 999, 517):
            a = rng.standard_normal(1000).astype(np.float32)
            a[pos] = bad
            assert O.has_nan_or_inf(a) == (not np.isfinite(a).all()) == True  # noqa: E712
    for _ in range(50):
        a = rng.standard_normal(257).astype(np.float32)
        if rng.random() < 0.5:
            a[rng.integers(0, 257)] = rng.choice([np.nan, np.inf, -np.inf, fmax])
        assert O.has_nan_or_inf(a) == (not np.isfinite(a).all())
