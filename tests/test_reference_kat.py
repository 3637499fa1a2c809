"""The reference's own known-answer tests, run through the restated tape on
two backends: the CPU oracle (pins the oracle) and HipBackend on the GPU
(pins the HIP trait ops).  Each test cites the reference test it restates."""
from __future__ import annotations

import numpy as np
import pytest

from orcaml_amd import autodiff as A

BACKENDS = [pytest.param("oracle", id="oracle"), pytest.param("hip", id="hip", marks=pytest.mark.gpu)]


@pytest.fixture(params=BACKENDS)
def ad(request):
    if request.param == "oracle":
        from tests.cpu_backend import OracleBackend

        return A.Autodiff(OracleBackend())
    ctx = request.getfixturevalue("ctx")
    from orcaml_amd.backend import HipBackend

    return A.Autodiff(HipBackend(ctx))


def T(ad, values, shape, requires_grad=False):
    return A.Tensor.from_numpy(ad, np.array(values, np.float32).reshape(shape), requires_grad)


def test_basic_autograd(ad):
    """orca-autograd/tests/autograd_tests.rs:6-53: loss = (x.w - 10)^2 => grad_w = [-20, -30]."""
    x = T(ad, [2.0, 3.0], (1, 2), True)
    w = T(ad, [1.0, 1.0], (2, 1), True)
    y = x @ w
    assert y.shape == (1, 1)
    ten = T(ad, [10.0], (1, 1))
    diff = y._bin(ten, "sub")
    loss = diff._bin(diff, "mul")
    loss.backward()
    g = w.grad().numpy().reshape(-1)
    assert abs(g[0] - (-20.0)) < 1e-5 and abs(g[1] - (-30.0)) < 1e-5


def test_autograd_activation(ad):
    """autograd_tests.rs:55-90: relu([-1, 2]) = [0, 2], grad = [0, 1] exactly."""
    x = T(ad, [-1.0, 2.0], (1, 2), True)
    y = x.relu()
    assert y.to_list() == [0.0, 2.0]
    ones = T(ad, [1.0, 1.0], (1, 2))
    loss = y._bin(ones, "mul")
    loss.backward()
    assert x.grad().to_list() == [0.0, 1.0]


@pytest.mark.parametrize("a,b,op", [([1.0, 2.0], [3.0, 4.0], "add"), ([2.0, 3.0], [4.0, 5.0], "sub"),
                                    ([1.0, 2.0], [3.0, 4.0], "mul")])
def test_tensor_ops(ad, a, b, op):
    """python/tests/test_api.py:33-51: exact elementwise results."""
    x, y = T(ad, a, (1, 2)), T(ad, b, (1, 2))
    c = {"add": x + y, "sub": x - y, "mul": x * y}[op]
    want = {"add": [p + q for p, q in zip(a, b)], "sub": [p - q for p, q in zip(a, b)],
            "mul": [p * q for p, q in zip(a, b)]}[op]
    assert c.to_list() == want


def test_autograd_basic(ad):
    """test_api.py:53-61: d(x^2)/dx at 2 = 4."""
    x = T(ad, [2.0], (1, 1), True)
    y = x * x
    y.backward()
    assert abs(x.grad().to_list()[0] - 4.0) < 1e-5


def test_shape_mismatch_exception(ad):
    """test_api.py:63-68."""
    a = T(ad, [1.0, 2.0], (1, 2))
    b = T(ad, [1.0, 2.0, 3.0], (1, 3))
    with pytest.raises(ValueError):
        _ = a + b


def test_crossentropy_loss_positive(ad):
    """test_api.py:83-89."""
    loss = A.CrossEntropyLoss()(T(ad, [1.0, 0.0], (1, 2)), T(ad, [1.0, 0.0], (1, 2)))
    assert loss.to_list()[0] > 0.0


def _cubic(ad, xv, requires_grad=False):
    x = T(ad, [xv], (1,), requires_grad)
    y = x * x * x + x * x * A.Tensor.scalar(ad, 2.0) + x * A.Tensor.scalar(ad, 5.0)
    return x, y


def test_numerical_gradients(ad):
    """test_api.py:196-218: y = x^3 + 2x^2 + 5x, dy/dx at 2 = 25."""
    x, y = _cubic(ad, 2.0, True)
    y.backward()
    ga = x.grad().to_list()[0]
    eps = 1e-4
    gn = (_cubic(ad, 2.0 + eps)[1].to_list()[0] - _cubic(ad, 2.0 - eps)[1].to_list()[0]) / (2 * eps)
    assert abs(ga - 25.0) < 1e-2
    assert abs(ga - gn) < 1e-2


def test_linear_numerical_gradient(ad):
    """test_api.py:250-279: y = x @ W => dW = x^T."""
    xv, wv = [1.5, -2.0], [0.8, 1.2]
    x = T(ad, xv, (1, 2))
    W = T(ad, wv, (2, 1), True)
    y = x @ W
    y.backward()
    g = W.grad().to_list()
    eps = 1e-4
    yp = (x @ T(ad, [wv[0] + eps, wv[1]], (2, 1))).to_list()[0]
    ym = (x @ T(ad, [wv[0] - eps, wv[1]], (2, 1))).to_list()[0]
    assert abs(g[0] - (yp - ym) / (2 * eps)) < 1e-2
    assert abs(g[0] - xv[0]) < 1e-3


def _chunk(t: A.Tensor, chunks: int):
    """python/orca/tensor.py:29-80 for a rank-2 tensor along the last dim:
    each chunk is t @ P with a 0/1 projection matrix."""
    rows, dim = t.shape
    cs = dim // chunks
    out = []
    for i in range(chunks):
        proj = np.zeros((dim, cs), np.float32)
        for j in range(cs):
            proj[i * cs + j, j] = 1.0
        out.append(t @ A.Tensor.from_numpy(t.ad, proj))
    return out


def test_tensor_chunk(ad):
    """test_api.py:323-346: gradients flow back through chunks as [10, 20, 30, ...]."""
    x = T(ad, [1.0, 2.0, 3.0, 4.0, 5.0, 6.0], (2, 3), True)
    c = _chunk(x, 3)
    assert [ch.to_list() for ch in c] == [[1.0, 4.0], [2.0, 5.0], [3.0, 6.0]]
    loss = c[0] * 10.0 + c[1] * 20.0 + c[2] * 30.0
    loss.sum_to_shape((1,)).backward()
    assert x.grad().to_list() == [10.0, 20.0, 30.0, 10.0, 20.0, 30.0]


def _num_grads(ad, model, x, y, loss_fn, eps=1e-4):
    grads = []
    for p in model.parameters():
        data = p.tensor.numpy().astype(np.float32).reshape(-1)
        g = np.zeros_like(data)
        for i in range(data.size):
            orig = data[i]
            vals = []
            for d in (eps, -eps):
                data[i] = orig + d
                p.update(A.Tensor.from_numpy(ad, data.reshape(p.tensor.shape), True))
                vals.append(loss_fn(model(x), y).to_list()[0])
            data[i] = orig
            g[i] = (vals[0] - vals[1]) / (2 * eps)
        p.update(A.Tensor.from_numpy(ad, data.reshape(p.tensor.shape), True))
        grads.append(g.reshape(p.tensor.shape))
    return grads


@pytest.mark.parametrize("case", ["linear_relu_mse", "linear_ce"])
def test_grad_check(ad, case):
    """examples/basics/test_grad_check.py:49-119: analytic vs finite-difference
    gradients, max abs diff < 5e-3 (fixed seeded data instead of randn)."""
    rng = np.random.default_rng(7)
    if case == "linear_relu_mse":
        model = A.Sequential(A.Linear(ad, rng.uniform(-0.5, 0.5, (4, 2)).astype(np.float32),
                                      rng.uniform(-0.5, 0.5, (1, 2)).astype(np.float32)), A.ReLU())
        x = A.Tensor.from_numpy(ad, rng.standard_normal((2, 4)).astype(np.float32))
        y = A.Tensor.from_numpy(ad, rng.standard_normal((2, 2)).astype(np.float32))
        loss_fn = A.MSELoss()
    else:
        model = A.Linear(ad, rng.uniform(-0.5, 0.5, (3, 3)).astype(np.float32),
                         rng.uniform(-0.5, 0.5, (1, 3)).astype(np.float32))
        x = A.Tensor.from_numpy(ad, rng.standard_normal((2, 3)).astype(np.float32))
        y = A.Tensor.from_numpy(ad, np.array([[1, 0, 0], [0, 1, 0]], np.float32))
        loss_fn = A.CrossEntropyLoss()
    loss = loss_fn(model(x), y)
    loss.backward()
    analytic = [p.tensor.grad().numpy() for p in model.parameters()]
    ad.tape.clear()
    numeric = _num_grads(ad, model, x, y, loss_fn)
    for a, n in zip(analytic, numeric):
        assert np.max(np.abs(a - n)) < 5e-3


def test_optimizers_update_weights(ad):
    """test_api.py:91-122 for SGD (momentum 0.9, wd 0.01) and AdamW."""
    rng = np.random.default_rng(3)
    for make in (lambda ps: A.SGD(ps, lr=0.1, momentum=0.9, weight_decay=0.01),
                 lambda ps: A.AdamW(ps, lr=0.01, weight_decay=0.01)):
        model = A.Sequential(A.Linear(ad, rng.uniform(-0.7, 0.7, (2, 2)).astype(np.float32),
                                      rng.uniform(-0.7, 0.7, (1, 2)).astype(np.float32)))
        opt = make(model.parameters())
        x = T(ad, [1.0, 1.0], (1, 2))
        y = T(ad, [1.0, 0.0], (1, 2))
        before = list(model.parameters())[0].tensor.to_list()
        opt.zero_grad()
        A.MSELoss()(model(x), y).backward()
        opt.step()
        assert list(model.parameters())[0].tensor.to_list() != before
