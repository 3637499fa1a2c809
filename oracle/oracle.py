"""TEST INFRASTRUCTURE ONLY -- ctypes binding of the CPU oracle library.

The oracle (oracle/*.c) restates the reference CPU backend
(orca-backend-cpu/src/backend.rs), the autograd tape order
(orca-autograd/src/tape.rs:107-118) and the Python frontend op sequence
(python/orca/nn/{linear,loss}.py, python/orca/optim/{sgd,adamw}.py).
Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module; the product package never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liborca_oracle.so")

_F = ctypes.POINTER(ctypes.c_float)
_SZ = ctypes.POINTER(ctypes.c_size_t)


class OrcOpt(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int),
        ("lr", ctypes.c_double),
        ("momentum", ctypes.c_double),
        ("weight_decay", ctypes.c_double),
        ("beta1", ctypes.c_double),
        ("beta2", ctypes.c_double),
        ("eps", ctypes.c_double),
    ]


def build() -> str:
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.orc_mul_scalar.argtypes = [_F, ctypes.c_float, _F, ctypes.c_size_t]
        _lib.orc_has_nan_or_inf.restype = ctypes.c_int
        _lib.orc_num_threads.restype = ctypes.c_int
    return _lib


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _dims(shape):
    arr = (ctypes.c_size_t * max(1, len(shape)))(*shape)
    return arr, len(shape)


def _check(rc: int, what: str):
    if rc != 0:
        raise ValueError(f"oracle {what} failed with status {rc}")


# ---- elementwise ------------------------------------------------------------
def _binary(name):
    def f(a, b):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        out = np.empty_like(a)
        getattr(lib(), "orc_" + name)(_fp(a), _fp(b), _fp(out), ctypes.c_size_t(a.size))
        return out

    f.__name__ = name
    return f


def _unary(name):
    def f(a):
        a = np.ascontiguousarray(a, np.float32)
        out = np.empty_like(a)
        getattr(lib(), "orc_" + name)(_fp(a), _fp(out), ctypes.c_size_t(a.size))
        return out

    f.__name__ = name
    return f


add = _binary("add")
sub = _binary("sub")
mul = _binary("mul")
div = _binary("div")
relu_backward = _binary("relu_backward")
sigmoid_backward = _binary("sigmoid_backward")
exp_backward = _binary("exp_backward")
log_backward = _binary("log_backward")
sqrt_backward = _binary("sqrt_backward")
div_backward_lhs = _binary("div_backward_lhs")
accumulate_grad = _binary("accumulate_grad")
relu = _unary("relu")
sigmoid = _unary("sigmoid")
exp = _unary("exp")
log = _unary("log")
sqrt = _unary("sqrt")


def div_backward_rhs(g, l, r):
    g, l, r = (np.ascontiguousarray(v, np.float32) for v in (g, l, r))
    out = np.empty_like(g)
    lib().orc_div_backward_rhs(_fp(g), _fp(l), _fp(r), _fp(out), ctypes.c_size_t(g.size))
    return out


def mul_scalar(a, s: float):
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty_like(a)
    lib().orc_mul_scalar(_fp(a), ctypes.c_float(s), _fp(out), ctypes.c_size_t(a.size))
    return out


def has_nan_or_inf(a) -> bool:
    a = np.ascontiguousarray(a, np.float32)
    return bool(lib().orc_has_nan_or_inf(_fp(a), ctypes.c_size_t(a.size)))


# ---- shape ops ----------------------------------------------------------------
def _shape_op(name, a, out_shape):
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty(tuple(out_shape), np.float32)
    ind, inr = _dims(a.shape)
    od, onr = _dims(out_shape)
    _check(getattr(lib(), "orc_" + name)(_fp(a), _fp(out), ind, ctypes.c_size_t(inr), od,
                                         ctypes.c_size_t(onr)), name)
    return out


def expand(a, out_shape):
    return _shape_op("expand", a, out_shape)


def sum_to_shape(a, out_shape):
    return _shape_op("sum_to_shape", a, out_shape)


def max_to_shape(a, out_shape):
    return _shape_op("max_to_shape", a, out_shape)


def max_to_shape_backward(g, x, y):
    g, x, y = (np.ascontiguousarray(v, np.float32) for v in (g, x, y))
    out = np.empty_like(x)
    ind, inr = _dims(x.shape)
    od, onr = _dims(y.shape)
    _check(lib().orc_max_to_shape_backward(_fp(g), _fp(x), _fp(y), _fp(out), ind, ctypes.c_size_t(inr),
                                           od, ctypes.c_size_t(onr)), "max_to_shape_backward")
    return out


def transpose(a, d0: int, d1: int):
    a = np.ascontiguousarray(a, np.float32)
    shape = list(a.shape)
    shape[d0], shape[d1] = shape[d1], shape[d0]
    out = np.empty(tuple(shape), np.float32)
    dd, r = _dims(a.shape)
    _check(lib().orc_transpose(_fp(a), _fp(out), dd, ctypes.c_size_t(r), ctypes.c_size_t(d0),
                               ctypes.c_size_t(d1)), "transpose")
    return out


def matmul(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty(a.shape[:-1] + (b.shape[-1],), np.float32)
    ad, ar = _dims(a.shape)
    bd, br = _dims(b.shape)
    _check(lib().orc_matmul(_fp(a), _fp(b), _fp(out), ad, ctypes.c_size_t(ar), bd, ctypes.c_size_t(br)),
           "matmul")
    return out


def argmax_rows(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape[0], np.int32)
    lib().orc_argmax_rows(_fp(x), ctypes.c_size_t(x.shape[0]), ctypes.c_size_t(x.shape[1]),
                          out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)))
    return out


# ---- composed cross-entropy, optimizers, training step --------------------------
def cross_entropy(logits, onehot):
    logits = np.ascontiguousarray(logits, np.float32)
    onehot = np.ascontiguousarray(onehot, np.float32)
    B, C = logits.shape
    loss = np.zeros(1, np.float32)
    d = np.empty_like(logits)
    _check(lib().orc_cross_entropy(_fp(logits), _fp(onehot), ctypes.c_size_t(B), ctypes.c_size_t(C),
                                   _fp(loss), _fp(d)), "cross_entropy")
    return float(loss[0]), d


def make_opt(kind: str, lr: float, weight_decay: float = 0.0, betas=(0.9, 0.999), eps: float = 1e-8):
    return OrcOpt(0 if kind == "sgd" else 1, lr, 0.0, weight_decay, betas[0], betas[1], eps)


def sgd_update(p, g, lr: float):
    p = np.array(p, np.float32, copy=True)
    g = np.ascontiguousarray(g, np.float32)
    opt = make_opt("sgd", lr)
    lib().orc_sgd_update(_fp(p), _fp(g), ctypes.c_size_t(p.size), ctypes.byref(opt))
    return p


def adamw_update(p, g, m, v, t: int, lr=1e-3, weight_decay=0.01, betas=(0.9, 0.999), eps=1e-8):
    p = np.array(p, np.float32, copy=True)
    m = np.array(m, np.float32, copy=True)
    v = np.array(v, np.float32, copy=True)
    g = np.ascontiguousarray(g, np.float32)
    opt = make_opt("adamw", lr, weight_decay, betas, eps)
    lib().orc_adamw_update(_fp(p), _fp(g), _fp(m), _fp(v), ctypes.c_size_t(p.size), ctypes.byref(opt),
                           ctypes.c_int64(t))
    return p, m, v


def mlp_train(dims, params, x, onehot, opt: OrcOpt, steps: int = 1, m=None, v=None, t: int = 0,
              want_grads: bool = True):
    """Runs `steps` reference training steps on copies of `params`.

    Returns a dict with params, m, v, t, losses, grads (last step), logits,
    preds and correct (last step)."""
    L = len(dims) - 1
    B = x.shape[0]
    params = [np.array(p, np.float32, copy=True) for p in params]
    if opt.kind == 1:
        m = [np.zeros_like(p) for p in params] if m is None else [np.array(a, np.float32, copy=True) for a in m]
        v = [np.zeros_like(p) for p in params] if v is None else [np.array(a, np.float32, copy=True) for a in v]
    grads = [np.empty_like(p) for p in params] if want_grads else None
    PP = _F * (2 * L)
    pp = PP(*[_fp(p) for p in params])
    mp = PP(*[_fp(a) for a in m]) if m is not None else None
    vp = PP(*[_fp(a) for a in v]) if v is not None else None
    gp = PP(*[_fp(a) for a in grads]) if grads is not None else None
    tt = ctypes.c_int64(t)
    losses = np.zeros(max(steps, 1), np.float32)
    logits = np.empty((B, dims[-1]), np.float32)
    preds = np.empty(B, np.int32)
    correct = ctypes.c_int64(0)
    dd, _ = _dims(dims)
    x = np.ascontiguousarray(x, np.float32)
    onehot = np.ascontiguousarray(onehot, np.float32)
    _check(lib().orc_mlp_train(dd, ctypes.c_size_t(L), ctypes.c_size_t(B), pp, mp, vp, ctypes.byref(tt),
                               _fp(x), _fp(onehot), ctypes.byref(opt), ctypes.c_int(steps), _fp(losses), gp,
                               _fp(logits), preds.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                               ctypes.byref(correct)), "mlp_train")
    return dict(params=params, m=m, v=v, t=tt.value, losses=losses[:steps], grads=grads, logits=logits,
                preds=preds, correct=correct.value)


def num_threads() -> int:
    return int(lib().orc_num_threads())
