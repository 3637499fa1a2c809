"""TEST INFRASTRUCTURE: the CPU oracle (orca-backend-cpu restated in C) behind
the same method names as the `Backend` trait, so the tape in
orcaml_amd.autodiff can run on it.  Storages are flat float32 numpy arrays."""
from __future__ import annotations

import sys

import numpy as np

from oracle import oracle as O


def _n(shape) -> int:
    return int(np.prod(shape, dtype=np.int64))


class OracleBackend:
    def device(self) -> str:
        return "cpu"

    def zeros(self, shape, dtype=0):
        return np.zeros(_n(shape), np.float32)

    def from_f32_slice(self, shape, data):
        a = np.array(data, np.float32).reshape(-1)
        assert a.size == _n(shape)
        return a

    def to_f32_vec(self, s):
        return np.array(s, np.float32)

    def matmul(self, a, b, a_shape, b_shape, dtype=0):
        return O.matmul(a.reshape(a_shape), b.reshape(b_shape)).reshape(-1)

    def transpose(self, s, shape, d0, d1, dtype=0):
        return O.transpose(s.reshape(shape), d0, d1).reshape(-1)

    def add(self, a, b, shape, dtype=0):
        return O.add(a, b)

    def sub(self, a, b, shape, dtype=0):
        return O.sub(a, b)

    def mul(self, a, b, shape, dtype=0):
        return O.mul(a, b)

    def div(self, a, b, shape, dtype=0):
        return O.div(a, b)

    def mul_scalar(self, s, scalar, shape, dtype=0):
        return O.mul_scalar(s, scalar)

    def relu(self, s, shape, dtype=0):
        return O.relu(s)

    def sigmoid(self, s, shape, dtype=0):
        return O.sigmoid(s)

    def exp(self, s, shape, dtype=0):
        return O.exp(s)

    def log(self, s, shape, dtype=0):
        return O.log(s)

    def sqrt(self, s, shape, dtype=0):
        return O.sqrt(s)

    def relu_backward(self, g, x, shape, dtype=0):
        return O.relu_backward(g, x)

    def sigmoid_backward(self, g, y, shape, dtype=0):
        return O.sigmoid_backward(g, y)

    def exp_backward(self, g, y, shape, dtype=0):
        return O.exp_backward(g, y)

    def log_backward(self, g, x, shape, dtype=0):
        return O.log_backward(g, x)

    def sqrt_backward(self, g, y, shape, dtype=0):
        return O.sqrt_backward(g, y)

    def div_backward_lhs(self, g, r, shape, dtype=0):
        return O.div_backward_lhs(g, r)

    def div_backward_rhs(self, g, l, r, shape, dtype=0):
        return O.div_backward_rhs(g, l, r)

    def accumulate_grad(self, a, b):
        return O.accumulate_grad(a, b)

    def expand(self, s, in_shape, out_shape, dtype=0):
        return O.expand(s.reshape(in_shape), tuple(out_shape)).reshape(-1)

    def sum_to_shape(self, s, in_shape, out_shape, dtype=0):
        return O.sum_to_shape(s.reshape(in_shape), tuple(out_shape)).reshape(-1)

    def reshape(self, s, in_shape, out_shape, dtype=0):
        if _n(in_shape) != _n(out_shape):
            raise ValueError("Shape mismatch during reshape")
        return s

    def max_to_shape(self, s, in_shape, out_shape, dtype=0):
        return O.max_to_shape(s.reshape(in_shape), tuple(out_shape)).reshape(-1)

    def max_to_shape_backward(self, g, x, y, in_shape, out_shape, dtype=0):
        return O.max_to_shape_backward(g.reshape(out_shape), x.reshape(in_shape), y.reshape(out_shape)).reshape(-1)

    def has_nan_or_inf(self, s, dtype=0):
        return O.has_nan_or_inf(s)

    def to_bytes(self, s):
        return np.ascontiguousarray(s, "<f4").tobytes()

    def from_bytes(self, shape, data, dtype=0):
        a = np.frombuffer(data, "<f4").copy()
        assert a.size == _n(shape)
        return a

    # ---- the fused paths' methods, on the oracle ----
    def clone(self, s):
        return np.array(s, np.float32, copy=True)

    def softmax_ce(self, logits, onehot, B, C, want_grad=True):
        loss, d = O.cross_entropy(logits.reshape(B, C), onehot.reshape(B, C))
        return np.array([loss], np.float32), (d.reshape(-1) if want_grad else None)

    def adamw_step_(self, p, g, m, v, n, lr, beta1, beta2, eps, weight_decay, t):
        p2, m2, v2 = O.adamw_update(p, g, m, v, t, lr=lr, weight_decay=weight_decay, betas=(beta1, beta2), eps=eps)
        p[:], m[:], v[:] = p2, m2, v2

    def sgd_step_(self, p, g, n, lr):
        p[:] = O.sgd_update(p, g, lr)

    # flat arenas (numpy views of one array) and the one-pass optimizers over them
    def arena(self, n, fill=None):
        return np.full(max(n, 1), 0.0 if fill is None else fill, np.float32)

    @staticmethod
    def view(arena, offset, n):
        return arena[offset:offset + n]

    def copy_into(self, dst, src):
        dst[:] = src

    def arena_exclusive(self, arena):
        # every numpy view (and array derived from one) holds its base array: the caller's
        # reference, the call's argument slot, this parameter and getrefcount's own argument
        # are the only ones when none is alive (CPython 3.10)
        return sys.getrefcount(arena) <= 4

    def adamw_multi_(self, segs, lr, beta1, beta2, eps, weight_decay, t):
        for ps, pd, g, m, v, n in segs:
            p2, m2, v2 = O.adamw_update(ps, g, m, v, t, lr=lr, weight_decay=weight_decay, betas=(beta1, beta2),
                                        eps=eps)
            pd[:], m[:], v[:] = p2, m2, v2

    def sgd_multi_(self, segs, lr):
        for ps, pd, g, n in segs:
            pd[:] = O.sgd_update(ps, g, lr)
