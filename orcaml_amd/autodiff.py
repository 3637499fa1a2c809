"""The reference's autograd tape and frontend op sequence, replayed on any
backend that has the `Backend` trait's methods (HipBackend, or the CPU
oracle backend of the tests).

The reference's `Autodiff<B>` decorator, tape and tensor layer are the
unchanged callers of a drop-in backend; there is no Rust toolchain here, so
this module restates them for the ops of the MLP hot path, op for op, to drive
the HIP backend exactly as they would:

* Tape / Autodiff -- orca-autograd/src/tape.rs:6-128 (ids from a counter,
  reverse walk over every node, gradients summed with accumulate_grad in
  arrival order) and orca-autograd/src/backend.rs (which op records which
  backward node, and the backward rules of lines 1379-1793);
* Tensor -- orca-tensor/src/tensor.rs (shape/dtype checks, matmul 267-345) with
  the orca-python dunder semantics (orca-python/src/lib.rs:513-669): binary
  operators expand BOTH operands to the broadcast shape, `x * float` is
  mul_scalar, other float operands become Tensor.scalar, `-x` is x * -1 and
  mean is sum * (1/n as f32);
* nn / optim -- python/orca/nn/{module,linear,activation,container,loss}.py and
  python/orca/optim/{optimizer,sgd,adamw}.py for the layers used by the MLP.
"""
from __future__ import annotations

import contextlib
import math
from typing import Iterable

import numpy as np

F32 = 0


class OrcaError(ValueError):
    """orca_core::OrcaError as orca-python raises it (ValueError)."""


# ============================================================ tape
class Tape:
    """orca-autograd/src/tape.rs:61-128."""

    def __init__(self):
        self.nodes = []
        self.next_id = 0
        self.grads = {}

    def generate_id(self) -> int:
        i = self.next_id
        self.next_id += 1
        return i

    def push_node(self, node) -> None:
        self.nodes.append(node)

    def clear(self) -> None:
        self.grads.clear()
        self.nodes.clear()

    def accumulate(self, node_id, grad, backend) -> None:
        """Gradients::accumulate (tape.rs:34-47)."""
        if node_id in self.grads:
            self.grads[node_id] = backend.accumulate_grad(self.grads[node_id], grad)
        else:
            self.grads[node_id] = grad

    def execute_backward(self, root_id, root_grad, backend) -> None:
        """tape.rs:107-118."""
        self.grads[root_id] = root_grad
        for node in reversed(self.nodes):
            node(self, backend)


class AdStorage:
    """AutodiffStorage (orca-autograd/src/backend.rs:9-13)."""

    __slots__ = ("primal", "node_id")

    def __init__(self, primal, node_id=None):
        self.primal = primal
        self.node_id = node_id


class Autodiff:
    """The backend decorator (orca-autograd/src/backend.rs:22-45)."""

    def __init__(self, inner):
        self.inner = inner
        self.tape = Tape()
        self.grad_enabled = True  # orca-autograd/src/lib.rs:5-20

    # --- recording helper: generate an id whenever grad is enabled, push the
    # node only if an input has a node id (e.g. backend.rs:83-117) ---
    def _record(self, primal, inputs, make_node):
        if not self.grad_enabled:
            return AdStorage(primal)
        out_id = self.tape.generate_id()
        for s in inputs:
            if s.node_id is not None:
                self.tape.push_node(make_node(out_id))
                return AdStorage(primal, out_id)
        return AdStorage(primal)

    # --- a node with its own backward.  The reference's tape knows a fixed set
    # of BackwardOp types; a fused op (one kernel for what is several ops)
    # needs one more kind of node, recorded the same way ---
    def custom(self, primal, inputs, backward):
        """Records `primal` as the output of one node over `inputs`;
        backward(g, backend) returns one gradient storage (or None) per input,
        accumulated like any other node's."""

        def node(out_id, ids=tuple(s.node_id for s in inputs)):
            def run(tape, be):
                g = tape.grads.get(out_id)
                if g is None:
                    return
                for i, gi in zip(ids, backward(g, be)):
                    if i is not None and gi is not None:
                        tape.accumulate(i, gi, be)
            return run
        return self._record(primal, inputs, node)

    def add(self, a, b, shape):
        primal = self.inner.add(a.primal, b.primal, shape)

        def node(out_id, l=a.node_id, r=b.node_id):
            def backward(tape, be):  # AddBackward (backend.rs:1387-1401)
                g = tape.grads.get(out_id)
                if g is None:
                    return
                if l is not None:
                    tape.accumulate(l, g, be)
                if r is not None:
                    tape.accumulate(r, g, be)
            return backward
        return self._record(primal, (a, b), node)

    def sub(self, a, b, shape):
        primal = self.inner.sub(a.primal, b.primal, shape)

        def node(out_id, l=a.node_id, r=b.node_id):
            def backward(tape, be):  # SubBackward (backend.rs:1542-1561)
                g = tape.grads.get(out_id)
                if g is None:
                    return
                if l is not None:
                    tape.accumulate(l, g, be)
                if r is not None:
                    tape.accumulate(r, be.mul_scalar(g, -1.0, shape), be)
            return backward
        return self._record(primal, (a, b), node)

    def mul(self, a, b, shape):
        primal = self.inner.mul(a.primal, b.primal, shape)

        def node(out_id, l=a.node_id, r=b.node_id, lp=a.primal, rp=b.primal):
            def backward(tape, be):  # MulBackward (backend.rs:1601-1620)
                g = tape.grads.get(out_id)
                if g is None:
                    return
                if l is not None:
                    tape.accumulate(l, be.mul(g, rp, shape), be)
                if r is not None:
                    tape.accumulate(r, be.mul(g, lp, shape), be)
            return backward
        return self._record(primal, (a, b), node)

    def div(self, a, b, shape):
        primal = self.inner.div(a.primal, b.primal, shape)

        def node(out_id, l=a.node_id, r=b.node_id, lp=a.primal, rp=b.primal):
            def backward(tape, be):  # DivBackward (backend.rs:1807-1833)
                g = tape.grads.get(out_id)
                if g is None:
                    return
                if l is not None:
                    tape.accumulate(l, be.div_backward_lhs(g, rp, shape), be)
                if r is not None:
                    tape.accumulate(r, be.div_backward_rhs(g, lp, rp, shape), be)
            return backward
        return self._record(primal, (a, b), node)

    def mul_scalar(self, a, scalar, shape):
        scalar = float(np.float32(scalar))
        primal = self.inner.mul_scalar(a.primal, scalar, shape)

        def node(out_id, i=a.node_id):
            def backward(tape, be):  # MulScalarBackward (backend.rs:1574-1586)
                g = tape.grads.get(out_id)
                if g is None:
                    return
                tape.accumulate(i, be.mul_scalar(g, scalar, shape), be)
            return backward
        return self._record(primal, (a,), node)

    def matmul(self, a, b, a_shape, b_shape):
        primal = self.inner.matmul(a.primal, b.primal, a_shape, b_shape)

        def node(out_id, l=a.node_id, r=b.node_id, lp=a.primal, rp=b.primal):
            def backward(tape, be):  # MatMulBackward (backend.rs:1448-1499)
                g = tape.grads.get(out_id)
                if g is None:
                    return
                out_shape = list(a_shape)
                out_shape[-1] = b_shape[-1]
                if l is not None:  # grad_x = grad_z @ y^T
                    rk = len(b_shape)
                    rt = be.transpose(rp, b_shape, rk - 2, rk - 1)
                    rt_shape = list(b_shape)
                    rt_shape[-2], rt_shape[-1] = rt_shape[-1], rt_shape[-2]
                    tape.accumulate(l, be.matmul(g, rt, out_shape, rt_shape), be)
                if r is not None:  # grad_y = x^T @ grad_z
                    lk = len(a_shape)
                    lt = be.transpose(lp, a_shape, lk - 2, lk - 1)
                    lt_shape = list(a_shape)
                    lt_shape[-2], lt_shape[-1] = lt_shape[-1], lt_shape[-2]
                    tape.accumulate(r, be.matmul(lt, g, lt_shape, out_shape), be)
            return backward
        return self._record(primal, (a, b), node)

    def transpose(self, a, shape, d0, d1):
        primal = self.inner.transpose(a.primal, shape, d0, d1)

        def node(out_id, i=a.node_id):
            def backward(tape, be):  # TransposeBackward (backend.rs:1514-1529)
                g = tape.grads.get(out_id)
                if g is None:
                    return
                out_shape = list(shape)
                out_shape[d0], out_shape[d1] = out_shape[d1], out_shape[d0]
                tape.accumulate(i, be.transpose(g, out_shape, d0, d1), be)
            return backward
        return self._record(primal, (a,), node)

    def _unary(self, name, bw_name, a, shape, keep):
        primal = getattr(self.inner, name)(a.primal, shape)

        def node(out_id, i=a.node_id, saved=(primal if keep == "out" else a.primal)):
            def backward(tape, be):
                g = tape.grads.get(out_id)
                if g is None:
                    return
                tape.accumulate(i, getattr(be, bw_name)(g, saved, shape), be)
            return backward
        return self._record(primal, (a,), node)

    def relu(self, a, shape):  # ReluBackward keeps the input (backend.rs:1633-1645)
        return self._unary("relu", "relu_backward", a, shape, "in")

    def sigmoid(self, a, shape):  # SigmoidBackward keeps the output (1658-1671)
        return self._unary("sigmoid", "sigmoid_backward", a, shape, "out")

    def exp(self, a, shape):  # ExpBackwardOp keeps the output (1759-1769)
        return self._unary("exp", "exp_backward", a, shape, "out")

    def log(self, a, shape):  # LogBackwardOp keeps the input (1782-1792)
        return self._unary("log", "log_backward", a, shape, "in")

    def sqrt(self, a, shape):  # SqrtBackwardOp keeps the output (1846-1857)
        return self._unary("sqrt", "sqrt_backward", a, shape, "out")

    def expand(self, a, in_shape, out_shape):
        primal = self.inner.expand(a.primal, in_shape, out_shape)

        def node(out_id, i=a.node_id):
            def backward(tape, be):  # ExpandBackward (backend.rs:1684-1697)
                g = tape.grads.get(out_id)
                if g is None:
                    return
                tape.accumulate(i, be.sum_to_shape(g, out_shape, in_shape), be)
            return backward
        return self._record(primal, (a,), node)

    def sum_to_shape(self, a, in_shape, out_shape):
        primal = self.inner.sum_to_shape(a.primal, in_shape, out_shape)

        def node(out_id, i=a.node_id):
            def backward(tape, be):  # SumToShapeBackward (backend.rs:1710-1722)
                g = tape.grads.get(out_id)
                if g is None:
                    return
                tape.accumulate(i, be.expand(g, out_shape, in_shape), be)
            return backward
        return self._record(primal, (a,), node)

    def reshape(self, a, in_shape, out_shape):
        primal = self.inner.reshape(a.primal, in_shape, out_shape)

        def node(out_id, i=a.node_id):
            def backward(tape, be):  # ReshapeBackward (backend.rs:1735-1746)
                g = tape.grads.get(out_id)
                if g is None:
                    return
                tape.accumulate(i, be.reshape(g, out_shape, in_shape), be)
            return backward
        return self._record(primal, (a,), node)

    def max_to_shape(self, a, in_shape, out_shape):
        primal = self.inner.max_to_shape(a.primal, in_shape, out_shape)

        def node(out_id, i=a.node_id, xp=a.primal, yp=primal):
            def backward(tape, be):  # MaxToShapeBackward (backend.rs:1416-1432)
                g = tape.grads.get(out_id)
                if g is None:
                    return
                tape.accumulate(i, be.max_to_shape_backward(g, xp, yp, in_shape, out_shape), be)
            return backward
        return self._record(primal, (a,), node)


# ============================================================ tensor
def broadcast_shape(a, b):
    """Shape::broadcast (orca-core/src/shape.rs:26-51)."""
    out = []
    i, j = len(a) - 1, len(b) - 1
    while i >= 0 or j >= 0:
        d1 = a[i] if i >= 0 else 1
        d2 = b[j] if j >= 0 else 1
        if d1 == d2 or d2 == 1:
            out.append(d1)
        elif d1 == 1:
            out.append(d2)
        else:
            return None
        i -= 1
        j -= 1
    return tuple(reversed(out))


class Tensor:
    """Tensor<Autodiff<B>> with the orca-python method surface used by the MLP path."""

    def __init__(self, ad: Autodiff, storage: AdStorage, shape):
        self.ad = ad
        self.storage = storage
        self.shape = shape if type(shape) is tuple else tuple(int(d) for d in shape)
        self.dtype = F32

    # ---- construction / host I/O ----
    @classmethod
    def from_numpy(cls, ad: Autodiff, arr, requires_grad: bool = False) -> "Tensor":
        arr = np.ascontiguousarray(arr, np.float32)
        shape = arr.shape if arr.ndim else (1,)
        t = cls(ad, AdStorage(ad.inner.from_f32_slice(shape, arr.reshape(-1))), shape)
        if requires_grad:
            t.require_grad()
        return t

    @classmethod
    def scalar(cls, ad: Autodiff, value: float) -> "Tensor":
        """Tensor::scalar (orca-tensor/src/tensor.rs:46-49): shape [1]."""
        return cls.from_numpy(ad, np.array([np.float32(value)], np.float32))

    @classmethod
    def zeros(cls, ad: Autodiff, shape, requires_grad: bool = False) -> "Tensor":
        t = cls(ad, AdStorage(ad.inner.zeros(tuple(shape))), shape)
        if requires_grad:
            t.require_grad()
        return t

    def numpy(self) -> np.ndarray:
        return np.asarray(self.ad.inner.to_f32_vec(self.storage.primal)).reshape(self.shape)

    def to_list(self):
        return [float(v) for v in self.numpy().reshape(-1)]

    @property
    def requires_grad(self) -> bool:
        return self.storage.node_id is not None

    # ---- autograd (orca-autograd/src/tensor.rs:36-140) ----
    def require_grad(self) -> None:
        self.storage = AdStorage(self.storage.primal, self.ad.tape.generate_id())

    def backward(self) -> None:
        if self.storage.node_id is None:
            raise OrcaError("Internal error: Cannot call backward on a tensor that doesn't require gradients")
        n = int(np.prod(self.shape))
        seed = self.ad.inner.from_f32_slice(self.shape, np.ones(n, np.float32))
        self.ad.tape.execute_backward(self.storage.node_id, seed, self.ad.inner)

    def grad(self):
        if self.storage.node_id is None:
            return None
        g = self.ad.tape.grads.get(self.storage.node_id)
        if g is None:
            return None
        return Tensor(self.ad, AdStorage(g), self.shape)

    def detach(self) -> "Tensor":
        return Tensor(self.ad, AdStorage(self.storage.primal), self.shape)

    # ---- ops ----
    def _check_same(self, other: "Tensor", op: str) -> None:
        if self.shape != other.shape:
            raise OrcaError(f"Shape mismatch during {op}: expected {list(self.shape)}, got {list(other.shape)}")
        if self.ad is not other.ad:
            raise OrcaError("Device mismatch: tensors must be on the same device")

    def _bin(self, other: "Tensor", op: str) -> "Tensor":
        self._check_same(other, op)
        return Tensor(self.ad, getattr(self.ad, op)(self.storage, other.storage, self.shape), self.shape)

    def expand(self, shape) -> "Tensor":
        shape = tuple(shape)
        return Tensor(self.ad, self.ad.expand(self.storage, self.shape, shape), shape)

    def sum_to_shape(self, shape) -> "Tensor":
        shape = tuple(shape)
        return Tensor(self.ad, self.ad.sum_to_shape(self.storage, self.shape, shape), shape)

    def max_to_shape(self, shape) -> "Tensor":
        shape = tuple(shape)
        return Tensor(self.ad, self.ad.max_to_shape(self.storage, self.shape, shape), shape)

    def reshape(self, shape) -> "Tensor":
        shape = tuple(shape)
        return Tensor(self.ad, self.ad.reshape(self.storage, self.shape, shape), shape)

    def transpose(self, d0: int, d1: int) -> "Tensor":
        shape = list(self.shape)
        shape[d0], shape[d1] = shape[d1], shape[d0]
        return Tensor(self.ad, self.ad.transpose(self.storage, self.shape, d0, d1), shape)

    def sum(self) -> "Tensor":
        return self.sum_to_shape((1,))

    def mean(self) -> "Tensor":
        n = int(np.prod(self.shape))
        return self.sum().mul_scalar(np.float32(1.0) / np.float32(n))

    def mul_scalar(self, s) -> "Tensor":
        return Tensor(self.ad, self.ad.mul_scalar(self.storage, s, self.shape), self.shape)

    def relu(self) -> "Tensor":
        return Tensor(self.ad, self.ad.relu(self.storage, self.shape), self.shape)

    def sigmoid(self) -> "Tensor":
        return Tensor(self.ad, self.ad.sigmoid(self.storage, self.shape), self.shape)

    def exp(self) -> "Tensor":
        return Tensor(self.ad, self.ad.exp(self.storage, self.shape), self.shape)

    def log(self) -> "Tensor":
        return Tensor(self.ad, self.ad.log(self.storage, self.shape), self.shape)

    def sqrt(self) -> "Tensor":
        return Tensor(self.ad, self.ad.sqrt(self.storage, self.shape), self.shape)

    def matmul(self, other: "Tensor") -> "Tensor":
        """orca-tensor/src/tensor.rs:267-345."""
        r1, r2 = len(self.shape), len(other.shape)
        if r1 < 2 or r2 < 2:
            raise OrcaError(f"Shape mismatch during matmul: expected >= 2D tensors, got {r1}D and {r2}D")
        if self.shape[-1] != other.shape[-2]:
            raise OrcaError(f"Shape mismatch during matmul: expected Inner dimensions must match: "
                            f"{self.shape[-1]} == {other.shape[-2]}")
        if r1 != r2:
            raise OrcaError("Shape mismatch during matmul: expected Same rank for batched matmul")
        if self.shape[:-2] != other.shape[:-2]:
            raise OrcaError("Shape mismatch during matmul: expected Matching batch dimensions")
        if self.ad is not other.ad:
            raise OrcaError("Device mismatch: tensors must be on the same device")
        out_shape = self.shape[:-1] + (other.shape[-1],)
        return Tensor(self.ad, self.ad.matmul(self.storage, other.storage, self.shape, other.shape), out_shape)

    __matmul__ = matmul

    # ---- PyO3 dunders (orca-python/src/lib.rs:513-669) ----
    def _resolve(self, other) -> "Tensor":
        if isinstance(other, Tensor):
            return other
        return Tensor.scalar(self.ad, float(other))

    def _broadcast_pair(self, other: "Tensor"):
        shape = broadcast_shape(self.shape, other.shape)
        if shape is None:
            raise OrcaError("Shapes are not broadcastable")
        return self.expand(shape), other.expand(shape)

    def __add__(self, other):
        a, b = self._broadcast_pair(self._resolve(other))
        return a._bin(b, "add")

    __radd__ = __add__

    def __sub__(self, other):
        a, b = self._broadcast_pair(self._resolve(other))
        return a._bin(b, "sub")

    def __rsub__(self, other):
        a, b = self._resolve(other)._broadcast_pair(self)
        return a._bin(b, "sub")

    def __mul__(self, other):
        if not isinstance(other, Tensor):
            return self.mul_scalar(float(other))
        a, b = self._broadcast_pair(other)
        return a._bin(b, "mul")

    __rmul__ = __mul__

    def __truediv__(self, other):
        a, b = self._broadcast_pair(self._resolve(other))
        return a._bin(b, "div")

    def __neg__(self):
        return self.mul_scalar(-1.0)


@contextlib.contextmanager
def no_grad(ad: Autodiff):
    """orca.no_grad (python/orca/__init__.py:22-37)."""
    prev = ad.grad_enabled
    ad.grad_enabled = False
    try:
        yield
    finally:
        ad.grad_enabled = prev


# ============================================================ nn
class Parameter:
    """python/orca/nn/parameter.py:5-41."""

    def __init__(self, tensor: Tensor):
        self.tensor = tensor

    def update(self, new_tensor: Tensor) -> None:
        self.tensor = new_tensor


class Module:
    """Parameter order: own parameters, then submodules in insertion order
    (python/orca/nn/module.py:32-44)."""

    def __init__(self):
        object.__setattr__(self, "_parameters", {})
        object.__setattr__(self, "_modules", {})

    def __setattr__(self, name, value):
        if isinstance(value, Parameter):
            self._parameters[name] = value
        elif isinstance(value, Module):
            self._modules[name] = value
        object.__setattr__(self, name, value)

    def parameters(self):
        for p in self._parameters.values():
            yield p
        for m in self._modules.values():
            yield from m.parameters()

    def named_parameters(self, prefix: str = ""):
        """(name, Parameter) with the names save_weights writes: own parameters,
        then each submodule's under "<submodule>." (python/orca/nn/module.py:176-184)."""
        for n, p in self._parameters.items():
            yield prefix + n, p
        for n, m in self._modules.items():
            yield from m.named_parameters(prefix + n + ".")

    def state_dict(self) -> dict:
        return {n: p.tensor for n, p in self.named_parameters()}

    def save_weights(self, filepath: str) -> None:
        """python/orca/nn/module.py:169-187: the parameters as a safetensors file."""
        from .serialize import save_tensors
        save_tensors(filepath, self.state_dict())

    def load_weights(self, filepath: str) -> None:
        """python/orca/nn/module.py:189-218: every parameter named in the file
        is replaced by the file's tensor (others are left alone), which
        requires grad if the parameter did."""
        from .serialize import load_tensors
        params = list(self.named_parameters())
        if not params:
            return
        state = load_tensors(filepath, params[0][1].tensor.ad)
        for n, p in params:
            if n in state:
                t = state[n]
                if p.tensor.requires_grad:
                    t.require_grad()
                p.tensor = t

    def __call__(self, *args):
        return self.forward(*args)


class Linear(Module):
    """python/orca/nn/linear.py:7-86: weight [in, out], bias [1, out],
    forward x @ W + bias.expand(out.shape).  Weights are given explicitly (the
    reference's init RNG is unseeded)."""

    def __init__(self, ad: Autodiff, weight: np.ndarray, bias: np.ndarray | None):
        super().__init__()
        self.in_features, self.out_features = weight.shape
        self.weight = Parameter(Tensor.from_numpy(ad, weight, requires_grad=True))
        self.bias = Parameter(Tensor.from_numpy(ad, np.asarray(bias, np.float32).reshape(1, -1),
                                                requires_grad=True)) if bias is not None else None

    def forward(self, x: Tensor) -> Tensor:
        shape = x.shape
        x_flat = x.reshape((int(np.prod(shape[:-1])), self.in_features)) if len(shape) > 2 else x
        out = x_flat @ self.weight.tensor
        if self.bias is not None:
            b = self.bias.tensor.expand(out.shape)
            out = out + b
        if len(shape) > 2:
            out = out.reshape(tuple(shape[:-1]) + (self.out_features,))
        return out


class ReLU(Module):
    """python/orca/nn/activation.py:5-21."""

    def forward(self, x: Tensor) -> Tensor:
        return x.relu()


class Sequential(Module):
    """python/orca/nn/container.py:1-17."""

    def __init__(self, *layers):
        super().__init__()
        for i, layer in enumerate(layers):
            setattr(self, str(i), layer)

    def forward(self, x):
        for m in self._modules.values():
            x = m(x)
        return x


class CrossEntropyLoss(Module):
    """python/orca/nn/loss.py:42-100 (one-hot targets).

    fused=True (opt-in): when the backend has a fused softmax cross-entropy
    (HipBackend.softmax_ce), a 2-D prediction with reduction "mean" takes one
    kernel for the loss and dL/dpred, recorded as one tape node whose backward
    scales the saved gradient by the incoming one.  The gradient is the
    composed tape's to rounding (the row sums run in a different order); with
    the usual seed of 1 it is passed on unchanged."""

    def __init__(self, reduction: str = "mean", fused: bool = False):
        super().__init__()
        if reduction not in ("mean", "sum", "none"):
            raise ValueError(f"Invalid reduction mode: {reduction}")
        self.reduction = reduction
        self.fused = fused

    def forward(self, pred: Tensor, target: Tensor) -> Tensor:
        if (self.fused and self.reduction == "mean" and len(pred.shape) == 2
                and hasattr(pred.ad.inner, "softmax_ce")):
            return _fused_cross_entropy(pred, target)
        batch = pred.shape[0]
        max_pred_base = pred.max_to_shape([batch, 1])
        max_pred = max_pred_base.expand(list(pred.shape))
        shifted_pred = pred - max_pred
        exp_pred = shifted_pred.exp()
        sum_exp_base = exp_pred.sum_to_shape([batch, 1])
        sum_exp = sum_exp_base.expand(list(pred.shape))
        log_sum_exp = max_pred + sum_exp.log()
        log_softmax = pred - log_sum_exp
        loss_matrix = -(target * log_softmax)
        per_batch_loss = loss_matrix.sum_to_shape([batch, 1])
        if self.reduction == "mean":
            return per_batch_loss.mean()
        if self.reduction == "sum":
            return per_batch_loss.sum()
        return per_batch_loss


def _fused_cross_entropy(pred: Tensor, target: Tensor) -> Tensor:
    if pred.shape != target.shape:
        raise OrcaError(f"Shape mismatch during cross_entropy: expected {list(pred.shape)}, got {list(target.shape)}")
    if pred.ad is not target.ad:
        raise OrcaError("Device mismatch: tensors must be on the same device")
    ad, (B, C) = pred.ad, pred.shape
    want_grad = ad.grad_enabled and pred.storage.node_id is not None
    loss, dpred = ad.inner.softmax_ce(pred.storage.primal, target.storage.primal, B, C, want_grad)

    def backward(g, be):  # g: the gradient of the loss, shape [1]
        return be.mul(be.expand(g, (1,), (B, C)), dpred, (B, C)), None
    return Tensor(ad, ad.custom(loss, (pred.storage, target.storage), backward), (1,))


class MSELoss(Module):
    """python/orca/nn/loss.py:4-40."""

    def __init__(self, reduction: str = "mean"):
        super().__init__()
        self.reduction = reduction

    def forward(self, pred: Tensor, target: Tensor) -> Tensor:
        diff = pred - target
        sq = diff * diff
        if self.reduction == "mean":
            return sq.mean()
        if self.reduction == "sum":
            return sq.sum()
        return sq


# ============================================================ optim
class Optimizer:
    """python/orca/optim/optimizer.py: zero_grad clears the whole tape (95-102)."""

    def __init__(self, parameters: Iterable[Parameter]):
        self.parameters = list(parameters)
        if not self.parameters:
            raise ValueError("optimizer got an empty parameter list")
        for p in self.parameters:
            if not isinstance(p, Parameter):
                raise TypeError("optimizer parameters must be Parameter instances")

    def zero_grad(self) -> None:
        self.parameters[0].tensor.ad.tape.clear()


class _FlatParams:
    """The parameters of a fused optimizer in flat device arenas, each parameter's storage a
    view of its slice, so one launch updates all of them (orca_hip_adamw_multi /
    orca_hip_sgd_multi).

    Every step reads the arena that holds the parameters and writes the other, and the
    parameters are then rebound to views of the written one: a storage of the previous
    values (a forward's tape, a pending op, the caller) keeps them unchanged, as the
    reference's functional update does.  The arena written is the one from two steps back
    only when no view of it is still referenced; otherwise a fresh arena is taken.  The
    moments live in two more arenas, updated in place (they belong to the optimizer)."""

    ALIGN = 64  # floats: 256-byte aligned slices

    def __init__(self, ad: "Autodiff", params, moments: bool):
        self.ad, self.be = ad, ad.inner
        self.params = params
        self.sizes = [_numel(p.tensor.shape) for p in params]
        self.offs, total = [], 0
        for n in self.sizes:
            self.offs.append(total)
            total += -(-n // self.ALIGN) * self.ALIGN
        self.total = total
        self.cur = self.be.arena(total)
        self.spare = None
        # The parameters move into the arena with their values: each tensor keeps its
        # identity and node id (a gradient already recorded for it stays attached); only
        # its storage becomes the arena slice.
        for p, off, n in zip(params, self.offs, self.sizes):
            view = self.be.view(self.cur, off, n)
            self.be.copy_into(view, p.tensor.storage.primal)
            p.tensor.storage.primal = view
        self.m = self.v = None
        if moments:
            self.m, self.v = self.be.arena(total, 0.0), self.be.arena(total, 0.0)

    def moment(self, which: str, i: int):
        return self.be.view(self.m if which == "m" else self.v, self.offs[i], self.sizes[i])

    def step(self, run) -> None:
        """run(segments) launches the update; segments are (i, p_src, p_dst, g) of the
        parameters with a gradient.  Parameters without one are copied across."""
        # Every view (and every storage derived from one: a lazy transpose, a pending op's
        # operand) holds the arena's memory, so an arena nothing else refers to has no
        # reader left (the backend tracks those references).
        if self.spare is not None and self.be.arena_exclusive(self.spare):
            dst = self.spare
        else:
            dst = self.be.arena(self.total)
        self.spare = None
        segs, rebind = [], []
        for i, p in enumerate(self.params):
            src = p.tensor.storage.primal
            view = self.be.view(dst, self.offs[i], self.sizes[i])
            g = p.tensor.grad() if p.tensor.requires_grad else None
            if g is None:
                self.be.copy_into(view, src)
            else:
                segs.append((i, src, view, g.storage.primal))
            rebind.append((p, view))
        if segs:
            run(segs)
        for p, view in rebind:
            p.update(_new_leaf(self.ad, view, p.tensor.shape))
        self.spare, self.cur = self.cur, dst


class SGD(Optimizer):
    """python/orca/optim/sgd.py:10-79.

    fused=True (opt-in): with momentum = weight_decay = 0, the update
    p - g * f32(lr) of all parameters is one launch over flat parameter
    arenas (_FlatParams) on a backend that has them, else one kernel per
    parameter on a copy of p; either way the old tensor is left as it was,
    as the composed update leaves it, with the same f32 operations, so the
    same bits."""

    def __init__(self, parameters, lr=0.01, momentum=0.0, weight_decay=0.0, dampening=0.0, fused: bool = False):
        super().__init__(parameters)
        self.lr, self.momentum, self.weight_decay, self.dampening = lr, momentum, weight_decay, dampening
        self.fused = fused
        self._velocity = [None] * len(self.parameters)
        ad = self.parameters[0].tensor.ad
        self._flat = None
        if fused and momentum == 0.0 and weight_decay == 0.0 and hasattr(ad.inner, "sgd_multi_"):
            self._flat = _FlatParams(ad, self.parameters, moments=False)

    def step(self) -> None:
        ad = self.parameters[0].tensor.ad
        if self._flat is not None:
            n = self._flat.sizes
            self._flat.step(lambda segs: ad.inner.sgd_multi_([(ps, pd, g, n[i]) for i, ps, pd, g in segs], self.lr))
            return
        if (self.fused and self.momentum == 0.0 and self.weight_decay == 0.0
                and hasattr(ad.inner, "sgd_step_")):
            for p in self.parameters:
                grad = p.tensor.grad()
                if grad is None:
                    continue
                new = ad.inner.clone(p.tensor.storage.primal)
                ad.inner.sgd_step_(new, grad.storage.primal, _numel(p.tensor.shape), self.lr)
                p.update(_new_leaf(ad, new, p.tensor.shape))
            return
        with no_grad(ad):
            for i, p in enumerate(self.parameters):
                grad = p.tensor.grad()
                if grad is None:
                    continue
                if self.weight_decay != 0.0:
                    grad = grad + p.tensor * self.weight_decay
                if self.momentum != 0.0:
                    if self._velocity[i] is None:
                        self._velocity[i] = grad.detach()
                    elif self.dampening != 0.0:
                        self._velocity[i] = self._velocity[i] * self.momentum + grad * (1.0 - self.dampening)
                    else:
                        self._velocity[i] = self._velocity[i] * self.momentum + grad
                    grad = self._velocity[i]
                update = grad * self.lr
                new_tensor = p.tensor - update
                new_leaf = new_tensor.detach()
                new_leaf.require_grad()
                p.update(new_leaf)


class AdamW(Optimizer):
    """python/orca/optim/adamw.py:12-99.

    fused=True (opt-in): the update of all parameters is one launch over flat
    parameter and moment arenas (_FlatParams) on a backend that has them,
    else one kernel per parameter on a copy of p; the same f32 operations in
    the same order, so the same bits.  m and v are updated in place (they
    belong to the optimizer alone).

    state_dict / load_state_dict carry m, v and t, which the reference does
    not save."""

    def __init__(self, parameters, lr=0.001, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, fused: bool = False):
        super().__init__(parameters)
        self.lr, (self.beta1, self.beta2), self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self.fused = fused
        self.t = 0
        ad = self.parameters[0].tensor.ad
        self._flat = None
        if fused and hasattr(ad.inner, "adamw_multi_"):
            self._flat = _FlatParams(ad, self.parameters, moments=True)
            self.m = [Tensor(ad, AdStorage(self._flat.moment("m", i)), p.tensor.shape)
                      for i, p in enumerate(self.parameters)]
            self.v = [Tensor(ad, AdStorage(self._flat.moment("v", i)), p.tensor.shape)
                      for i, p in enumerate(self.parameters)]
            return
        self.m = [Tensor.zeros(p.tensor.ad, p.tensor.shape) for p in self.parameters]
        self.v = [Tensor.zeros(p.tensor.ad, p.tensor.shape) for p in self.parameters]

    def state_dict(self) -> dict:
        """{"m.<i>": Tensor, "v.<i>": Tensor, "t": int} for parameter i in optimizer order.
        With fused=True the moments are updated in place by later steps, so the
        returned tensors are copies: a snapshot stays what it was when taken."""
        out = {"t": self.t}
        for i in range(len(self.parameters)):
            m, v = self.m[i], self.v[i]
            if self.fused and hasattr(m.ad.inner, "clone"):
                m = Tensor(m.ad, AdStorage(m.ad.inner.clone(m.storage.primal)), m.shape)
                v = Tensor(v.ad, AdStorage(v.ad.inner.clone(v.storage.primal)), v.shape)
            out[f"m.{i}"], out[f"v.{i}"] = m, v
        return out

    def load_state_dict(self, state: dict) -> None:
        n = len(self.parameters)
        for i in range(n):
            for key, slots in ((f"m.{i}", self.m), (f"v.{i}", self.v)):
                t = state[key]
                if tuple(t.shape) != tuple(self.parameters[i].tensor.shape):
                    raise OrcaError(f"Shape mismatch during load_state_dict: {key} expected "
                                    f"{list(self.parameters[i].tensor.shape)}, got {list(t.shape)}")
                if self._flat is not None:  # into the moment arena's slice
                    t.ad.inner.copy_into(slots[i].storage.primal, t.storage.primal)
                else:  # a private copy: the fused step updates moments in place
                    slots[i] = Tensor(t.ad, AdStorage(t.ad.inner.clone(t.storage.primal)), t.shape)
        self.t = int(state["t"])

    def step(self) -> None:
        grads = []
        for i, p in enumerate(self.parameters):
            if not p.tensor.requires_grad:
                continue
            g = p.tensor.grad()
            if g is not None:
                grads.append((i, p, g))
        if not grads:
            return
        self.t += 1
        ad = self.parameters[0].tensor.ad
        if self._flat is not None:
            flat = self._flat
            active = {i for i, _, _ in grads}

            def run(segs):
                ad.inner.adamw_multi_([(ps, pd, g, self.m[i].storage.primal, self.v[i].storage.primal, flat.sizes[i])
                                       for i, ps, pd, g in segs if i in active],
                                      self.lr, self.beta1, self.beta2, self.eps, self.weight_decay, self.t)

            flat.step(run)
            return
        if self.fused and hasattr(ad.inner, "adamw_step_"):
            for i, p, grad in grads:
                new = ad.inner.clone(p.tensor.storage.primal)
                ad.inner.adamw_step_(new, grad.storage.primal, self.m[i].storage.primal, self.v[i].storage.primal,
                                     _numel(p.tensor.shape), self.lr, self.beta1, self.beta2, self.eps,
                                     self.weight_decay, self.t)
                p.update(_new_leaf(ad, new, p.tensor.shape))
            return
        with no_grad(ad):
            for i, p, grad in grads:
                decayed = p.tensor * (1.0 - self.lr * self.weight_decay)
                m_new = self.m[i] * self.beta1 + grad * (1.0 - self.beta1)
                v_new = self.v[i] * self.beta2 + (grad * grad) * (1.0 - self.beta2)
                self.m[i] = m_new
                self.v[i] = v_new
                m_hat = m_new * (1.0 / (1.0 - self.beta1 ** self.t))
                v_hat = v_new * (1.0 / (1.0 - self.beta2 ** self.t))
                eps_tensor = Tensor.scalar(ad, self.eps).expand(v_hat.shape)
                denom = v_hat.sqrt() + eps_tensor
                update = (m_hat / denom) * self.lr
                new_tensor = decayed - update
                new_leaf = new_tensor.detach()
                new_leaf.require_grad()
                p.update(new_leaf)


def _numel(shape) -> int:
    return int(np.prod(shape, dtype=np.int64))


def _new_leaf(ad: Autodiff, storage, shape) -> Tensor:
    """detach() + require_grad() of an updated parameter (sgd.py:76-79, adamw.py:95-99)."""
    t = Tensor(ad, AdStorage(storage), shape)
    t.require_grad()
    return t


def build_mlp(ad: Autodiff, params) -> Sequential:
    """Sequential(Linear, ReLU, ..., Linear) from [W0, b0, W1, b1, ...]."""
    layers = []
    n = len(params) // 2
    for l in range(n):
        layers.append(Linear(ad, params[2 * l], params[2 * l + 1]))
        if l + 1 < n:
            layers.append(ReLU())
    return Sequential(*layers)


def argmax_rows(logits: np.ndarray) -> np.ndarray:
    """python/orca/nn/model.py:65-75 (first maximum, strict >)."""
    out = np.zeros(logits.shape[0], np.int32)
    for r, row in enumerate(logits):
        best, bv = 0, row[0]
        for c in range(1, row.shape[0]):
            if row[c] > bv:
                best, bv = c, row[c]
        out[r] = best
    return out


__all__ = ["Autodiff", "Tensor", "Tape", "no_grad", "Linear", "ReLU", "Sequential", "CrossEntropyLoss", "MSELoss",
           "SGD", "AdamW", "Parameter", "Module", "build_mlp", "argmax_rows", "OrcaError", "math"]
