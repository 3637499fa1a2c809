"""HipBackend: the reference's `Backend` trait (orca-tensor/src/backend.rs:19-315)
over the C ABI of liborca_hip.so.

A storage is a `HipStorage`: a shared device buffer plus its element count
and a view flag.  Like the trait's storages it is cheap to clone (buffers are
reference counted by Python) and every op returns a new storage.  Two ops are
zero-copy here, as the trait allows (orca-backend-cpu/src/backend.rs:546
returns a clone for reshape): `reshape`, identity `expand`, and
`transpose` of the last two dims, which returns a lazy view that `matmul`
consumes with the transpose folded into its loads (the MatMulBackward
pattern, orca-autograd/src/backend.rs:1467-1495).  Any other consumer of a
view materialises it first.  Errors surface as `_lib.OrcaHipError`
(a ValueError, as orca-python maps OrcaError).

Two more internal shortcuts, invisible to the tape, serve Linear's backward
(ExpandBackward then MatMulBackward on the same upstream gradient G,
orca-autograd/src/backend.rs:1684-1697, 1448-1499):

* an identity `sum_to_shape` ([B, N] -> [B, N], one `0 + g` pass) computed
  once per source storage: the expand-both broadcast of `x @ W + b` asks for
  it twice on the same G, and storages are immutable, so the second call
  returns the first result;
* a column sum `sum_to_shape(G, [B, N] -> [1, N])` is returned pending; the
  next `matmul(X^T, G)` on that storage computes it inside the product
  (orca_hip_matmul_colsum, the same bits as the sum_to_shape kernel), and any
  other use computes it with the sum_to_shape kernel first.
"""
from __future__ import annotations

import ctypes
import math
import weakref

import numpy as np

from . import _lib
from .device import Buffer, Context


class HipStorage:
    __slots__ = ("_buf", "n", "transposed_shape", "_fill", "colsum_waiters", "ident", "__weakref__")

    def __init__(self, buf: Buffer | None, n: int, transposed_shape=None):
        self._buf = buf
        self.n = n
        # Logical shape of a lazy last-two-dims transpose (buffer holds the
        # untransposed data), or None for contiguous storage.
        self.transposed_shape = transposed_shape
        # Pending values: fill(self) sets _buf; run at the first use.
        self._fill = None
        # Weak references to pending column sums of this storage.
        self.colsum_waiters = None
        # This storage's identity sum_to_shape result, once computed.
        self.ident = None

    def __len__(self) -> int:
        return self.n

    @property
    def pending(self) -> bool:
        return self._fill is not None

    @property
    def buf(self) -> Buffer:
        if self._fill is not None:
            fill, self._fill = self._fill, None
            fill(self)
        return self._buf

    @property
    def ptr(self) -> int:
        return self.buf.ptr


def _dims(shape):
    return _lib.dims(shape)


def _numel(shape) -> int:
    return math.prod(int(d) for d in shape)


class HipBackend:
    """Drop-in for `GpuBackend` (orca-backend-gpu/src/backend.rs:45-50)."""

    def __init__(self, ctx: Context | None = None, deferred: bool = True):
        self.ctx = ctx if ctx is not None else Context(0)
        # The identity-reduction memo and the deferred column sum (module
        # docstring); off, every sum_to_shape runs its kernel at once.
        self.deferred = deferred

    def __repr__(self) -> str:
        return f"HipBackend(device=gpu:{self.ctx.device})"

    # ---- helpers ----
    def _wrap(self, ptr: ctypes.c_void_p, n: int) -> HipStorage:
        return HipStorage(Buffer(self.ctx, ptr.value, 4 * max(n, 1)), n)

    def _plain(self, s: HipStorage) -> HipStorage:
        """Materialises a lazy transpose view."""
        if s.transposed_shape is None:
            return s
        shape = list(s.transposed_shape)
        src_shape = shape[:-2] + [shape[-1], shape[-2]]
        out = ctypes.c_void_p()
        d, r = _dims(src_shape)
        _lib.call("orca_hip_transpose", self.ctx.handle, s.ptr, d, r, r - 2, r - 1, _lib.F32, ctypes.byref(out))
        return self._wrap(out, s.n)

    def _op1(self, name, s, shape, dtype):
        s = self._plain(s)
        out = ctypes.c_void_p()
        d, r = _dims(shape)
        _lib.call("orca_hip_" + name, self.ctx.handle, s.ptr, d, r, dtype, ctypes.byref(out))
        return self._wrap(out, _numel(shape))

    def _op2(self, name, a, b, shape, dtype):
        a, b = self._plain(a), self._plain(b)
        out = ctypes.c_void_p()
        d, r = _dims(shape)
        _lib.call("orca_hip_" + name, self.ctx.handle, a.ptr, b.ptr, d, r, dtype, ctypes.byref(out))
        return self._wrap(out, _numel(shape))

    def _reshape_like(self, name, s, in_shape, out_shape, dtype):
        s = self._plain(s)
        out = ctypes.c_void_p()
        di, ri = _dims(in_shape)
        do, ro = _dims(out_shape)
        _lib.call("orca_hip_" + name, self.ctx.handle, s.ptr, di, ri, do, ro, dtype, ctypes.byref(out))
        return self._wrap(out, _numel(out_shape))

    # ---- trait methods (orca-tensor/src/backend.rs) ----
    def device(self) -> str:
        return f"gpu:{self.ctx.device}"

    def zeros(self, shape, dtype=_lib.F32):
        out = ctypes.c_void_p()
        d, r = _dims(shape)
        _lib.call("orca_hip_zeros", self.ctx.handle, d, r, dtype, ctypes.byref(out))
        return self._wrap(out, _numel(shape))

    def from_f32_slice(self, shape, data):
        data = np.ascontiguousarray(data, np.float32).reshape(-1)
        out = ctypes.c_void_p()
        d, r = _dims(shape)
        _lib.call("orca_hip_from_f32_slice", self.ctx.handle, d, r, data.ctypes.data_as(ctypes.c_void_p), data.size,
                  ctypes.byref(out))
        return self._wrap(out, data.size)

    def to_f32_vec(self, s: HipStorage) -> np.ndarray:
        s = self._plain(s)
        out = np.empty(s.n, np.float32)
        _lib.call("orca_hip_to_f32_vec", self.ctx.handle, s.ptr, s.n, out.ctypes.data_as(ctypes.c_void_p))
        return out

    def from_bytes(self, shape, data: bytes, dtype=_lib.F32):
        arr = np.frombuffer(data, np.uint8)
        out = ctypes.c_void_p()
        d, r = _dims(shape)
        _lib.call("orca_hip_from_bytes", self.ctx.handle, d, r, arr.ctypes.data_as(ctypes.c_void_p), arr.size, dtype,
                  ctypes.byref(out))
        return self._wrap(out, _numel(shape))

    def to_bytes(self, s: HipStorage) -> bytes:
        s = self._plain(s)
        out = np.empty(4 * s.n, np.uint8)
        _lib.call("orca_hip_to_bytes", self.ctx.handle, s.ptr, out.size, out.ctypes.data_as(ctypes.c_void_p))
        return out.tobytes()

    def matmul(self, lhs: HipStorage, rhs: HipStorage, lhs_shape, rhs_shape, dtype=_lib.F32):
        if (rhs.colsum_waiters and dtype == _lib.F32 and len(lhs_shape) == 2 and len(rhs_shape) == 2
                and rhs.transposed_shape is None and lhs_shape[1] == rhs_shape[0]):
            target = self._take_colsum_waiter(rhs, int(rhs_shape[1]))
            if target is not None:
                M, K, N = int(lhs_shape[0]), int(lhs_shape[1]), int(rhs_shape[1])
                lv = _lib.VIEW_TRANSPOSED if lhs.transposed_shape is not None else _lib.VIEW_CONTIGUOUS
                cs = self.ctx.alloc(4 * max(N, 1))
                out = ctypes.c_void_p()
                _lib.call("orca_hip_matmul_colsum", self.ctx.handle, lhs.ptr, rhs.ptr, M, K, N, lv, dtype, cs.ptr,
                          ctypes.byref(out))
                target._buf, target._fill = cs, None
                return self._wrap(out, M * N)
        out = ctypes.c_void_p()
        dl, rl = _dims(lhs_shape)
        dr, rr = _dims(rhs_shape)
        lv = _lib.VIEW_TRANSPOSED if lhs.transposed_shape is not None else _lib.VIEW_CONTIGUOUS
        rv = _lib.VIEW_TRANSPOSED if rhs.transposed_shape is not None else _lib.VIEW_CONTIGUOUS
        _lib.call("orca_hip_matmul", self.ctx.handle, lhs.ptr, rhs.ptr, dl, rl, dr, rr, dtype, lv, rv,
                  ctypes.byref(out))
        n = _numel(lhs_shape[:-1]) * int(rhs_shape[-1])
        return self._wrap(out, n)

    def transpose(self, s: HipStorage, shape, dim0: int, dim1: int, dtype=_lib.F32):
        rank = len(shape)
        if dim0 >= rank or dim1 >= rank:
            raise _lib.OrcaHipError(_lib.ERR_INTERNAL, "Invalid transpose dimensions")
        out_shape = list(shape)
        out_shape[dim0], out_shape[dim1] = out_shape[dim1], out_shape[dim0]
        if rank >= 2 and {dim0, dim1} == {rank - 2, rank - 1} and dtype == _lib.F32:
            if s.transposed_shape is not None:  # transposing a view gives back the buffer's own layout
                return HipStorage(s.buf, s.n, None)
            return HipStorage(s.buf, s.n, tuple(out_shape))
        s = self._plain(s)
        out = ctypes.c_void_p()
        d, r = _dims(shape)
        _lib.call("orca_hip_transpose", self.ctx.handle, s.ptr, d, r, dim0, dim1, dtype, ctypes.byref(out))
        return self._wrap(out, s.n)

    def add(self, a, b, shape, dtype=_lib.F32):
        return self._op2("add", a, b, shape, dtype)

    def sub(self, a, b, shape, dtype=_lib.F32):
        return self._op2("sub", a, b, shape, dtype)

    def mul(self, a, b, shape, dtype=_lib.F32):
        return self._op2("mul", a, b, shape, dtype)

    def div(self, a, b, shape, dtype=_lib.F32):
        return self._op2("div", a, b, shape, dtype)

    def mul_scalar(self, s, scalar: float, shape, dtype=_lib.F32):
        s = self._plain(s)
        out = ctypes.c_void_p()
        d, r = _dims(shape)
        _lib.call("orca_hip_mul_scalar", self.ctx.handle, s.ptr, ctypes.c_float(scalar), d, r, dtype,
                  ctypes.byref(out))
        return self._wrap(out, _numel(shape))

    def relu(self, s, shape, dtype=_lib.F32):
        return self._op1("relu", s, shape, dtype)

    def sigmoid(self, s, shape, dtype=_lib.F32):
        return self._op1("sigmoid", s, shape, dtype)

    def exp(self, s, shape, dtype=_lib.F32):
        return self._op1("exp", s, shape, dtype)

    def log(self, s, shape, dtype=_lib.F32):
        return self._op1("log", s, shape, dtype)

    def sqrt(self, s, shape, dtype=_lib.F32):
        return self._op1("sqrt", s, shape, dtype)

    def relu_backward(self, g, x, shape, dtype=_lib.F32):
        return self._op2("relu_backward", g, x, shape, dtype)

    def sigmoid_backward(self, g, y, shape, dtype=_lib.F32):
        return self._op2("sigmoid_backward", g, y, shape, dtype)

    def exp_backward(self, g, y, shape, dtype=_lib.F32):
        return self._op2("exp_backward", g, y, shape, dtype)

    def log_backward(self, g, x, shape, dtype=_lib.F32):
        return self._op2("log_backward", g, x, shape, dtype)

    def sqrt_backward(self, g, y, shape, dtype=_lib.F32):
        return self._op2("sqrt_backward", g, y, shape, dtype)

    def div_backward_lhs(self, g, r, shape, dtype=_lib.F32):
        return self._op2("div_backward_lhs", g, r, shape, dtype)

    def div_backward_rhs(self, g, l, r, shape, dtype=_lib.F32):
        g, l, r = self._plain(g), self._plain(l), self._plain(r)
        out = ctypes.c_void_p()
        d, rk = _dims(shape)
        _lib.call("orca_hip_div_backward_rhs", self.ctx.handle, g.ptr, l.ptr, r.ptr, d, rk, dtype, ctypes.byref(out))
        return self._wrap(out, _numel(shape))

    def accumulate_grad(self, a, b):
        a, b = self._plain(a), self._plain(b)
        out = ctypes.c_void_p()
        _lib.call("orca_hip_accumulate_grad", self.ctx.handle, a.ptr, b.ptr, a.n, ctypes.byref(out))
        return self._wrap(out, a.n)

    def expand(self, s, in_shape, out_shape, dtype=_lib.F32):
        if tuple(in_shape) == tuple(out_shape) and dtype == _lib.F32:
            return s  # identity broadcast: share the storage
        return self._reshape_like("expand", s, in_shape, out_shape, dtype)

    def sum_to_shape(self, s, in_shape, out_shape, dtype=_lib.F32):
        in_shape, out_shape = tuple(int(d) for d in in_shape), tuple(int(d) for d in out_shape)
        if self.deferred and dtype == _lib.F32 and s.transposed_shape is None and not s.pending:
            if in_shape == out_shape:
                if s.ident is None:
                    s.ident = self._reshape_like("sum_to_shape", s, in_shape, out_shape, dtype)
                return s.ident
            if len(in_shape) == 2 and out_shape in ((1, in_shape[1]), (in_shape[1],)):
                return self._deferred_colsum(s, in_shape)
        return self._reshape_like("sum_to_shape", s, in_shape, out_shape, dtype)

    def _deferred_colsum(self, s: HipStorage, in_shape) -> HipStorage:
        """sum_to_shape(s, [R, N] -> [1, N]) left pending on s (see the module docstring)."""
        cols = in_shape[1]
        out = HipStorage(None, cols)

        def fill(st, src=s, shape=in_shape):
            st._buf = self._reshape_like("sum_to_shape", src, shape, (1, shape[1]), _lib.F32)._buf

        out._fill = fill
        if s.colsum_waiters is None:
            s.colsum_waiters = []
        s.colsum_waiters.append(weakref.ref(out))
        return out

    @staticmethod
    def _take_colsum_waiter(s: HipStorage, cols: int):
        """Removes and returns a still-pending column sum of s with `cols` columns, or None."""
        found = None
        live = []
        for ref in s.colsum_waiters:
            t = ref()
            if t is None or not t.pending:
                continue
            if found is None and t.n == cols:
                found = t
            else:
                live.append(ref)
        s.colsum_waiters = live or None
        return found

    @staticmethod
    def _mutating(*storages) -> None:
        """Before an in-place update: values derived lazily from these storages are computed
        from their current contents, and their memoised identity reductions are dropped."""
        for s in storages:
            if s.colsum_waiters:
                for ref in s.colsum_waiters:
                    t = ref()
                    if t is not None:
                        t.buf  # runs a pending fill
            s.colsum_waiters = None
            s.ident = None

    def reshape(self, s, in_shape, out_shape, dtype=_lib.F32):
        n_in = _numel(in_shape)
        n_out = _numel(out_shape)
        if n_in != n_out:
            raise _lib.OrcaHipError(_lib.ERR_SHAPE, f"Shape mismatch during reshape: expected {n_in} elements, "
                                                    f"got {n_out} elements")
        return self._plain(s)

    def max_to_shape(self, s, in_shape, out_shape, dtype=_lib.F32):
        return self._reshape_like("max_to_shape", s, in_shape, out_shape, dtype)

    def max_to_shape_backward(self, g, x, y, in_shape, out_shape, dtype=_lib.F32):
        g, x, y = self._plain(g), self._plain(x), self._plain(y)
        out = ctypes.c_void_p()
        di, ri = _dims(in_shape)
        do, ro = _dims(out_shape)
        _lib.call("orca_hip_max_to_shape_backward", self.ctx.handle, g.ptr, x.ptr, y.ptr, di, ri, do, ro, dtype,
                  ctypes.byref(out))
        return self._wrap(out, _numel(in_shape))

    def has_nan_or_inf(self, s, dtype=_lib.F32) -> bool:
        s = self._plain(s)
        res = ctypes.c_int()
        _lib.call("orca_hip_has_nan_or_inf", self.ctx.handle, s.ptr, s.n, dtype, ctypes.byref(res))
        return bool(res.value)

    # ---- fused paths: inherent methods beside the trait (the reference's
    # trait has no loss or optimizer op; nn.CrossEntropyLoss(fused=True),
    # optim.SGD / AdamW(fused=True) call these when the backend has them) ----
    def clone(self, s: HipStorage) -> HipStorage:
        """A new buffer holding the same values (device to device)."""
        s = self._plain(s)
        out = HipStorage(self.ctx.alloc(4 * max(s.n, 1)), s.n)
        if s.n:
            self.ctx.d2d(out.buf, s.buf, 4 * s.n)
        return out

    def softmax_ce(self, logits: HipStorage, onehot: HipStorage, B: int, C: int, want_grad: bool = True):
        """Mean softmax cross-entropy of [B, C] logits against one-hot targets
        and, if want_grad, dL/dlogits for a loss seed of 1, in one kernel
        (orca_hip_softmax_ce).  Returns (loss [1], dlogits [B, C] or None)."""
        logits, onehot = self._plain(logits), self._plain(onehot)
        loss = HipStorage(self.ctx.alloc(4), 1)
        dl = HipStorage(self.ctx.alloc(4 * max(B * C, 1)), B * C) if want_grad else None
        _lib.call("orca_hip_softmax_ce", self.ctx.handle, logits.ptr, B, C, onehot.ptr, None, loss.ptr,
                  dl.ptr if dl is not None else None, None, None)
        return loss, dl

    def adamw_step_(self, p: HipStorage, g: HipStorage, m: HipStorage, v: HipStorage, n: int, lr: float,
                    beta1: float, beta2: float, eps: float, weight_decay: float, t: int) -> None:
        """In place on p, m, v (orca_hip_adamw_step)."""
        g = self._plain(g)
        self._mutating(p, m, v)
        _lib.call("orca_hip_adamw_step", self.ctx.handle, p.ptr, g.ptr, m.ptr, v.ptr, n, lr, beta1, beta2, eps,
                  weight_decay, t)

    def sgd_step_(self, p: HipStorage, g: HipStorage, n: int, lr: float) -> None:
        """In place on p (orca_hip_sgd_step)."""
        g = self._plain(g)
        self._mutating(p)
        _lib.call("orca_hip_sgd_step", self.ctx.handle, p.ptr, g.ptr, n, lr)
