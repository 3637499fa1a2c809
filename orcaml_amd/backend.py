"""HipBackend: the reference's `Backend` trait (orca-tensor/src/backend.rs:19-315)
over the storage handles of liborca_hip.so (include/orca_hip.h, "storage handles").

Each trait method is one call into the library (`orca_hip_trait_<method>`), which
takes and returns reference-counted storage handles.  The planning that makes the
composed step cheap -- lazy transpose views, pending elementwise chains fused into
one program, pending products run with their epilogue, the deferred bias column
sum and identity-reduction memo, one-element host constants, and the events of the
fused optimizer's second-stream pass -- lives behind those handles in the library
(orcaml_amd/csrc/storage.cpp), as it does behind a Rust `HipBackend`'s storages.

A `HipStorage` owns one reference to its handle and releases it when Python drops
it: the library decides from reference counts which pending values something still
holds, so a handle must be released as soon as its last holder goes.  A call that
returns a storage this backend already wraps (an identity `expand`, the identity
`sum_to_shape` memo, `reshape`) gives back the same Python object.  Errors surface
as `_lib.OrcaHipError` (a ValueError, as orca-python maps OrcaError).
"""
from __future__ import annotations

import ctypes
import math
import weakref

import numpy as np

from . import _lib
from ._lib import (EW_ADD, EW_ADD_SCALAR, EW_COPY, EW_DIV, EW_DIV_BW_RHS, EW_EXP, EW_EXP_BW, EW_LOG,  # noqa: F401
                   EW_LOG_BW, EW_MAX_INPUTS, EW_MAX_OPS, EW_MAX_OUTPUTS, EW_MAX_REGS, EW_MAX_VISIT, EW_MUL,
                   EW_MUL_SCALAR, EW_RELU, EW_RELU_BW, EW_SIGMOID, EW_SIGMOID_BW, EW_SQRT, EW_SQRT_BW, EW_SUB,
                   EW_SUM_VISIT, EwInput)
from .device import Context

_VP = ctypes.c_void_p
_byref = ctypes.byref
_FLAG_PENDING, _FLAG_TRANSPOSED, _FLAG_MARKED, _FLAG_CONSTANT = 1, 2, 4, 8


def _dims(shape):
    return _lib.dims(shape)


def _numel(shape) -> int:
    return math.prod(int(d) for d in shape)


class HipStorage:
    """A storage handle (`HipBackend::Storage`): cheap to share, immutable, possibly not yet
    computed."""

    __slots__ = ("be", "h", "_n", "__weakref__")

    def __init__(self, be: "HipBackend", h: int):
        self.be = be
        self.h = h
        self._n = None

    @property
    def n(self) -> int:
        if self._n is None:
            v = ctypes.c_size_t()
            _lib.call("orca_hip_storage_len", self.h, ctypes.byref(v))
            self._n = v.value
        return self._n

    def __len__(self) -> int:
        return self.n

    def flags(self) -> int:
        v = ctypes.c_uint32()
        _lib.call("orca_hip_storage_flags", self.h, ctypes.byref(v))
        return v.value

    @property
    def pending(self) -> bool:
        """Not computed yet (a pending op, product, column sum or host constant)."""
        return bool(self.flags() & _FLAG_PENDING)

    @property
    def transposed(self) -> bool:
        """A lazy transpose view of its buffer."""
        return bool(self.flags() & _FLAG_TRANSPOSED)

    @property
    def marked(self) -> bool:
        """Written on the second stream; its first use makes the context stream wait."""
        return bool(self.flags() & _FLAG_MARKED)

    @property
    def ptr(self) -> int:
        """The device address of its values (computing them first)."""
        p = _VP()
        _lib.call("orca_hip_storage_device_ptr", self.be.handle, self.h, ctypes.byref(p))
        return p.value

    def __del__(self):
        be = self.be
        h = self.h
        if be is None or not h:
            return
        try:
            live = be._live
            r = live.get(h)
            if r is not None and r() is None:
                del live[h]
            if be.ctx.handle:
                rc = be._release_fn(h)
                if rc != _lib.OK:
                    _lib.check(rc)
        except Exception:
            pass
        self.h = None


class HipBackend:
    """Drop-in for `GpuBackend` (orca-backend-gpu/src/backend.rs:45-50): an `orca_hip_backend`
    on a context.  The switches select the library's planning (include/orca_hip.h
    orca_hip_backend_options); None keeps the default (environment overrides included)."""

    def __init__(self, ctx: Context | None = None, deferred: bool = True, lazy: bool = True, fold: bool = True,
                 overlap: bool | None = None, side_frac: float | None = None, side_bpc: int | None = None):
        self.ctx = ctx if ctx is not None else Context(0)
        opts = _lib.BackendOptions()
        _lib.call("orca_hip_backend_default_options", ctypes.byref(opts))
        opts.deferred, opts.lazy, opts.fold = int(deferred), int(lazy), int(fold and lazy)
        if overlap is not None:
            opts.overlap = int(overlap)
        if side_frac is not None:
            opts.side_frac = float(side_frac)
        if side_bpc is not None:
            opts.side_bpc = int(side_bpc)
        self.options = opts
        h = _VP()
        _lib.call("orca_hip_backend_create", self.ctx.handle, ctypes.byref(opts), ctypes.byref(h))
        self.handle = h.value
        self._live = {}  # handle -> weak reference to its HipStorage
        lib = _lib.load()
        self._release_fn = lib.orca_hip_storage_release

    @property
    def deferred(self) -> bool:
        return bool(self.options.deferred)

    @property
    def lazy(self) -> bool:
        return bool(self.options.lazy)

    @property
    def overlap(self) -> bool:
        return bool(self.options.overlap)

    def __repr__(self) -> str:
        return f"HipBackend(device=gpu:{self.ctx.device})"

    def __del__(self):
        try:
            if self.handle and self.ctx.handle:
                _lib.call("orca_hip_backend_destroy", self.handle)
            self.handle = None
        except Exception:
            pass

    # ---- handles ----
    def _release(self, h: int) -> None:
        rc = self._release_fn(h)
        if rc != _lib.OK:
            _lib.check(rc)

    def _forget(self, h: int) -> None:
        r = self._live.get(h)
        if r is not None and r() is None:
            del self._live[h]

    def _wrap(self, h: int) -> HipStorage:
        r = self._live.get(h)
        if r is not None:
            w = r()
            if w is not None:
                self._release(h)  # the call's reference: the wrapper holds one already
                return w
        w = HipStorage(self, h)
        self._live[h] = weakref.ref(w)
        return w

    def _out(self, name: str, *args) -> HipStorage:
        fn = _lib._FNS.get(name)
        if fn is None:
            fn = _lib._FNS[name] = getattr(_lib.load(), name)
        out = _VP()
        rc = fn(self.handle, *args, _byref(out))
        if rc != _lib.OK:
            _lib.check(rc)
        h = out.value
        r = self._live.get(h)
        if r is not None:
            w = r()
            if w is not None:
                self._release(h)  # the call's reference: the wrapper holds one already
                return w
        w = HipStorage(self, h)
        self._live[h] = weakref.ref(w)
        return w

    # ---- trait methods (orca-tensor/src/backend.rs) ----
    def device(self) -> str:
        kind, index = ctypes.c_int(), ctypes.c_int()
        _lib.call("orca_hip_trait_device", self.handle, ctypes.byref(kind), ctypes.byref(index))
        return f"gpu:{index.value}"

    def zeros(self, shape, dtype=_lib.F32):
        d, r = _dims(shape)
        return self._out("orca_hip_trait_zeros", d, r, dtype)

    def from_f32_slice(self, shape, data):
        data = np.ascontiguousarray(data, np.float32).reshape(-1)
        d, r = _dims(shape)
        return self._out("orca_hip_trait_from_f32_slice", d, r, data.ctypes.data_as(_VP), data.size)

    def to_f32_vec(self, s: HipStorage) -> np.ndarray:
        out = np.empty(s.n, np.float32)
        _lib.call("orca_hip_trait_to_f32_vec", self.handle, s.h, out.ctypes.data_as(_VP), out.size)
        return out

    def from_bytes(self, shape, data: bytes, dtype=_lib.F32):
        arr = np.frombuffer(data, np.uint8)
        d, r = _dims(shape)
        return self._out("orca_hip_trait_from_bytes", d, r, arr.ctypes.data_as(_VP), arr.size, dtype)

    def to_bytes(self, s: HipStorage) -> bytes:
        out = np.empty(4 * s.n, np.uint8)
        _lib.call("orca_hip_trait_to_bytes", self.handle, s.h, out.ctypes.data_as(_VP), out.size)
        return out.tobytes()

    def has_nan_or_inf(self, s, dtype=_lib.F32) -> bool:
        res = ctypes.c_int()
        _lib.call("orca_hip_trait_has_nan_or_inf", self.handle, s.h, dtype, ctypes.byref(res))
        return bool(res.value)

    def matmul(self, lhs: HipStorage, rhs: HipStorage, lhs_shape, rhs_shape, dtype=_lib.F32):
        dl, rl = _dims(lhs_shape)
        dr, rr = _dims(rhs_shape)
        return self._out("orca_hip_trait_matmul", lhs.h, rhs.h, dl, rl, dr, rr, dtype)

    def transpose(self, s: HipStorage, shape, dim0: int, dim1: int, dtype=_lib.F32):
        d, r = _dims(shape)
        return self._out("orca_hip_trait_transpose", s.h, d, r, dim0, dim1, dtype)

    def _binary(self, name, a, b, shape, dtype):
        d, r = _dims(shape)
        return self._out(name, a.h, b.h, d, r, dtype)

    def _unary(self, name, s, shape, dtype):
        d, r = _dims(shape)
        return self._out(name, s.h, d, r, dtype)

    def add(self, a, b, shape, dtype=_lib.F32):
        return self._binary("orca_hip_trait_add", a, b, shape, dtype)

    def sub(self, a, b, shape, dtype=_lib.F32):
        return self._binary("orca_hip_trait_sub", a, b, shape, dtype)

    def mul(self, a, b, shape, dtype=_lib.F32):
        return self._binary("orca_hip_trait_mul", a, b, shape, dtype)

    def div(self, a, b, shape, dtype=_lib.F32):
        return self._binary("orca_hip_trait_div", a, b, shape, dtype)

    def mul_scalar(self, s, scalar: float, shape, dtype=_lib.F32):
        d, r = _dims(shape)
        return self._out("orca_hip_trait_mul_scalar", s.h, ctypes.c_float(scalar), d, r, dtype)

    def relu(self, s, shape, dtype=_lib.F32):
        return self._unary("orca_hip_trait_relu", s, shape, dtype)

    def sigmoid(self, s, shape, dtype=_lib.F32):
        return self._unary("orca_hip_trait_sigmoid", s, shape, dtype)

    def exp(self, s, shape, dtype=_lib.F32):
        return self._unary("orca_hip_trait_exp", s, shape, dtype)

    def log(self, s, shape, dtype=_lib.F32):
        return self._unary("orca_hip_trait_log", s, shape, dtype)

    def sqrt(self, s, shape, dtype=_lib.F32):
        return self._unary("orca_hip_trait_sqrt", s, shape, dtype)

    def relu_backward(self, g, x, shape, dtype=_lib.F32):
        return self._binary("orca_hip_trait_relu_backward", g, x, shape, dtype)

    def sigmoid_backward(self, g, y, shape, dtype=_lib.F32):
        return self._binary("orca_hip_trait_sigmoid_backward", g, y, shape, dtype)

    def exp_backward(self, g, y, shape, dtype=_lib.F32):
        return self._binary("orca_hip_trait_exp_backward", g, y, shape, dtype)

    def log_backward(self, g, x, shape, dtype=_lib.F32):
        return self._binary("orca_hip_trait_log_backward", g, x, shape, dtype)

    def sqrt_backward(self, g, y, shape, dtype=_lib.F32):
        return self._binary("orca_hip_trait_sqrt_backward", g, y, shape, dtype)

    def div_backward_lhs(self, g, r, shape, dtype=_lib.F32):
        return self._binary("orca_hip_trait_div_backward_lhs", g, r, shape, dtype)

    def div_backward_rhs(self, g, l, r, shape, dtype=_lib.F32):
        d, rk = _dims(shape)
        return self._out("orca_hip_trait_div_backward_rhs", g.h, l.h, r.h, d, rk, dtype)

    def accumulate_grad(self, a, b):
        return self._out("orca_hip_trait_accumulate_grad", a.h, b.h)

    def _reshape_like(self, name, s, in_shape, out_shape, dtype):
        di, ri = _dims(in_shape)
        do, ro = _dims(out_shape)
        return self._out(name, s.h, di, ri, do, ro, dtype)

    def expand(self, s, in_shape, out_shape, dtype=_lib.F32):
        if dtype == _lib.F32 and s.be.ctx is self.ctx and tuple(in_shape) == tuple(out_shape):
            return s  # the library's identity broadcast gives back the same storage: no call needed
        return self._reshape_like("orca_hip_trait_expand", s, in_shape, out_shape, dtype)

    def sum_to_shape(self, s, in_shape, out_shape, dtype=_lib.F32):
        return self._reshape_like("orca_hip_trait_sum_to_shape", s, in_shape, out_shape, dtype)

    def reshape(self, s, in_shape, out_shape, dtype=_lib.F32):
        return self._reshape_like("orca_hip_trait_reshape", s, in_shape, out_shape, dtype)

    def max_to_shape(self, s, in_shape, out_shape, dtype=_lib.F32):
        return self._reshape_like("orca_hip_trait_max_to_shape", s, in_shape, out_shape, dtype)

    def max_to_shape_backward(self, g, x, y, in_shape, out_shape, dtype=_lib.F32):
        di, ri = _dims(in_shape)
        do, ro = _dims(out_shape)
        return self._out("orca_hip_trait_max_to_shape_backward", g.h, x.h, y.h, di, ri, do, ro, dtype)

    def cast(self, s, shape, current_dtype, target_dtype):
        d, r = _dims(shape)
        return self._out("orca_hip_trait_cast", s.h, d, r, current_dtype, target_dtype)

    # ---- fused paths: inherent methods beside the trait (the reference's trait has no loss
    # or optimizer op; nn.CrossEntropyLoss(fused=True), optim.SGD / AdamW(fused=True) call
    # these when the backend has them) ----
    def clone(self, s: HipStorage) -> HipStorage:
        """A new buffer holding the same values (device to device)."""
        return self._out("orca_hip_be_clone", s.h)

    def softmax_ce(self, logits: HipStorage, onehot: HipStorage, B: int, C: int, want_grad: bool = True):
        """Mean softmax cross-entropy of [B, C] logits against one-hot targets and, if
        want_grad, dL/dlogits for a loss seed of 1, in one kernel (orca_hip_be_softmax_ce).
        Returns (loss [1], dlogits [B, C] or None)."""
        loss, dl = _VP(), _VP()
        _lib.call("orca_hip_be_softmax_ce", self.handle, logits.h, onehot.h, B, C, int(want_grad), ctypes.byref(loss),
                  ctypes.byref(dl))
        return self._wrap(loss.value), (self._wrap(dl.value) if want_grad else None)

    def adamw_step_(self, p: HipStorage, g: HipStorage, m: HipStorage, v: HipStorage, n: int, lr: float,
                    beta1: float, beta2: float, eps: float, weight_decay: float, t: int) -> None:
        """In place on p, m, v (orca_hip_be_adamw_step)."""
        _lib.call("orca_hip_be_adamw_step", self.handle, p.h, g.h, m.h, v.h, n, lr, beta1, beta2, eps, weight_decay, t)

    def sgd_step_(self, p: HipStorage, g: HipStorage, n: int, lr: float) -> None:
        """In place on p (orca_hip_be_sgd_step)."""
        _lib.call("orca_hip_be_sgd_step", self.handle, p.h, g.h, n, lr)

    # ---- flat arenas and one-launch optimizer passes ----
    def arena(self, n: int, fill: float | None = None) -> HipStorage:
        """A flat device storage of n floats (set to `fill` if given)."""
        return self._out("orca_hip_be_arena", n, int(fill is not None), ctypes.c_float(fill or 0.0))

    def view(self, arena: HipStorage, offset: int, n: int) -> HipStorage:
        """The storage of n floats at `offset` (floats) of an arena, sharing its memory."""
        return self._out("orca_hip_be_view", arena.h, offset, n)

    def copy_into(self, dst: HipStorage, src: HipStorage) -> None:
        """dst <- src, device to device (dst a fresh arena slice nobody reads yet)."""
        _lib.call("orca_hip_be_copy_into", self.handle, dst.h, src.h)

    def arena_exclusive(self, arena: HipStorage) -> bool:
        """No view, storage or pending work refers to the arena's memory (besides `arena`)."""
        v = ctypes.c_int()
        _lib.call("orca_hip_be_arena_exclusive", self.handle, arena.h, ctypes.byref(v))
        return bool(v.value)

    @staticmethod
    def _rows(segs, moments: bool):
        table = (_lib.OptRow * max(1, len(segs)))()
        for i, seg in enumerate(segs):
            if moments:
                ps, pd, g, m, v, n = seg
                table[i] = _lib.OptRow(ps.h, pd.h, g.h, m.h, v.h, n)
            else:
                ps, pd, g, n = seg
                table[i] = _lib.OptRow(ps.h, pd.h, g.h, None, None, n)
        return table

    def adamw_multi_(self, segs, lr: float, beta1: float, beta2: float, eps: float, weight_decay: float,
                     t: int) -> None:
        """One AdamW pass over many parameters (orca_hip_be_adamw_multi): segs holds
        (p_src, p_dst, g, m, v, n) storages; p_dst, m and v are written."""
        _lib.call("orca_hip_be_adamw_multi", self.handle, self._rows(segs, True), len(segs), lr, beta1, beta2, eps,
                  weight_decay, t)

    def sgd_multi_(self, segs, lr: float) -> None:
        """One SGD pass over many parameters (orca_hip_be_sgd_multi): segs holds (p_src, p_dst, g, n)."""
        _lib.call("orca_hip_be_sgd_multi", self.handle, self._rows(segs, False), len(segs), lr)
