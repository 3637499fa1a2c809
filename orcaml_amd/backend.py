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

And elementwise ops are lazy: add ... div_backward_rhs, accumulate_grad and
the identity sum_to_shape / max_to_shape return a storage holding the op and
its operands.  The first use that needs its values (any other op, a host
read, an in-place update of one of its inputs) compiles the pending chain into
one program of per-element instructions (orca_hip_ew_program): one launch and
one pass over memory instead of one per op.  Pending values that something
outside the chain still references (a tape node's saved primal, an optimizer's
moment) are written by the same launch.  Each instruction is the op's own f32
operation, so every value has the bits the ops run one by one would give.

Products are lazy too: a 2-D f32 `matmul` returns a storage that runs the GEMM
at its first use.  When that use is a pending chain that is exactly a GEMM
epilogue over a product nothing else references -- Linear's `x @ W +
b.expand(..)` with or without the ReLU after it (orca-autograd/src/backend.rs:
1625-1646 keeps the pre-activation, so both are written), or ReluBackward's
`relu_backward(g @ W^T, z)` (the product, a gradient the tape keeps, is written
too) -- the product runs once with that epilogue (orca_hip_gemm) instead of a
product and a program.  The epilogue computes the
same f32 operations on the same product, so the bits are those of the ops.

The fused optimizer passes (`adamw_multi_`, `sgd_multi_`, one launch over many
parameters) may run part of the update on the context's second stream: a
weight-gradient product (`matmul` of a transposed view) leaves a mark (an
event) on its output, and the parameters whose gradients came from a product
before the step's last one are updated on the side stream as soon as those
gradients exist, beside the backward's remaining products.  The parameters it
writes carry the side stream's mark: their first use waits for it on the
context stream, and what that update reads stays referenced until then, so no
block is reused early.  Same kernel, same bits.
"""
from __future__ import annotations

import collections
import ctypes
import itertools
import math
import os
import struct
import sys
import weakref

import numpy as np

from . import _lib
from .device import Buffer, Context


# Elementwise program opcodes (include/orca_hip.h ORCA_HIP_EW_*) and interpreter limits.
EW_ADD, EW_SUB, EW_MUL, EW_DIV, EW_MUL_SCALAR, EW_RELU, EW_RELU_BW, EW_EXP, EW_LOG, EW_SQRT = range(10)
EW_SIGMOID, EW_EXP_BW, EW_LOG_BW, EW_SQRT_BW, EW_SIGMOID_BW, EW_DIV_BW_RHS, EW_SUM_VISIT, EW_MAX_VISIT = range(10, 18)
EW_COPY, EW_ADD_SCALAR = 18, 19
EW_MAX_INPUTS, EW_MAX_OUTPUTS, EW_MAX_OPS, EW_MAX_REGS = 8, 8, 64, 16
_INSTR = struct.Struct("<BBBBBxxxf")  # orca_hip_ew_instr
_SCALAR = struct.Struct("<f")  # its scalar field, at byte 8


class EwInput(ctypes.Structure):
    """orca_hip_ew_input: element e of a program reads ptr[(e / div) % mod]."""
    _fields_ = [("ptr", ctypes.c_void_p), ("div", ctypes.c_uint64), ("mod", ctypes.c_uint64)]


class _Broadcast:
    """A program input that reads `src` broadcast to `n` elements through the index map
    (e / div) % mod -- Backend::expand of a contiguous block of dims, run in place."""

    __slots__ = ("src", "n", "div", "mod", "_expr", "_ew_ops", "_ew_leaves", "__weakref__")

    def __init__(self, src, n, div, mod):
        self.src, self.n, self.div, self.mod = src, n, div, mod
        self._expr, self._ew_ops, self._ew_leaves = None, 0, 1

    @property
    def ptr(self) -> int:
        return self.src.ptr


def _broadcast_map(in_shape, out_shape):
    """(div, mod) when expanding in_shape to out_shape reads input element (e / div) % mod for
    output element e (the input's non-broadcast dims are one contiguous block of the output's),
    else None."""
    r = len(out_shape)
    pin = (1,) * (r - len(in_shape)) + tuple(in_shape)
    kept = [d for d in range(r) if pin[d] != 1]
    if any(pin[d] != out_shape[d] for d in kept):
        return None
    if not kept:
        return 1, 1
    i0, i1 = kept[0], kept[-1] + 1
    if any(pin[d] == 1 and out_shape[d] != 1 for d in range(i0, i1)):
        return None
    return math.prod(out_shape[i1:]), math.prod(out_shape[i0:i1])


class _Mark:
    """A point in one stream's work (an event), to order the context's two streams.  `keep`
    holds what work before the mark reads: it stays referenced until the context stream has
    been made to wait for the mark, so its blocks are not reused before that work is done."""

    __slots__ = ("ctx", "ev", "seq", "keep", "settled")
    _seq = itertools.count()

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.ev = ctx.event_record()  # on the current stream
        self.seq = next(_Mark._seq)
        self.keep = None
        self.settled = False

    def wait(self) -> None:
        """The current stream waits for the mark (no host wait)."""
        self.ctx.event_wait(self.ev)

    def settle(self) -> None:
        """The context stream waits for the mark (once); the kept storages can go."""
        if self.ctx.on_side:
            raise RuntimeError("a marked storage was used while launches go to the second stream")
        if not self.settled:
            self.settled = True
            self.ctx.event_wait(self.ev)
            self.keep = None

    def __del__(self):
        try:
            if self.ctx.handle:
                if self.keep is not None:
                    self.settle()
                self.ctx.event_release(self.ev)
        except Exception:
            pass


class HipStorage:
    __slots__ = ("_buf", "n", "transposed_shape", "_fill", "colsum_waiters", "ident", "_expr", "_ew_ops",
                 "_ew_leaves", "_prod", "_const", "_ready", "_made", "__weakref__")

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
        # A pending elementwise op: (backend, opcode, operand storages, scalar), with
        # upper bounds of the ops and distinct inputs of its pending chain.
        self._expr = None
        self._ew_ops = 0
        self._ew_leaves = 1
        # A pending product (with _fill set): (lhs, rhs, M, K, N, lhs transposed, rhs transposed).
        self._prod = None
        # The value of a one-element storage known on the host (a small upload, uploaded at
        # its first use on the device); dropped by an in-place update.
        self._const = None
        # Written on the side stream: the mark its first use waits for on the context stream.
        self._ready = None
        # Made by a weight-gradient product: the mark just after that launch.
        self._made = None

    def __len__(self) -> int:
        return self.n

    @property
    def pending(self) -> bool:
        return self._fill is not None or self._expr is not None

    @property
    def buf(self) -> Buffer:
        if self._ready is not None:
            mark, self._ready = self._ready, None
            mark.settle()
        if self._expr is not None:
            self._expr[0]._flush(self)
        if self._fill is not None:
            fill, self._fill = self._fill, None
            fill(self)
        return self._buf

    @property
    def ptr(self) -> int:
        return self.buf.ptr


class _ArenaView:
    """n floats at `offset` of a flat device arena: the buffer of one parameter (or moment)
    of a fused optimizer.  Keeps the arena alive; frees nothing itself."""

    __slots__ = ("arena", "ptr", "nbytes")

    def __init__(self, arena: Buffer, offset: int, n: int):
        self.arena = arena
        self.ptr = arena.ptr + 4 * offset
        self.nbytes = 4 * n

    def free(self) -> None:
        pass


_wref = weakref.ref


def _dims(shape):
    return _lib.dims(shape)


def _numel(shape) -> int:
    return math.prod(int(d) for d in shape)


def _split_rows(ptrs, frac):
    """Splits optimizer segments (p_src, p_dst, g, m, v, n pointers) at `frac` of their elements,
    on a 64-element boundary (256 bytes, so a split segment keeps its alignment)."""
    total = sum(p[5] for p in ptrs)
    cut = int(total * frac) // 64 * 64
    a, b, acc = [], [], 0
    for p in ptrs:
        n = p[5]
        if acc + n <= cut:
            a.append(p)
        elif acc >= cut:
            b.append(p)
        else:
            k = (cut - acc) // 64 * 64
            shift = tuple(None if q is None else q + 4 * k for q in p[:5])
            a.append(p[:5] + (k,))
            b.append(shift + (n - k,))
        acc += n
    return [p for p in a if p[5]], [p for p in b if p[5]]


class HipBackend:
    """Drop-in for `GpuBackend` (orca-backend-gpu/src/backend.rs:45-50)."""

    def __init__(self, ctx: Context | None = None, deferred: bool = True, lazy: bool = True, fold: bool = True,
                 overlap: bool | None = None):
        self.ctx = ctx if ctx is not None else Context(0)
        # Part of a fused optimizer pass on the second stream (module docstring); off
        # (or ORCA_HIP_OVERLAP=0), the whole pass runs on the context stream.
        self.overlap = os.environ.get("ORCA_HIP_OVERLAP", "1") != "0" if overlap is None else overlap
        # Backward products (a transposed operand) leave marks once a fused optimizer pass has
        # asked for them (the last few kept: the pass splits its side-stream part at the one
        # before the last weight gradient).
        self._marking = False
        self._recent = collections.deque(maxlen=8)
        # The side-stream part: side_frac of it on side_bpc blocks per CU beside the product
        # after the first weight gradients, the rest on the full grid once the product before
        # the last weight gradient is done (which leaves CUs idle beside it).
        self.side_frac = float(os.environ.get("ORCA_HIP_OPT_SIDE_FRAC", "70")) / 100.0
        self.side_bpc = int(os.environ.get("ORCA_HIP_OPT_SIDE_BPC", "3")) or -1
        # The identity-reduction memo and the deferred column sum (module
        # docstring); off, every sum_to_shape runs its kernel at once.
        self.deferred = deferred
        # Lazy elementwise ops run as fused programs (module docstring); off,
        # every elementwise op runs its own kernel at once.
        self.lazy = lazy
        # Pending products whose consumer is a GEMM epilogue run with it (module
        # docstring; needs lazy); off, every product runs by itself.
        self.fold = fold
        # weak references to storages created with a pending elementwise op or product (some
        # since computed or gone; pruned when the list grows, emptied by _mutating)
        self._pending = []
        self._programs = {}  # compiled elementwise programs by chain structure

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
        if self.lazy and data.size == 1 and _numel(shape) == 1 and not math.isnan(data[0]):
            return self._const_node(float(data[0]), 1)
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
                res = self._wrap(out, M * N)
                if self._marking:
                    mark = self._mark()
                    if lv == _lib.VIEW_TRANSPOSED:  # a weight gradient X^T G and its bias gradient
                        res._made = target._made = mark
                return res
        if (self.lazy and dtype == _lib.F32 and len(lhs_shape) == 2 and len(rhs_shape) == 2
                and lhs_shape[1] == rhs_shape[0]):
            M, K, N = int(lhs_shape[0]), int(lhs_shape[1]), int(rhs_shape[1])
            if lhs.n == M * K and rhs.n == K * N and M * N > 0 and K > 0:
                out = HipStorage(None, M * N)
                out._prod = (lhs, rhs, M, K, N, lhs.transposed_shape is not None, rhs.transposed_shape is not None)
                out._fill = self._run_product
                pending = self._pending
                pending.append(_wref(out))
                if len(pending) > 4096:
                    pending[:] = [r for r in pending if (x := r()) is not None and x.pending]
                return out
        out = ctypes.c_void_p()
        dl, rl = _dims(lhs_shape)
        dr, rr = _dims(rhs_shape)
        lv = _lib.VIEW_TRANSPOSED if lhs.transposed_shape is not None else _lib.VIEW_CONTIGUOUS
        rv = _lib.VIEW_TRANSPOSED if rhs.transposed_shape is not None else _lib.VIEW_CONTIGUOUS
        _lib.call("orca_hip_matmul", self.ctx.handle, lhs.ptr, rhs.ptr, dl, rl, dr, rr, dtype, lv, rv,
                  ctypes.byref(out))
        n = _numel(lhs_shape[:-1]) * int(rhs_shape[-1])
        return self._wrap(out, n)

    def _run_product(self, st: HipStorage) -> None:
        """The _fill of a pending product: runs it by itself (orca_hip_matmul)."""
        lhs, rhs, M, K, N, lt, rt = st._prod
        st._prod = None
        out = ctypes.c_void_p()
        dl, rl = _dims((M, K))
        dr, rr = _dims((K, N))
        _lib.call("orca_hip_matmul", self.ctx.handle, lhs.ptr, rhs.ptr, dl, rl, dr, rr, _lib.F32,
                  _lib.VIEW_TRANSPOSED if lt else _lib.VIEW_CONTIGUOUS,
                  _lib.VIEW_TRANSPOSED if rt else _lib.VIEW_CONTIGUOUS, ctypes.byref(out))
        st._buf = Buffer(self.ctx, out.value, 4 * M * N)
        if self._marking and (lt or rt):  # a backward product
            mark = self._mark()
            if lt:  # a weight gradient X^T G
                st._made = mark

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

    # ---- lazy elementwise ops ----
    def _ew(self, op: int, operands, n: int, scalar: float = 0.0) -> HipStorage:
        """A pending elementwise op over equally long operands (lazy transposes are
        materialised first).  Operands whose pending chains would push this one past the
        interpreter's limits are run first."""
        for o in operands:
            if type(o) is HipStorage and o.transposed_shape is not None:
                operands = tuple(o if type(o) is _Broadcast else self._plain(o) for o in operands)
                break
        while True:
            ops, leaves = 1, 0
            for o in operands:
                if o._expr is not None:
                    ops += o._ew_ops
                    leaves += o._ew_leaves
                else:
                    leaves += 1
            if ops <= EW_MAX_OPS // 2 and leaves <= EW_MAX_INPUTS:
                break
            biggest = max((o for o in operands if o._expr is not None), key=lambda o: o._ew_ops)
            self._flush(biggest)
        out = HipStorage(None, n)
        out._expr = (self, op, operands, scalar)
        out._ew_ops = ops
        out._ew_leaves = leaves
        pending = self._pending
        pending.append(_wref(out))
        if len(pending) > 4096:
            pending[:] = [r for r in pending if (x := r()) is not None and x.pending]
        return out

    def _lazy_ok(self, dtype, *operands) -> bool:
        if not self.lazy or dtype != _lib.F32:
            return False
        n = operands[0].n
        for o in operands:
            if o.n != n:
                return False
        return True

    def _flush(self, root: HipStorage) -> None:
        """Runs root's pending elementwise chain as one program; pending values in the chain
        that are referenced from outside it (beyond the chain's own operand links) are
        written too.  A chain's program (register allocation and instructions) is compiled
        once per structure -- opcodes, operand slots, outputs -- and reused with the
        chain's scalars written into it.  Falls back to running the operands' chains first
        when the program would exceed the interpreter's registers or outputs."""
        order, leaves, ref, inner, sig, scalars = [], [], {}, {}, [], []

        def visit(node):  # post-order (chains hold at most EW_MAX_OPS / 2 ops)
            refs = []
            for c in node._expr[2]:
                i = ref.get(id(c))
                if c._expr is None:  # an input: -1, -2, ...
                    if i is None:
                        i = ref[id(c)] = -1 - len(leaves)
                        leaves.append(c)
                else:
                    inner[id(c)] = inner.get(id(c), 0) + 1
                    if i is None:
                        i = ref[id(c)] = visit(c)
                refs.append(i)
            k = len(order)
            order.append(node)
            e = node._expr
            sig.append((e[1], *refs))
            scalars.append(e[3])
            return k

        visit(root)
        visit = None  # the closure refers to itself: break that cycle, which holds the chain's storages
        # externally referenced: references beyond the chain's links, the `order` list and
        # getrefcount's own argument
        out_idx = []
        for k in range(len(order) - 1):
            if sys.getrefcount(order[k]) > inner.get(id(order[k]), 0) + 2:
                out_idx.append(k)
        out_idx.append(len(order) - 1)  # the root
        if self.fold and type(leaves[0]) is HipStorage and leaves[0]._prod is not None:
            if self._fold(order, leaves, sig, out_idx):
                return
        key = (tuple(sig), tuple(out_idx), len(leaves))
        prog = self._programs.get(key)
        if prog is None:
            prog = self._programs[key] = self._compile(sig, out_idx, len(leaves))
        if prog is False:
            return self._flush_operands_first(root)
        instrs, oregs, n_regs, scalar_at, written = prog
        if scalar_at:
            cur = [scalars[k] for k in scalar_at]
            if cur != written:
                for k, v in zip(scalar_at, cur):
                    _SCALAR.pack_into(instrs, _INSTR.size * k + 8, v)
                prog[4] = cur
        n = root.n
        bufs = [self.ctx.alloc(4 * max(n, 1)) for _ in out_idx]
        ins = (EwInput * max(1, len(leaves)))(
            *[(lf.ptr, lf.div, lf.mod) if type(lf) is _Broadcast else (lf.ptr, 1, n) for lf in leaves])
        outs = (ctypes.c_void_p * len(out_idx))(*[b.ptr for b in bufs])
        _lib.call("orca_hip_ew_program", self.ctx.handle, n, ins, len(leaves), outs, oregs, len(out_idx), instrs,
                  len(order), n_regs)
        for k, b in zip(out_idx, bufs):
            X = order[k]
            X._buf, X._expr, X._ew_ops, X._ew_leaves = b, None, 0, 1

    # Chains that are a GEMM epilogue over their first input, a pending product P (leaf -1):
    # add(P, expand(b)) with b broadcast along rows, optionally relu of it, and
    # relu_backward(P, z).
    _FOLD_BIAS = ((EW_COPY, -2), (EW_ADD, -1, 0))
    _FOLD_BIAS_RELU = ((EW_COPY, -2), (EW_ADD, -1, 0), (EW_RELU, 1))
    _FOLD_MASK = ((EW_RELU_BW, -1, -2),)
    # ... and its identity sum_to_shape (0 + x, Linear's expand-both broadcast in backward).
    # A product never holds -0 (every sum starts from +0 and adds in round-to-nearest, where
    # +0 + -0 = +0) and the mask writes +0, so 0 + x is x bit for bit (a NaN stays the same
    # quiet NaN): both values share one buffer.
    _FOLD_MASK_IDENT = ((EW_RELU_BW, -1, -2), (EW_SUM_VISIT, 0))

    @staticmethod
    def _narrow(kind, lt, rt, N, K) -> bool:
        """Whether orca_hip_gemm runs the product on its narrow kernels with this epilogue: the
        planner's rule (orcaml_amd/csrc/gemm.hip plan_gemm).  A fold is taken only where the
        plain product and the one with the epilogue run on the same kernel (the same sums)."""
        if not lt and not rt and N <= 16:
            return kind in (_lib.EPI_NONE, _lib.EPI_BIAS)
        if not lt and rt and K <= 16:
            return kind in (_lib.EPI_NONE, _lib.EPI_RELU_MASK, _lib.EPI_RELU_MASK_PRE)
        if lt and not rt and N <= 16:
            return kind == _lib.EPI_NONE
        return False

    def _fold(self, order, leaves, sig, out_idx) -> bool:
        """Runs the chain as its product's epilogue when it is one of the three forms above.
        The `leaves` list, the one operand tuple that holds the product, `prod` and
        getrefcount's argument account for 4 references to it; a product referenced beyond
        them (a gradient the tape holds) is written as well by the mask epilogue, and is not
        folded into the bias ones."""
        prod = leaves[0]
        if prod._fill is None:
            return False
        shared = sys.getrefcount(prod) > 4
        lhs, rhs, M, K, N, lt, rt = prod._prod
        sig = tuple(sig)
        pre = None
        if (sig == self._FOLD_MASK and out_idx == [0]) or (sig == self._FOLD_MASK_IDENT and out_idx in ([0, 1], [1])):
            z = leaves[1]
            if type(z) is not HipStorage or z.transposed_shape is not None or z.n != M * N:
                return False
            kind, bias, mask = _lib.EPI_RELU_MASK_PRE if shared else _lib.EPI_RELU_MASK, None, z
        elif shared:
            return False
        elif (sig == self._FOLD_BIAS and out_idx == [1]) or (sig == self._FOLD_BIAS_RELU and out_idx in ([1, 2], [2])):
            b = leaves[1]
            if type(b) is not _Broadcast or b.div != 1 or b.mod != N or b.src.n != N or b.src.transposed_shape:
                return False
            kind = _lib.EPI_BIAS if len(sig) == 2 else (_lib.EPI_BIAS_RELU_PRE if out_idx == [1, 2] else
                                                        _lib.EPI_BIAS_RELU)
            bias, mask = b.src, None
        else:
            return False
        if self._narrow(kind, lt, rt, N, K) != self._narrow(_lib.EPI_NONE, lt, rt, N, K):
            return False  # the plain product runs on another kernel (other sums, other bits)
        # The operands first: pending work they need is launched before a wait on a mark that a
        # bias or mask written on the second stream brings in.
        lp, rp = lhs.ptr, rhs.ptr
        c = self.ctx.alloc(4 * M * N)
        e = _lib.Epilogue(kind, bias.ptr if bias is not None else None, mask.ptr if mask is not None else None,
                          N if mask is not None else 0, None)
        if kind in (_lib.EPI_BIAS_RELU_PRE, _lib.EPI_RELU_MASK_PRE):
            pre = self.ctx.alloc(4 * M * N)
            e.pre = pre.ptr
        _lib.call("orca_hip_gemm", self.ctx.handle, int(lt), int(rt), M, N, K, lp, M if lt else K, rp,
                  K if rt else N, c.ptr, N, ctypes.byref(e))
        if self._marking and (lt or rt):  # a backward product
            self._mark()
        prod._prod = prod._fill = None
        if kind == _lib.EPI_RELU_MASK_PRE:
            prod._buf, pre = pre, None  # the product itself, for its other holders
        if sig == self._FOLD_MASK_IDENT:
            outs = [c] * len(out_idx)  # the masked product and its identity sum: one buffer
        else:
            outs = [c] if pre is None else [pre, c]  # out_idx order: the add (pre-activation) before the relu
        for k, buf in zip(out_idx, outs):
            X = order[k]
            X._buf, X._expr, X._ew_ops, X._ew_leaves = buf, None, 0, 1
        return True

    @staticmethod
    def _compile(sig, out_idx, n_leaves):
        """[instructions, output registers, register count, indices of the instructions
        that carry a scalar, the scalars last written into them] of a chain, or False when
        it needs more registers or outputs than the interpreter has.  Inputs take registers
        0..n_leaves-1; each op result takes the lowest free register; a register is freed
        after its value's last use (an output keeps its register to the end)."""
        if len(out_idx) > EW_MAX_OUTPUTS or len(sig) > EW_MAX_OPS:
            return False
        last = {}
        for k, (_, *refs) in enumerate(sig):
            for r in refs:
                last[r] = k
        outs = set(out_idx)
        free, reg, n_regs = [], {}, n_leaves
        instrs = bytearray()
        scalar_at = []
        for k, (op, *refs) in enumerate(sig):
            regs = [(-1 - r) if r < 0 else reg[r] for r in refs]
            for r in set(refs):
                if last[r] == k and (r < 0 or r not in outs):
                    free.append((-1 - r) if r < 0 else reg[r])
            if free:
                free.sort()
                dst = free.pop(0)
            else:
                dst = n_regs
                n_regs += 1
            reg[k] = dst
            regs += [regs[0]] * (3 - len(regs))
            instrs += _INSTR.pack(op, dst, regs[0], regs[1], regs[2], 0.0)
            if op in (EW_MUL_SCALAR, EW_ADD_SCALAR):
                scalar_at.append(k)
        if n_regs > EW_MAX_REGS:
            return False
        oregs = (ctypes.c_uint8 * len(out_idx))(*[reg[k] for k in out_idx])
        return [ctypes.create_string_buffer(bytes(instrs), max(1, len(instrs))), oregs, n_regs, scalar_at, None]

    def _flush_operands_first(self, root: HipStorage) -> None:
        for c in root._expr[2]:
            if c._expr is not None:
                self._flush(c)
        self._flush(root)

    def _unary(self, name, op, s, shape, dtype):
        if self._lazy_ok(dtype, s):
            return self._ew(op, (s,), s.n)
        return self._op1(name, s, shape, dtype)

    def _binary(self, name, op, a, b, shape, dtype):
        if self._lazy_ok(dtype, a, b):
            return self._ew(op, (a, b), a.n)
        return self._op2(name, a, b, shape, dtype)

    def add(self, a, b, shape, dtype=_lib.F32):
        if self._lazy_ok(dtype, a, b):
            r = self._fold_const(EW_ADD, a, b)
            if r is not None:
                return r
        return self._binary("add", EW_ADD, a, b, shape, dtype)

    def sub(self, a, b, shape, dtype=_lib.F32):
        return self._binary("sub", EW_SUB, a, b, shape, dtype)

    def mul(self, a, b, shape, dtype=_lib.F32):
        if self._lazy_ok(dtype, a, b):
            r = self._fold_const(EW_MUL, a, b)
            if r is not None:
                return r
        return self._binary("mul", EW_MUL, a, b, shape, dtype)

    def div(self, a, b, shape, dtype=_lib.F32):
        return self._binary("div", EW_DIV, a, b, shape, dtype)

    def mul_scalar(self, s, scalar: float, shape, dtype=_lib.F32):
        if self._lazy_ok(dtype, s):
            f = float(ctypes.c_float(scalar).value)
            c = self._const_src(s)
            if c is not None:
                v = np.float32(c._const) * np.float32(f)
                if not math.isnan(v):
                    return self._const_node(float(v), s.n)
            return self._ew(EW_MUL_SCALAR, (s,), s.n, f)
        s = self._plain(s)
        out = ctypes.c_void_p()
        d, r = _dims(shape)
        _lib.call("orca_hip_mul_scalar", self.ctx.handle, s.ptr, ctypes.c_float(scalar), d, r, dtype,
                  ctypes.byref(out))
        return self._wrap(out, _numel(shape))

    def relu(self, s, shape, dtype=_lib.F32):
        return self._unary("relu", EW_RELU, s, shape, dtype)

    def sigmoid(self, s, shape, dtype=_lib.F32):
        return self._unary("sigmoid", EW_SIGMOID, s, shape, dtype)

    def exp(self, s, shape, dtype=_lib.F32):
        return self._unary("exp", EW_EXP, s, shape, dtype)

    def log(self, s, shape, dtype=_lib.F32):
        return self._unary("log", EW_LOG, s, shape, dtype)

    def sqrt(self, s, shape, dtype=_lib.F32):
        return self._unary("sqrt", EW_SQRT, s, shape, dtype)

    def relu_backward(self, g, x, shape, dtype=_lib.F32):
        return self._binary("relu_backward", EW_RELU_BW, g, x, shape, dtype)

    def sigmoid_backward(self, g, y, shape, dtype=_lib.F32):
        return self._binary("sigmoid_backward", EW_SIGMOID_BW, g, y, shape, dtype)

    def exp_backward(self, g, y, shape, dtype=_lib.F32):
        return self._binary("exp_backward", EW_EXP_BW, g, y, shape, dtype)

    def log_backward(self, g, x, shape, dtype=_lib.F32):
        return self._binary("log_backward", EW_LOG_BW, g, x, shape, dtype)

    def sqrt_backward(self, g, y, shape, dtype=_lib.F32):
        return self._binary("sqrt_backward", EW_SQRT_BW, g, y, shape, dtype)

    def div_backward_lhs(self, g, r, shape, dtype=_lib.F32):
        return self._binary("div_backward_lhs", EW_DIV, g, r, shape, dtype)

    def div_backward_rhs(self, g, l, r, shape, dtype=_lib.F32):
        if self._lazy_ok(dtype, g, l, r):
            return self._ew(EW_DIV_BW_RHS, (g, l, r), g.n)
        g, l, r = self._plain(g), self._plain(l), self._plain(r)
        out = ctypes.c_void_p()
        d, rk = _dims(shape)
        _lib.call("orca_hip_div_backward_rhs", self.ctx.handle, g.ptr, l.ptr, r.ptr, d, rk, dtype, ctypes.byref(out))
        return self._wrap(out, _numel(shape))

    def accumulate_grad(self, a, b):
        if self._lazy_ok(_lib.F32, a, b):
            r = self._fold_const(EW_ADD, a, b)
            return r if r is not None else self._ew(EW_ADD, (a, b), a.n)
        a, b = self._plain(a), self._plain(b)
        out = ctypes.c_void_p()
        _lib.call("orca_hip_accumulate_grad", self.ctx.handle, a.ptr, b.ptr, a.n, ctypes.byref(out))
        return self._wrap(out, a.n)

    def expand(self, s, in_shape, out_shape, dtype=_lib.F32):
        if tuple(in_shape) == tuple(out_shape) and dtype == _lib.F32:
            return s  # identity broadcast: share the storage
        c = self._const_src(s) if self.lazy and dtype == _lib.F32 else None
        if c is not None and len(out_shape) >= len(in_shape):
            n = _numel(out_shape)
            if n > 0 and s.n == _numel(in_shape):
                return self._ew(EW_COPY, (_Broadcast(c, n, 1, 1),), n)
        if self.lazy and dtype == _lib.F32 and len(out_shape) >= len(in_shape):
            m = _broadcast_map(tuple(int(d) for d in in_shape), tuple(int(d) for d in out_shape))
            n = _numel(out_shape)
            if m is not None and n > 0 and s.n == _numel(in_shape):
                return self._ew(EW_COPY, (_Broadcast(self._plain(s), n, *m),), n)
        return self._reshape_like("expand", s, in_shape, out_shape, dtype)

    def sum_to_shape(self, s, in_shape, out_shape, dtype=_lib.F32):
        in_shape, out_shape = tuple(int(d) for d in in_shape), tuple(int(d) for d in out_shape)
        if self.deferred and dtype == _lib.F32 and s.transposed_shape is None and s._fill is None:
            if in_shape == out_shape:
                if s.ident is None:
                    s.ident = (self._ew(EW_SUM_VISIT, (s,), s.n) if self.lazy else
                               self._reshape_like("sum_to_shape", s, in_shape, out_shape, dtype))
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

    # ---- one-element constants ----
    # A one-element upload (the backward seed, Tensor::scalar) stays on the host until the
    # device needs it.  An expand of it is a single-value broadcast of the same storage, and
    # add / mul / accumulate_grad with such a value take it as an instruction's scalar
    # (x + c, x * c: the ops' own f32 operations; the constant is never NaN, so the operand
    # order does not matter), mul_scalar of it is computed on the host in f32.
    def _const_node(self, value: float, n: int) -> HipStorage:
        c = HipStorage(None, 1)
        c._const = value
        c._fill = lambda st, v=value: self._upload_const(st, v)
        return c if n == 1 else self._ew(EW_COPY, (_Broadcast(c, n, 1, 1),), n)

    def _upload_const(self, st: HipStorage, value: float) -> None:
        data = np.array([value], np.float32)
        out = ctypes.c_void_p()
        d, r = _dims((1,))
        _lib.call("orca_hip_from_f32_slice", self.ctx.handle, d, r, data.ctypes.data_as(ctypes.c_void_p), 1,
                  ctypes.byref(out))
        st._buf = Buffer(self.ctx, out.value, 4)

    @staticmethod
    def _const_src(s):
        """The one-element constant storage whose value s holds everywhere, or None."""
        if type(s) is not HipStorage:
            return None
        if s._const is not None:
            return s
        e = s._expr
        if e is not None and e[1] == EW_COPY:
            b = e[2][0]
            if type(b) is _Broadcast and b.mod == 1 and type(b.src) is HipStorage and b.src._const is not None:
                return b.src
        return None

    def _fold_const(self, op, a, b):
        """add / mul (op EW_ADD / EW_MUL) with a constant operand as a scalar instruction, or of
        two constants on the host; None when neither operand is a constant."""
        ca, cb = self._const_src(a), self._const_src(b)
        if ca is None and cb is None:
            return None
        n = a.n
        if ca is not None and cb is not None:
            x, y = np.float32(ca._const), np.float32(cb._const)
            v = x + y if op == EW_ADD else x * y
            return None if math.isnan(v) else self._const_node(float(v), n)
        x, c = (a, cb._const) if cb is not None else (b, ca._const)
        return self._ew(EW_ADD_SCALAR if op == EW_ADD else EW_MUL_SCALAR, (x,), n, c)

    def _mutating(self, *storages) -> None:
        """Before an in-place update: values derived lazily from these storages are computed
        from their current contents, and their memoised identity reductions are dropped."""
        pending, self._pending = self._pending, []
        for r in pending:
            node = r()
            if node is not None and node.pending:
                node.buf  # runs its pending elementwise chain or product
        for s in storages:
            if s.colsum_waiters:
                for ref in s.colsum_waiters:
                    t = ref()
                    if t is not None:
                        t.buf  # runs a pending fill
            s.colsum_waiters = None
            s.ident = None
            if s._const is not None:
                s.buf  # a constant not yet on the device is uploaded before it changes there
                s._const = None

    def reshape(self, s, in_shape, out_shape, dtype=_lib.F32):
        n_in = _numel(in_shape)
        n_out = _numel(out_shape)
        if n_in != n_out:
            raise _lib.OrcaHipError(_lib.ERR_SHAPE, f"Shape mismatch during reshape: expected {n_in} elements, "
                                                    f"got {n_out} elements")
        return self._plain(s)

    def max_to_shape(self, s, in_shape, out_shape, dtype=_lib.F32):
        if tuple(in_shape) == tuple(out_shape) and self._lazy_ok(dtype, s):
            return self._ew(EW_MAX_VISIT, (s,), s.n)
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

    # ---- flat arenas and one-launch optimizer passes ----
    def arena(self, n: int, fill: float | None = None) -> Buffer:
        """A flat device buffer of n floats (set to `fill` if given)."""
        buf = self.ctx.alloc(4 * max(n, 1))
        if fill is not None and n:
            self.ctx.fill(buf, fill, n)
        return buf

    @staticmethod
    def view(arena: Buffer, offset: int, n: int) -> HipStorage:
        """The storage of n floats at `offset` (floats) of an arena."""
        return HipStorage(_ArenaView(arena, offset, n), n)

    def copy_into(self, dst: HipStorage, src: HipStorage) -> None:
        """dst <- src, device to device (dst a fresh arena slice nobody reads yet)."""
        src = self._plain(src)
        if src.n:
            self.ctx.d2d(dst.buf, src.buf, 4 * src.n)

    def adamw_multi_(self, segs, lr: float, beta1: float, beta2: float, eps: float, weight_decay: float,
                     t: int) -> None:
        """One AdamW pass over many parameters (orca_hip_adamw_multi): segs holds
        (p_src, p_dst, g, m, v, n) storages; p_dst, m and v are written."""
        rows = [(self._plain(ps), pd, self._plain(g), m, v, n) for ps, pd, g, m, v, n in segs]
        self._mutating(*[r[k] for r in rows for k in (1, 3, 4)])

        def launch(ptrs):
            table = (_lib.OptSegment * max(1, len(ptrs)))(*ptrs)
            _lib.call("orca_hip_adamw_multi", self.ctx.handle, table, len(ptrs), lr, beta1, beta2, eps, weight_decay,
                      t)

        self._optimizer_pass(rows, 2, (1, 3, 4), lambda r: (r[0].ptr, r[1].ptr, r[2].ptr, r[3].ptr, r[4].ptr, r[5]),
                             launch)

    def _mark(self) -> _Mark:
        mark = _Mark(self.ctx)
        self._recent.append(mark)
        return mark

    def _optimizer_pass(self, rows, gi: int, written, ptrs_of, launch) -> None:
        """Runs launch(pointer rows) for an optimizer pass; rows[k][gi] is a gradient, rows[k][w]
        for w in `written` the storages written (parameter, moments).  With overlap, the rows whose
        gradients come from a weight-gradient product before the latest one among them run first,
        on the side stream, after that product (beside the rest of the backward); the storages
        they write are marked, and what they only read is kept until the context stream waits
        for the mark.  The other rows (gradients
        of the latest product, or of no marked product) run on the context stream.  Gradients
        still pending are computed first, the last row's last, as a backward pass makes them.
        The side-stream part is split like the trainer's update: side_frac of it on a bounded grid
        beside the product after those gradients, the rest on the full grid once the product
        before the latest weight gradient is done."""
        self._marking = self.overlap
        if self.overlap:  # gradients still pending run now, the last parameter's last (backward order)
            for r in reversed(rows):
                if r[gi].pending:
                    r[gi].buf
        marks = [r[gi]._made for r in rows] if self.overlap else []
        known = [m for m in marks if m is not None]
        last = max((m.seq for m in known), default=None)
        early = [m for m in known if m.seq != last]
        side = [r for r, m in zip(rows, marks) if m is not None and m.seq != last] if early else []
        here = [r for r, m in zip(rows, marks) if m is None or m.seq == last] if early else rows
        if side:
            after = max(early, key=lambda m: m.seq)  # the same stream's earlier marks come before it
            mid = max((m for m in self._recent if after.seq < m.seq < last), key=lambda m: m.seq, default=None)
            ptrs = [ptrs_of(r) for r in side]  # pending values settled on the context stream first
            parts = [(after, self.side_bpc, ptrs)]
            if mid is not None and self.side_frac < 1.0:
                a, b = _split_rows(ptrs, self.side_frac)
                parts = [(after, self.side_bpc, a), (mid, -1, b)]
            done = None
            for mark, bpc, part in parts:
                if not part:
                    continue
                self.ctx.use_side_stream(bpc)
                try:
                    mark.wait()
                    launch(part)
                    done = _Mark(self.ctx)  # the side stream's work so far
                finally:
                    self.ctx.use_side_stream(0)
            if done is not None:
                done.keep = [tuple(x for k, x in enumerate(r) if k not in written) for r in side]
                for r in side:
                    for k in written:
                        r[k]._ready = done
        if here:
            launch([ptrs_of(r) for r in here])

    def sgd_multi_(self, segs, lr: float) -> None:
        """One SGD pass over many parameters (orca_hip_sgd_multi): segs holds (p_src, p_dst, g, n)."""
        rows = [(self._plain(ps), pd, self._plain(g), n) for ps, pd, g, n in segs]
        self._mutating(*[r[1] for r in rows])

        def launch(ptrs):
            table = (_lib.OptSegment * max(1, len(ptrs)))(*ptrs)
            _lib.call("orca_hip_sgd_multi", self.ctx.handle, table, len(ptrs), lr)

        self._optimizer_pass(rows, 2, (1,), lambda r: (r[0].ptr, r[1].ptr, r[2].ptr, None, None, r[3]), launch)

    def sgd_step_(self, p: HipStorage, g: HipStorage, n: int, lr: float) -> None:
        """In place on p (orca_hip_sgd_step)."""
        g = self._plain(g)
        self._mutating(p)
        _lib.call("orca_hip_sgd_step", self.ctx.handle, p.ptr, g.ptr, n, lr)
