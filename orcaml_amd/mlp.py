"""Device-resident MLP training step (orca_hip_mlp_* in include/orca_hip.h).

Equivalent to the reference's
    model = nn.Sequential(nn.Linear(d0, d1), nn.ReLU(), ..., nn.Linear(dL-1, dL))
    loss = nn.CrossEntropyLoss()(model(x), onehot); loss.backward(); opt.step()
(python/orca/nn/{container,linear,activation,loss}.py, python/orca/optim)
with fused HIP kernels and flat parameter / gradient / moment arenas.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .device import Context


class MLPTrainer:
    def __init__(self, ctx: Context, dims, batch: int, kind: str = "sgd", lr: float = 0.01,
                 weight_decay: float = 0.0, betas=(0.9, 0.999), eps: float = 1e-8):
        if kind not in ("sgd", "adamw"):
            raise ValueError(f"unknown optimizer {kind!r}")
        self.ctx = ctx
        self.kind = kind
        self.dims = tuple(int(d) for d in dims)
        self.batch = int(batch)
        self.n_layers = len(self.dims) - 1
        opt = _lib.Optim(0 if kind == "sgd" else 1, lr, weight_decay, betas[0], betas[1], eps)
        dd, n = _lib.dims(self.dims)
        h = ctypes.c_void_p()
        _lib.call("orca_hip_mlp_create", ctx.handle, dd, self.n_layers, self.batch, ctypes.byref(opt), ctypes.byref(h))
        self.handle = h

    def close(self) -> None:
        if self.handle and self.ctx.handle:
            _lib.call("orca_hip_mlp_destroy", self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def param_shape(self, i: int):
        l = i // 2
        return (self.dims[l], self.dims[l + 1]) if i % 2 == 0 else (1, self.dims[l + 1])

    def set_params(self, params) -> None:
        for i, p in enumerate(params):
            p = np.ascontiguousarray(p, np.float32)
            _lib.call("orca_hip_mlp_set_param", self.handle, i, p.ctypes.data_as(ctypes.c_void_p), p.size)

    def _read(self, fn: str, i: int, *extra) -> np.ndarray:
        shape = self.param_shape(i)
        out = np.empty(shape, np.float32)
        _lib.call(fn, self.handle, *extra, i, out.ctypes.data_as(ctypes.c_void_p), out.size)
        return out

    def params(self):
        return [self._read("orca_hip_mlp_get_param", i) for i in range(2 * self.n_layers)]

    def grads(self):
        return [self._read("orca_hip_mlp_get_grad", i) for i in range(2 * self.n_layers)]

    def moments(self, which: int):
        return [self._read("orca_hip_mlp_get_moment", i, which) for i in range(2 * self.n_layers)]

    def set_batch(self, x: np.ndarray, onehot: np.ndarray | None = None, labels: np.ndarray | None = None) -> None:
        x = np.ascontiguousarray(x, np.float32)
        if x.shape != (self.batch, self.dims[0]):
            raise ValueError(f"x must be {(self.batch, self.dims[0])}, got {x.shape}")
        oh = lb = None
        if onehot is not None:
            onehot = np.ascontiguousarray(onehot, np.float32)
            if onehot.shape != (self.batch, self.dims[-1]):
                raise ValueError("one-hot targets have the wrong shape")
            oh = onehot.ctypes.data_as(ctypes.c_void_p)
        if labels is not None:
            labels = np.ascontiguousarray(labels, np.int32)
            if labels.shape != (self.batch,):
                raise ValueError("labels have the wrong shape")
            lb = labels.ctypes.data_as(ctypes.c_void_p)
        _lib.call("orca_hip_mlp_set_batch", self.handle, x.ctypes.data_as(ctypes.c_void_p), oh, lb)

    def step(self) -> None:
        _lib.call("orca_hip_mlp_step", self.handle)

    def metrics(self):
        loss = ctypes.c_float()
        correct = ctypes.c_int64()
        _lib.call("orca_hip_mlp_read_metrics", self.handle, ctypes.byref(loss), ctypes.byref(correct))
        return float(loss.value), int(correct.value)

    def logits(self) -> np.ndarray:
        out = np.empty((self.batch, self.dims[-1]), np.float32)
        _lib.call("orca_hip_mlp_get_logits", self.handle, out.ctypes.data_as(ctypes.c_void_p), out.size)
        return out

    def preds(self) -> np.ndarray:
        out = np.empty(self.batch, np.int32)
        _lib.call("orca_hip_mlp_get_preds", self.handle, out.ctypes.data_as(ctypes.c_void_p), out.size)
        return out

    def activation(self, layer: int) -> np.ndarray:
        """ReLU output of layer `layer` (< L-1) or the logits (layer L-1) of the last step."""
        out = np.empty((self.batch, self.dims[layer + 1]), np.float32)
        _lib.call("orca_hip_mlp_get_activation", self.handle, layer, out.ctypes.data_as(ctypes.c_void_p), out.size)
        return out

    def step_count(self) -> int:
        t = ctypes.c_int64()
        _lib.call("orca_hip_mlp_get_step_count", self.handle, ctypes.byref(t))
        return int(t.value)

    def set_moments(self, which: int, arrays) -> None:
        """Restores AdamW's m (which = 0) or v (which = 1) for every parameter."""
        for i, a in enumerate(arrays):
            a = np.ascontiguousarray(a, np.float32)
            _lib.call("orca_hip_mlp_set_moment", self.handle, which, i, a.ctypes.data_as(ctypes.c_void_p), a.size)

    def set_step_count(self, t: int) -> None:
        _lib.call("orca_hip_mlp_set_step_count", self.handle, int(t))

    def set_update_shard(self, index: int, count: int) -> None:
        """One rank's share of a data-parallel step with the optimizer state sharded over
        `count` ranks: each step's update passes cover slice `index` of their ranges only
        (the other slices keep their current values); count = 1 restores the whole update."""
        _lib.call("orca_hip_mlp_set_update_shard", self.handle, int(index), int(count))

    def save(self, path: str) -> None:
        """Parameters (named as the equivalent nn.Sequential's) and AdamW state, as safetensors."""
        from .serialize import save_trainer
        save_trainer(path, self)

    def load(self, path: str) -> None:
        from .serialize import load_trainer
        load_trainer(path, self)
