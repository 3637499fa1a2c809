"""Checkpoints in the safetensors format, written and read straight from
device storage.

* save_tensors / load_tensors: orca-serialize/src/lib.rs:6-79 (one tensor per
  name with its shape and dtype; the data comes from Backend::to_bytes and
  goes back through Backend::from_bytes, orca-tensor/src/backend.rs:296-297),
  so a checkpoint never passes through a host list of floats.  Only f32 is on
  this path.
* save_optimizer / load_optimizer: AdamW's m, v and step count t, which the
  reference does not save (python/orca/optim/adamw.py:30-33 keeps them in
  Python lists).
* save_trainer / load_trainer: the device-resident MLP trainer's parameters
  under the names the equivalent nn.Sequential gives them ("0.weight",
  "0.bias", "2.weight", ...; python/orca/nn/module.py:176-184), so
  Module.load_weights of that model reads the file, plus the AdamW state.
"""
from __future__ import annotations

import numpy as np
from safetensors import safe_open
from safetensors.numpy import load_file, save_file

from .autodiff import AdStorage, OrcaError, Tensor

_F32 = np.dtype("<f4")


def save_tensors(path: str, tensors: dict, metadata: dict | None = None) -> None:
    """name -> Tensor, as a safetensors file (F32 tensors, the shapes given)."""
    arrays = {}
    for name, t in tensors.items():
        data = t.ad.inner.to_bytes(t.storage.primal)
        arrays[name] = np.frombuffer(data, _F32).reshape(t.shape)
    save_file(arrays, path, metadata=metadata)


def load_tensors(path: str, ad) -> dict:
    """The file's tensors as name -> Tensor on the backend of `ad` (no grad)."""
    out = {}
    for name, arr in load_file(path).items():
        if arr.dtype != _F32:
            raise OrcaError(f"Unsupported dtype {arr.dtype} for {name!r}: only F32 tensors are on this path")
        shape = tuple(arr.shape) if arr.ndim else (1,)
        storage = ad.inner.from_bytes(shape, np.ascontiguousarray(arr).tobytes())
        out[name] = Tensor(ad, AdStorage(storage), shape)
    return out


def read_metadata(path: str) -> dict:
    with safe_open(path, framework="numpy") as f:
        return dict(f.metadata() or {})


def save_optimizer(path: str, optim) -> None:
    """AdamW state: tensors "m.<i>", "v.<i>" (parameter order) and metadata t."""
    state = optim.state_dict()
    t = state.pop("t")
    save_tensors(path, state, metadata={"t": str(int(t))})


def load_optimizer(path: str, optim) -> None:
    ad = optim.parameters[0].tensor.ad
    state = load_tensors(path, ad)
    meta = read_metadata(path)
    if "t" not in meta:
        raise OrcaError(f"{path}: no optimizer step count in the file")
    state["t"] = int(meta["t"])
    optim.load_state_dict(state)


def trainer_param_names(n_layers: int):
    """Names of W_l, b_l in nn.Sequential(Linear, ReLU, ..., Linear): Linear l is module 2l."""
    names = []
    for l in range(n_layers):
        names += [f"{2 * l}.weight", f"{2 * l}.bias"]
    return names


def save_trainer(path: str, trainer) -> None:
    names = trainer_param_names(trainer.n_layers)
    arrays = {n: np.ascontiguousarray(p, _F32) for n, p in zip(names, trainer.params())}
    meta = {"dims": ",".join(str(d) for d in trainer.dims), "optimizer": trainer.kind}
    if trainer.kind == "adamw":
        for which, key in ((0, "m"), (1, "v")):
            for n, a in zip(names, trainer.moments(which)):
                arrays[f"adamw.{key}.{n}"] = np.ascontiguousarray(a, _F32)
        meta["adamw.t"] = str(trainer.step_count())
    save_file(arrays, path, metadata=meta)


def load_trainer(path: str, trainer) -> None:
    meta = read_metadata(path)
    dims = meta.get("dims")
    if dims is not None and tuple(int(d) for d in dims.split(",")) != trainer.dims:
        raise OrcaError(f"Shape mismatch during load_trainer: expected dims {list(trainer.dims)}, got [{dims}]")
    arrays = load_file(path)
    names = trainer_param_names(trainer.n_layers)
    missing = [n for n in names if n not in arrays]
    if missing:
        raise OrcaError(f"{path}: missing parameters {missing}")
    for i, n in enumerate(names):
        if tuple(arrays[n].shape) != trainer.param_shape(i):
            raise OrcaError(f"Shape mismatch during load_trainer: {n} expected {list(trainer.param_shape(i))}, "
                            f"got {list(arrays[n].shape)}")
    trainer.set_params([arrays[n] for n in names])
    if trainer.kind == "adamw":
        if "adamw.t" in meta:
            for which, key in ((0, "m"), (1, "v")):
                trainer.set_moments(which, [arrays[f"adamw.{key}.{n}"] for n in names])
            trainer.set_step_count(int(meta["adamw.t"]))
        else:  # weights only: a fresh optimizer state
            zeros = [np.zeros(trainer.param_shape(i), np.float32) for i in range(len(names))]
            trainer.set_moments(0, zeros)
            trainer.set_moments(1, zeros)
            trainer.set_step_count(0)
