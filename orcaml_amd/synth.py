"""Seeded synthetic inputs for the MLP training-step workloads.

The reference draws inputs and weights from an unseeded thread RNG
(orca-tensor/src/tensor.rs:63,90,110), so identical inputs for the HIP backend
and the CPU oracle come from this counter-based generator instead:

* stream(seed, tensor_id): SplitMix64 started at
  ``seed ^ (tensor_id * 0x9E3779B97F4A7C15)``; output i is the (i+1)-th
  SplitMix64 value, so any element can be produced independently;
* uniform f32 in [0,1): ``(u64 >> 40) * 2**-24`` (exact in f32);
* integers in [0, k): ``u64 % k``;
* normal: Box-Muller in f64 on the pair (2j, 2j+1) -> element 2j uses cos,
  2j+1 uses sin; ``u1 = ((a >> 11) + 1) * 2**-53``, ``u2 = (b >> 11) * 2**-53``;
  the f64 value ``mu + sigma * n`` is rounded to f32;
* Kaiming-uniform weights: ``f32((2u - 1) * bound)`` with u the f64 uniform
  above and ``bound = 1/sqrt(fan_in)`` (python/orca/nn/init.py:40-50 with
  a = sqrt(5): gain sqrt(1/3), bound = sqrt(3) * gain / sqrt(fan_in));
  biases are zero.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream(seed: int, tensor_id: int, n: int, offset: int = 0) -> np.ndarray:
    """Raw SplitMix64 outputs offset .. offset+n-1 of one tensor's stream."""
    s0 = np.uint64((seed ^ ((tensor_id * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF)) & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        idx = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        return _mix(s0 + idx * GAMMA)


def uniform(seed: int, tensor_id: int, shape, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    u = (stream(seed, tensor_id, n) >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
    if lo == 0.0 and hi == 1.0:
        return u.reshape(shape)
    return (lo + (hi - lo) * u.astype(np.float64)).astype(np.float32).reshape(shape)


def integers(seed: int, tensor_id: int, n: int, k: int) -> np.ndarray:
    return (stream(seed, tensor_id, n) % np.uint64(k)).astype(np.int32)


def normal_range(seed: int, tensor_id: int, offset: int, count: int, mu: float = 0.0,
                 sigma: float = 1.0) -> np.ndarray:
    """Elements offset .. offset+count-1 of the flat normal stream (offset even)."""
    if offset % 2:
        raise ValueError("offset must be even (elements come in Box-Muller pairs)")
    out = np.empty(count, np.float32)
    pairs = (count + 1) // 2
    for p0 in range(0, pairs, _CHUNK):
        np_ = min(_CHUNK, pairs - p0)
        raw = stream(seed, tensor_id, 2 * np_, offset=offset + 2 * p0)
        a, b = raw[0::2], raw[1::2]
        u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
        u2 = (b >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
        r = np.sqrt(-2.0 * np.log(u1))
        th = 2.0 * np.pi * u2
        vals = np.empty(2 * np_, np.float64)
        vals[0::2] = r * np.cos(th)
        vals[1::2] = r * np.sin(th)
        lo = 2 * p0
        hi = min(count, lo + 2 * np_)
        out[lo:hi] = (mu + sigma * vals[: hi - lo]).astype(np.float32)
    return out


def normal(seed: int, tensor_id: int, shape, mu: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    return normal_range(seed, tensor_id, 0, int(np.prod(shape)), mu, sigma).reshape(shape)


def kaiming_weight(seed: int, tensor_id: int, fan_in: int, fan_out: int) -> np.ndarray:
    n = fan_in * fan_out
    u = (stream(seed, tensor_id, n) >> np.uint64(40)).astype(np.float64) * 2.0 ** -24
    bound = 1.0 / np.sqrt(float(fan_in))
    return ((2.0 * u - 1.0) * bound).astype(np.float32).reshape(fan_in, fan_out)


def one_hot(labels: np.ndarray, classes: int) -> np.ndarray:
    out = np.zeros((labels.shape[0], classes), np.float32)
    out[np.arange(labels.shape[0]), labels] = 1.0
    return out


# Tensor ids of the MLP workloads: x = 1, labels = 2, W_l = 10 + 2l, b_l = zeros.
def mlp_problem(seed: int, dims, batch: int):
    """Returns (params [W1, b1, ...], x [B, dims[0]], labels [B], onehot [B, C])."""
    x = uniform(seed, 1, (batch, dims[0]))
    labels = integers(seed, 2, batch, dims[-1])
    params = []
    for l in range(len(dims) - 1):
        params.append(kaiming_weight(seed, 10 + 2 * l, dims[l], dims[l + 1]))
        params.append(np.zeros((1, dims[l + 1]), np.float32))
    return params, x, labels, one_hot(labels, dims[-1])


# The MLP workloads of the hot path by name: generator seed, dims, batch,
# optimizer, and the number of steps their parity tests run.
MLP_SMALL = "mlp784-128-128-10_b64_sgd"
MLP_MEDIUM = "mlp784-1024-1024-10_b256_adamw"
MLP_LARGE = "mlp784-4096-4096-10_b1024_adamw"
WORKLOADS = {
    MLP_SMALL: dict(name=MLP_SMALL, seed=1, dims=(784, 128, 128, 10), batch=64,
                    opt=dict(kind="sgd", lr=0.1), steps=1),
    MLP_MEDIUM: dict(name=MLP_MEDIUM, seed=2, dims=(784, 1024, 1024, 10), batch=256,
                     opt=dict(kind="adamw", lr=1e-3, weight_decay=0.01, betas=(0.9, 0.999), eps=1e-8), steps=100),
    MLP_LARGE: dict(name=MLP_LARGE, seed=3, dims=(784, 4096, 4096, 10), batch=1024,
                    opt=dict(kind="adamw", lr=1e-3, weight_decay=0.01, betas=(0.9, 0.999), eps=1e-8), steps=1),
}
