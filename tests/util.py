"""Shared helpers of the parity tests."""
from __future__ import annotations

import numpy as np

# Tolerance of the MLP hot path for f32 losses, gradients and parameters:
# |gpu - cpu| <= ATOL + RTOL * |cpu|.
RTOL = 1e-4
ATOL = 1e-5


def assert_close(got, want, rtol: float = RTOL, atol: float = ATOL, what: str = "") -> None:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    err = np.abs(got - want)
    bound = atol + rtol * np.abs(want)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} elements outside tolerance; worst at {i}: "
                             f"got {got[i]!r} want {want[i]!r}")


def assert_close_scaled(got, want, rtol: float = RTOL, what: str = "") -> None:
    """Stricter check for tensors whose entries sit far below ATOL (e.g.
    gradients of a mean loss over a large batch): the absolute slack is
    scaled to the tensor's largest magnitude."""
    want = np.asarray(want, np.float64)
    scale = float(np.max(np.abs(want))) if want.size else 0.0
    assert_close(got, want, rtol=rtol, atol=rtol * scale + 1e-30, what=what)


def outside_tolerance(got, want, rtol: float = RTOL, atol: float = ATOL) -> int:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return int((np.abs(got - want) > atol + rtol * np.abs(want)).sum())


def int_matrix(rng: np.random.Generator, shape, lo: int = -8, hi: int = 8) -> np.ndarray:
    """Small-integer f32 data: every product sum is exact in f32."""
    return rng.integers(lo, hi, size=shape).astype(np.float32)
