"""The tolerance policy for comparing float32 transforms with the float64 references.

Restates python/spectral/testing.py:26-78 of the reference: per transform, the normwise relative
L2 error ||actual - expected|| / ||expected|| must not exceed 8 * eps32 * max(1, log2 N)
(N = N1 N2 in 2D). Float32 error grows with the stage count log2 N; the factor 8 leaves room for
fast twiddle evaluation. Real bugs give errors of order 1.

TEST INFRASTRUCTURE: see oracle/__init__.py for who may import this.
"""

from __future__ import annotations

import math

import numpy as np

FLOAT32_EPS = float(np.finfo(np.float32).eps)  # 2^-23
FFT_TOLERANCE_FACTOR = 8.0

POW2_SIZES = [2**p for p in range(1, 13)]  # 2 .. 4096, the single-kernel range
BATCHES = [1, 3, 64]


def fft_tolerance(n: int, eps: float = FLOAT32_EPS) -> float:
    """Largest relative L2 error allowed for one transform of n points (testing.py:33-35)."""
    return FFT_TOLERANCE_FACTOR * eps * max(1.0, math.log2(n))


def to_numpy(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.asarray(x)


def relative_error(actual, expected, axes: tuple[int, ...]) -> np.ndarray:
    """||actual - expected|| / ||expected|| per transform, norms over `axes` (testing.py:44-52)."""
    a = to_numpy(actual).astype(np.complex128)
    e = to_numpy(expected).astype(np.complex128)
    if a.shape != e.shape:
        raise AssertionError(f"shape {a.shape} differs from the expected {e.shape}")
    num = np.sqrt(np.sum(np.abs(a - e) ** 2, axis=axes))
    den = np.sqrt(np.sum(np.abs(e) ** 2, axis=axes))
    return num / np.maximum(den, np.finfo(np.float64).tiny)


def assert_transform_close(actual, expected, n: int, axes: tuple[int, ...] = (-1,),
                           tol: float | None = None) -> None:
    """Fails if any transform of the batch exceeds the tolerance for n points (testing.py:55-68)."""
    tol = fft_tolerance(n) if tol is None else tol
    err = relative_error(actual, expected, axes)
    worst = float(np.max(err))
    if worst > tol:
        where = np.unravel_index(int(np.argmax(err)), np.shape(err)) if np.ndim(err) else ()
        raise AssertionError(
            f"relative L2 error {worst:.3e} exceeds the tolerance {tol:.3e} "
            f"(n = {n}) in transform {tuple(int(i) for i in where)}"
        )


def random_complex(rng: np.random.Generator, shape, dtype=np.complex64) -> np.ndarray:
    """Unit-variance complex Gaussian samples (testing.py:71-74)."""
    z = rng.standard_normal(shape) + 1j * rng.standard_normal(shape)
    return (z / math.sqrt(2.0)).astype(dtype)


def random_real(rng: np.random.Generator, shape, dtype=np.float32) -> np.ndarray:
    """testing.py:77-78"""
    return rng.standard_normal(shape).astype(dtype)
