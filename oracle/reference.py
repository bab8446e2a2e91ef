"""Float64 NumPy references for every transform on the hot path.

Restates the reference's oracle, python/spectral/reference.py:28-105 (Jeanm2005/gpu-spectral-stack):
transforms act on the last axis (1D) or last two axes (2D); forward unnormalized; inverse divided
by N (N1 N2 in 2D); real transforms keep N // 2 + 1 bins of the last axis; truncated transforms keep
the low-frequency modes of the FNO layout. Everything is computed in complex128 / float64 on the
same float32 input the kernel saw, so a comparison measures the transform's error alone.

TEST INFRASTRUCTURE: see oracle/__init__.py for who may import this.
"""

from __future__ import annotations

import numpy as np


def _c128(x) -> np.ndarray:
    return np.asarray(x, dtype=np.complex128)


def _f64(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float64)


def dft(x) -> np.ndarray:
    """The DFT by its definition, O(N^2) (reference.py:28-34): X[k] = sum_m x[m] e^{-2 pi i k m/N}."""
    x = _c128(x)
    n = x.shape[-1]
    k = np.arange(n)
    # exponent reduced mod n in integers first, so large k*m lose no accuracy
    w = np.exp(-2j * np.pi * (np.outer(k, k) % max(n, 1)) / max(n, 1))
    return x @ w


def fft(x) -> np.ndarray:
    """reference.py:37-38"""
    return np.fft.fft(_c128(x), axis=-1)


def ifft(x) -> np.ndarray:
    """reference.py:41-42"""
    return np.fft.ifft(_c128(x), axis=-1)


def rfft(x) -> np.ndarray:
    """reference.py:45-46"""
    return np.fft.rfft(_f64(x), axis=-1)


def irfft(x, n: int) -> np.ndarray:
    """reference.py:49-52: imaginary parts of bin 0 (and n/2, n even) are ignored."""
    return np.fft.irfft(_c128(x), n=n, axis=-1)


def fft2(x) -> np.ndarray:
    """reference.py:55-56"""
    return np.fft.fft2(_c128(x), axes=(-2, -1))


def ifft2(x) -> np.ndarray:
    """reference.py:59-60"""
    return np.fft.ifft2(_c128(x), axes=(-2, -1))


def rfft2(x) -> np.ndarray:
    """reference.py:63-64"""
    return np.fft.rfft2(_f64(x), axes=(-2, -1))


def irfft2(x, shape: tuple[int, int]) -> np.ndarray:
    """reference.py:67-68"""
    return np.fft.irfft2(_c128(x), s=shape, axes=(-2, -1))


def fft_truncate(x, k: int) -> np.ndarray:
    """The first k outputs of fft(x) (reference.py:71-76)."""
    n = np.shape(x)[-1]
    if not 0 < k <= n:
        raise ValueError(f"k must be in [1, {n}], got {k}")
    return fft(x)[..., :k]


def ifft_from_modes(modes, n: int) -> np.ndarray:
    """Inverse FFT of n points whose first k inputs are `modes`, the rest zero (the layout of
    test_pruned.py:19-22)."""
    modes = _c128(modes)
    full = np.zeros(modes.shape[:-1] + (n,), dtype=np.complex128)
    full[..., : modes.shape[-1]] = modes
    return ifft(full)


def rfft2_truncate(x, m1: int, m2: int) -> np.ndarray:
    """Modes of rfft2(x) an FNO keeps (reference.py:79-91): rows 0 .. m1-1 (positive frequencies)
    then n1-m1 .. n1-1 (negative), columns 0 .. m2-1; shape (..., 2 m1, m2)."""
    n1, n2 = np.shape(x)[-2:]
    if not (0 < 2 * m1 <= n1 and 0 < m2 <= n2 // 2 + 1):
        raise ValueError(f"need 0 < 2*m1 <= {n1} and 0 < m2 <= {n2 // 2 + 1}, got {m1}, {m2}")
    full = rfft2(x)
    return np.concatenate([full[..., :m1, :m2], full[..., n1 - m1 :, :m2]], axis=-2)


def irfft2_from_modes(modes, shape: tuple[int, int]) -> np.ndarray:
    """Inverse of rfft2_truncate (reference.py:94-105): zero-fill the dropped modes, irfft2."""
    modes = _c128(modes)
    n1, n2 = shape
    two_m1, m2 = modes.shape[-2:]
    m1 = two_m1 // 2
    if two_m1 % 2 or not (0 < two_m1 <= n1 and 0 < m2 <= n2 // 2 + 1):
        raise ValueError(f"modes of shape {modes.shape[-2:]} do not fit an output of {shape}")
    full = np.zeros(modes.shape[:-2] + (n1, n2 // 2 + 1), dtype=np.complex128)
    full[..., :m1, :m2] = modes[..., :m1, :]
    full[..., n1 - m1 :, :m2] = modes[..., m1:, :]
    return irfft2(full, shape)
