"""Python entry points for the torch.ops.spectral operators (reference python/spectral/ops.py).

Signatures, defaults and docstring contracts are the reference's; the operators underneath run
this repository's gfx950 kernels through libspectral_hip.so.
"""

from __future__ import annotations

import torch

from . import _C

# Every FFT implementation, in registry order, read from the C++ table so that a new
# implementation reaches every test (reference ops.py:9-10).
FFT_IMPLS: tuple[str, ...] = _C.fft_impls()


def scale(x: torch.Tensor, alpha: float) -> torch.Tensor:
    """alpha * x by our kernel; x complex64 on the GPU. Non-contiguous inputs are copied first."""
    return torch.ops.spectral.scale.default(x, alpha)


def fft_c2c(x: torch.Tensor, *, inverse: bool = False, impl: str = "naive") -> torch.Tensor:
    """Batched complex FFT along the last dimension (power of two); leading dimensions are batch.
    Forward unnormalized, inverse divided by n, like torch.fft.fft / ifft."""
    return torch.ops.spectral.fft_c2c.default(x, inverse, impl)


def rfft(x: torch.Tensor, *, impl: str = "naive") -> torch.Tensor:
    """Batched real-to-complex FFT along the last dimension (n >= 2, a power of two), like
    torch.fft.rfft: complex64 with n // 2 + 1 values in the last dimension."""
    return torch.ops.spectral.fft_r2c.default(x, impl)


def irfft(x: torch.Tensor, n: int, *, impl: str = "naive") -> torch.Tensor:
    """Inverse of rfft, divided by n, like torch.fft.irfft(x, n). The imaginary parts of the
    zero and n/2 frequencies are ignored."""
    return torch.ops.spectral.fft_c2r.default(x, n, impl)


def fft2(
    x: torch.Tensor, *, inverse: bool = False, impl: str = "naive", columns: str = "auto"
) -> torch.Tensor:
    """Batched 2D complex FFT over the last two dimensions, like torch.fft.fft2 (or ifft2).
    `columns`: "strided" (in place, column kernel), "transpose", or "auto" (strided if any)."""
    return torch.ops.spectral.fft2_c2c.default(x, inverse, impl, columns)


def rfft2(x: torch.Tensor, *, impl: str = "naive", columns: str = "auto") -> torch.Tensor:
    """Batched 2D real-to-complex FFT, like torch.fft.rfft2: (..., n1, n2) float32 ->
    (..., n1, n2 // 2 + 1) complex64."""
    return torch.ops.spectral.fft2_r2c.default(x, impl, columns)


def irfft2(x: torch.Tensor, n2: int, *, impl: str = "naive", columns: str = "auto") -> torch.Tensor:
    """Inverse of rfft2, like torch.fft.irfft2(x, s=(x.shape[-2], n2)): divides by n1 * n2."""
    return torch.ops.spectral.fft2_c2r.default(x, n2, impl, columns)


def fft_truncated(x: torch.Tensor, k: int, *, impl: str = "naive") -> torch.Tensor:
    """The first k outputs of fft_c2c(x): (..., n) complex64 -> (..., k)."""
    return torch.ops.spectral.fft_c2c_pruned.default(x, x.shape[-1], k, False, impl)


def ifft_from_modes(modes: torch.Tensor, n: int, *, impl: str = "naive") -> torch.Tensor:
    """Inverse FFT of n points whose first k = modes.shape[-1] inputs are `modes`, the rest
    zero: (..., k) complex64 -> (..., n), divided by n."""
    return torch.ops.spectral.fft_c2c_pruned.default(modes, n, modes.shape[-1], True, impl)


def rfft2_truncated(x: torch.Tensor, m1: int, m2: int, *, impl: str = "naive") -> torch.Tensor:
    """The low-frequency modes of rfft2(x): (..., n1, n2) float32 -> (..., 2 m1, m2) complex64,
    rows 0 .. m1-1 then n1-m1 .. n1-1, columns 0 .. m2-1."""
    return torch.ops.spectral.rfft2_modes.default(x, m1, m2, impl)


def irfft2_from_modes(
    modes: torch.Tensor, shape: tuple[int, int], *, impl: str = "naive"
) -> torch.Tensor:
    """Inverse of rfft2_truncated: (..., 2 m1, m2) complex64 -> (..., n1, n2) float32, every
    dropped mode taken as zero."""
    n1, n2 = shape
    return torch.ops.spectral.irfft2_modes.default(modes, n1, n2, impl)
