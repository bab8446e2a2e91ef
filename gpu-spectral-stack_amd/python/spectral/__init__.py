"""spectral: batched FFTs for AMD MI355X (gfx950), hand-written HIP kernels behind the API of
Jeanm2005/gpu-spectral-stack (python/spectral/__init__.py:1-34).

The operators live in libspectral_hip.so (HIP kernels, C ABI) and are registered with PyTorch
by the extension module spectral._C. Build both with `python gpu-spectral-stack_amd/build.py`;
importing this package without them fails: there is no fallback path.
"""

import torch  # noqa: F401  # loads PyTorch's HIP runtime first, so the extension shares it

try:
    from . import _C  # noqa: F401  # registers the torch.ops.spectral operators
except ImportError as err:  # pragma: no cover - exercised only on a broken install
    raise ImportError(
        "spectral._C is not built: run `python gpu-spectral-stack_amd/build.py` "
        f"(or __graft_entry__.build()) first ({err})"
    ) from err

from .ops import (
    FFT_IMPLS,
    fft2,
    fft_c2c,
    fft_truncated,
    ifft_from_modes,
    irfft,
    irfft2,
    irfft2_from_modes,
    rfft,
    rfft2,
    rfft2_truncated,
    scale,
)

__all__ = [
    "FFT_IMPLS",
    "fft2",
    "fft_c2c",
    "fft_truncated",
    "ifft_from_modes",
    "irfft",
    "irfft2",
    "irfft2_from_modes",
    "rfft",
    "rfft2",
    "rfft2_truncated",
    "scale",
]
