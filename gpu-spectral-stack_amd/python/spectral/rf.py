"""Radio signal processing on this stack's FFTs (reference python/spectral/rf.py:1-212: the same
API, options and command line): window functions, the framed spectrum, and FIR filtering by
overlap-save, each with a selectable FFT backend.

    fft_impl="rocfft"        torch.fft (rocFFT on ROCm): the library baseline
    fft_impl="cufft"         the reference's name for the same torch.fft backend
    fft_impl="stockham_r8"   one of this stack's kernels (any name in spectral.FFT_IMPLS)

With a Stockham implementation, spectrum() and fir() each run as ONE kernel
(torch.ops.spectral.rf_spectrum / rf_fir): the frames or overlap-save blocks are read straight
from the signal (zero padding by bounds), windowed or multiplied by the filter's spectrum in
registers, and written once. With "naive" or the torch.fft backend, they run the reference's
composition of padding, framing, transforms and products. The command line reads and writes the
.cf32 / .f32 files of gpu-rf-pipeline (interleaved little-endian float32 I/Q, raw float32 taps):

    python -m spectral.rf spectrum --in x.cf32 --out spec.cf32 --nfft 1024 --window hann
    python -m spectral.rf fir --in x.cf32 --taps h.f32 --out y.cf32 --fft-impl stockham_r8
"""

from __future__ import annotations

import argparse
import math
import sys
from pathlib import Path

import numpy as np
import torch

from . import _C, ops  # noqa: F401  # _C registers torch.ops.spectral

TORCH_BACKENDS: tuple[str, ...] = ("rocfft", "cufft")
FFT_BACKENDS: tuple[str, ...] = (*TORCH_BACKENDS, *ops.FFT_IMPLS)
WINDOWS: tuple[str, ...] = ("rect", "hann", "hamming", "blackman")
FUSED_MAX_NFFT = 16384  # the largest frame or block the single-kernel paths take


# --- FFT backend ------------------------------------------------------------------------------


def _check_backend(fft_impl: str) -> None:
    if fft_impl not in FFT_BACKENDS:
        raise ValueError(f"unknown fft_impl '{fft_impl}' (available: {', '.join(FFT_BACKENDS)})")


def _fused(fft_impl: str, nfft: int) -> bool:
    return fft_impl.startswith("stockham") and 2 <= nfft <= FUSED_MAX_NFFT


def fft(x: torch.Tensor, *, inverse: bool = False, fft_impl: str = "rocfft") -> torch.Tensor:
    """Complex FFT along the last dimension (inverse divided by n) with the chosen backend
    (reference rf.py:43-48)."""
    _check_backend(fft_impl)
    if fft_impl in TORCH_BACKENDS:
        return torch.fft.ifft(x) if inverse else torch.fft.fft(x)
    return ops.fft_c2c(x, inverse=inverse, impl=fft_impl)


# --- Windows ----------------------------------------------------------------------------------


def window(name: str, n: int, *, device: torch.device | str | None = None) -> torch.Tensor:
    """The periodic window of n points (scipy.signal.get_window with fftbins=True), computed in
    float64 and returned as float32 (reference rf.py:54-83):

    rect      all ones
    hann      0.5 - 0.5 cos(2 pi k / n)
    hamming   0.54 - 0.46 cos(2 pi k / n)
    blackman  0.42 - 0.5 cos(2 pi k / n) + 0.08 cos(4 pi k / n)

    A window of one point is [1] whatever its name, as in scipy.
    """
    if n < 1:
        raise ValueError(f"a window needs at least one point, got {n}")
    if name not in WINDOWS:
        raise ValueError(f"unknown window '{name}' (available: {', '.join(WINDOWS)})")
    if n == 1 or name == "rect":
        return torch.ones(n, device=device)
    phase = 2.0 * np.pi * np.arange(n) / n
    if name == "hann":
        w = 0.5 - 0.5 * np.cos(phase)
    elif name == "hamming":
        w = 0.54 - 0.46 * np.cos(phase)
    else:
        w = 0.42 - 0.5 * np.cos(phase) + 0.08 * np.cos(2.0 * phase)
    return torch.from_numpy(w.astype(np.float32)).to(device)


# --- Spectrum ---------------------------------------------------------------------------------


def frames(x: torch.Tensor, nfft: int) -> torch.Tensor:
    """(..., n) -> (..., ceil(n / nfft), nfft): back-to-back frames, the last one zero-padded
    (at least one frame)."""
    n = x.shape[-1]
    count = max(1, math.ceil(n / nfft))
    padded = torch.nn.functional.pad(x, (0, count * nfft - n))
    return padded.reshape(*x.shape[:-1], count, nfft)


def spectrum(
    x: torch.Tensor, nfft: int, *, window_name: str = "rect", fft_impl: str = "rocfft"
) -> torch.Tensor:
    """FFT of each nfft-sample frame of x after applying the window: complex64 (..., n) ->
    (..., frames, nfft) (reference rf.py:94-105)."""
    _check_complex(x, "x")
    _check_backend(fft_impl)
    if nfft < 1:
        raise ValueError(f"nfft must be at least 1, got {nfft}")
    w = _device_window(window_name, nfft, x.device)
    if _fused(fft_impl, nfft):
        return torch.ops.spectral.rf_spectrum.default(
            x, None if window_name == "rect" else w, nfft, fft_impl
        )
    return fft(frames(x, nfft) * w, fft_impl=fft_impl)


_WINDOWS: dict[tuple[str, int, torch.device], torch.Tensor] = {}


def _device_window(name: str, n: int, device: torch.device) -> torch.Tensor:
    """window(name, n) on `device`, built and copied once per (name, n, device): spectrum()
    only reads it, so repeated calls skip the host computation and the host-to-device copy."""
    key = (name, n, device)
    w = _WINDOWS.get(key)
    if w is None:
        w = window(name, n, device=device)
        _WINDOWS[key] = w
    return w


# --- FIR by overlap-save ----------------------------------------------------------------------


def default_nfft(num_taps: int) -> int:
    """The block size fir() uses (reference rf.py:108-117): a power of two about four times the
    filter length, from 64 up to 4096; longer filters get the next power of two above their
    length."""
    if num_taps < 1:
        raise ValueError("the filter needs at least one tap")
    nfft = 1 << max(6, math.ceil(math.log2(4 * num_taps)))
    if nfft > 4096:
        nfft = max(4096, 1 << math.ceil(math.log2(num_taps)))
    return nfft


def fir(
    x: torch.Tensor, taps: torch.Tensor, *, nfft: int | None = None, fft_impl: str = "rocfft"
) -> torch.Tensor:
    """Causal FIR filter y[n] = sum_k taps[k] x[n - k] with zero initial state, as
    scipy.signal.lfilter(taps, 1, x): complex64 (..., n) -> (..., n), each row its own signal
    (reference rf.py:120-153). Overlap-save in blocks of nfft samples overlapping by
    len(taps) - 1; the first len(taps) - 1 outputs of each block wrap around and are dropped.
    taps may be real or complex."""
    _check_complex(x, "x")
    _check_backend(fft_impl)
    if taps.dim() != 1 or taps.numel() < 1:
        raise ValueError("taps must be a non-empty 1D tensor")
    m = taps.numel()
    nfft = default_nfft(m) if nfft is None else nfft
    if nfft < m or nfft & (nfft - 1):
        raise ValueError(f"nfft must be a power of two of at least len(taps) = {m}, got {nfft}")

    if _fused(fft_impl, nfft):
        # The filter spectrum in one launch from the taps as they are (float32 or complex64).
        t = taps.to(device=x.device)
        if t.dtype not in (torch.float32, torch.complex64):
            t = t.to(torch.complex64 if t.is_complex() else torch.float32)
        spectrum_h = torch.ops.spectral.rf_fir_spectrum.default(t, nfft, fft_impl)
        return torch.ops.spectral.rf_fir.default(x, spectrum_h, m, nfft, fft_impl)

    h = torch.zeros(nfft, dtype=torch.complex64, device=x.device)
    h[:m] = taps.to(device=x.device, dtype=torch.complex64)
    spectrum_h = fft(h, fft_impl=fft_impl)

    step = nfft - m + 1  # new outputs per block
    n = x.shape[-1]
    blocks = max(1, math.ceil(n / step))
    # Block b covers padded[b * step : b * step + nfft], where padded is x after m - 1 zeros.
    padded = torch.nn.functional.pad(x, (m - 1, blocks * step - n))
    segments = padded.unfold(-1, nfft, step).contiguous()  # (..., blocks, nfft)
    filtered = fft(fft(segments, fft_impl=fft_impl) * spectrum_h, inverse=True, fft_impl=fft_impl)
    y = filtered[..., m - 1 :].reshape(*x.shape[:-1], blocks * step)
    return y[..., :n].contiguous()


def _check_complex(x: torch.Tensor, name: str) -> None:
    if x.dtype != torch.complex64 or not x.is_cuda:
        raise ValueError(f"{name} must be a complex64 CUDA tensor, got {x.dtype} on {x.device}")


# --- Files and command line -------------------------------------------------------------------


def read_cf32(path: Path) -> np.ndarray:
    """Interleaved little-endian float32 I/Q samples as complex64."""
    return np.fromfile(path, dtype="<f4").view(np.complex64)


def write_cf32(path: Path, x: np.ndarray) -> None:
    np.asarray(x, dtype=np.complex64).view("<f4").tofile(path)


def read_f32(path: Path) -> np.ndarray:
    return np.fromfile(path, dtype="<f4")


def main(argv: list[str] | None = None) -> int:
    """The reference's command line (rf.py:177-208)."""
    parser = argparse.ArgumentParser(
        prog="python -m spectral.rf",
        description="Spectrum and FIR filtering of .cf32 recordings on the GPU.",
    )
    sub = parser.add_subparsers(dest="op", required=True)

    sp = sub.add_parser("spectrum", help="windowed FFT of back-to-back frames")
    sp.add_argument("--in", dest="inp", type=Path, required=True)
    sp.add_argument("--out", type=Path, required=True)
    sp.add_argument("--nfft", type=int, default=1024)
    sp.add_argument("--window", choices=WINDOWS, default="rect")

    fp = sub.add_parser("fir", help="FIR filter by overlap-save")
    fp.add_argument("--in", dest="inp", type=Path, required=True)
    fp.add_argument("--taps", type=Path, required=True, help="raw float32 taps (.f32)")
    fp.add_argument("--out", type=Path, required=True)
    fp.add_argument("--nfft", type=int, default=None, help="block size (default: about 4x taps)")

    for p in (sp, fp):
        p.add_argument("--fft-impl", choices=FFT_BACKENDS, default="rocfft")
    args = parser.parse_args(argv)

    x = torch.from_numpy(read_cf32(args.inp)).cuda()
    if args.op == "spectrum":
        y = spectrum(x, args.nfft, window_name=args.window, fft_impl=args.fft_impl)
    else:
        taps = torch.from_numpy(read_f32(args.taps)).cuda()
        y = fir(x, taps, nfft=args.nfft, fft_impl=args.fft_impl)
    write_cf32(args.out, y.reshape(-1).cpu().numpy())
    print(f"{args.op}[{args.fft_impl}]: {x.numel()} samples in, {y.numel()} out -> {args.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
