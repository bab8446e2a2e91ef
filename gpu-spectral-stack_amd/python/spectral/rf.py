"""Radio processing on this stack's FFTs: periodic windows, the spectrum of back-to-back frames,
and FIR filtering by overlap-save, each with a selectable FFT backend. The public names, their
arguments and results, and the command line are the reference's (python/spectral/rf.py:1-212),
so its callers and its RF tests run unchanged.

Backends (fft_impl):
    "rocfft" / "cufft"   torch.fft (rocFFT on ROCm); "cufft" is the reference's name for it
    a spectral.FFT_IMPLS name   this stack's kernels

With a Stockham backend and a frame or block of 2 .. 16384 samples, spectrum() and fir() are one
kernel launch each (torch.ops.spectral.rf_spectrum, rf_fir; the filter's spectrum is one more,
rf_fir_spectrum): frames and overlap-save blocks are read from the signal in place, with the zero
padding decided by bounds, and the window or the filter's spectrum is applied in registers.
Otherwise the same results are composed from tensor operations around the chosen FFT.

Files are gpu-rf-pipeline's: .cf32 interleaved little-endian float32 I/Q, .f32 raw float32 taps.

    python -m spectral.rf spectrum --in x.cf32 --out spec.cf32 --nfft 1024 --window hann
    python -m spectral.rf fir --in x.cf32 --taps h.f32 --out y.cf32 --fft-impl stockham_r8
"""

from __future__ import annotations

import argparse
import sys
from pathlib import Path

import numpy as np
import torch

from . import _C, ops  # noqa: F401  # _C registers torch.ops.spectral

TORCH_BACKENDS: tuple[str, ...] = ("rocfft", "cufft")
FFT_BACKENDS: tuple[str, ...] = (*TORCH_BACKENDS, *ops.FFT_IMPLS)
WINDOWS: tuple[str, ...] = ("rect", "hann", "hamming", "blackman")
FUSED_MAX_NFFT = 16384  # the longest frame or block the one-launch paths take

# Each window as a generalized cosine sum w[k] = sum_j (-1)^j a_j cos(2 pi j k / n), periodic
# (scipy.signal.get_window's fftbins=True convention).
_COSINE_TERMS: dict[str, tuple[float, ...]] = {
    "rect": (1.0,),
    "hann": (0.5, 0.5),
    "hamming": (0.54, 0.46),
    "blackman": (0.42, 0.5, 0.08),
}


def _check_backend(fft_impl: str) -> None:
    if fft_impl not in FFT_BACKENDS:
        raise ValueError(f"unknown fft_impl '{fft_impl}' (available: {', '.join(FFT_BACKENDS)})")


def _check_complex(x: torch.Tensor, name: str) -> None:
    if x.dtype != torch.complex64 or not x.is_cuda:
        raise ValueError(f"{name} must be a complex64 CUDA tensor, got {x.dtype} on {x.device}")


def _one_launch(fft_impl: str, nfft: int) -> bool:
    return fft_impl.startswith("stockham") and 2 <= nfft <= FUSED_MAX_NFFT


def _ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def fft(x: torch.Tensor, *, inverse: bool = False, fft_impl: str = "rocfft") -> torch.Tensor:
    """Complex FFT over the last dimension with the chosen backend; the inverse divides by n."""
    _check_backend(fft_impl)
    if fft_impl in TORCH_BACKENDS:
        return (torch.fft.ifft if inverse else torch.fft.fft)(x)
    return ops.fft_c2c(x, inverse=inverse, impl=fft_impl)


def window(name: str, n: int, *, device: torch.device | str | None = None) -> torch.Tensor:
    """The n-point periodic window `name`, evaluated in float64 and returned as float32:

    rect      1
    hann      0.5 - 0.5 cos(2 pi k / n)
    hamming   0.54 - 0.46 cos(2 pi k / n)
    blackman  0.42 - 0.5 cos(2 pi k / n) + 0.08 cos(4 pi k / n)

    A one-point window is [1] whatever the name (scipy's convention)."""
    if n < 1:
        raise ValueError(f"a window needs at least one point, got {n}")
    terms = _COSINE_TERMS.get(name)
    if terms is None:
        raise ValueError(f"unknown window '{name}' (available: {', '.join(WINDOWS)})")
    if n == 1:
        return torch.ones(1, device=device)
    angle = (2.0 * np.pi / n) * np.arange(n)
    w = sum((-1.0) ** j * a * np.cos(j * angle) for j, a in enumerate(terms))
    return torch.from_numpy(np.asarray(w, dtype=np.float32)).to(device)


_DEVICE_WINDOWS: dict[tuple[str, int, torch.device], torch.Tensor] = {}


def _window_on(name: str, n: int, device: torch.device) -> torch.Tensor:
    """window(name, n) on `device`, computed and copied once: callers only read it."""
    key = (name, n, device)
    if key not in _DEVICE_WINDOWS:
        _DEVICE_WINDOWS[key] = window(name, n, device=device)
    return _DEVICE_WINDOWS[key]


def frames(x: torch.Tensor, nfft: int) -> torch.Tensor:
    """(..., n) -> (..., max(1, ceil(n / nfft)), nfft): consecutive frames of x, the last one
    completed with zeros."""
    n = x.shape[-1]
    count = max(1, _ceil_div(n, nfft))
    out = x.new_zeros((*x.shape[:-1], count * nfft))
    out[..., :n] = x
    return out.view(*x.shape[:-1], count, nfft)


def spectrum(
    x: torch.Tensor, nfft: int, *, window_name: str = "rect", fft_impl: str = "rocfft"
) -> torch.Tensor:
    """The FFT of every nfft-sample frame of x times the window: complex64 (..., n) ->
    (..., frames, nfft)."""
    _check_complex(x, "x")
    _check_backend(fft_impl)
    if nfft < 1:
        raise ValueError(f"nfft must be at least 1, got {nfft}")
    w = _window_on(window_name, nfft, x.device)
    if _one_launch(fft_impl, nfft):
        return torch.ops.spectral.rf_spectrum.default(
            x, None if window_name == "rect" else w, nfft, fft_impl
        )
    return fft(frames(x, nfft) * w, fft_impl=fft_impl)


def default_nfft(num_taps: int) -> int:
    """fir()'s block size for a filter of num_taps taps: the power of two nearest above four
    times the length, at least 64 and at most 4096, unless the filter alone needs more (then the
    power of two just above its length)."""
    if num_taps < 1:
        raise ValueError("the filter needs at least one tap")
    above = lambda v: 1 << (v - 1).bit_length()  # noqa: E731  # smallest power of two >= v
    nfft = max(64, above(4 * num_taps))
    return nfft if nfft <= 4096 else max(4096, above(num_taps))


def _taps_spectrum(taps: torch.Tensor, nfft: int, fft_impl: str, device) -> torch.Tensor:
    """The nfft-point FFT of the taps followed by zeros."""
    t = taps.to(device=device)
    if _one_launch(fft_impl, nfft):
        if t.dtype not in (torch.float32, torch.complex64):
            t = t.to(torch.complex64 if t.is_complex() else torch.float32)
        return torch.ops.spectral.rf_fir_spectrum.default(t, nfft, fft_impl)
    padded = torch.zeros(nfft, dtype=torch.complex64, device=device)
    padded[: t.numel()] = t.to(torch.complex64)
    return fft(padded, fft_impl=fft_impl)


def fir(
    x: torch.Tensor, taps: torch.Tensor, *, nfft: int | None = None, fft_impl: str = "rocfft"
) -> torch.Tensor:
    """y[n] = sum_k taps[k] x[n - k], zero initial state (scipy.signal.lfilter(taps, 1, x)), each
    row of complex64 (..., n) its own signal; taps real or complex. Overlap-save: block b is the
    nfft samples x[b L - (M - 1) .. b L + L - 1] (zeros before the start and past the end), with
    M = len(taps) and L = nfft - M + 1; its circular convolution with the taps is exact in its
    last L outputs, which are y[b L .. b L + L - 1]."""
    _check_complex(x, "x")
    _check_backend(fft_impl)
    if taps.dim() != 1 or taps.numel() < 1:
        raise ValueError("taps must be a non-empty 1D tensor")
    m = taps.numel()
    nfft = default_nfft(m) if nfft is None else nfft
    if nfft < m or nfft & (nfft - 1):
        raise ValueError(f"nfft must be a power of two of at least len(taps) = {m}, got {nfft}")
    h = _taps_spectrum(taps, nfft, fft_impl, x.device)
    if _one_launch(fft_impl, nfft):
        return torch.ops.spectral.rf_fir.default(x, h, m, nfft, fft_impl)

    n = x.shape[-1]
    step = nfft - m + 1
    blocks = max(1, _ceil_div(n, step))
    # The signal behind m - 1 leading zeros, long enough for every block; block b starts at b step.
    padded = x.new_zeros((*x.shape[:-1], (blocks - 1) * step + nfft))
    padded[..., m - 1 : m - 1 + n] = x
    starts = torch.arange(blocks, device=x.device)[:, None] * step
    segments = padded[..., starts + torch.arange(nfft, device=x.device)]  # (..., blocks, nfft)
    circular = fft(fft(segments, fft_impl=fft_impl) * h, inverse=True, fft_impl=fft_impl)
    return circular[..., m - 1 :].reshape(*x.shape[:-1], blocks * step)[..., :n].contiguous()


def read_cf32(path: Path) -> np.ndarray:
    """A .cf32 file as complex64 samples."""
    return np.frombuffer(Path(path).read_bytes(), dtype="<c8").astype(np.complex64)


def write_cf32(path: Path, x: np.ndarray) -> None:
    Path(path).write_bytes(np.asarray(x, dtype="<c8").tobytes())


def read_f32(path: Path) -> np.ndarray:
    """A .f32 file as float32 values."""
    return np.frombuffer(Path(path).read_bytes(), dtype="<f4").astype(np.float32)


def _run_spectrum(args, x: torch.Tensor) -> torch.Tensor:
    return spectrum(x, args.nfft, window_name=args.window, fft_impl=args.fft_impl)


def _run_fir(args, x: torch.Tensor) -> torch.Tensor:
    taps = torch.from_numpy(read_f32(args.taps)).cuda()
    return fir(x, taps, nfft=args.nfft, fft_impl=args.fft_impl)


def main(argv: list[str] | None = None) -> int:
    """`python -m spectral.rf {spectrum,fir} ...`: a .cf32 file in, a .cf32 file out."""
    parser = argparse.ArgumentParser(
        prog="python -m spectral.rf",
        description="Spectrum and FIR filtering of .cf32 recordings on the GPU.",
    )
    ops_parser = parser.add_subparsers(dest="op", required=True)
    commands = {
        "spectrum": ("windowed FFT of back-to-back frames", _run_spectrum,
                     [("--nfft", dict(type=int, default=1024)),
                      ("--window", dict(choices=WINDOWS, default="rect"))]),
        "fir": ("FIR filter by overlap-save", _run_fir,
                [("--taps", dict(type=Path, required=True, help="raw float32 taps (.f32)")),
                 ("--nfft", dict(type=int, default=None,
                                 help="block size (default: about 4x taps)"))]),
    }
    for name, (summary, run, options) in commands.items():
        p = ops_parser.add_parser(name, help=summary)
        p.add_argument("--in", dest="inp", type=Path, required=True)
        p.add_argument("--out", type=Path, required=True)
        for flag, kwargs in options:
            p.add_argument(flag, **kwargs)
        p.add_argument("--fft-impl", choices=FFT_BACKENDS, default="rocfft")
        p.set_defaults(run=run)
    args = parser.parse_args(argv)

    x = torch.from_numpy(read_cf32(args.inp)).cuda()
    y = args.run(args, x)
    write_cf32(args.out, y.reshape(-1).cpu().numpy())
    print(f"{args.op}[{args.fft_impl}]: {x.numel()} samples in, {y.numel()} out -> {args.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
