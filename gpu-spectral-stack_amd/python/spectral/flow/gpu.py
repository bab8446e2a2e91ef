"""Batched 2D Navier-Stokes in vorticity form on the GPU, the caller of this stack's pruned and full
real 2D transforms. The API, options and discretization are the reference's
(python/spectral/flow/gpu.py:1-146); the numerics of one step are:

    state       w = omega_hat, in the rfft2 layout, or (pruned=True) in the FNO mode layout of
                spectral.rfft2_truncated with m = n/3 + 1 (rows ky = 0 .. m-1 and -m .. -1,
                columns kx = 0 .. m-1); the row ky = -m lies outside the 2/3 set and stays zero
    tendency    F(w) = f_hat - mask * FFT(u d omega/dx + v d omega/dy), where (u, v, d omega/dx,
                d omega/dy) come from w by one multiplier each (u = i ky psi, v = -i kx psi,
                psi = w / |k|^2) and one batched inverse transform of the four fields
    step        L = -nu |k|^2 - alpha treated by Crank-Nicolson, F by Heun:
                w* = [(1 + dt/2 L) w + dt F(w)] / (1 - dt/2 L)
                w' = [(1 + dt/2 L) w + dt/2 (F(w) + F(w*))] / (1 - dt/2 L)

fft_impl names one of spectral.FFT_IMPLS, or "rocfft" for torch.fft (rocFFT on ROCm); "cufft", the
reference's name for the torch.fft backend, means the same.

fused (this stack's own option): with pruned=True, a Stockham fft_impl and n = 64 or 128, a field's
step is one workgroup running both stages, each holding the derived fields, their product and its
spectrum in LDS: the arithmetic above in float32 without the intermediate HBM traffic. step() is
one launch (torch.ops.spectral.ns_advance with one step); advance(w, k), which frames() and
simulate() use between frames, runs k steps as one launch. The single stages are also exposed
(torch.ops.spectral.ns_predict / ns_correct). fused=None uses it wherever it applies, True
requires it, False never.
"""

from __future__ import annotations

from collections.abc import Callable, Iterator

import numpy as np
import torch

from .. import _C, ops
from .params import Flow, Grid, forcing

TORCH_BACKENDS = ("rocfft", "cufft")

Transform = Callable[[torch.Tensor], torch.Tensor]


def _layout_rows(n: int, pruned: bool) -> np.ndarray:
    """Which rfft2 row (vertical frequency index mod n) each row of the layout holds."""
    if not pruned:
        return np.arange(n)
    m = n // 3 + 1
    return np.concatenate([np.arange(m), np.arange(n - m, n)])


def _torch_pair(n: int, rows: np.ndarray, width: int, pruned: bool,
                device) -> tuple[Transform, Transform]:
    """rfft2 / irfft2 of torch.fft, restricted to (forward) or extended from (inverse) the kept
    rows and the first `width` columns."""
    if not pruned:
        return torch.fft.rfft2, lambda h: torch.fft.irfft2(h, s=(n, n))
    index = torch.as_tensor(rows, device=device)

    def forward(x: torch.Tensor) -> torch.Tensor:
        return torch.fft.rfft2(x).index_select(-2, index)[..., :width]

    def inverse(h: torch.Tensor) -> torch.Tensor:
        full = h.new_zeros((*h.shape[:-2], n, n // 2 + 1))
        full[..., :width].index_copy_(-2, index, h)
        return torch.fft.irfft2(full, s=(n, n))

    return forward, inverse


def _stack_pair(n: int, impl: str, pruned: bool) -> tuple[Transform, Transform]:
    if pruned:
        m = n // 3 + 1
        return (lambda x: ops.rfft2_truncated(x, m, m, impl=impl),
                lambda h: ops.irfft2_from_modes(h, (n, n), impl=impl))
    return (lambda x: ops.rfft2(x, impl=impl), lambda h: ops.irfft2(h, n, impl=impl))


class Spectral:
    """A forward / inverse real 2D transform pair and the wavenumbers of its layout: ky (rows, 1),
    kx (1, columns) and the 2/3-rule mask, float32 on `device`."""

    def __init__(self, n: int, fft_impl: str, pruned: bool, device: torch.device | str):
        if fft_impl not in TORCH_BACKENDS and fft_impl not in ops.FFT_IMPLS:
            raise ValueError(
                f"unknown fft_impl '{fft_impl}' (available: rocfft, {', '.join(ops.FFT_IMPLS)})"
            )
        self.n, self.fft_impl, self.pruned = n, fft_impl, pruned
        rows = _layout_rows(n, pruned)
        width = n // 3 + 1 if pruned else n // 2 + 1
        if pruned:
            self.m = width
        signed = np.where(rows < n // 2, rows, rows - n)
        self.ky = torch.as_tensor(signed, dtype=torch.float32, device=device)[:, None]
        self.kx = torch.arange(width, dtype=torch.float32, device=device)[None, :]
        limit = n / 3
        self.mask = ((self.ky.abs() <= limit) & (self.kx <= limit)).to(torch.float32)
        if fft_impl in TORCH_BACKENDS:
            self._forward, self._inverse = _torch_pair(n, rows, width, pruned, device)
        else:
            self._forward, self._inverse = _stack_pair(n, fft_impl, pruned)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Real (..., n, n) float32 -> complex64 spectrum in this layout."""
        return self._forward(x)

    def inverse(self, x_hat: torch.Tensor) -> torch.Tensor:
        """Complex64 spectrum in this layout -> real (..., n, n) float32."""
        return self._inverse(x_hat)


class GpuSolver:
    """Advances a batch of vorticity fields; viscosity a float or one value per trajectory."""

    def __init__(
        self,
        n: int,
        flow: Flow,
        dt: float,
        *,
        fft_impl: str = "stockham_r8",
        pruned: bool = False,
        fused: bool | None = None,
        device: torch.device | str = "cuda",
    ):
        self.n, self.flow, self.dt = n, flow, dt
        self.spectral = s = Spectral(n, fft_impl, pruned, device)
        fusable = pruned and fft_impl.startswith("stockham") and _C.ns_supports(n)
        if fused and not fusable:
            raise ValueError(
                "fused=True needs pruned=True, a stockham fft_impl and n = 64 or 128 "
                f"(got pruned={pruned}, fft_impl='{fft_impl}', n={n})"
            )
        self.fused = fusable if fused is None else bool(fused)

        k2 = s.kx**2 + s.ky**2
        over_k2 = torch.where(k2 > 0, 1.0 / k2.clamp(min=1.0), torch.zeros_like(k2))
        ikx = 1j * s.kx.to(torch.complex64)
        iky = 1j * s.ky.to(torch.complex64)
        # omega_hat -> (u, v, d omega/dx, d omega/dy) spectra, one multiplier each: (4, rows, cols)
        self.derivatives = torch.stack(
            [iky * over_k2, -ikx * over_k2, torch.broadcast_to(ikx, k2.shape),
             torch.broadcast_to(iky, k2.shape)]
        ).contiguous()

        f = torch.as_tensor(forcing(Grid(n), flow), dtype=torch.float32, device=device)
        self.forcing_hat = s.forward(f) * s.mask
        nu = torch.as_tensor(np.asarray(flow.viscosity), dtype=torch.float32, device=device)
        self.nu = nu.reshape(-1).contiguous()  # one value, or one per trajectory (fused stages)
        per_field = nu.reshape(*nu.shape, 1, 1)
        half_l = 0.5 * dt * (-per_field * k2 - flow.drag)
        self.explicit = (1.0 + half_l).to(torch.complex64)
        self.implicit = (1.0 / (1.0 - half_l)).to(torch.complex64)

    def to_spectral(self, w: torch.Tensor) -> torch.Tensor:
        """omega_hat of physical vorticity (..., n, n), projected onto the dealiased modes."""
        return self.spectral.forward(w.to(torch.float32).contiguous()) * self.spectral.mask

    def to_physical(self, w_hat: torch.Tensor) -> torch.Tensor:
        return self.spectral.inverse(w_hat)

    def tendency(self, w_hat: torch.Tensor) -> torch.Tensor:
        """F = f_hat - N_hat with N = u d omega/dx + v d omega/dy, dealiased."""
        lead = (1,) * (w_hat.dim() - 2)
        fields_hat = self.derivatives.view(4, *lead, *w_hat.shape[-2:]) * w_hat
        u, v, wx, wy = self.spectral.inverse(fields_hat)  # one batched inverse of four fields
        product = torch.addcmul(u * wx, v, wy)
        return self.forcing_hat - self.spectral.forward(product) * self.spectral.mask

    def step(self, w_hat: torch.Tensor) -> torch.Tensor:
        if self.fused:
            return self.advance(w_hat, 1)
        carried = self.explicit * w_hat
        f0 = self.tendency(w_hat)
        predicted = (carried + self.dt * f0) * self.implicit
        f1 = self.tendency(predicted)
        return (carried + (0.5 * self.dt) * (f0 + f1)) * self.implicit

    def advance(self, w_hat: torch.Tensor, steps: int) -> torch.Tensor:
        """`steps` calls of step(). The fused path runs them as one launch (each field's state,
        tendency and predictor stay in its XCD's L2 from stage to stage), with the same
        arithmetic as step()."""
        if steps < 0:
            raise ValueError("need steps >= 0")
        if self.fused:
            return torch.ops.spectral.ns_advance.default(
                w_hat, self.forcing_hat, self.nu, float(self.flow.drag), float(self.dt), self.n,
                steps)
        for _ in range(steps):
            w_hat = self.step(w_hat)
        return w_hat

    def frames(self, w0: torch.Tensor, steps: int, record_every: int = 1) -> Iterator[torch.Tensor]:
        """Physical vorticity at step 0 (the dealiased initial condition) and after every
        record_every steps up to `steps`, produced one at a time so a caller can stream them."""
        if steps < 0 or record_every < 1:
            raise ValueError("need steps >= 0 and record_every >= 1")
        w_hat = self.to_spectral(w0)
        yield self.to_physical(w_hat)
        for _ in range(steps // record_every):
            w_hat = self.advance(w_hat, record_every)
            yield self.to_physical(w_hat)
        self.advance(w_hat, steps % record_every)  # the tail past the last recorded frame

    def simulate(self, w0: torch.Tensor, steps: int, record_every: int = 1) -> torch.Tensor:
        """Every frame of frames(), stacked: (frames, ..., n, n)."""
        return torch.stack(list(self.frames(w0, steps, record_every)))
