"""Batched pseudo-spectral 2D Navier-Stokes on the GPU (reference python/spectral/flow/gpu.py:1-146:
the same discretization, API and options).

Vorticity form, state omega_hat in the rfft2 layout, 2/3-rule dealiasing, IMEX time stepping:
the linear terms L = -nu |k|^2 - alpha implicit (Crank-Nicolson), the forcing and the nonlinear
term F = f_hat - N_hat explicit (Heun predictor-corrector):

    w*  = [(1 + dt/2 L) w + dt F(w)] / (1 - dt/2 L)
    w'  = [(1 + dt/2 L) w + dt/2 (F(w) + F(w*))] / (1 - dt/2 L)

N = u . grad omega is formed in physical space from one batched inverse transform of four fields
(u, v, d omega/dx, d omega/dy) and one forward transform of the product, then masked.

pruned=True keeps the state only on the modes the 2/3 rule can keep, in the FNO layout of
spectral.rfft2_truncated with m = n/3 + 1: rows ky = 0 .. m-1 and -m .. -1, columns kx = 0 .. m-1.
The transforms then move only those modes. The row ky = -m lies outside the 2/3 set and stays
masked, so the pruned state equals the full one's kept modes.

fft_impl: one of spectral.FFT_IMPLS (this stack's kernels), or "rocfft" for torch.fft (rocFFT on
ROCm). "cufft", the reference's name for the torch.fft backend, is accepted as the same thing.

fused (this stack's addition; the reference has no such option): with pruned=True, a Stockham
fft_impl and n = 64 or 128, each of the step's two stages runs as one kernel per field
(torch.ops.spectral.ns_predict / ns_correct) that keeps the four derived fields, their product and
its spectrum in LDS: the same arithmetic as tendency() and the update below, in float32, without
the intermediate HBM traffic. fused=None picks it whenever it applies; True requires it; False
turns it off.
"""

from __future__ import annotations

from collections.abc import Iterator

import numpy as np
import torch

from .. import _C, ops
from .params import Flow, Grid, forcing

TORCH_BACKENDS = ("rocfft", "cufft")


class Spectral:
    """A forward / inverse real 2D transform pair and the wavenumbers of its layout."""

    def __init__(self, n: int, fft_impl: str, pruned: bool, device: torch.device | str):
        if fft_impl not in TORCH_BACKENDS and fft_impl not in ops.FFT_IMPLS:
            raise ValueError(
                f"unknown fft_impl '{fft_impl}' (available: rocfft, {', '.join(ops.FFT_IMPLS)})"
            )
        self.n, self.fft_impl, self.pruned = n, fft_impl, pruned
        self.torch_backend = fft_impl in TORCH_BACKENDS
        grid = Grid(n)
        ky = grid.ky[:, 0]
        kx = grid.kx[0]
        if pruned:
            self.m = n // 3 + 1
            ky = np.concatenate([ky[: self.m], ky[n - self.m :]])
            kx = kx[: self.m]
        self.ky = torch.as_tensor(ky, dtype=torch.float32, device=device)[:, None]
        self.kx = torch.as_tensor(kx, dtype=torch.float32, device=device)[None, :]
        self.mask = ((self.kx.abs() <= n / 3) & (self.ky.abs() <= n / 3)).to(torch.float32)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Real (..., n, n) float32 -> complex64 spectrum in this layout."""
        if self.torch_backend:
            full = torch.fft.rfft2(x)
            if not self.pruned:
                return full
            m, n = self.m, self.n
            return torch.cat([full[..., :m, :m], full[..., n - m :, :m]], dim=-2)
        if self.pruned:
            return ops.rfft2_truncated(x, self.m, self.m, impl=self.fft_impl)
        return ops.rfft2(x, impl=self.fft_impl)

    def inverse(self, x_hat: torch.Tensor) -> torch.Tensor:
        """Complex64 spectrum in this layout -> real (..., n, n) float32."""
        n = self.n
        if self.torch_backend:
            if self.pruned:
                m = self.m
                full = x_hat.new_zeros((*x_hat.shape[:-2], n, n // 2 + 1))
                full[..., :m, :m] = x_hat[..., :m, :]
                full[..., n - m :, :m] = x_hat[..., m:, :]
                x_hat = full
            return torch.fft.irfft2(x_hat, s=(n, n))
        if self.pruned:
            return ops.irfft2_from_modes(x_hat, (n, n), impl=self.fft_impl)
        return ops.irfft2(x_hat, n, impl=self.fft_impl)


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
        fusable = (
            pruned
            and fft_impl.startswith("stockham")
            and _C.ns_supports(n)
        )
        if fused and not fusable:
            raise ValueError(
                "fused=True needs pruned=True, a stockham fft_impl and n = 64 or 128 "
                f"(got pruned={pruned}, fft_impl='{fft_impl}', n={n})"
            )
        self.fused = fusable if fused is None else bool(fused)
        self.ikx = (1j * s.kx).to(torch.complex64)
        self.iky = (1j * s.ky).to(torch.complex64)
        k2 = s.kx**2 + s.ky**2
        self.inverse_k2 = torch.where(k2 > 0, 1.0 / k2.clamp(min=1.0), torch.zeros_like(k2))
        f = torch.as_tensor(forcing(Grid(n), flow), dtype=torch.float32, device=device)
        self.forcing_hat = s.forward(f) * s.mask
        nu = torch.as_tensor(np.asarray(flow.viscosity), dtype=torch.float32, device=device)
        self.nu = nu.reshape(-1).contiguous()  # one value, or one per trajectory
        nu = nu[..., None, None] if nu.dim() else nu
        linear = -nu * k2 - flow.drag
        self.explicit = (1.0 + 0.5 * dt * linear).to(torch.complex64)
        self.implicit = (1.0 / (1.0 - 0.5 * dt * linear)).to(torch.complex64)

    def to_spectral(self, w: torch.Tensor) -> torch.Tensor:
        """omega_hat of physical vorticity (..., n, n), projected onto the dealiased modes."""
        return self.spectral.forward(w.to(torch.float32).contiguous()) * self.spectral.mask

    def to_physical(self, w_hat: torch.Tensor) -> torch.Tensor:
        return self.spectral.inverse(w_hat)

    def tendency(self, w_hat: torch.Tensor) -> torch.Tensor:
        """F = f_hat - N_hat, N = u . grad omega, dealiased."""
        psi_hat = w_hat * self.inverse_k2
        fields_hat = torch.stack(
            [self.iky * psi_hat, -self.ikx * psi_hat, self.ikx * w_hat, self.iky * w_hat]
        )
        u, v, wx, wy = self.spectral.inverse(fields_hat)  # one batched inverse transform
        nonlinear_hat = self.spectral.forward(u * wx + v * wy) * self.spectral.mask
        return self.forcing_hat - nonlinear_hat

    def step(self, w_hat: torch.Tensor) -> torch.Tensor:
        if self.fused:
            drag, dt, n = float(self.flow.drag), float(self.dt), self.n
            f0, predicted = torch.ops.spectral.ns_predict.default(
                w_hat, self.forcing_hat, self.nu, drag, dt, n
            )
            return torch.ops.spectral.ns_correct.default(
                predicted, w_hat, f0, self.forcing_hat, self.nu, drag, dt, n
            )
        f0 = self.tendency(w_hat)
        predicted = (self.explicit * w_hat + self.dt * f0) * self.implicit
        f1 = self.tendency(predicted)
        return (self.explicit * w_hat + (0.5 * self.dt) * (f0 + f1)) * self.implicit

    def frames(self, w0: torch.Tensor, steps: int, record_every: int = 1) -> Iterator[torch.Tensor]:
        """Physical vorticity every record_every steps, starting with the dealiased initial
        condition (reference gpu.py:131-141)."""
        if steps < 0 or record_every < 1:
            raise ValueError("need steps >= 0 and record_every >= 1")
        w_hat = self.to_spectral(w0)
        yield self.to_physical(w_hat)
        for k in range(1, steps + 1):
            w_hat = self.step(w_hat)
            if k % record_every == 0:
                yield self.to_physical(w_hat)

    def simulate(self, w0: torch.Tensor, steps: int, record_every: int = 1) -> torch.Tensor:
        """All frames stacked: (frames, ..., n, n)."""
        return torch.stack(list(self.frames(w0, steps, record_every)))
