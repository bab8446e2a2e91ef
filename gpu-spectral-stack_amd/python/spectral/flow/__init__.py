"""2D incompressible Navier-Stokes in vorticity form on this stack's FFTs: the caller of the
batched-FFT hot path in the reference's data pipeline (python/spectral/flow/__init__.py)."""

from .params import Flow, Grid, forcing, forcing_velocity, laminar_kolmogorov, taylor_green

__all__ = ["Flow", "Grid", "forcing", "forcing_velocity", "laminar_kolmogorov", "taylor_green"]
