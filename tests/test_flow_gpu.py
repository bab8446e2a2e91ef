"""The composed Navier-Stokes solver (spectral.flow.gpu.GpuSolver with fused=False: this stack's
transforms plus torch elementwise products) on the GPU, for every transform backend in the full
and the pruned layout. Pinned by closed-form solutions, the float64 oracle solver (oracle/flow.py)
and its exact energy and enstrophy budgets; the reference checks the same properties
(tests/test_flow_gpu.py). The fused single-kernel stages have their own file, test_flow_fused.py."""

import numpy as np
import pytest
import torch

from oracle import flow as oracle
from spectral.flow import Flow, Grid
from spectral.flow.gpu import GpuSolver
from spectral.flow.params import laminar_kolmogorov, taylor_green

pytestmark = pytest.mark.gpu

BACKENDS = {
    "rocfft-full": ("rocfft", False),
    "rocfft-pruned": ("rocfft", True),
    "r8-full": ("stockham_r8", False),
    "r8-pruned": ("stockham_r8", True),
    "r4-pruned": ("stockham_r4", True),
    "naive-full": ("naive", False),
    "naive-pruned": ("naive", True),
}


@pytest.fixture(params=list(BACKENDS), ids=list(BACKENDS))
def backend(request):
    return BACKENDS[request.param]


def evolve(w0: np.ndarray, flow: Flow, dt: float, steps: int, backend, every: int | None = None):
    """Frames (float64 on the host) of the composed solver from physical vorticity w0."""
    impl, pruned = backend
    solver = GpuSolver(w0.shape[-1], flow, dt, fft_impl=impl, pruned=pruned, fused=False)
    frames = solver.simulate(torch.tensor(w0, dtype=torch.float32, device="cuda"), steps,
                             every or max(steps, 1))
    return frames.double().cpu().numpy()


def rel(a: np.ndarray, b: np.ndarray) -> float:
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_unforced_taylor_green_vortex_decays_at_its_exact_rate(backend):
    nu, drag, t_end, dt = 0.01, 0.1, 2.0, 0.01
    grid = Grid(32)
    flow = Flow(viscosity=nu, drag=drag, forcing_amplitude=0.0)
    last = evolve(taylor_green(grid, 0.0, nu, drag), flow, dt, round(t_end / dt), backend)[-1]
    assert rel(last, taylor_green(grid, t_end, nu, drag)) < 1e-5


def test_laminar_kolmogorov_flow_does_not_move(backend):
    flow = Flow(viscosity=0.01)
    w = laminar_kolmogorov(Grid(32), flow)
    assert rel(evolve(w, flow, 0.05, 100, backend)[-1], w) < 1e-5


def test_forced_flow_follows_the_float64_solver(rng, backend):
    # 200 steps of a nonlinear, forced flow: long enough to exercise every term, short enough that
    # the float32 rounding is not amplified by the chaotic dynamics.
    w0 = oracle.smooth_random_field(rng, 64)
    ours = evolve(w0, Flow(viscosity=1e-3, drag=0.1), 5e-3, 200, backend)[-1]
    exact = oracle.simulate(w0, 1e-3, 0.1, 1.0, 4, 5e-3, 200, record_every=200)[-1]
    assert rel(ours, exact) < 1e-4


def test_one_tendency_matches_the_float64_solver(rng, backend):
    # The nonlinear term alone, no time stepping: F(w) against the oracle's, mode by mode.
    impl, pruned = backend
    n, nu = 64, 2e-3
    solver = GpuSolver(n, Flow(viscosity=nu, drag=0.1), 1e-3, fft_impl=impl, pruned=pruned,
                       fused=False)
    w_hat = solver.to_spectral(torch.tensor(oracle.smooth_random_field(rng, n, batch=(2,)),
                                            dtype=torch.float32, device="cuda"))
    ours = solver.tendency(w_hat)
    w64 = solver.to_physical(w_hat).double().cpu().numpy()
    full = oracle.Solver(n, nu, 0.1, 1.0, 4, 1e-3).tendency(oracle.rfft2(w64))
    if pruned:
        m = n // 3 + 1
        full = np.concatenate([full[..., :m, :m], full[..., n - m:, :m]], axis=-2)
    assert rel(ours.cpu().numpy(), full) < 1e-5


def test_energy_and_enstrophy_change_at_the_budget_rates(rng, backend):
    # Centred differences over two steps against the exact budget of the truncated system.
    dt, nu, drag = 1e-3, 0.01, 0.1
    frames = evolve(oracle.smooth_random_field(rng, 32), Flow(viscosity=nu, drag=drag), dt, 2,
                    backend, every=1)
    before = oracle.diagnostics(frames[0], nu, drag, 1.0, 4)
    after = oracle.diagnostics(frames[2], nu, drag, 1.0, 4)
    d_energy, d_enstrophy = oracle.budget_rates(frames[1], nu, drag, 1.0, 4)
    for key, rate in (("energy", d_energy), ("enstrophy", d_enstrophy)):
        assert (after[key] - before[key]) / (2 * dt) == pytest.approx(rate, rel=2e-3), key


def test_the_pruned_state_is_the_full_state_on_the_kept_modes(rng):
    w0 = oracle.smooth_random_field(rng, 128, batch=(2,))
    full = evolve(w0, Flow(viscosity=1e-3), 2e-3, 100, ("stockham_r8", False))
    pruned = evolve(w0, Flow(viscosity=1e-3), 2e-3, 100, ("stockham_r8", True))
    assert rel(pruned, full) < 1e-5


def test_each_trajectory_keeps_its_own_viscosity(rng):
    nus = np.array([1e-3, 4e-3, 1e-2])
    w0 = oracle.smooth_random_field(rng, 32, batch=(3,))
    ours = evolve(w0, Flow(viscosity=nus), 5e-3, 100, ("stockham_r8", True))[-1]
    exact = oracle.simulate(w0, nus, 0.1, 1.0, 4, 5e-3, 100, record_every=100)[-1]
    for b, nu in enumerate(nus):
        assert rel(ours[b], exact[b]) < 1e-4, nu
    # and a trajectory run alone evolves exactly as it does inside the batch
    alone = evolve(w0[1], Flow(viscosity=nus[1]), 5e-3, 100, ("stockham_r8", True))[-1]
    assert rel(alone, ours[1]) < 1e-6


@pytest.mark.parametrize(("steps", "every", "count"), [(10, 5, 3), (11, 5, 3), (4, 5, 1),
                                                       (0, 1, 1)])
def test_frames_are_produced_every_record_every_steps(rng, steps, every, count):
    solver = GpuSolver(16, Flow(), 0.01)
    w0 = torch.tensor(oracle.smooth_random_field(rng, 16), dtype=torch.float32, device="cuda")
    frames = list(solver.frames(w0, steps=steps, record_every=every))
    assert len(frames) == count
    assert all(f.shape == (16, 16) and f.dtype == torch.float32 for f in frames)
    # the k-th frame is k * every steps from the start
    if count > 1:
        w_hat = solver.to_spectral(w0)
        for _ in range(every):
            w_hat = solver.step(w_hat)
        assert torch.equal(frames[1], solver.to_physical(w_hat))


def test_cufft_names_the_torch_fft_backend(rng):
    w0 = oracle.smooth_random_field(rng, 32)
    assert np.array_equal(evolve(w0, Flow(), 0.01, 5, ("cufft", True)),
                          evolve(w0, Flow(), 0.01, 5, ("rocfft", True)))


def test_an_unknown_backend_is_rejected():
    with pytest.raises(ValueError, match="unknown fft_impl"):
        GpuSolver(16, Flow(), 0.01, fft_impl="fftw")
