"""The float64 Navier-Stokes oracle (oracle/flow.py) against exact solutions, its own budgets and
its order of accuracy, and the product's grid (spectral.flow.params) against the oracle's: CPU
only. Mirrors the reference's tests/test_flow_reference.py."""

import numpy as np
import pytest

from oracle import flow as ref
from spectral.flow import Flow, Grid
from spectral.flow.params import forcing, laminar_kolmogorov, taylor_green


def relative(a, b) -> float:
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_grid_wavenumbers_follow_the_rfft2_layout():
    g = Grid(8)
    assert g.kx.ravel().tolist() == [0, 1, 2, 3, 4]
    assert g.ky.ravel().tolist() == [0, 1, 2, 3, -4, -3, -2, -1]
    assert g.inverse_k2[0, 0] == 0 and g.inverse_k2[1, 2] == pytest.approx(1 / 5)
    kx, ky = ref.wavenumbers(32)
    assert np.array_equal(Grid(32).kx, kx) and np.array_equal(Grid(32).ky, ky)


def test_two_thirds_rule_keeps_wavenumbers_up_to_n_over_3():
    mask = Grid(64).dealias
    assert np.flatnonzero(mask[0]).max() == 21  # 64 / 3 = 21.3
    assert mask[21, 0] and not mask[22, 0] and mask[64 - 21, 0] and not mask[64 - 22, 0]
    assert np.array_equal(mask, ref.dealias_mask(64))


def test_rejects_a_grid_that_is_not_a_power_of_two():
    with pytest.raises(ValueError, match="power of two"):
        Grid(48)


def test_product_exact_solutions_match_the_oracle():
    g, flow = Grid(16), Flow(viscosity=0.02, drag=0.1)
    assert np.allclose(forcing(g, flow), ref.forcing(16, 1.0, 4))
    assert np.allclose(laminar_kolmogorov(g, flow), ref.laminar_kolmogorov(16, 0.02, 0.1, 1.0, 4))
    assert np.allclose(taylor_green(g, 0.5, 0.02, 0.1), ref.taylor_green(16, 0.5, 0.02, 0.1))


def test_taylor_green_decays_exactly():
    nu, alpha, dt, steps = 0.01, 0.1, 0.01, 200
    w0 = ref.taylor_green(32, 0.0, nu, alpha)
    frames = ref.simulate(w0, nu, alpha, 0.0, 4, dt, steps, record_every=steps)
    assert relative(frames[-1], ref.taylor_green(32, dt * steps, nu, alpha)) < 1e-6


def test_laminar_kolmogorov_flow_is_a_fixed_point():
    w = ref.laminar_kolmogorov(32, 0.01, 0.1, 1.0, 4)
    frames = ref.simulate(w, 0.01, 0.1, 1.0, 4, 0.05, 100, record_every=100)
    assert relative(frames[-1], w) < 1e-12


def test_the_dealiased_nonlinear_term_conserves_energy_and_enstrophy(rng):
    n = 32
    solver = ref.Solver(n, 0.0, 0.0, 0.0, 4, 1.0)
    w_hat = ref.rfft2(ref.smooth_random_field(rng, n)) * solver.mask
    nl = ref.irfft2(solver.nonlinear_hat(w_hat), n)
    psi = ref.irfft2(w_hat * solver.inverse_k2, n)
    w = ref.irfft2(w_hat, n)
    # d/dt of enstrophy and energy from the nonlinear term alone: <w N> and <psi N> vanish.
    assert abs(np.mean(w * nl)) < 1e-12 * np.mean(w**2) * np.abs(nl).max()
    assert abs(np.mean(psi * nl)) < 1e-12 * np.abs(psi).max() * np.abs(nl).max()


def test_budgets_hold(rng):
    nu, alpha, dt = 0.01, 0.1, 1e-4
    frames = ref.simulate(ref.smooth_random_field(rng, 32), nu, alpha, 1.0, 4, dt, 2, 1)
    d0 = ref.diagnostics(frames[0], nu, alpha, 1.0, 4)
    d2 = ref.diagnostics(frames[2], nu, alpha, 1.0, 4)
    de, dz = ref.budget_rates(frames[1], nu, alpha, 1.0, 4)
    assert (d2["energy"] - d0["energy"]) / (2 * dt) == pytest.approx(de, rel=1e-4)
    assert (d2["enstrophy"] - d0["enstrophy"]) / (2 * dt) == pytest.approx(dz, rel=1e-4)


def test_time_stepping_is_second_order(rng):
    w0 = ref.smooth_random_field(rng, 32)
    t = 0.4

    def final(dt):
        return ref.simulate(w0, 0.01, 0.1, 1.0, 4, dt, round(t / dt), round(t / dt))[-1]

    fine = final(0.0025)
    e1 = np.linalg.norm(final(0.02) - fine)
    e2 = np.linalg.norm(final(0.01) - fine)
    assert 3.0 < e1 / e2 < 5.0  # ~4 for a second-order method


def test_batched_viscosity_matches_separate_runs(rng):
    w0 = ref.smooth_random_field(rng, 16, batch=(2,))
    both = ref.simulate(w0, np.array([1e-3, 1e-2]), 0.1, 1.0, 4, 0.01, 10, 10)[-1]
    for b, nu in enumerate([1e-3, 1e-2]):
        single = ref.simulate(w0[b], nu, 0.1, 1.0, 4, 0.01, 10, 10)[-1]
        assert relative(both[b], single) < 1e-13
