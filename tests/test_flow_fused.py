"""The fused Navier-Stokes stages (torch.ops.spectral.ns_predict / ns_correct, C ABI spx_ns_stage):
one kernel per field and stage, against the composed GpuSolver path on the same state, against the
float64 oracle over many steps, and against the exact Taylor-Green and laminar Kolmogorov
solutions and the energy budget of the truncated system. The many-step launch
(torch.ops.spectral.ns_advance, C ABI spx_ns_steps, GpuSolver.advance) against the same steps
taken one stage at a time."""

import numpy as np
import pytest
import torch

from oracle import flow as ref
from spectral.flow import Flow, Grid
from spectral.flow.gpu import GpuSolver
from spectral.flow.params import laminar_kolmogorov, taylor_green

SIZES = [64, 128]


def relative(a, b):
    a = a.cpu().numpy() if torch.is_tensor(a) else a
    b = b.cpu().numpy() if torch.is_tensor(b) else b
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_fused_needs_a_supported_configuration():
    for n, impl, pruned in [(32, "stockham_r8", True), (64, "stockham_r8", False),
                            (64, "rocfft", True), (64, "naive", True)]:
        with pytest.raises(ValueError, match="fused=True needs"):
            GpuSolver(n, Flow(), 0.01, fft_impl=impl, pruned=pruned, fused=True, device="cpu")


@pytest.mark.gpu
def test_fused_is_the_default_where_it_applies():
    assert GpuSolver(64, Flow(), 0.01, pruned=True).fused
    assert GpuSolver(128, Flow(), 0.01, fft_impl="stockham_r4", pruned=True).fused
    assert not GpuSolver(64, Flow(), 0.01, pruned=False).fused
    assert not GpuSolver(256, Flow(), 0.01, pruned=True).fused
    assert not GpuSolver(64, Flow(), 0.01, pruned=True, fused=False).fused


def random_state(rng, n, batch, solver):
    w0 = ref.smooth_random_field(rng, n, batch=batch)
    # Add small-scale content up to the 2/3 cutoff, so every kept mode carries energy.
    w0 = w0 + 0.3 * rng.standard_normal(w0.shape)
    return solver.to_spectral(torch.as_tensor(w0, dtype=torch.float32, device="cuda"))


@pytest.mark.gpu
@pytest.mark.parametrize("n", SIZES)
def test_stages_match_the_composed_step(rng, n):
    nus = np.array([1e-3, 2e-3, 5e-3, 3e-3, 1e-2])
    flow, dt = Flow(viscosity=nus, drag=0.1), 2.5e-3
    fused = GpuSolver(n, flow, dt, pruned=True, fused=True)
    composed = GpuSolver(n, flow, dt, pruned=True, fused=False)
    w = random_state(rng, n, (5,), composed)
    drag, nu = 0.1, fused.nu
    f0, predicted = torch.ops.spectral.ns_predict(w, fused.forcing_hat, nu, drag, dt, n)
    f0_ref = composed.tendency(w)
    predicted_ref = (composed.explicit * w + dt * f0_ref) * composed.implicit
    assert relative(f0, f0_ref) < 2e-6
    assert relative(predicted, predicted_ref) < 2e-6
    out = torch.ops.spectral.ns_correct(predicted, w, f0, fused.forcing_hat, nu, drag, dt, n)
    f1_ref = composed.tendency(predicted)
    out_ref = (composed.explicit * w + (0.5 * dt) * (f0_ref + f1_ref)) * composed.implicit
    assert relative(out, out_ref) < 2e-6
    assert relative(fused.step(w), composed.step(w)) < 2e-6
    # The modes outside the 2/3 set (the row ky = -m) stay exactly zero.
    assert torch.count_nonzero(out[:, n // 3 + 1, :]) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("n", SIZES)
def test_tendency_matches_the_float64_oracle(rng, n):
    # One tendency evaluation, without time stepping: the fused kernel's nonlinear term against
    # the oracle's float64 rfft2 / irfft2 on the same (float32-representable) state.
    flow = Flow(viscosity=2e-3, drag=0.1)
    solver = GpuSolver(n, flow, 1e-3, pruned=True, fused=True)
    w_hat = random_state(rng, n, (3,), solver)
    w = solver.to_physical(w_hat).double().cpu().numpy()
    f0, _ = torch.ops.spectral.ns_predict(w_hat, solver.forcing_hat, solver.nu, 0.1, 1e-3, n)
    oracle = ref.Solver(n, 2e-3, 0.1, 1.0, 4, 1e-3)
    expected_full = oracle.tendency(ref.rfft2(w) * oracle.mask)
    m = n // 3 + 1
    expected = np.concatenate([expected_full[:, :m, :m], expected_full[:, n - m:, :m]], axis=1)
    assert relative(f0.cpu().numpy().astype(np.complex128), expected) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("n", SIZES)
def test_agrees_with_the_float64_oracle_over_many_steps(rng, n):
    nus = np.array([1e-3, 4e-3])
    w0 = ref.smooth_random_field(rng, n, batch=(2,))
    solver = GpuSolver(n, Flow(viscosity=nus, drag=0.1), 5e-3, pruned=True, fused=True)
    w = torch.as_tensor(w0, dtype=torch.float32, device="cuda")
    gpu = solver.simulate(w, 200, 200).double().cpu().numpy()
    cpu = ref.simulate(w0, nus, 0.1, 1.0, 4, 5e-3, 200, record_every=200)
    for b in range(2):
        assert relative(gpu[-1, b], cpu[-1, b]) < 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("n", SIZES)
def test_taylor_green_decays_exactly(n):
    grid, nu, alpha = Grid(n), 0.01, 0.1
    flow = Flow(viscosity=nu, drag=alpha, forcing_amplitude=0.0)
    solver = GpuSolver(n, flow, 0.01, pruned=True, fused=True)
    w = torch.as_tensor(taylor_green(grid, 0.0, nu, alpha), dtype=torch.float32, device="cuda")
    final = solver.simulate(w, 200, 200)[-1].double().cpu().numpy()
    assert relative(final, taylor_green(grid, 2.0, nu, alpha)) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("n", SIZES)
def test_laminar_kolmogorov_flow_is_a_fixed_point(n):
    grid, flow = Grid(n), Flow(viscosity=0.01)
    w = laminar_kolmogorov(grid, flow)
    solver = GpuSolver(n, flow, 0.05, pruned=True, fused=True)
    final = solver.simulate(torch.as_tensor(w, dtype=torch.float32, device="cuda"), 100, 100)[-1]
    assert relative(final.double().cpu().numpy(), w) < 1e-5


@pytest.mark.gpu
def test_energy_budget_holds(rng):
    n, flow, dt = 64, Flow(viscosity=0.01, drag=0.1), 1e-3
    solver = GpuSolver(n, flow, dt, pruned=True, fused=True)
    w0 = torch.as_tensor(ref.smooth_random_field(rng, n), dtype=torch.float32, device="cuda")
    frames = solver.simulate(w0, 2, 1).double().cpu().numpy()
    d0 = ref.diagnostics(frames[0], 0.01, 0.1, 1.0, 4)
    d2 = ref.diagnostics(frames[2], 0.01, 0.1, 1.0, 4)
    de, dz = ref.budget_rates(frames[1], 0.01, 0.1, 1.0, 4)
    assert (d2["energy"] - d0["energy"]) / (2 * dt) == pytest.approx(de, rel=2e-3)
    assert (d2["enstrophy"] - d0["enstrophy"]) / (2 * dt) == pytest.approx(dz, rel=2e-3)


@pytest.mark.gpu
def test_one_viscosity_for_every_field_and_batch_shapes(rng):
    n, dt = 64, 2.5e-3
    fused = GpuSolver(n, Flow(viscosity=3e-3), dt, pruned=True, fused=True)
    composed = GpuSolver(n, Flow(viscosity=3e-3), dt, pruned=True, fused=False)
    assert fused.nu.numel() == 1
    w = random_state(rng, n, (2, 3), composed)
    out = fused.step(w)
    assert out.shape == w.shape
    assert relative(out, composed.step(w)) < 2e-6
    # A non-contiguous state is read through a contiguous copy.
    wt = w.transpose(0, 1)
    assert relative(fused.step(wt), composed.step(wt.contiguous())) < 2e-6
    # An empty batch launches nothing.
    empty = w[:0]
    assert fused.step(empty).shape == empty.shape


@pytest.mark.gpu
def test_operators_reject_bad_arguments(rng):
    n = 64
    solver = GpuSolver(n, Flow(viscosity=np.array([1e-3, 2e-3])), 1e-3, pruned=True, fused=True)
    w = random_state(rng, n, (2,), solver)
    fh, nu = solver.forcing_hat, solver.nu
    with pytest.raises(RuntimeError, match="supports n = 64 and 128"):
        torch.ops.spectral.ns_predict(w, fh, nu, 0.1, 1e-3, 32)
    with pytest.raises(RuntimeError, match="state must hold"):
        torch.ops.spectral.ns_predict(w[..., :-1], fh, nu, 0.1, 1e-3, n)
    with pytest.raises(RuntimeError, match="one viscosity or one per field"):
        torch.ops.spectral.ns_predict(w[:1], fh, nu, 0.1, 1e-3, n)
    with pytest.raises(RuntimeError, match="float32 CUDA"):
        torch.ops.spectral.ns_predict(w, fh, nu.double(), 0.1, 1e-3, n)
    with pytest.raises(RuntimeError, match="same shape"):
        torch.ops.spectral.ns_correct(w, w[:1], w, fh, nu, 0.1, 1e-3, n)
    with pytest.raises(RuntimeError, match="steps must be >= 0"):
        torch.ops.spectral.ns_advance(w, fh, nu, 0.1, 1e-3, n, -1)
    with pytest.raises(ValueError, match="steps >= 0"):
        solver.advance(w, -1)


@pytest.mark.gpu
@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("viscosity", [np.array([1e-3, 4e-3, 2e-2]), 3e-3],
                         ids=["per-field", "shared"])
def test_advance_equals_the_stages_one_at_a_time(rng, n, viscosity):
    # The many-step kernel runs the stage kernel's code on the same values; the compiler may
    # contract a few products into fused multiply-adds differently in the two kernels, so the
    # states agree to float32 rounding after every count of steps (none: exactly).
    dt = 2.5e-3
    solver = GpuSolver(n, Flow(viscosity=viscosity, drag=0.1), dt, pruned=True, fused=True)
    w = random_state(rng, n, (3,), solver)
    stepped, done = w, 0
    for steps in (0, 1, 2, 5):
        while done < steps:
            f0, predicted = torch.ops.spectral.ns_predict(stepped, solver.forcing_hat, solver.nu,
                                                          0.1, dt, n)
            stepped = torch.ops.spectral.ns_correct(predicted, stepped, f0, solver.forcing_hat,
                                                    solver.nu, 0.1, dt, n)
            done += 1
        advanced = solver.advance(w, steps)
        assert advanced.data_ptr() != w.data_ptr()
        if steps == 0:
            assert torch.equal(advanced, w)
        else:
            assert relative(advanced, stepped) < 1e-6, f"{steps} steps"


@pytest.mark.gpu
def test_advance_keeps_its_input_and_batch_shapes(rng):
    n, dt = 128, 2.5e-3
    fused = GpuSolver(n, Flow(viscosity=3e-3), dt, pruned=True, fused=True)
    composed = GpuSolver(n, Flow(viscosity=3e-3), dt, pruned=True, fused=False)
    w = random_state(rng, n, (2, 3), composed)
    kept = w.clone()
    out = fused.advance(w, 4)
    assert torch.equal(w, kept) and out.shape == w.shape
    expected = w
    for _ in range(4):
        expected = composed.step(expected)
    assert relative(out, expected) < 1e-5
    # A non-contiguous state is read through a contiguous copy; an empty batch launches nothing.
    wt = w.transpose(0, 1)
    assert torch.equal(fused.advance(wt, 2), fused.advance(wt.contiguous(), 2))  # same launch
    assert fused.advance(w[:0], 3).shape == w[:0].shape


@pytest.mark.gpu
def test_frames_take_the_many_step_path(rng):
    # frames() advances between frames with advance(); step() is advance() by one step, and the
    # many-step kernel does the same arithmetic every step, so the frames equal those of step()
    # calls bit for bit.
    n, dt = 64, 2.5e-3
    solver = GpuSolver(n, Flow(viscosity=np.array([2e-3, 5e-3])), dt, pruned=True, fused=True)
    w0 = torch.as_tensor(ref.smooth_random_field(rng, n, batch=(2,)), dtype=torch.float32,
                         device="cuda")
    frames = list(solver.frames(w0, 7, record_every=3))
    assert len(frames) == 3
    w_hat = solver.to_spectral(w0)
    expected = [solver.to_physical(w_hat)]
    for _ in range(2):
        for _ in range(3):
            w_hat = solver.step(w_hat)
        expected.append(solver.to_physical(w_hat))
    for got, want in zip(frames, expected):
        assert torch.equal(got, want)
