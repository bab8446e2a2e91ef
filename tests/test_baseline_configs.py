"""The BASELINE configurations at their full sizes, on the GPU, with the inputs the benchmark
uses (C1 U[-1, 1) complex from seed 0, C2-C4 standard normal, C5 a k^-3 Gaussian random field).

The kernels run the same code per transform at any batch, but not the same grid: persistent tile
loops, XCD ordering, partial last groups and the batch-wide index math only reach these shapes
at full size. Each test checks:
  - transforms sampled across the batch (the first, the last and random ones) against the float64
    oracle, within the policy tolerance;
  - a property over every transform of the batch that needs no oracle: the round trip back to
    the input, Parseval's identity, or the projection identity of the FNO mode transforms.
"""

import numpy as np
import pytest
import torch

import spectral
from oracle import reference as ref
from oracle.tolerance import assert_transform_close, fft_tolerance

pytestmark = pytest.mark.gpu

IMPL = "stockham_r8"
POINTS = 1 << 24


def sample(rng, count: int, picks: int = 24) -> np.ndarray:
    """The first and last index and `picks` random ones, sorted."""
    return np.unique(np.concatenate([[0, count - 1], rng.choice(count, picks, replace=False)]))


def worst_relative(actual: torch.Tensor, expected: torch.Tensor, dims) -> float:
    """Largest per-transform ||actual - expected|| / ||expected||, in float64 on the GPU."""
    a = actual.to(torch.complex128) if actual.is_complex() else actual.double()
    e = expected.to(torch.complex128) if expected.is_complex() else expected.double()
    num = (a - e).abs().pow(2).sum(dim=dims).sqrt()
    den = e.abs().pow(2).sum(dim=dims).sqrt()
    return float((num / den).max())


def test_c1_complex_1024_x_16384():
    rng = np.random.default_rng(0)
    n, batch = 1024, 16384
    x = (rng.uniform(-1, 1, (batch, n)) + 1j * rng.uniform(-1, 1, (batch, n))).astype(np.complex64)
    xd = torch.from_numpy(x).cuda()
    y = spectral.fft_c2c(xd, impl=IMPL)
    rows = sample(rng, batch)
    assert_transform_close(y[rows].cpu().numpy(), ref.fft(x[rows]), n)
    # Parseval over every row: sum |X|^2 = n sum |x|^2.
    energy_x = xd.to(torch.complex128).abs().pow(2).sum(-1)
    energy_y = y.to(torch.complex128).abs().pow(2).sum(-1)
    assert float(((energy_y / n - energy_x) / energy_x).abs().max()) < 2 * fft_tolerance(n)
    back = spectral.fft_c2c(y, inverse=True, impl=IMPL)
    assert_transform_close(back[rows].cpu().numpy(), x[rows], n, tol=2 * fft_tolerance(n))
    assert worst_relative(back, xd, -1) < 2 * fft_tolerance(n)


@pytest.mark.parametrize("n", [2 ** p for p in range(1, 13)])
def test_c2_real_sweep_at_2e24_points(n):
    rng = np.random.default_rng(n)
    batch = POINTS // n
    x = rng.standard_normal((batch, n)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    half = spectral.rfft(xd, impl=IMPL)
    assert tuple(half.shape) == (batch, n // 2 + 1)
    rows = sample(rng, batch)
    assert_transform_close(half[rows].cpu().numpy(), ref.rfft(x[rows]), n)
    back = spectral.irfft(half, n, impl=IMPL)
    assert_transform_close(back[rows].cpu().numpy(), ref.irfft(ref.rfft(x[rows]), n), n,
                           tol=2 * fft_tolerance(n))
    assert worst_relative(back, xd, -1) < 2 * fft_tolerance(n)


@pytest.mark.parametrize("columns", ["strided", "transpose"])
@pytest.mark.parametrize(("side", "arrays"), [(128, 1024), (512, 64)])
def test_c3_real_2d(side, arrays, columns):
    rng = np.random.default_rng(side)
    x = rng.standard_normal((arrays, side, side)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    points = side * side
    half = spectral.rfft2(xd, impl=IMPL, columns=columns)
    picks = sample(rng, arrays, 6)
    assert_transform_close(half[picks].cpu().numpy(), ref.rfft2(x[picks]), points, axes=(-2, -1))
    back = spectral.irfft2(half, side, impl=IMPL, columns=columns)
    assert_transform_close(back[picks].cpu().numpy(), x[picks], points, axes=(-2, -1),
                           tol=2 * fft_tolerance(points))
    assert worst_relative(back, xd, (-2, -1)) < 2 * fft_tolerance(points)


def test_c4_fno_modes_64_x_32_x_128_x_128():
    rng = np.random.default_rng(4)
    m1 = m2 = 16
    x = rng.standard_normal((64, 32, 128, 128)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    modes = spectral.rfft2_truncated(xd, m1, m2, impl=IMPL)
    assert tuple(modes.shape) == (64, 32, 2 * m1, m2)
    flat_x, flat_modes = x.reshape(-1, 128, 128), modes.reshape(-1, 2 * m1, m2)
    picks = sample(rng, flat_x.shape[0], 6)
    assert_transform_close(flat_modes[picks].cpu().numpy(), ref.rfft2_truncate(flat_x[picks], m1, m2),
                           128 * 128, axes=(-2, -1))
    field = spectral.irfft2_from_modes(modes, (128, 128), impl=IMPL)
    flat_field = field.reshape(-1, 128, 128)
    given = flat_modes[picks].cpu().numpy()
    assert_transform_close(flat_field[picks].cpu().numpy(),
                           ref.irfft2_from_modes(given, (128, 128)), 128 * 128, axes=(-2, -1))
    # Projection over every array: the modes of the band-limited field are the given modes,
    # except where a real field ties a kept mode to a dropped one. In column 0, row -m1 (block
    # row m1) pairs with row +m1, which is not kept, so the field carries half of it.
    again = spectral.rfft2_truncated(field, m1, m2, impl=IMPL)
    expected = modes.clone()
    expected[..., m1, 0] = modes[..., m1, 0] / 2
    assert worst_relative(again, expected, (-2, -1)) < 2 * fft_tolerance(128 * 128)


def test_c5_navier_stokes_128_x_256_from_a_k3_field():
    import bench
    from oracle import flow as flow_ref
    from spectral.flow import Flow
    from spectral.flow.gpu import GpuSolver

    n, batch, dt, steps = 128, 256, 0.0025, 40
    rng = np.random.default_rng(0)
    nu = rng.uniform(1e-3, 5e-3, batch)
    w0 = bench.random_vorticity(rng, n, batch)
    solver = GpuSolver(n, Flow(viscosity=nu), dt, pruned=True, fused=True)
    frames = solver.simulate(torch.as_tensor(w0, device="cuda"), steps, steps)
    assert bool(torch.isfinite(frames).all())
    final = frames[-1].double().cpu().numpy()
    picks = sample(rng, batch, 3)
    expected = flow_ref.simulate(w0[picks].astype(np.float64), nu[picks], 0.1, 1.0, 4, dt, steps,
                                 record_every=steps)[-1]
    for i, b in enumerate(picks):
        err = np.linalg.norm(final[b] - expected[i]) / np.linalg.norm(expected[i])
        assert err < 1e-4, (b, err)
