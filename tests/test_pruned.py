"""Pruned transforms against the float64 oracle, every implementation (reference
tests/test_pruned.py): the Stockham kernels prune inside the kernel, naive gathers from (or
scatters into) a full transform. The mode layout is checked bit for bit: through the transforms
on integer-valued modes (rounded after the transform), and through the C ABI's gather and scatter
in tests/test_capi.py."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import spectral
from oracle import reference as ref
from oracle.tolerance import assert_transform_close, fft_tolerance, random_complex, random_real

pytestmark = pytest.mark.gpu

IMPLS = spectral.FFT_IMPLS
AXES = (-2, -1)


def cuda(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(x).cuda()


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize(("n", "k"), [(1, 1), (8, 1), (8, 3), (64, 16), (256, 255), (4096, 32)])
@pytest.mark.parametrize("batch", [1, 3, 300])
def test_fft_truncated_matches_the_oracle(rng, impl, n, k, batch):
    x = random_complex(rng, (batch, n))
    y = spectral.fft_truncated(cuda(x), k, impl=impl)
    assert y.shape == (batch, k)
    assert_transform_close(y, ref.fft_truncate(x, k), n)


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize(("n", "k"), [(1, 1), (8, 1), (8, 3), (64, 16), (256, 255), (4096, 32)])
@pytest.mark.parametrize("batch", [1, 3, 300])
def test_ifft_from_modes_matches_the_oracle(rng, impl, n, k, batch):
    modes = random_complex(rng, (batch, k))
    y = spectral.ifft_from_modes(cuda(modes), n, impl=impl)
    assert y.shape == (batch, n)
    assert_transform_close(y, ref.ifft_from_modes(modes, n), n)


@pytest.mark.parametrize("impl", IMPLS)
def test_keeping_every_mode_is_the_full_transform(rng, impl):
    x = cuda(random_complex(rng, (5, 128)))
    full = spectral.fft_c2c(x, impl=impl)
    assert torch.equal(spectral.fft_truncated(x, 128, impl=impl), full)


CASES_2D = [
    (2, 2, 1, 1),
    (8, 8, 2, 3),
    (16, 16, 8, 9),
    (64, 32, 12, 12),
    (32, 128, 4, 20),
    (256, 256, 16, 16),
    (1024, 16, 100, 5),
    (128, 1024, 16, 300),
    (4096, 2, 2, 2),
    (2, 8192, 1, 64),
    (128, 128, 16, 16),
    (128, 128, 43, 43),
]


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize(("n1", "n2", "m1", "m2"), CASES_2D)
def test_rfft2_truncated_matches_the_oracle(rng, impl, n1, n2, m1, m2):
    x = random_real(rng, (3, n1, n2))
    y = spectral.rfft2_truncated(cuda(x), m1, m2, impl=impl)
    assert y.shape == (3, 2 * m1, m2)
    assert_transform_close(y, ref.rfft2_truncate(x, m1, m2), n1 * n2, axes=AXES)


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize(("n1", "n2", "m1", "m2"), CASES_2D)
def test_irfft2_from_modes_matches_the_oracle(rng, impl, n1, n2, m1, m2):
    modes = random_complex(rng, (3, 2 * m1, m2))
    y = spectral.irfft2_from_modes(cuda(modes), (n1, n2), impl=impl)
    assert y.shape == (3, n1, n2)
    assert_transform_close(y, ref.irfft2_from_modes(modes, (n1, n2)), n1 * n2, axes=AXES)


# Every shape with a narrow-tile single-pass pruned kernel (at most n2/8 kept columns). Their
# inverse is built for compile-time bounds on the kept columns (n2/16 or n2/8) and rows (n1/8,
# n1/4 or n1/2): each case sits at a bound or just past one, in both directions.
NARROW_SHAPES = [(64, 64), (128, 64), (32, 128), (64, 128), (128, 128), (32, 256), (64, 256)]


def narrow_cases():
    for n1, n2 in NARROW_SHAPES:
        wmax = n2 // 8
        for m2 in sorted({1, wmax // 2, wmax // 2 + 1, wmax}):
            for m1 in sorted({1, n1 // 8, n1 // 8 + 1, n1 // 4 + 1, n1 // 2}):
                yield n1, n2, m1, m2


@pytest.mark.parametrize("impl", ["stockham_r4", "stockham_r8", "stockham_r8_table"])
@pytest.mark.parametrize(("n1", "n2", "m1", "m2"), list(narrow_cases()))
def test_narrow_tile_kernels_at_their_bounds(rng, impl, n1, n2, m1, m2):
    x = random_real(rng, (3, n1, n2))
    y = spectral.rfft2_truncated(cuda(x), m1, m2, impl=impl)
    assert_transform_close(y, ref.rfft2_truncate(x, m1, m2), n1 * n2, axes=AXES)
    modes = random_complex(rng, (3, 2 * m1, m2))
    back = spectral.irfft2_from_modes(cuda(modes), (n1, n2), impl=impl)
    assert_transform_close(back, ref.irfft2_from_modes(modes, (n1, n2)), n1 * n2, axes=AXES)


def golden_positions(n1: int, n2: int, m1: int, m2: int) -> np.ndarray:
    data = json.loads((Path(__file__).parent / "golden" / "modes_index.json").read_text())
    case = next(c for c in data if (c["n1"], c["n2"], c["m1"], c["m2"]) == (n1, n2, m1, m2))
    return np.array(case["positions"])


# Golden-fixture shapes with at least one column between DC and Nyquist.
LAYOUT_CASES = [(8, 8, 2, 3), (16, 16, 3, 4), (16, 16, 8, 9), (64, 32, 12, 12), (32, 128, 4, 20),
                (128, 128, 16, 16)]


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize(("n1", "n2", "m1", "m2"), LAYOUT_CASES)
def test_mode_layout_is_exact_through_the_transforms(impl, n1, n2, m1, m2):
    # Distinct integers placed at the fixture's positions of a half spectrum (columns 0 and n2/2,
    # where a real field ties a mode to its conjugate partner, left zero), turned into a real
    # field on the CPU. The GPU forward must return every integer in its own slot of the mode
    # block: its float32 error is far below 0.5 at these sizes, so rounding to the nearest
    # integer compares the layout bit for bit. The GPU inverse of the integer block, taken back
    # through the float64 forward and rounded, must be the same half spectrum, zeros included.
    w = n2 // 2 + 1
    pos = golden_positions(n1, n2, m1, m2)
    free = (pos % w != 0) & (pos % w != n2 // 2)
    count = int(free.sum())
    ids = np.zeros((2, pos.size), dtype=np.complex128)
    ids[:, free] = (np.arange(1, 2 * count + 1) - 1j * np.arange(2 * count, 0, -1)).reshape(2, -1)
    full = np.zeros((2, n1 * w), dtype=np.complex128)
    full[:, pos] = ids
    field = ref.irfft2(full.reshape(2, n1, w), (n1, n2)).astype(np.float32)

    modes = spectral.rfft2_truncated(cuda(field), m1, m2, impl=impl).cpu().numpy()
    got = modes.reshape(2, -1).astype(np.complex128)
    assert np.array_equal(np.round(got.real) + 1j * np.round(got.imag), ids)

    block = cuda(ids.reshape(2, 2 * m1, m2).astype(np.complex64))
    back = spectral.irfft2_from_modes(block, (n1, n2), impl=impl).cpu().numpy()
    spec = ref.rfft2(back).reshape(2, -1)
    assert np.array_equal(np.round(spec.real) + 1j * np.round(spec.imag), full)


@pytest.mark.parametrize("impl", IMPLS)
def test_a_band_limited_field_survives_the_round_trip(rng, impl):
    n1, n2, m1, m2 = 64, 64, 8, 8
    modes = ref.rfft2_truncate(random_real(rng, (2, n1, n2)), m1, m2)
    modes[..., m1, 0] = 0
    field = ref.irfft2_from_modes(modes, (n1, n2)).astype(np.float32)
    back = spectral.irfft2_from_modes(
        spectral.rfft2_truncated(cuda(field), m1, m2, impl=impl), (n1, n2), impl=impl
    )
    assert_transform_close(back, field, n1 * n2, axes=AXES, tol=2 * fft_tolerance(n1 * n2))


@pytest.mark.parametrize("impl", IMPLS)
def test_many_arrays_and_leading_dimensions(rng, impl):
    x = random_real(rng, (2, 70, 16, 32))
    y = spectral.rfft2_truncated(cuda(x), 4, 5, impl=impl)
    assert y.shape == (2, 70, 8, 5)
    assert_transform_close(y, ref.rfft2_truncate(x, 4, 5), 512, axes=AXES)


def test_every_implementation_agrees(rng):
    x = cuda(random_real(rng, (4, 128, 128)))
    results = [spectral.rfft2_truncated(x, 12, 12, impl=impl) for impl in IMPLS]
    for r in results[1:]:
        assert_transform_close(r, results[0], 128 * 128, axes=AXES, tol=2 * fft_tolerance(2**14))


def test_rejects_modes_that_do_not_fit():
    x = torch.zeros(8, 8, device="cuda")
    with pytest.raises(RuntimeError, match="1 <= m1 <= n1/2"):
        spectral.rfft2_truncated(x, 5, 2)
    with pytest.raises(RuntimeError, match="1 <= m1 <= n1/2"):
        spectral.rfft2_truncated(x, 2, 6)
    with pytest.raises(RuntimeError, match="do not fit"):
        spectral.irfft2_from_modes(torch.zeros(3, 2, dtype=torch.complex64, device="cuda"), (8, 8))


def test_rejects_keep_out_of_range():
    x = torch.zeros(2, 8, dtype=torch.complex64, device="cuda")
    with pytest.raises(RuntimeError, match="1 <= keep <= n"):
        spectral.fft_truncated(x, 9)
    with pytest.raises(RuntimeError, match="1 <= keep <= n"):
        spectral.ifft_from_modes(x, 4)


# Every shape with a single-pass kernel, with random kept-mode counts and a partial last workgroup.
FUSED_SHAPES = [(4, 4), (8, 4), (16, 4), (4, 8), (8, 8), (16, 8), (4, 16), (8, 16), (16, 16),
                (32, 32), (64, 32), (128, 32), (256, 32), (32, 64), (64, 64), (128, 64),
                (256, 64), (32, 128), (64, 128), (128, 128), (32, 256), (64, 256)]


@pytest.mark.parametrize("impl", ["stockham_r4", "stockham_r8", "stockham_r8_table"])
@pytest.mark.parametrize(("n1", "n2"), FUSED_SHAPES)
def test_single_pass_modes_round_trip(rng, impl, n1, n2):
    m1 = int(rng.integers(1, n1 // 2 + 1))
    m2 = int(rng.integers(1, n2 // 2 + 2))
    x = random_real(rng, (17, n1, n2))
    modes = spectral.rfft2_truncated(cuda(x), m1, m2, impl=impl)
    assert_transform_close(modes, ref.rfft2_truncate(x, m1, m2), n1 * n2, axes=AXES)
    given = random_complex(rng, (17, 2 * m1, m2))
    y = spectral.irfft2_from_modes(cuda(given), (n1, n2), impl=impl)
    assert_transform_close(y, ref.irfft2_from_modes(given, (n1, n2)), n1 * n2, axes=AXES)


# Shapes whose pruned transforms with m2 <= n2/8 take the narrow-tile kernels (one array per
# workgroup, only the kept columns in LDS); the edges of that path: one and n1/2 kept row pairs,
# one and n2/8 kept columns, and n2/8 + 1 (the first width past it, back on the general kernel).
NARROW_SHAPES = [(64, 64), (128, 64), (32, 128), (64, 128), (128, 128), (32, 256), (64, 256)]


@pytest.mark.parametrize("impl", ["stockham_r4", "stockham_r8", "stockham_r8_table"])
@pytest.mark.parametrize(("n1", "n2"), NARROW_SHAPES)
@pytest.mark.parametrize(("m1_of", "m2_of"), [(lambda n: 1, lambda n: 1),
                                              (lambda n: n // 2, lambda n: n // 8),
                                              (lambda n: 1, lambda n: n // 8),
                                              (lambda n: n // 4, lambda n: n // 8 + 1)])
def test_narrow_modes_match_the_oracle(rng, impl, n1, n2, m1_of, m2_of):
    m1, m2 = m1_of(n1), m2_of(n2)
    x = random_real(rng, (5, n1, n2))
    modes = spectral.rfft2_truncated(cuda(x), m1, m2, impl=impl)
    assert modes.shape == (5, 2 * m1, m2)
    assert_transform_close(modes, ref.rfft2_truncate(x, m1, m2), n1 * n2, axes=AXES)
    given = random_complex(rng, (5, 2 * m1, m2))
    y = spectral.irfft2_from_modes(cuda(given), (n1, n2), impl=impl)
    assert_transform_close(y, ref.irfft2_from_modes(given, (n1, n2)), n1 * n2, axes=AXES)
