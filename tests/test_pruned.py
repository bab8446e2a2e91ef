"""Pruned transforms on the GPU for every implementation (reference tests/test_pruned.py covers
the same ground): the Stockham implementations prune inside their kernels, naive gathers from or
scatters into a full transform. Parity with the float64 oracle for the 1D truncated transforms
and the 2D FNO mode transforms; the mode layout bit for bit through the product kernels, the DC
and Nyquist columns included; band-limited round trips; batch layouts; agreement between
implementations; and the rejections with the reference's messages. The gather and scatter of the
C ABI are checked bit for bit in tests/test_capi.py."""

import numpy as np
import pytest
import torch

import spectral
from oracle import reference as ref
from oracle.tolerance import assert_transform_close, fft_tolerance, random_complex, random_real
from mode_labels import (
    LAYOUT_CASES,
    golden_positions,
    hermitian_join,
    labelled_half_spectrum,
    rounded,
)

pytestmark = pytest.mark.gpu

IMPLS = spectral.FFT_IMPLS
AXES = (-2, -1)
DIRECTIONS = ["forward", "inverse"]
CASES_1D = [(1, 1), (8, 1), (8, 3), (64, 16), (256, 255), (4096, 32)]  # (n, keep)


def dev(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(x).cuda()


# --- 1D: the first `keep` outputs, or the inverse from the first `keep` modes -------------------

@pytest.mark.parametrize("direction", DIRECTIONS)
@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize(("n", "keep"), CASES_1D)
@pytest.mark.parametrize("batch", [1, 3, 300])
def test_truncated_1d_parity(rng, batch, n, keep, impl, direction):
    if direction == "forward":
        x = random_complex(rng, (batch, n))
        y = spectral.fft_truncated(dev(x), keep, impl=impl)
        expected = ref.fft_truncate(x, keep)
    else:
        modes = random_complex(rng, (batch, keep))
        y = spectral.ifft_from_modes(dev(modes), n, impl=impl)
        expected = ref.ifft_from_modes(modes, n)
    assert tuple(y.shape) == expected.shape
    assert_transform_close(y, expected, n)


@pytest.mark.parametrize("impl", IMPLS)
def test_keeping_all_modes_is_the_unpruned_transform_bit_for_bit(rng, impl):
    x = dev(random_complex(rng, (5, 128)))
    assert torch.equal(spectral.fft_truncated(x, 128, impl=impl), spectral.fft_c2c(x, impl=impl))


# --- 2D FNO modes: rows 0 .. m1-1 and n1-m1 .. n1-1, columns 0 .. m2-1 of the half spectrum --

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


@pytest.mark.parametrize("direction", DIRECTIONS)
@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize(("n1", "n2", "m1", "m2"), CASES_2D)
def test_modes_2d_parity(rng, n1, n2, m1, m2, impl, direction):
    if direction == "forward":
        field = random_real(rng, (3, n1, n2))
        y = spectral.rfft2_truncated(dev(field), m1, m2, impl=impl)
        expected = ref.rfft2_truncate(field, m1, m2)
    else:
        modes = random_complex(rng, (3, 2 * m1, m2))
        y = spectral.irfft2_from_modes(dev(modes), (n1, n2), impl=impl)
        expected = ref.irfft2_from_modes(modes, (n1, n2))
    assert tuple(y.shape) == expected.shape
    assert_transform_close(y, expected, n1 * n2, axes=AXES)


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
    y = spectral.rfft2_truncated(dev(x), m1, m2, impl=impl)
    assert_transform_close(y, ref.rfft2_truncate(x, m1, m2), n1 * n2, axes=AXES)
    modes = random_complex(rng, (3, 2 * m1, m2))
    back = spectral.irfft2_from_modes(dev(modes), (n1, n2), impl=impl)
    assert_transform_close(back, ref.irfft2_from_modes(modes, (n1, n2)), n1 * n2, axes=AXES)


# --- the mode layout, bit for bit ------------------------------------------------------------

@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize(("n1", "n2", "m1", "m2"), LAYOUT_CASES)
def test_mode_layout_is_exact_through_the_transforms(impl, n1, n2, m1, m2):
    # Forward: the real field of the labelled spectrum (made on the CPU in float64) must give
    # back every label in its own slot. Float32 error is far below 0.5 at these sizes, so
    # rounding compares the layout bit for bit, DC and Nyquist columns included (the single-pass
    # kernels carry those two columns packed as one complex column until the last step).
    full, kept = labelled_half_spectrum(n1, n2, m1, m2)
    field = ref.irfft2(full, (n1, n2)).astype(np.float32)
    modes = spectral.rfft2_truncated(dev(field), m1, m2, impl=impl).cpu().numpy()
    assert np.array_equal(rounded(modes.reshape(2, -1).astype(np.complex128)), kept)

    # Inverse: the label block, every dropped mode zero. Its float64 spectrum, rounded, must be
    # the labels at their positions and zero elsewhere, except that columns 0 and n2/2 come back
    # as their Hermitian join (the partner of row n1 - m1 is dropped, so both get half).
    block = dev(kept.reshape(2, 2 * m1, m2).astype(np.complex64))
    back = spectral.irfft2_from_modes(block, (n1, n2), impl=impl).cpu().numpy()
    only_kept = np.zeros_like(full).reshape(2, -1)
    only_kept[:, golden_positions(n1, n2, m1, m2)] = kept
    expected = hermitian_join(only_kept.reshape(full.shape), n2)
    assert np.array_equal(rounded(ref.rfft2(back)), expected)


@pytest.mark.parametrize("impl", IMPLS)
def test_band_limited_field_round_trips(rng, impl):
    # A field with no energy outside the kept modes is reproduced by forward then inverse. Row m1
    # of the DC column is zeroed: its conjugate partner -m1 is kept, so the pair is not complete.
    n1, n2, m1, m2 = 64, 64, 8, 8
    modes = ref.rfft2_truncate(random_real(rng, (2, n1, n2)), m1, m2)
    modes[..., m1, 0] = 0
    field = ref.irfft2_from_modes(modes, (n1, n2)).astype(np.float32)
    there = spectral.rfft2_truncated(dev(field), m1, m2, impl=impl)
    back = spectral.irfft2_from_modes(there, (n1, n2), impl=impl)
    assert_transform_close(back, field, n1 * n2, axes=AXES, tol=2 * fft_tolerance(n1 * n2))


@pytest.mark.parametrize("impl", IMPLS)
def test_modes_of_arrays_over_leading_dimensions(rng, impl):
    field = random_real(rng, (2, 70, 16, 32))
    y = spectral.rfft2_truncated(dev(field), 4, 5, impl=impl)
    assert tuple(y.shape) == (2, 70, 8, 5)
    assert_transform_close(y, ref.rfft2_truncate(field, 4, 5), 16 * 32, axes=AXES)


def test_pruned_implementations_agree_with_each_other(rng):
    field = dev(random_real(rng, (4, 128, 128)))
    first, *rest = (spectral.rfft2_truncated(field, 12, 12, impl=impl) for impl in IMPLS)
    for other in rest:
        assert_transform_close(other, first, 128 * 128, axes=AXES,
                               tol=2 * fft_tolerance(128 * 128))


# --- rejections (the reference's messages) ---------------------------------------------------

@pytest.mark.parametrize(("call", "message"), [
    (lambda: spectral.rfft2_truncated(torch.zeros(8, 8, device="cuda"), 5, 2), "1 <= m1 <= n1/2"),
    (lambda: spectral.rfft2_truncated(torch.zeros(8, 8, device="cuda"), 2, 6), "1 <= m1 <= n1/2"),
    (lambda: spectral.irfft2_from_modes(
        torch.zeros(3, 2, dtype=torch.complex64, device="cuda"), (8, 8)), "do not fit"),
    (lambda: spectral.fft_truncated(
        torch.zeros(2, 8, dtype=torch.complex64, device="cuda"), 9), "1 <= keep <= n"),
    (lambda: spectral.ifft_from_modes(
        torch.zeros(2, 8, dtype=torch.complex64, device="cuda"), 4), "1 <= keep <= n"),
], ids=["m1-too-large", "m2-too-large", "modes-too-many", "keep-too-large", "keep-above-n"])
def test_modes_that_do_not_fit_are_refused(call, message):
    with pytest.raises(RuntimeError, match=message):
        call()


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
    modes = spectral.rfft2_truncated(dev(x), m1, m2, impl=impl)
    assert_transform_close(modes, ref.rfft2_truncate(x, m1, m2), n1 * n2, axes=AXES)
    given = random_complex(rng, (17, 2 * m1, m2))
    y = spectral.irfft2_from_modes(dev(given), (n1, n2), impl=impl)
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
    modes = spectral.rfft2_truncated(dev(x), m1, m2, impl=impl)
    assert modes.shape == (5, 2 * m1, m2)
    assert_transform_close(modes, ref.rfft2_truncate(x, m1, m2), n1 * n2, axes=AXES)
    given = random_complex(rng, (5, 2 * m1, m2))
    y = spectral.irfft2_from_modes(dev(given), (n1, n2), impl=impl)
    assert_transform_close(y, ref.irfft2_from_modes(given, (n1, n2)), n1 * n2, axes=AXES)
