"""The CPU oracle, checked before any kernel is compared against it: the float64 references
against the DFT's definition, closed forms and each other; the tolerance policy against float32
rounding and production FFTs (reference tests/test_reference.py)."""

import numpy as np
import pytest
import torch

from oracle import reference as ref
from oracle.tolerance import (
    FLOAT32_EPS,
    POW2_SIZES,
    assert_transform_close,
    fft_tolerance,
    random_complex,
    random_real,
)

# --- the references ------------------------------------------------------------------------


@pytest.mark.parametrize("n", [1, 2, 3, 5, 8, 12, 16, 31, 64])
def test_fft_matches_the_definition(rng, n):
    x = random_complex(rng, (4, n))
    np.testing.assert_allclose(ref.fft(x), ref.dft(x), rtol=0, atol=1e-10 * n)


def test_dft_of_closed_forms():
    # Independent of numpy.fft: impulse -> ones, tone k0 -> n at bin k0, constant -> n at bin 0.
    n = 16
    imp = np.zeros((1, n))
    imp[0, 0] = 1
    np.testing.assert_allclose(ref.dft(imp), np.ones((1, n)), atol=1e-12)
    m = np.arange(n)
    tone = np.exp(2j * np.pi * 3 * m / n)[None]
    want = np.zeros((1, n), complex)
    want[0, 3] = n
    np.testing.assert_allclose(ref.dft(tone), want, atol=1e-11)
    np.testing.assert_allclose(ref.fft(tone), want, atol=1e-11)


@pytest.mark.parametrize("n", [2, 64, 4096])
def test_ifft_inverts_fft(rng, n):
    x = random_complex(rng, (3, n))
    np.testing.assert_allclose(ref.ifft(ref.fft(x)), x, rtol=0, atol=1e-12)


@pytest.mark.parametrize("n", [8, 9, 64])
def test_rfft_is_the_nonnegative_half_of_fft(rng, n):
    x = random_real(rng, (3, n))
    np.testing.assert_allclose(ref.rfft(x), ref.fft(x)[..., : n // 2 + 1], rtol=0, atol=1e-10)


@pytest.mark.parametrize("n", [8, 9, 64])
def test_irfft_inverts_rfft(rng, n):
    x = random_real(rng, (3, n))
    np.testing.assert_allclose(ref.irfft(ref.rfft(x), n), x, rtol=0, atol=1e-12)


def test_irfft_ignores_imaginary_dc_and_nyquist(rng):
    x = random_complex(rng, (2, 9)).astype(np.complex128)
    y = x.copy()
    y[:, 0] = y[:, 0].real
    y[:, 8] = y[:, 8].real
    np.testing.assert_allclose(ref.irfft(x, 16), ref.irfft(y, 16), atol=1e-14)
    # and equals the definition applied to the Hermitian extension of the real parts there
    full = np.concatenate([y, np.conj(y[:, 1:8][:, ::-1])], axis=1)
    np.testing.assert_allclose(ref.irfft(x, 16), (ref.dft(np.conj(full)).conj() / 16).real,
                               atol=1e-12)


def test_fft2_is_row_transforms_then_column_transforms(rng):
    x = random_complex(rng, (2, 8, 16))
    rows_then_columns = np.fft.fft(ref.fft(x), axis=-2)
    np.testing.assert_allclose(ref.fft2(x), rows_then_columns, rtol=0, atol=1e-10)


def test_rfft2_truncate_keeps_the_lowest_modes(rng):
    # The reference's known answer (test_reference.py:53-59), restated.
    x = random_real(rng, (2, 16, 16))
    full = ref.rfft2(x)
    modes = ref.rfft2_truncate(x, m1=3, m2=4)
    assert modes.shape == (2, 6, 4)
    np.testing.assert_array_equal(modes[..., :3, :], full[..., :3, :4])
    np.testing.assert_array_equal(modes[..., 3:, :], full[..., 13:, :4])


def test_truncation_layout_by_frequency(rng):
    # Independent of the slicing: row r of the modes holds frequency r for r < m1 and r - 2 m1
    # (negative) after; compute each kept mode from the 2D DFT definition at that frequency.
    n1, n2, m1, m2 = 8, 8, 2, 3
    x = random_real(rng, (n1, n2)).astype(np.float64)
    modes = ref.rfft2_truncate(x, m1, m2)
    i, j = np.meshgrid(np.arange(n1), np.arange(n2), indexing="ij")
    for r in range(2 * m1):
        f1 = r if r < m1 else r - 2 * m1
        for c in range(m2):
            want = np.sum(x * np.exp(-2j * np.pi * (f1 * i / n1 + c * j / n2)))
            assert abs(modes[r, c] - want) < 1e-10


def test_keeping_every_mode_round_trips(rng):
    x = random_real(rng, (2, 8, 8))
    modes = ref.rfft2_truncate(x, m1=4, m2=5)
    np.testing.assert_allclose(ref.irfft2_from_modes(modes, (8, 8)), x, rtol=0, atol=1e-12)


def test_truncation_is_a_low_pass_filter():
    i, j = np.meshgrid(np.arange(32), np.arange(32), indexing="ij")
    low = np.cos(2 * np.pi * (1 * i + 2 * j) / 32)
    high = np.cos(2 * np.pi * (10 * i + 12 * j) / 32)
    modes = ref.rfft2_truncate(low + high, m1=4, m2=4)
    np.testing.assert_allclose(ref.irfft2_from_modes(modes, (32, 32)), low, rtol=0, atol=1e-12)


def test_reference_rejects_bad_modes():
    with pytest.raises(ValueError):
        ref.rfft2_truncate(np.zeros((8, 8)), 5, 2)
    with pytest.raises(ValueError):
        ref.irfft2_from_modes(np.zeros((3, 2)), (8, 8))
    with pytest.raises(ValueError):
        ref.fft_truncate(np.zeros((2, 8)), 9)


# --- the tolerance policy ------------------------------------------------------------------


@pytest.mark.parametrize("n", POW2_SIZES)
def test_policy_accepts_float32_rounding_of_the_exact_result(rng, n):
    x = random_complex(rng, (8, n))
    exact = ref.fft(x)
    assert_transform_close(exact.astype(np.complex64), exact, n)


def test_policy_rejects_one_bad_transform_in_a_batch(rng):
    n = 1024
    x = random_complex(rng, (64, n))
    exact = ref.fft(x)
    actual = exact.copy()
    actual[17, 5] += 10 * fft_tolerance(n) * np.linalg.norm(exact[17])
    with pytest.raises(AssertionError, match=r"exceeds the tolerance .* in transform \(17,\)"):
        assert_transform_close(actual, exact, n)


def test_policy_limit_is_eight_eps_per_stage():
    assert fft_tolerance(4096) == pytest.approx(8 * FLOAT32_EPS * 12)
    assert fft_tolerance(1024) == pytest.approx(9.5367e-06, rel=1e-4)
    assert fft_tolerance(2) == pytest.approx(8 * FLOAT32_EPS)
    assert fft_tolerance(1) == pytest.approx(8 * FLOAT32_EPS)  # max(1, log2 N)


def test_policy_catches_plausible_mistakes(rng):
    # A dropped twiddle, a sign flip or a transposed index must each fail the policy.
    n = 64
    x = random_complex(rng, (4, n))
    good = ref.fft(x)
    assert_transform_close(good.astype(np.complex64), good, n)
    wrong_sign = np.fft.ifft(x, axis=-1) * n
    swapped = good[..., np.r_[1, 0, 2:n]]
    for bad in (wrong_sign, swapped, np.fft.fft(x[..., ::-1], axis=-1)):
        with pytest.raises(AssertionError):
            assert_transform_close(bad, good, n)


def test_torch_fft_meets_the_policy_on_cpu(rng):
    for n in POW2_SIZES:
        x = random_complex(rng, (64, n))
        assert_transform_close(torch.fft.fft(torch.from_numpy(x)), ref.fft(x), n)


def test_torch_rfft2_meets_the_policy_on_cpu(rng):
    for n1, n2 in [(64, 64), (128, 256)]:
        x = random_real(rng, (8, n1, n2))
        actual = torch.fft.rfft2(torch.from_numpy(x))
        assert_transform_close(actual, ref.rfft2(x), n1 * n2, axes=(-2, -1))
