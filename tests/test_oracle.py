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


def idft_by_sum(modes: np.ndarray, n: int, freqs) -> np.ndarray:
    """x[m] = (1/n) sum_j modes[j] e^{+2 pi i f_j m / n}, one frequency at a time: the inverse
    DFT's definition over an explicit list of input frequencies, independent of numpy.fft."""
    m = np.arange(n)
    out = np.zeros(modes.shape[:-1] + (n,), dtype=np.complex128)
    for j, f in enumerate(freqs):
        out += modes[..., j : j + 1] * np.exp(2j * np.pi * ((f * m) % n) / n)
    return out / n


@pytest.mark.parametrize(("n", "k"), [(1, 1), (8, 1), (8, 3), (16, 16), (64, 17)])
def test_fft_truncate_is_the_first_outputs_of_the_definition(rng, n, k):
    x = random_complex(rng, (3, n))
    np.testing.assert_allclose(ref.fft_truncate(x, k), ref.dft(x)[..., :k], rtol=0,
                               atol=1e-10 * n)
    # the last kept bin is frequency k - 1, not k or n - k (a shifted or mirrored slice fails)
    if 1 < k < n:
        m = np.arange(n)
        tone = np.exp(2j * np.pi * (k - 1) * m / n)[None]
        got = ref.fft_truncate(tone, k)
        assert np.argmax(np.abs(got[0])) == k - 1 and abs(got[0, k - 1] - n) < 1e-9


@pytest.mark.parametrize(("n", "k"), [(1, 1), (8, 1), (8, 3), (32, 32), (64, 17)])
def test_ifft_from_modes_is_the_inverse_definition_over_the_kept_inputs(rng, n, k):
    modes = random_complex(rng, (3, k))
    want = idft_by_sum(modes, n, range(k))
    np.testing.assert_allclose(ref.ifft_from_modes(modes, n), want, rtol=0, atol=1e-12)


@pytest.mark.parametrize(("n", "k0"), [(8, 0), (8, 3), (64, 5), (64, 63)])
def test_ifft_from_modes_of_a_unit_mode_is_the_closed_form(n, k0):
    # One unit input at k0: x[m] = e^{+2 pi i k0 m / n} / n (a wrong sign, scale or slot fails).
    modes = np.zeros((1, k0 + 1), dtype=np.complex128)
    modes[0, k0] = 1.0
    m = np.arange(n)
    np.testing.assert_allclose(ref.ifft_from_modes(modes, n)[0],
                               np.exp(2j * np.pi * k0 * m / n) / n, rtol=0, atol=1e-15)


@pytest.mark.parametrize("n", [1, 8, 64])
def test_ifft_from_modes_of_every_mode_inverts_fft(rng, n):
    x = random_complex(rng, (4, n))
    np.testing.assert_allclose(ref.ifft_from_modes(ref.fft(x), n), x, rtol=0, atol=1e-12)


@pytest.mark.parametrize(("n1", "n2"), [(1, 8), (4, 4), (8, 16), (16, 2)])
def test_ifft2_is_the_inverse_definition(rng, n1, n2):
    # x[a, b] = (1 / (n1 n2)) sum_{p,q} X[p, q] e^{+2 pi i (p a / n1 + q b / n2)}, evaluated as the
    # conjugate of the forward definition on both axes.
    spec = random_complex(rng, (2, n1, n2))
    rows = ref.dft(np.conj(spec))
    both = np.swapaxes(ref.dft(np.swapaxes(rows, -1, -2)), -1, -2)
    np.testing.assert_allclose(ref.ifft2(spec), np.conj(both) / (n1 * n2), rtol=0, atol=1e-12)


def test_ifft2_is_column_inverses_of_row_inverses_and_inverts_fft2(rng):
    x = random_complex(rng, (3, 8, 32))
    spec = ref.fft2(x)
    rows_then_columns = np.fft.ifft(ref.ifft(spec), axis=-2)
    np.testing.assert_allclose(ref.ifft2(spec), rows_then_columns, rtol=0, atol=1e-14)
    np.testing.assert_allclose(ref.ifft2(spec), x, rtol=0, atol=1e-13)
    # a separable tone comes back at its own frequency pair with amplitude 1 / (n1 n2)
    tone = np.zeros((8, 32), dtype=np.complex128)
    tone[3, 30] = 1.0
    a, b = np.meshgrid(np.arange(8), np.arange(32), indexing="ij")
    np.testing.assert_allclose(ref.ifft2(tone), np.exp(2j * np.pi * (3 * a / 8 + 30 * b / 32))
                               / 256, rtol=0, atol=1e-16)


def test_the_pruned_pins_reject_plausible_mistakes(rng):
    # Mistakes planted in copies of the helpers (on the CPU), each caught by a check above.
    n, k = 16, 5
    modes = random_complex(rng, (2, k))
    want = idft_by_sum(modes, n, range(k))

    def modes_at_the_end(md, nn):  # kept inputs placed at n - k .. n - 1
        full = np.zeros(md.shape[:-1] + (nn,), dtype=np.complex128)
        full[..., nn - md.shape[-1]:] = md
        return np.fft.ifft(full, axis=-1)

    def forward_sign(md, nn):  # e^{-2 pi i k m / n}
        return np.fft.fft(np.pad(md, [(0, 0), (0, nn - md.shape[-1])]), axis=-1) / nn

    def unscaled(md, nn):  # the 1/n dropped
        return ref.ifft_from_modes(md, nn) * nn

    for bad in (modes_at_the_end, forward_sign, unscaled):
        assert not np.allclose(bad(modes, n), want, rtol=0, atol=1e-6), bad.__name__
    x = random_complex(rng, (2, n))
    assert not np.allclose(ref.fft(x)[..., 1 : k + 1], ref.dft(x)[..., :k], atol=1e-6)
    spec = random_complex(rng, (8, 16))
    rows = ref.dft(np.conj(spec))
    defn = np.conj(np.swapaxes(ref.dft(np.swapaxes(rows, -1, -2)), -1, -2)) / 128
    for bad in (np.fft.ifft(spec, axis=-1),  # rows only
                np.fft.fft2(spec) / 128,  # forward sign
                np.fft.ifft2(spec) * 128):  # unscaled
        assert not np.allclose(bad, defn, rtol=0, atol=1e-6)


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
