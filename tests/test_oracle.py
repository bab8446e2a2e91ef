"""The CPU oracle, checked before any kernel is compared against it (reference
tests/test_reference.py covers the same ground): the float64 references against the DFT written
out as sums, closed forms, invariants (Parseval, conjugation, Hermitian symmetry) and the golden
mode-index fixture; mistakes planted in copies of them must fail those checks. Then the
tolerance policy against float32 FFTs and the values it is quoted with."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from mode_labels import LAYOUT_CASES, hermitian_join, labelled_half_spectrum, rounded
from oracle import reference as ref
from oracle.tolerance import (
    FLOAT32_EPS,
    POW2_SIZES,
    assert_transform_close,
    fft_tolerance,
    random_complex,
    random_real,
)

GOLDEN = Path(__file__).parent / "golden"


def dft_by_sums(x: np.ndarray) -> np.ndarray:
    """X[k] = sum_m x[m] (cos - i sin)(2 pi k m / n), the angle reduced exactly in integers."""
    n = x.shape[-1]
    km = np.outer(np.arange(n), np.arange(n)) % n
    angle = 2 * np.pi * km / n
    return x.astype(np.complex128) @ (np.cos(angle) - 1j * np.sin(angle)).T


# --- the 1D references -----------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 2, 3, 5, 8, 12, 16, 31, 64, 100])
def test_fft_is_the_dft_sum(rng, n):
    x = random_complex(rng, (4, n))
    got = ref.fft(x)
    assert np.max(np.abs(got - dft_by_sums(x))) <= 1e-10 * n
    assert np.max(np.abs(ref.dft(x) - dft_by_sums(x))) <= 1e-10 * n  # the oracle's own sum


@pytest.mark.parametrize("n", [2, 64, 4096])
def test_fft_keeps_energy_and_ifft_is_its_conjugate_form(rng, n):
    x = random_complex(rng, (3, n)).astype(np.complex128)
    spectrum = ref.fft(x)
    # Parseval: sum |x|^2 = sum |X|^2 / n.
    np.testing.assert_allclose(np.sum(np.abs(spectrum) ** 2, -1) / n, np.sum(np.abs(x) ** 2, -1),
                               rtol=1e-12)
    # ifft(X) = conj(fft(conj X)) / n, and it returns x.
    np.testing.assert_allclose(ref.ifft(spectrum), np.conj(ref.fft(np.conj(spectrum))) / n,
                               rtol=0, atol=1e-13)
    assert np.max(np.abs(ref.ifft(spectrum) - x)) <= 1e-12


@pytest.mark.parametrize("n", [8, 9, 64])
def test_rfft_is_the_cosine_and_sine_sums_for_k_up_to_n_over_2(rng, n):
    x = random_real(rng, (3, n)).astype(np.float64)
    k = np.arange(n // 2 + 1)[:, None]
    m = np.arange(n)[None, :]
    angle = 2 * np.pi * (k * m % n) / n
    expected = x @ np.cos(angle).T - 1j * (x @ np.sin(angle).T)
    assert np.max(np.abs(ref.rfft(x) - expected)) <= 1e-11 * n


@pytest.mark.parametrize("n", [8, 9, 64])
def test_irfft_rebuilds_the_real_signal_from_its_half_spectrum(rng, n):
    x = random_real(rng, (3, n)).astype(np.float64)
    half = ref.rfft(x)
    assert np.max(np.abs(ref.irfft(half, n) - x)) <= 1e-12
    # and the full spectrum it stands for is Hermitian: X[n - k] = conj X[k]
    full = ref.fft(x)
    np.testing.assert_allclose(full[..., 1:][..., ::-1], np.conj(full[..., 1:]), atol=1e-11)


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


@pytest.mark.parametrize(("n1", "n2"), [(2, 8), (8, 16), (5, 3)])
def test_fft2_is_the_2d_dft_sum_and_separates_in_either_order(rng, n1, n2):
    x = random_complex(rng, (2, n1, n2))
    a, b = np.arange(n1), np.arange(n2)
    kernel = np.exp(-2j * np.pi * ((np.multiply.outer(a, a) % n1)[:, None, :, None] / n1
                                   + (np.multiply.outer(b, b) % n2)[None, :, None, :] / n2))
    by_sum = np.einsum("zmn,pqmn->zpq", x.astype(np.complex128), kernel)
    np.testing.assert_allclose(ref.fft2(x), by_sum, rtol=0, atol=1e-10 * n1 * n2)
    columns_first = ref.fft(np.fft.fft(x.astype(np.complex128), axis=-2))
    np.testing.assert_allclose(ref.fft2(x), columns_first, rtol=0, atol=1e-10 * n1 * n2)


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


def test_rfft2_truncate_takes_the_golden_positions_of_the_half_spectrum(rng):
    # tests/golden/modes_index.json holds, per shape, the half-spectrum position of every mode
    # slot, enumerated from the frequency semantics alone. The oracle's modes must be exactly the
    # values at those positions (the reference's known answer, test_reference.py:53-59, is the
    # (16, 16, 3, 4) case).
    for case in json.loads((GOLDEN / "modes_index.json").read_text()):
        n1, n2, m1, m2 = case["n1"], case["n2"], case["m1"], case["m2"]
        x = random_real(rng, (2, n1, n2))
        flat = ref.rfft2(x).reshape(2, -1)
        modes = ref.rfft2_truncate(x, m1, m2)
        assert modes.shape == (2, 2 * m1, m2)
        np.testing.assert_array_equal(modes.reshape(2, -1), flat[:, case["positions"]])


def test_labelled_spectra_of_the_layout_tests_are_exact_targets():
    # The GPU layout test (test_pruned.py) labels the kept modes with Gaussian integers and
    # compares rounded results: the labels must be distinct, survive a float64 round trip
    # through a real field, and be a fixed point of the real inverse's Hermitian join.
    for n1, n2, m1, m2 in LAYOUT_CASES:
        full, kept = labelled_half_spectrum(n1, n2, m1, m2)
        assert np.count_nonzero(kept) == kept.size
        assert len(set(kept[0].tolist())) == kept.shape[1]
        assert np.array_equal(rounded(ref.rfft2(ref.irfft2(full, (n1, n2)))), full)
        assert np.array_equal(hermitian_join(full, n2), full)
    # A mistake planted in the join (rows mirrored without the wrap of row 0) is caught.
    full, _ = labelled_half_spectrum(16, 16, 3, 4)
    shifted = full.copy()
    shifted[..., :, 0] = (full[..., :, 0] + np.conj(full[..., ::-1, 0])) / 2
    assert not np.array_equal(shifted, hermitian_join(full, 16))


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


@pytest.mark.parametrize(("n1", "n2"), [(8, 8), (4, 16), (16, 2)])
def test_keeping_the_whole_half_spectrum_loses_nothing(rng, n1, n2):
    # m1 = n1/2 rows of each sign and m2 = n2/2 + 1 columns are every stored frequency.
    x = random_real(rng, (2, n1, n2))
    modes = ref.rfft2_truncate(x, n1 // 2, n2 // 2 + 1)
    assert np.max(np.abs(ref.irfft2_from_modes(modes, (n1, n2)) - x)) <= 1e-12


@pytest.mark.parametrize(("kept", "dropped"), [([(1, 2), (-3, 1)], [(10, 12), (-7, 9)]),
                                               ([(0, 3), (2, 0)], [(4, 1), (-12, 5)])])
def test_truncation_passes_kept_cosines_and_removes_the_rest(kept, dropped):
    # Cosines at frequencies (f1, f2) inside m1 = m2 = 4 come back unchanged; those outside go.
    i, j = np.meshgrid(np.arange(32), np.arange(32), indexing="ij")

    def cosines(freqs):
        return sum(np.cos(2 * np.pi * (f1 * i + f2 * j) / 32) for f1, f2 in freqs)

    modes = ref.rfft2_truncate(cosines(kept) + cosines(dropped), m1=4, m2=4)
    back = ref.irfft2_from_modes(modes, (32, 32))
    assert np.max(np.abs(back - cosines(kept))) <= 1e-12


def test_reference_rejects_bad_modes():
    with pytest.raises(ValueError):
        ref.rfft2_truncate(np.zeros((8, 8)), 5, 2)
    with pytest.raises(ValueError):
        ref.irfft2_from_modes(np.zeros((3, 2)), (8, 8))
    with pytest.raises(ValueError):
        ref.fft_truncate(np.zeros((2, 8)), 9)


# --- the tolerance policy ------------------------------------------------------------------


@pytest.mark.parametrize("n", POW2_SIZES)
def test_policy_passes_numpys_own_single_precision_fft(rng, n):
    # pocketfft computes complex64 in single precision: a production float32 FFT must pass.
    x = random_complex(rng, (8, n))
    single = np.fft.fft(x.astype(np.complex64), axis=-1)
    assert single.dtype == np.complex64
    assert_transform_close(single, ref.fft(x), n)


def test_policy_names_the_transform_that_fails():
    n = 256
    exact = ref.fft(random_complex(np.random.default_rng(7), (4, 8, n)))
    bad = exact.copy()
    bad[2, 5, 100] += 20 * fft_tolerance(n) * np.linalg.norm(exact[2, 5])
    with pytest.raises(AssertionError, match=r"exceeds the tolerance .* in transform \(2, 5\)"):
        assert_transform_close(bad, exact, n)
    bad[2, 5, 100] = exact[2, 5, 100] + 0.5 * fft_tolerance(n) * np.linalg.norm(exact[2, 5])
    assert_transform_close(bad, exact, n)  # half the allowance passes


@pytest.mark.parametrize(("n", "quoted"), [(1, 9.54e-7), (2, 9.54e-7), (1024, 9.54e-6),
                                          (4096, 1.14e-5), (128 * 128, 1.34e-5),
                                          (512 * 512, 1.72e-5)])
def test_policy_values_are_eight_float32_epsilons_per_stage(n, quoted):
    assert FLOAT32_EPS == 2.0 ** -23
    assert fft_tolerance(n) == pytest.approx(quoted, rel=5e-3)  # quoted to 3 digits
    assert fft_tolerance(n) == 8 * 2.0 ** -23 * max(1, int(np.log2(n)))


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


@pytest.mark.parametrize("shape", [(64, 2), (64, 1024), (16, 4096), (8, 64, 64), (4, 128, 256)])
def test_torch_fft_on_the_cpu_meets_the_policy(rng, shape):
    if len(shape) == 2:
        x = random_complex(rng, shape)
        assert_transform_close(torch.fft.fft(torch.from_numpy(x)), ref.fft(x), shape[-1])
    else:
        x = random_real(rng, shape)
        n = shape[-2] * shape[-1]
        assert_transform_close(torch.fft.rfft2(torch.from_numpy(x)), ref.rfft2(x), n,
                               axes=(-2, -1))
