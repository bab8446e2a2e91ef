"""rfft / irfft on the GPU, every implementation: naive's generic path (an n/2-point complex
transform and a separate combine or prepare pass) and the Stockham kernels (the n/2 combine fused
into the store, the prepare into the load). Checked against the float64 oracle over the sizes and
batches the reference covers (tests/test_real.py), against closed forms that need no FFT at all,
and for the API's shapes, dtypes and error messages."""

import numpy as np
import pytest
import torch

import spectral
from oracle import reference as ref
from oracle.tolerance import (
    BATCHES,
    assert_transform_close,
    fft_tolerance,
    random_complex,
    random_real,
)

pytestmark = pytest.mark.gpu

IMPLS = spectral.FFT_IMPLS
# n real points run an n/2-point complex transform, so single-kernel sizes reach 8192.
SIZES = [1 << p for p in range(1, 14)]
LIMITED = [impl for impl in IMPLS if impl.startswith("stockham")]


def on_gpu(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def forward(x: np.ndarray, impl: str) -> np.ndarray:
    return spectral.rfft(on_gpu(x), impl=impl).cpu().numpy()


def inverse(h: np.ndarray, n: int, impl: str) -> np.ndarray:
    return spectral.irfft(on_gpu(h), n, impl=impl).cpu().numpy()


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("batch", BATCHES)
@pytest.mark.parametrize("n", SIZES)
def test_both_directions_match_the_oracle(rng, impl, n, batch):
    x = random_real(rng, (batch, n))
    spectrum = forward(x, impl)
    assert spectrum.shape == (batch, n // 2 + 1) and spectrum.dtype == np.complex64
    assert_transform_close(spectrum, ref.rfft(x), n)
    # the inverse on a Hermitian spectrum of the oracle's, then on our own forward's output
    given = ref.rfft(random_real(rng, (batch, n))).astype(np.complex64)
    y = inverse(given, n, impl)
    assert y.shape == (batch, n) and y.dtype == np.float32
    assert_transform_close(y, ref.irfft(given, n), n)
    assert_transform_close(inverse(spectrum, n, impl), x, n, tol=2 * fft_tolerance(n))


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("n", [2, 16, 1024, 8192])
def test_an_impulse_gives_a_pure_phase_ramp(impl, n):
    # x = delta at p: X[k] = exp(-2 pi i k p / n), |X[k]| = 1, with no FFT in the expectation.
    p = n // 2 - 1 if n > 2 else 1
    x = np.zeros((1, n), dtype=np.float32)
    x[0, p] = 1.0
    k = np.arange(n // 2 + 1)
    assert_transform_close(forward(x, impl), np.exp(-2j * np.pi * k * p / n)[None], n)


@pytest.mark.parametrize("impl", IMPLS)
def test_constant_and_alternating_signals_land_in_dc_and_nyquist(impl):
    n = 128
    x = np.stack([np.ones(n), (-1.0) ** np.arange(n)]).astype(np.float32)
    want = np.zeros((2, n // 2 + 1), dtype=np.complex128)
    want[0, 0] = n
    want[1, n // 2] = n
    np.testing.assert_allclose(forward(x, impl), want, rtol=0, atol=1e-4)


@pytest.mark.parametrize("impl", IMPLS)
def test_a_cosine_is_half_its_length_at_its_own_bin(impl):
    n, k0 = 2048, 100
    x = np.cos(2 * np.pi * k0 * np.arange(n) / n).astype(np.float32)[None]
    want = np.zeros((1, n // 2 + 1), dtype=np.complex128)
    want[0, k0] = n / 2
    assert_transform_close(forward(x, impl), want, n)


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("n", [8, 256])
def test_irfft_drops_the_imaginary_parts_of_dc_and_nyquist(rng, impl, n):
    # numpy's semantics, also for inputs no real signal has: only Re X[0] and Re X[n/2] count.
    spectrum = random_complex(rng, (3, n // 2 + 1))
    cleaned = spectrum.copy()
    cleaned[:, 0] = cleaned[:, 0].real
    cleaned[:, -1] = cleaned[:, -1].real
    assert_transform_close(inverse(spectrum, n, impl), ref.irfft(cleaned, n), n)
    expected = torch.fft.irfft(torch.from_numpy(spectrum).to(torch.complex128), n).numpy()
    assert_transform_close(inverse(spectrum, n, impl), expected, n)


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("batch", [255, 257, 1000])
def test_batches_that_leave_the_last_workgroup_partly_empty(rng, impl, batch):
    x = random_real(rng, (batch, 16))
    assert_transform_close(forward(x, impl), ref.rfft(x), 16)
    given = ref.rfft(random_real(rng, (batch, 16))).astype(np.complex64)
    assert_transform_close(inverse(given, 16, impl), ref.irfft(given, 16), 16)


@pytest.mark.parametrize("impl", IMPLS)
def test_leading_dimensions_and_strided_views(rng, impl):
    x = on_gpu(random_real(rng, (64, 2, 3))).permute(1, 2, 0)  # a (2, 3, 64) view, not contiguous
    assert not x.is_contiguous()
    y = spectral.rfft(x, impl=impl)
    assert y.shape == (2, 3, 33)
    assert_transform_close(y, ref.rfft(x.cpu().numpy()), 64)
    back = spectral.irfft(y.transpose(0, 1), 64, impl=impl)
    assert back.shape == (3, 2, 64)
    assert_transform_close(back, x.transpose(0, 1), 64, tol=2 * fft_tolerance(64))


@pytest.mark.parametrize("impl", IMPLS)
def test_no_rows_in_no_rows_out(impl):
    assert spectral.rfft(torch.zeros(0, 8, device="cuda"), impl=impl).shape == (0, 5)
    empty = torch.zeros(0, 5, dtype=torch.complex64, device="cuda")
    assert spectral.irfft(empty, 8, impl=impl).shape == (0, 8)


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("n", [1, 12])
def test_sizes_must_be_powers_of_two_from_2(impl, n):
    with pytest.raises(RuntimeError, match="power of two of at least 2"):
        spectral.rfft(torch.zeros(2, n, device="cuda"), impl=impl)


@pytest.mark.parametrize("impl", LIMITED)
def test_sizes_beyond_the_kernels_are_rejected(impl):
    with pytest.raises(RuntimeError, match="real sizes up to 8192"):
        spectral.rfft(torch.zeros(2, 16384, device="cuda"), impl=impl)


def test_the_spectrum_length_must_fit_n():
    with pytest.raises(RuntimeError, match="n/2 \\+ 1 = 5 inputs"):
        spectral.irfft(torch.zeros(2, 8, dtype=torch.complex64, device="cuda"), 8)


def test_dtypes_are_checked():
    with pytest.raises(RuntimeError, match="float32"):
        spectral.rfft(torch.zeros(2, 8, dtype=torch.complex64, device="cuda"))
    with pytest.raises(RuntimeError, match="complex64"):
        spectral.irfft(torch.zeros(2, 5, device="cuda"), 8)
