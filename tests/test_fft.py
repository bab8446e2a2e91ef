"""spectral.fft_c2c on the GPU for every implementation of spectral.FFT_IMPLS (reference
tests/test_fft.py covers the same ground): parity with the float64 oracle in both directions at
every power of two up to 4096 and every batch of the policy, the multi-pass sizes up to 2^24,
closed-form spectra, batch layouts, streams, agreement between implementations, and the
rejections with the reference's messages."""

import numpy as np
import pytest
import torch

import spectral
from oracle import reference as ref
from oracle.tolerance import (
    BATCHES,
    POW2_SIZES,
    assert_transform_close,
    fft_tolerance,
    random_complex,
)

pytestmark = pytest.mark.gpu

IMPLS = spectral.FFT_IMPLS
STOCKHAM = [impl for impl in IMPLS if impl.startswith("stockham")]
DIRECTIONS = ["forward", "inverse"]
# 8192 and 16384: one workgroup per transform; to 2^20 a column pass and a transposing row pass;
# beyond, the column pass runs as two (64 x n1/64 points) before the rows.
MULTI_PASS = [1 << p for p in range(13, 24)]


def c2c(x, impl: str, direction: str = "forward") -> torch.Tensor:
    """The transform on the GPU; `x` is a numpy array or a device tensor."""
    xd = torch.from_numpy(x).cuda() if isinstance(x, np.ndarray) else x
    return spectral.fft_c2c(xd, inverse=direction == "inverse", impl=impl)


def oracle(x: np.ndarray, direction: str) -> np.ndarray:
    return ref.fft(x) if direction == "forward" else ref.ifft(x)


# --- parity ----------------------------------------------------------------------------------

@pytest.mark.parametrize("direction", DIRECTIONS)
@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("batch", BATCHES)
@pytest.mark.parametrize("n", [1, *POW2_SIZES])
def test_c2c_parity(rng, n, batch, impl, direction):
    x = random_complex(rng, (batch, n))
    assert_transform_close(c2c(x, impl, direction), oracle(x, direction), n)


@pytest.mark.parametrize("direction", DIRECTIONS)
@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("batch", [1, 2])
@pytest.mark.parametrize("n", MULTI_PASS)
def test_c2c_parity_multi_pass(rng, n, batch, impl, direction):
    x = random_complex(rng, (batch, n))
    assert_transform_close(c2c(x, impl, direction), oracle(x, direction), n)


@pytest.mark.parametrize("impl", IMPLS)
def test_c2c_parity_at_the_size_limit(rng, impl):
    n = 1 << 24  # 32768 x 512: two 64 x 512 column passes, then the rows
    x = random_complex(rng, (1, n))
    assert_transform_close(c2c(x, impl), ref.fft(x), n)


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("n", [8, 64, 1024])
@pytest.mark.parametrize("batch", [255, 257, 1000])
def test_c2c_parity_with_a_partly_filled_last_workgroup(rng, impl, n, batch):
    # Small sizes pack many transforms per workgroup: these counts leave the last one partial.
    x = random_complex(rng, (batch, n))
    assert_transform_close(c2c(x, impl), ref.fft(x), n)


@pytest.mark.parametrize("direction", DIRECTIONS)
@pytest.mark.parametrize("impl", STOCKHAM)
@pytest.mark.parametrize(("n", "batch"), [(8192, 513), (8192, 1283), (16384, 300), (16384, 600)])
def test_c2c_parity_with_more_large_transforms_than_cus(rng, n, batch, impl, direction):
    # Every workgroup of 1024 lanes owns one whole transform. At 16384 points it loops over
    # transforms g, g + G, ... (G = 256 resident workgroups); the batches take the loop round twice
    # and three times, the last time for some workgroups only. At 8192 the grid covers the batch.
    x = random_complex(rng, (batch, n))
    assert_transform_close(c2c(x, impl, direction), oracle(x, direction), n)


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("n", [2, 64, 4096])
def test_c2c_round_trip(rng, impl, n):
    x = torch.from_numpy(random_complex(rng, (3, n))).cuda()
    back = c2c(c2c(x, impl), impl, "inverse")
    assert_transform_close(back, x, n, tol=2 * fft_tolerance(n))  # two transforms of error


@pytest.mark.parametrize("impl", IMPLS)
def test_c2c_is_linear(rng, impl):
    # F(a x + b y) = a F(x) + b F(y), with complex a and b, at two transforms of tolerance.
    n = 512
    x, y = random_complex(rng, (4, n)), random_complex(rng, (4, n))
    a, b = 0.75 - 0.5j, -1.25 + 2j
    lhs = c2c((a * x + b * y).astype(np.complex64), impl)
    rhs = a * c2c(x, impl) + b * c2c(y, impl)
    assert_transform_close(lhs, rhs, n, tol=2 * fft_tolerance(n))


# --- closed forms: an index or sign error moves or flips these, where random data only blurs

def tone(n: int, k0: int) -> np.ndarray:
    return np.exp(2j * np.pi * k0 * np.arange(n) / n)[None, :].astype(np.complex64)


def bin_at(n: int, k0: int, value: complex) -> np.ndarray:
    spectrum = np.zeros((1, n), np.complex128)
    spectrum[0, k0] = value
    return spectrum


@pytest.mark.parametrize("impl", IMPLS)
def test_unit_impulse_has_a_flat_spectrum(impl):
    x = np.zeros((1, 256), np.complex64)
    x[0, 0] = 1
    y = c2c(x, impl).cpu().numpy()
    assert np.max(np.abs(y - 1)) <= 1e-6


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("direction", DIRECTIONS)
def test_delayed_impulse_gives_a_phase_ramp_of_the_right_sign(impl, direction):
    # x = delta(m - 3): forward exp(-2 pi i k 3 / n), inverse exp(+2 pi i k 3 / n) / n.
    n, m0 = 512, 3
    x = np.zeros((1, n), np.complex64)
    x[0, m0] = 1
    sign, scale = (-1, 1.0) if direction == "forward" else (1, 1.0 / n)
    expected = scale * np.exp(sign * 2j * np.pi * np.arange(n) * m0 / n)[None, :]
    assert_transform_close(c2c(x, impl, direction), expected, n)


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize(("n", "k0"), [(256, 5), (1024, 333), (4096, 4095)])
def test_tone_lands_in_its_bin(impl, n, k0):
    assert_transform_close(c2c(tone(n, k0), impl), bin_at(n, k0, n), n)


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("n", [16384, 1 << 20])
def test_tone_lands_in_its_bin_through_the_multi_pass_splits(impl, n):
    # A wrong transpose or twiddle index of the splits moves the peak.
    assert_transform_close(c2c(tone(n, 12345), impl), bin_at(n, 12345, n), n)


@pytest.mark.parametrize("impl", IMPLS)
def test_inverse_of_a_single_bin_is_a_tone(impl):
    n, k0 = 2048, 77
    assert_transform_close(c2c(bin_at(n, k0, n).astype(np.complex64), impl, "inverse"),
                           tone(n, k0), n)


# --- layouts, streams, implementations -------------------------------------------------------

@pytest.mark.parametrize("impl", IMPLS)
def test_every_leading_dimension_is_a_batch_dimension(rng, impl):
    x = random_complex(rng, (2, 3, 64))
    y = c2c(x, impl)
    assert tuple(y.shape) == (2, 3, 64)
    assert_transform_close(y, ref.fft(x), 64)


@pytest.mark.parametrize("impl", IMPLS)
def test_strided_view_is_transformed_as_its_values(rng, impl):
    xd = torch.from_numpy(random_complex(rng, (64, 128))).cuda().transpose(0, 1)
    assert not xd.is_contiguous()
    assert_transform_close(c2c(xd, impl), ref.fft(xd.cpu().numpy()), 64)


@pytest.mark.parametrize("impl", IMPLS)
def test_no_transforms_give_an_empty_result(impl):
    y = c2c(torch.zeros(0, 8, dtype=torch.complex64, device="cuda"), impl)
    assert tuple(y.shape) == (0, 8)


@pytest.mark.parametrize("impl", STOCKHAM)
def test_multi_pass_scratch_follows_the_callers_stream(rng, impl):
    # The two-pass scratch is allocated and freed in stream order on the stream of the call.
    x = random_complex(rng, (2, 1 << 16))
    xd = torch.from_numpy(x).cuda()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        y = c2c(xd, impl)
    side.synchronize()
    assert_transform_close(y, ref.fft(x), 1 << 16)


def test_implementations_agree_with_each_other(rng):
    xd = torch.from_numpy(random_complex(rng, (16, 2048))).cuda()
    first, *rest = (c2c(xd, impl) for impl in IMPLS)
    for other in rest:
        assert_transform_close(other, first, 2048, tol=2 * fft_tolerance(2048))


# --- rejections (the reference's messages) ---------------------------------------------------

@pytest.mark.parametrize("impl", IMPLS)
def test_size_must_be_a_power_of_two(impl):
    with pytest.raises(RuntimeError, match="power of two"):
        c2c(torch.zeros(4, 12, dtype=torch.complex64, device="cuda"), impl)


@pytest.mark.parametrize("impl", STOCKHAM)
def test_size_beyond_the_limit_is_refused(impl):
    unread = torch.empty(1, 1 << 25, dtype=torch.complex64, device="cuda")
    with pytest.raises(RuntimeError, match="sizes up to 16777216"):
        c2c(unread, impl)


def test_unknown_implementation_is_refused():
    with pytest.raises(RuntimeError, match="unknown FFT implementation"):
        c2c(torch.zeros(4, 8, dtype=torch.complex64, device="cuda"), "nope")
