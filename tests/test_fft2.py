"""2D transforms against the float64 oracle (reference tests/test_fft2.py): every implementation
with the transpose method, and the ones with a strided column kernel with that method too."""

import numpy as np
import pytest
import torch

import spectral
from oracle import reference as ref
from oracle.tolerance import assert_transform_close, fft_tolerance, random_complex, random_real

pytestmark = pytest.mark.gpu

AXES = (-2, -1)
STOCKHAM = [impl for impl in spectral.FFT_IMPLS if impl.startswith("stockham")]
METHODS = [(impl, "transpose") for impl in spectral.FFT_IMPLS] + [
    (impl, "strided") for impl in STOCKHAM
]
METHOD_IDS = [f"{impl}-{cols}" for impl, cols in METHODS]

# (1024, 8) and (1024, 16): 1024-point strided columns, the persistent kernel in XCD order.
SHAPES = [(1, 8), (8, 1), (2, 2), (16, 16), (64, 32), (8, 256), (256, 8), (4096, 4), (4, 4096),
          (1024, 8), (64, 512), (128, 256)]
# (128, 128) and (512, 512) are BASELINE C3's grids, run here with both column methods.
REAL_SHAPES = [(1, 8), (8, 2), (16, 16), (64, 32), (8, 256), (256, 8), (4096, 4), (2, 8192),
               (128, 128), (512, 512), (1024, 16), (64, 1024), (128, 512)]


def cuda(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(x).cuda()


@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
@pytest.mark.parametrize(("n1", "n2"), SHAPES)
def test_fft2_matches_the_oracle(rng, impl, columns, n1, n2):
    x = random_complex(rng, (3, n1, n2))
    y = spectral.fft2(cuda(x), impl=impl, columns=columns)
    assert_transform_close(y, ref.fft2(x), n1 * n2, axes=AXES)


@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
@pytest.mark.parametrize(("n1", "n2"), SHAPES)
def test_ifft2_matches_the_oracle(rng, impl, columns, n1, n2):
    x = random_complex(rng, (3, n1, n2))
    y = spectral.fft2(cuda(x), inverse=True, impl=impl, columns=columns)
    assert_transform_close(y, ref.ifft2(x), n1 * n2, axes=AXES)


@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
@pytest.mark.parametrize(("n1", "n2"), REAL_SHAPES)
def test_rfft2_matches_the_oracle(rng, impl, columns, n1, n2):
    x = random_real(rng, (3, n1, n2))
    y = spectral.rfft2(cuda(x), impl=impl, columns=columns)
    assert y.shape == (3, n1, n2 // 2 + 1)
    assert_transform_close(y, ref.rfft2(x), n1 * n2, axes=AXES)


@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
@pytest.mark.parametrize(("n1", "n2"), REAL_SHAPES)
def test_irfft2_matches_the_oracle(rng, impl, columns, n1, n2):
    spectrum = ref.rfft2(random_real(rng, (3, n1, n2))).astype(np.complex64)
    y = spectral.irfft2(cuda(spectrum), n2, impl=impl, columns=columns)
    assert y.shape == (3, n1, n2)
    assert_transform_close(y, ref.irfft2(spectrum, (n1, n2)), n1 * n2, axes=AXES)


@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
def test_irfft2_of_a_non_hermitian_spectrum_matches_torch(rng, impl, columns):
    spectrum = random_complex(rng, (2, 16, 9))
    expected = torch.fft.irfft2(torch.from_numpy(spectrum).to(torch.complex128), s=(16, 16))
    y = spectral.irfft2(cuda(spectrum), 16, impl=impl, columns=columns)
    assert_transform_close(y, expected.numpy(), 256, axes=AXES)


@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
def test_round_trips(rng, impl, columns):
    x = cuda(random_complex(rng, (2, 32, 64)))
    back = spectral.fft2(
        spectral.fft2(x, impl=impl, columns=columns), inverse=True, impl=impl, columns=columns
    )
    assert_transform_close(back, x, 32 * 64, axes=AXES, tol=2 * fft_tolerance(32 * 64))
    r = cuda(random_real(rng, (2, 32, 64)))
    back = spectral.irfft2(spectral.rfft2(r, impl=impl, columns=columns), 64, impl=impl)
    assert_transform_close(back, r, 32 * 64, axes=AXES, tol=2 * fft_tolerance(32 * 64))


@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
def test_many_arrays_and_leading_dimensions(rng, impl, columns):
    # 300 arrays of 8 x 16: column groups of one workgroup straddle arrays.
    x = random_real(rng, (2, 3, 50, 8, 16))
    y = spectral.rfft2(cuda(x), impl=impl, columns=columns)
    assert y.shape == (2, 3, 50, 8, 9)
    assert_transform_close(y, ref.rfft2(x), 128, axes=AXES)


@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
def test_non_contiguous_input(rng, impl, columns):
    x = cuda(random_complex(rng, (16, 32, 3))).permute(2, 0, 1)
    assert not x.is_contiguous()
    y = spectral.fft2(x, impl=impl, columns=columns)
    assert_transform_close(y, ref.fft2(x.cpu().numpy()), 16 * 32, axes=AXES)


def test_auto_picks_strided_when_available(rng):
    x = cuda(random_real(rng, (4, 32, 32)))
    for impl in STOCKHAM:
        auto = spectral.rfft2(x, impl=impl)
        assert torch.equal(auto, spectral.rfft2(x, impl=impl, columns="strided"))
    naive = spectral.rfft2(x, impl="naive")
    assert torch.equal(naive, spectral.rfft2(x, impl="naive", columns="transpose"))


def test_empty_input_gives_empty_output():
    x = torch.zeros(0, 4, 8, device="cuda")
    assert spectral.rfft2(x).shape == (0, 4, 5)
    assert spectral.fft2(x.to(torch.complex64)).shape == (0, 4, 8)
    empty = torch.zeros(0, 4, 5, dtype=torch.complex64, device="cuda")
    assert spectral.irfft2(empty, 8).shape == (0, 4, 8)


def test_rejects_strided_without_a_column_kernel():
    x = torch.zeros(4, 8, dtype=torch.complex64, device="cuda")
    with pytest.raises(RuntimeError, match="no strided column kernel"):
        spectral.fft2(x, impl="naive", columns="strided")


def test_rejects_an_unknown_column_method():
    x = torch.zeros(4, 8, dtype=torch.complex64, device="cuda")
    with pytest.raises(RuntimeError, match="columns must be"):
        spectral.fft2(x, impl="naive", columns="sideways")


@pytest.mark.parametrize("impl", STOCKHAM)
def test_rejects_columns_longer_than_the_kernel_supports(impl):
    # Raised by the driver as an invalid argument: ValueError, as in the reference.
    x = torch.zeros(8192, 2, dtype=torch.complex64, device="cuda")
    with pytest.raises(ValueError, match="n1 to be a power of two up to 4096"):
        spectral.fft2(x, impl=impl)


def test_rejects_one_dimensional_input():
    with pytest.raises(RuntimeError, match="at least two dimensions"):
        spectral.rfft2(torch.zeros(8, device="cuda"))


def test_rejects_a_spectrum_of_the_wrong_width():
    x = torch.zeros(4, 8, dtype=torch.complex64, device="cuda")
    with pytest.raises(RuntimeError, match="n2/2 \\+ 1 = 5 input columns"):
        spectral.irfft2(x, 8)


# Every shape with a single-pass kernel (n1, n2 in 4 .. 16, or in 32 .. 256 with the half spectrum
# within the LDS tile), with a batch of 17 that leaves the last workgroup partly empty.
FUSED_SHAPES = [(4, 4), (8, 4), (16, 4), (4, 8), (8, 8), (16, 8), (4, 16), (8, 16), (16, 16),
                (32, 32), (64, 32), (128, 32), (256, 32), (32, 64), (64, 64), (128, 64),
                (256, 64), (32, 128), (64, 128), (128, 128), (32, 256), (64, 256)]
FUSED_IMPLS = ["stockham_r4", "stockham_r8", "stockham_r8_table"]


@pytest.mark.parametrize("impl", FUSED_IMPLS)
@pytest.mark.parametrize(("n1", "n2"), FUSED_SHAPES)
def test_single_pass_rfft2_and_irfft2(rng, impl, n1, n2):
    x = random_real(rng, (17, n1, n2))
    y = spectral.rfft2(cuda(x), impl=impl)
    assert_transform_close(y, ref.rfft2(x), n1 * n2, axes=AXES)
    two_pass = spectral.rfft2(cuda(x), impl=impl, columns="transpose")
    assert_transform_close(y, two_pass.cpu().numpy(), n1 * n2, axes=AXES)
    spectrum = random_complex(rng, (17, n1, n2 // 2 + 1))
    back = spectral.irfft2(cuda(spectrum), n2, impl=impl)
    assert_transform_close(back, ref.irfft2(spectrum, (n1, n2)), n1 * n2, axes=AXES)


# Shapes past the single-pass kernels with n2 >= 32 run column-first: columns over the real array
# read as complex, then one pass over pairs of rows (k1, -k1). n1 = 1 and 2 make every row its own
# partner; batches of 3 leave the last workgroup's pairs partly empty. The inverse takes random,
# non-Hermitian spectra: columns 0 and n2/2 are symmetrized across the pair as numpy does.
# 512-row shapes cover C3's column kernel from one 16-column tile per array (512 x 32) to 256.
COLUMN_FIRST_SHAPES = [(1, 64), (2, 32), (8, 256), (32, 512), (256, 256), (512, 512), (2048, 64),
                       (16, 4096), (4, 8192), (512, 32), (512, 64), (512, 2048), (512, 8192)]
STOCKHAM_IMPLS = [impl for impl in spectral.FFT_IMPLS if impl.startswith("stockham")]


@pytest.mark.parametrize("impl", STOCKHAM_IMPLS)
@pytest.mark.parametrize(("n1", "n2"), COLUMN_FIRST_SHAPES)
def test_column_first_rfft2_and_irfft2(rng, impl, n1, n2):
    x = random_real(rng, (3, n1, n2))
    y = spectral.rfft2(cuda(x), impl=impl)
    assert_transform_close(y, ref.rfft2(x), n1 * n2, axes=AXES)
    spectrum = random_complex(rng, (3, n1, n2 // 2 + 1))
    back = spectral.irfft2(cuda(spectrum), n2, impl=impl)
    assert_transform_close(back, ref.irfft2(spectrum, (n1, n2)), n1 * n2, axes=AXES)
    hermitian = ref.rfft2(x).astype(np.complex64)
    again = spectral.irfft2(cuda(hermitian), n2, impl=impl)
    assert_transform_close(again, x, n1 * n2, tol=2 * fft_tolerance(n1 * n2), axes=AXES)


# Complex 2D arrays whose n1 x n2 tile fits a workgroup's LDS run as one kernel (fft2_c2c,
# strided method); batches of 17 leave the last workgroup partly empty.
FUSED_C2C_SHAPES = [(4, 4), (8, 8), (16, 16), (32, 32), (32, 64), (64, 32), (64, 64), (64, 128),
                    (128, 64), (128, 128)]


@pytest.mark.parametrize("impl", FUSED_IMPLS)
@pytest.mark.parametrize(("n1", "n2"), FUSED_C2C_SHAPES)
def test_single_pass_fft2_and_ifft2(rng, impl, n1, n2):
    x = random_complex(rng, (17, n1, n2))
    y = spectral.fft2(cuda(x), impl=impl)
    assert_transform_close(y, ref.fft2(x), n1 * n2, axes=AXES)
    two_pass = spectral.fft2(cuda(x), impl=impl, columns="transpose")
    assert_transform_close(y, two_pass.cpu().numpy(), n1 * n2, axes=AXES)
    back = spectral.fft2(cuda(x), inverse=True, impl=impl)
    assert_transform_close(back, ref.ifft2(x), n1 * n2, axes=AXES)


# Columns of 2048 and 4096 points run as two passes of 64 x (n1 / 64) (tiles of 32 or more
# columns), for complex 2D and for the column passes of the real column-first transforms.
LONG_COLUMN_SHAPES = [(2048, 32), (2048, 64), (4096, 32), (4096, 128)]


@pytest.mark.parametrize("impl", STOCKHAM_IMPLS)
@pytest.mark.parametrize(("n1", "n2"), LONG_COLUMN_SHAPES)
def test_long_columns(rng, impl, n1, n2):
    x = random_complex(rng, (2, n1, n2))
    assert_transform_close(spectral.fft2(cuda(x), impl=impl), ref.fft2(x), n1 * n2, axes=AXES)
    assert_transform_close(spectral.fft2(cuda(x), inverse=True, impl=impl), ref.ifft2(x),
                           n1 * n2, axes=AXES)
    r = random_real(rng, (2, n1, 2 * n2))
    assert_transform_close(spectral.rfft2(cuda(r), impl=impl), ref.rfft2(r), 2 * n1 * n2,
                           axes=AXES)
    spectrum = random_complex(rng, (2, n1, n2 + 1))
    assert_transform_close(spectral.irfft2(cuda(spectrum), 2 * n2, impl=impl),
                           ref.irfft2(spectrum, (n1, 2 * n2)), 2 * n1 * n2, axes=AXES)
