"""spectral.fft2 / rfft2 / irfft2 on the GPU (reference tests/test_fft2.py covers the same
ground): parity with the float64 oracle for every implementation with the transpose column
method and every Stockham implementation with the strided one, in both directions, over square,
flat, tall and BASELINE C3 shapes; the inverse's reading of a non-Hermitian spectrum; round trips;
batch layouts; `columns="auto"`; and the rejections with the reference's messages. Then the
shapes of this stack's own single-pass, column-first and long-column kernels."""

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
DIRECTIONS = ["forward", "inverse"]

# (1024, 8) and (1024, 16): 1024-point strided columns, the persistent kernel in XCD order.
SHAPES = [(1, 8), (8, 1), (2, 2), (16, 16), (64, 32), (8, 256), (256, 8), (4096, 4), (4, 4096),
          (1024, 8), (64, 512), (128, 256)]
# (128, 128) and (512, 512) are BASELINE C3's grids, run here with both column methods.
REAL_SHAPES = [(1, 8), (8, 2), (16, 16), (64, 32), (8, 256), (256, 8), (4096, 4), (2, 8192),
               (128, 128), (512, 512), (1024, 16), (64, 1024), (128, 512)]


def dev(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(x).cuda()


def close_2d(actual, expected, n1: int, n2: int, *, passes: int = 1) -> None:
    """Within `passes` transforms' tolerance for n1 * n2 points, per array."""
    n = n1 * n2
    assert_transform_close(actual, expected, n, axes=AXES, tol=passes * fft_tolerance(n))


@pytest.mark.parametrize("direction", DIRECTIONS)
@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
@pytest.mark.parametrize(("n1", "n2"), SHAPES)
def test_complex_2d_parity(rng, n1, n2, impl, columns, direction):
    x = random_complex(rng, (3, n1, n2))
    inverse = direction == "inverse"
    y = spectral.fft2(dev(x), inverse=inverse, impl=impl, columns=columns)
    close_2d(y, ref.ifft2(x) if inverse else ref.fft2(x), n1, n2)


@pytest.mark.parametrize("direction", DIRECTIONS)
@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
@pytest.mark.parametrize(("n1", "n2"), REAL_SHAPES)
def test_real_2d_parity(rng, n1, n2, impl, columns, direction):
    field = random_real(rng, (3, n1, n2))
    if direction == "forward":
        y = spectral.rfft2(dev(field), impl=impl, columns=columns)
        assert tuple(y.shape) == (3, n1, n2 // 2 + 1)
        close_2d(y, ref.rfft2(field), n1, n2)
    else:
        half = ref.rfft2(field).astype(np.complex64)
        y = spectral.irfft2(dev(half), n2, impl=impl, columns=columns)
        assert tuple(y.shape) == (3, n1, n2)
        close_2d(y, ref.irfft2(half, (n1, n2)), n1, n2)


@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
def test_inverse_reads_a_non_hermitian_half_spectrum_as_numpy_does(rng, impl, columns):
    # The inverse is defined as complex inverses down the columns, then real inverses along the
    # rows that ignore the imaginary parts of bins 0 and n2/2; written out here in float64.
    half = random_complex(rng, (2, 16, 9))
    expected = np.fft.irfft(np.fft.ifft(half.astype(np.complex128), axis=-2), n=16, axis=-1)
    close_2d(spectral.irfft2(dev(half), 16, impl=impl, columns=columns), expected, 16, 16)


@pytest.mark.parametrize("kind", ["complex", "real"])
@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
def test_2d_round_trip(rng, impl, columns, kind):
    if kind == "complex":
        x = dev(random_complex(rng, (2, 32, 64)))
        there = spectral.fft2(x, impl=impl, columns=columns)
        back = spectral.fft2(there, inverse=True, impl=impl, columns=columns)
    else:
        x = dev(random_real(rng, (2, 32, 64)))
        back = spectral.irfft2(spectral.rfft2(x, impl=impl, columns=columns), 64, impl=impl)
    close_2d(back, x, 32, 64, passes=2)


@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
def test_arrays_spread_over_several_leading_dimensions(rng, impl, columns):
    # 300 arrays of 8 x 16: one workgroup's column group spans several arrays.
    field = random_real(rng, (2, 3, 50, 8, 16))
    y = spectral.rfft2(dev(field), impl=impl, columns=columns)
    assert tuple(y.shape) == (2, 3, 50, 8, 9)
    close_2d(y, ref.rfft2(field), 8, 16)


@pytest.mark.parametrize(("impl", "columns"), METHODS, ids=METHOD_IDS)
def test_permuted_view_is_transformed_as_its_values(rng, impl, columns):
    view = dev(random_complex(rng, (16, 32, 3))).permute(2, 0, 1)
    assert not view.is_contiguous()
    close_2d(spectral.fft2(view, impl=impl, columns=columns), ref.fft2(view.cpu().numpy()),
             16, 32)


def test_auto_columns_is_strided_where_a_column_kernel_exists(rng):
    # The same kernels in the same order: equal bits, not merely close values.
    field = dev(random_real(rng, (4, 32, 32)))
    for impl in spectral.FFT_IMPLS:
        method = "strided" if impl in STOCKHAM else "transpose"
        assert torch.equal(spectral.rfft2(field, impl=impl),
                           spectral.rfft2(field, impl=impl, columns=method)), impl


@pytest.mark.parametrize("op", ["rfft2", "fft2", "irfft2"])
def test_no_arrays_give_an_empty_result(op):
    if op == "rfft2":
        shape = spectral.rfft2(torch.zeros(0, 4, 8, device="cuda")).shape
        assert tuple(shape) == (0, 4, 5)
    elif op == "fft2":
        shape = spectral.fft2(torch.zeros(0, 4, 8, dtype=torch.complex64, device="cuda")).shape
        assert tuple(shape) == (0, 4, 8)
    else:
        half = torch.zeros(0, 4, 5, dtype=torch.complex64, device="cuda")
        assert tuple(spectral.irfft2(half, 8).shape) == (0, 4, 8)


# --- rejections (the reference's messages) ---------------------------------------------------

def _complex(*shape) -> torch.Tensor:
    return torch.zeros(*shape, dtype=torch.complex64, device="cuda")


@pytest.mark.parametrize(("call", "error", "message"), [
    (lambda: spectral.fft2(_complex(4, 8), impl="naive", columns="strided"), RuntimeError,
     "no strided column kernel"),
    (lambda: spectral.fft2(_complex(4, 8), impl="naive", columns="sideways"), RuntimeError,
     "columns must be"),
    (lambda: spectral.rfft2(torch.zeros(8, device="cuda")), RuntimeError,
     "at least two dimensions"),
    (lambda: spectral.irfft2(_complex(4, 8), 8), RuntimeError, r"n2/2 \+ 1 = 5 input columns"),
], ids=["strided-without-kernel", "unknown-method", "one-dimension", "spectrum-width"])
def test_bad_2d_requests_are_refused(call, error, message):
    with pytest.raises(error, match=message):
        call()


@pytest.mark.parametrize("impl", STOCKHAM)
def test_columns_past_the_kernel_limit_are_a_value_error(impl):
    # An invalid argument of the driver: ValueError, as the reference's std::invalid_argument.
    with pytest.raises(ValueError, match="n1 to be a power of two up to 4096"):
        spectral.fft2(_complex(8192, 2), impl=impl)


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
    y = spectral.rfft2(dev(x), impl=impl)
    assert_transform_close(y, ref.rfft2(x), n1 * n2, axes=AXES)
    two_pass = spectral.rfft2(dev(x), impl=impl, columns="transpose")
    assert_transform_close(y, two_pass.cpu().numpy(), n1 * n2, axes=AXES)
    spectrum = random_complex(rng, (17, n1, n2 // 2 + 1))
    back = spectral.irfft2(dev(spectrum), n2, impl=impl)
    assert_transform_close(back, ref.irfft2(spectrum, (n1, n2)), n1 * n2, axes=AXES)


# The whole-spectrum irfft2 of 16384-point arrays runs persistent: workgroup g transforms arrays
# g, g + G, g + 2G, ... (G = the workgroups resident at once, 512 on a 256-CU MI355X). 1283 arrays
# take the loop round three times, the third time for only some workgroups. Arrays on either side
# of each turn are checked against the oracle; every array's forward (one array per workgroup,
# 1283 workgroups) against torch.fft (rocFFT), and its inverse through the round trip.
PERSISTENT_SHAPES = [(128, 128), (256, 64), (64, 256)]
TURN_EDGES = [0, 1, 511, 512, 513, 1023, 1024, 1025, 1281, 1282]


@pytest.mark.parametrize("impl", FUSED_IMPLS)
@pytest.mark.parametrize(("n1", "n2"), PERSISTENT_SHAPES)
def test_single_pass_real_2d_over_more_arrays_than_resident_workgroups(rng, impl, n1, n2):
    batch, n = 1283, n1 * n2
    x = random_real(rng, (batch, n1, n2))
    xd = dev(x)
    y = spectral.rfft2(xd, impl=impl)
    assert_transform_close(y[TURN_EDGES].cpu().numpy(), ref.rfft2(x[TURN_EDGES]), n, axes=AXES)
    assert_transform_close(y.cpu().numpy(), torch.fft.rfft2(xd).cpu().numpy(), n, axes=AXES,
                           tol=2 * fft_tolerance(n))
    back = spectral.irfft2(y, n2, impl=impl)
    assert_transform_close(back.cpu().numpy(), x, n, axes=AXES, tol=2 * fft_tolerance(n))

    # A general half spectrum (not one of a real field) at the turn edges.
    spectrum = random_complex(rng, (batch, n1, n2 // 2 + 1))
    field = spectral.irfft2(dev(spectrum), n2, impl=impl)
    assert_transform_close(field[TURN_EDGES].cpu().numpy(),
                           ref.irfft2(spectrum[TURN_EDGES], (n1, n2)), n, axes=AXES)


# Shapes past the single-pass kernels with n2 >= 32 run column-first: columns over the real array
# read as complex, then one pass over pairs of rows (k1, -k1). n1 = 1 and 2 make every row its own
# partner; batches of 3 leave the last workgroup's pairs partly empty. The inverse takes random,
# non-Hermitian spectra: columns 0 and n2/2 are symmetrized across the pair as numpy does.
# 512-row shapes cover C3's column kernel from one 16-column tile per array (512 x 32) to 256.
COLUMN_FIRST_SHAPES = [(1, 64), (2, 32), (8, 256), (32, 512), (256, 256), (512, 512), (2048, 64),
                       (16, 4096), (4, 8192), (512, 32), (512, 64), (512, 2048), (512, 8192)]
STOCKHAM_IMPLS = STOCKHAM


@pytest.mark.parametrize("impl", STOCKHAM_IMPLS)
@pytest.mark.parametrize(("n1", "n2"), COLUMN_FIRST_SHAPES)
def test_column_first_rfft2_and_irfft2(rng, impl, n1, n2):
    x = random_real(rng, (3, n1, n2))
    y = spectral.rfft2(dev(x), impl=impl)
    assert_transform_close(y, ref.rfft2(x), n1 * n2, axes=AXES)
    spectrum = random_complex(rng, (3, n1, n2 // 2 + 1))
    back = spectral.irfft2(dev(spectrum), n2, impl=impl)
    assert_transform_close(back, ref.irfft2(spectrum, (n1, n2)), n1 * n2, axes=AXES)
    hermitian = ref.rfft2(x).astype(np.complex64)
    again = spectral.irfft2(dev(hermitian), n2, impl=impl)
    assert_transform_close(again, x, n1 * n2, tol=2 * fft_tolerance(n1 * n2), axes=AXES)


# Complex 2D arrays whose n1 x n2 tile fits a workgroup's LDS run as one kernel (fft2_c2c,
# strided method); batches of 17 leave the last workgroup partly empty.
FUSED_C2C_SHAPES = [(4, 4), (8, 8), (16, 16), (32, 32), (32, 64), (64, 32), (64, 64), (64, 128),
                    (128, 64), (128, 128)]


@pytest.mark.parametrize("impl", FUSED_IMPLS)
@pytest.mark.parametrize(("n1", "n2"), FUSED_C2C_SHAPES)
def test_single_pass_fft2_and_ifft2(rng, impl, n1, n2):
    x = random_complex(rng, (17, n1, n2))
    y = spectral.fft2(dev(x), impl=impl)
    assert_transform_close(y, ref.fft2(x), n1 * n2, axes=AXES)
    two_pass = spectral.fft2(dev(x), impl=impl, columns="transpose")
    assert_transform_close(y, two_pass.cpu().numpy(), n1 * n2, axes=AXES)
    back = spectral.fft2(dev(x), inverse=True, impl=impl)
    assert_transform_close(back, ref.ifft2(x), n1 * n2, axes=AXES)


# The single-pass complex 2D of 16384-point arrays runs persistent: workgroup g transforms arrays
# g, g + G, ... (G = the workgroups resident at once: one per CU at 128 x 128, two at 64 x 128).
# The batches take the loop round three times, the third time for only some workgroups; every
# array is checked against the oracle in both directions.
@pytest.mark.parametrize("impl", FUSED_IMPLS)
@pytest.mark.parametrize(("n1", "n2", "batch"), [(128, 128, 600), (64, 128, 1283)])
def test_single_pass_fft2_over_more_arrays_than_resident_workgroups(rng, impl, n1, n2, batch):
    x = random_complex(rng, (batch, n1, n2))
    y = spectral.fft2(dev(x), impl=impl)
    assert_transform_close(y, ref.fft2(x), n1 * n2, axes=AXES)
    back = spectral.fft2(dev(x), inverse=True, impl=impl)
    assert_transform_close(back, ref.ifft2(x), n1 * n2, axes=AXES)


# Columns of 2048 and 4096 points run as two passes of 64 x (n1 / 64) (tiles of 32 or more
# columns), for complex 2D and for the column passes of the real column-first transforms.
LONG_COLUMN_SHAPES = [(2048, 32), (2048, 64), (4096, 32), (4096, 128)]


@pytest.mark.parametrize("impl", STOCKHAM_IMPLS)
@pytest.mark.parametrize(("n1", "n2"), LONG_COLUMN_SHAPES)
def test_long_columns(rng, impl, n1, n2):
    x = random_complex(rng, (2, n1, n2))
    assert_transform_close(spectral.fft2(dev(x), impl=impl), ref.fft2(x), n1 * n2, axes=AXES)
    assert_transform_close(spectral.fft2(dev(x), inverse=True, impl=impl), ref.ifft2(x),
                           n1 * n2, axes=AXES)
    r = random_real(rng, (2, n1, 2 * n2))
    assert_transform_close(spectral.rfft2(dev(r), impl=impl), ref.rfft2(r), 2 * n1 * n2,
                           axes=AXES)
    spectrum = random_complex(rng, (2, n1, n2 + 1))
    assert_transform_close(spectral.irfft2(dev(spectrum), 2 * n2, impl=impl),
                           ref.irfft2(spectrum, (n1, 2 * n2)), 2 * n1 * n2, axes=AXES)
