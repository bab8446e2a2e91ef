"""The radio callers (spectral.rf; reference tests/test_rf.py): windows, the framed spectrum,
overlap-save FIR, the command line and the chirp / BPSK / QPSK recordings the reference ships
(copied as data into tests/golden/rf). Every GPU check runs with the torch.fft backend and with
each of this stack's implementations; the Stockham ones take the single-kernel paths
(torch.ops.spectral.rf_spectrum / rf_fir), "naive" the composed one. Expected values come from
numpy.fft and scipy.signal.lfilter in float64."""

import ctypes
import json
from pathlib import Path

import numpy as np
import pytest
import scipy.signal
import torch

from oracle.tolerance import random_complex, random_real
from spectral import rf

FIXTURES = Path(__file__).resolve().parent / "golden" / "rf"
BACKENDS = rf.FFT_BACKENDS
OURS = [b for b in BACKENDS if b.startswith("stockham")]
LIB = Path(__file__).resolve().parents[1] / "gpu-spectral-stack_amd" / "python" / "spectral"

gpu = pytest.mark.gpu


def cuda(x) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def relative_error(actual, expected) -> float:
    actual = np.asarray(actual, dtype=np.complex128)
    expected = np.asarray(expected, dtype=np.complex128)
    return float(np.linalg.norm(actual - expected) / max(np.linalg.norm(expected), 1e-30))


def load_fixture(name: str) -> tuple[np.ndarray, dict]:
    return rf.read_cf32(FIXTURES / f"{name}.cf32"), json.loads(
        (FIXTURES / f"{name}.json").read_text()
    )


def framed_spectrum(x: np.ndarray, nfft: int, window_name: str) -> np.ndarray:
    """numpy.fft of the zero-padded, windowed frames of each row (float64)."""
    n = x.shape[-1]
    count = max(1, -(-n // nfft))
    padded = np.zeros((*x.shape[:-1], count * nfft), dtype=np.complex128)
    padded[..., :n] = x
    if window_name == "rect" or nfft == 1:
        w = np.ones(nfft)
    else:
        w = scipy.signal.get_window(window_name, nfft, fftbins=True)
    return np.fft.fft(padded.reshape(*x.shape[:-1], count, nfft) * w, axis=-1)


# --- Windows, block sizes, fixtures (CPU) -----------------------------------------------------


@pytest.mark.parametrize("name", ["hann", "hamming", "blackman"])
@pytest.mark.parametrize("n", [1, 2, 7, 64, 1024])
def test_windows_match_scipy_periodic_windows(name, n):
    expected = scipy.signal.get_window(name, n, fftbins=True)
    np.testing.assert_allclose(rf.window(name, n).numpy(), expected, rtol=0, atol=1e-7)


def test_rect_window_is_all_ones():
    assert torch.equal(rf.window("rect", 5), torch.ones(5))


def test_rejects_an_unknown_window_and_an_empty_one():
    with pytest.raises(ValueError, match="unknown window"):
        rf.window("kaiser", 8)
    with pytest.raises(ValueError, match="at least one point"):
        rf.window("hann", 0)


def test_default_block_size():
    assert rf.default_nfft(1) == 64
    assert rf.default_nfft(63) == 256
    assert rf.default_nfft(1025) == 4096
    assert rf.default_nfft(5000) == 8192
    with pytest.raises(ValueError, match="at least one tap"):
        rf.default_nfft(0)


def test_rejects_an_unknown_backend():
    with pytest.raises(ValueError, match="unknown fft_impl"):
        rf.fft(torch.zeros(4, dtype=torch.complex64), fft_impl="fftw")


def test_backends_name_torch_fft_and_every_implementation():
    assert rf.FFT_BACKENDS[:2] == ("rocfft", "cufft")
    assert set(OURS) <= set(rf.FFT_BACKENDS)


def test_fixtures_are_small_and_described():
    for path in FIXTURES.glob("*.cf32"):
        x, meta = load_fixture(path.stem)
        assert path.stat().st_size < 1 << 20
        assert meta["num_samples"] == len(x)
        assert {"sample_rate", "generator", "seed"} <= meta.keys()


def test_chirp_frequency_rises_linearly():
    x, meta = load_fixture("chirp")
    inst = np.angle(x[1:] * np.conj(x[:-1])) / (2 * np.pi) * meta["sample_rate"]  # Hz
    ramp = np.linspace(meta["f0_hz"], meta["f1_hz"], len(x), endpoint=False)[:-1]
    assert np.max(np.abs(inst - ramp)) < 0.002 * meta["sample_rate"]


@pytest.mark.parametrize("name", ["bpsk", "qpsk"])
def test_fixtures_decode_with_the_float64_matched_filter(name):
    # Pins the recordings and their metadata without the GPU: scipy's direct-form filter.
    x, meta = load_fixture(name)
    taps = rf.read_f32(FIXTURES / meta["pulse"])
    y = scipy.signal.lfilter(taps.astype(np.float64), 1.0, x.astype(np.complex128))
    samples = y[meta["first_symbol_after_matched_filter"] :: meta["samples_per_symbol"]]
    if name == "bpsk":
        assert np.array_equal((samples.real > 0).astype(int), np.array(meta["bits"])[: len(samples)])
    else:
        decided = (samples.real < 0).astype(int) + 2 * (samples.imag < 0).astype(int)
        assert np.array_equal(decided, np.array(meta["symbols"])[: len(samples)])


def test_c_abi_validates_radio_arguments():
    import spectral  # noqa: F401  # loads the library the way the package does

    lib = ctypes.CDLL(str(LIB / "libspectral_hip.so"))
    lib.spx_last_error.restype = ctypes.c_char_p
    ll = ctypes.c_longlong
    p, q = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x100000)
    assert lib.spx_rf_max_nfft(0) == 0  # naive: composed path only
    assert lib.spx_rf_max_nfft(3) == 16384
    assert lib.spx_rf_spectrum(3, p, None, q, ll(100), 3, ll(1), None) == 1
    assert b"power of two from 2 to 16384" in lib.spx_last_error()
    assert lib.spx_rf_spectrum(3, p, None, q, ll(100), 32768, ll(1), None) == 1
    assert lib.spx_rf_fir(3, p, p, q, ll(100), 65, 64, ll(1), None) == 1
    assert b"at least len(taps) = 65" in lib.spx_last_error()
    assert lib.spx_rf_fir(0, p, p, q, ll(100), 3, 64, ll(1), None) == 1
    assert b"no fused radio kernels" in lib.spx_last_error()


# --- Spectrum ---------------------------------------------------------------------------------


@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
@pytest.mark.parametrize("window_name", ["rect", "hann", "blackman"])
@pytest.mark.parametrize("n", [1, 1000, 4096])
def test_spectrum_matches_numpy(rng, fft_impl, window_name, n):
    nfft = 256
    x = random_complex(rng, n)
    y = rf.spectrum(cuda(x), nfft, window_name=window_name, fft_impl=fft_impl)
    assert y.shape == (-(-n // nfft), nfft)
    assert relative_error(y.cpu().numpy(), framed_spectrum(x, nfft, window_name)) < 1e-5


@gpu
@pytest.mark.parametrize("fft_impl", OURS)
@pytest.mark.parametrize("nfft", [2, 4, 8, 16, 32, 64, 128, 512, 1024, 2048, 4096, 8192, 16384])
def test_single_kernel_spectrum_at_every_frame_size(rng, fft_impl, nfft):
    # Rows of a length that leaves the last frame partly filled.
    x = random_complex(rng, (3, 2 * nfft + nfft // 2 + 1))
    y = rf.spectrum(cuda(x), nfft, window_name="hamming", fft_impl=fft_impl)
    assert y.shape == (3, 3, nfft)
    tol = 1e-5 * max(1.0, np.log2(nfft) / 8)
    assert relative_error(y.cpu().numpy(), framed_spectrum(x, nfft, "hamming")) < tol


@gpu
@pytest.mark.parametrize("fft_impl", OURS)
def test_spectrum_of_many_frames_and_of_an_empty_signal(rng, fft_impl):
    x = random_complex(rng, (2, 300_001))
    y = rf.spectrum(cuda(x), 1024, window_name="hann", fft_impl=fft_impl)
    assert relative_error(y.cpu().numpy(), framed_spectrum(x, 1024, "hann")) < 1e-5
    empty = torch.zeros(2, 0, dtype=torch.complex64, device="cuda")
    z = rf.spectrum(empty, 64, fft_impl=fft_impl)
    assert z.shape == (2, 1, 64) and torch.count_nonzero(z) == 0


# --- FIR by overlap-save ----------------------------------------------------------------------

# (signal length, number of taps): one tap, a signal shorter than the filter, lengths that do not
# fill the last block, a filter longer than the default block's quarter, and long filters (4096
# taps take 16384-sample blocks).
FIR_CASES = [(1000, 1), (5, 63), (63, 63), (1000, 63), (4097, 64), (10_000, 1025), (3000, 4096)]


@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
@pytest.mark.parametrize(("n", "m"), FIR_CASES)
def test_fir_matches_lfilter(rng, fft_impl, n, m):
    x = random_complex(rng, n)
    taps = random_real(rng, m)
    expected = scipy.signal.lfilter(taps.astype(np.float64), 1.0, x.astype(np.complex128))
    y = rf.fir(cuda(x), cuda(taps), fft_impl=fft_impl)
    assert y.shape == (n,)
    assert relative_error(y.cpu().numpy(), expected) < 2e-5


@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
def test_fir_with_complex_taps_rows_and_a_chosen_block_size(rng, fft_impl):
    x = random_complex(rng, (3, 777))
    taps = random_complex(rng, 31)
    expected = scipy.signal.lfilter(taps.astype(np.complex128), 1.0, x.astype(np.complex128))
    y = rf.fir(cuda(x), cuda(taps), nfft=64, fft_impl=fft_impl)
    assert relative_error(y.cpu().numpy(), expected) < 2e-5


@gpu
@pytest.mark.parametrize("fft_impl", OURS)
@pytest.mark.parametrize("nfft", [2, 8, 32, 128, 1024, 8192])
def test_single_kernel_fir_at_every_block_size(rng, fft_impl, nfft):
    m = max(1, nfft // 3)
    x = random_complex(rng, (2, 5 * nfft + 7))
    taps = random_real(rng, m)
    expected = scipy.signal.lfilter(taps.astype(np.float64), 1.0, x.astype(np.complex128))
    y = rf.fir(cuda(x), cuda(taps), nfft=nfft, fft_impl=fft_impl)
    assert relative_error(y.cpu().numpy(), expected) < 2e-5


@gpu
@pytest.mark.parametrize("fft_impl", OURS)
def test_single_kernel_fir_matches_the_composed_path(rng, fft_impl):
    x = cuda(random_complex(rng, (4, 50_000)))
    taps = cuda(random_real(rng, 63))
    fused = rf.fir(x, taps, fft_impl=fft_impl)
    composed = rf.fir(x, taps, fft_impl="rocfft")
    assert relative_error(fused.cpu().numpy(), composed.cpu().numpy()) < 1e-5


@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
def test_fir_of_zeros_is_zeros(fft_impl):
    x = torch.zeros(500, dtype=torch.complex64, device="cuda")
    taps = torch.ones(17, device="cuda")
    assert torch.count_nonzero(rf.fir(x, taps, fft_impl=fft_impl)) == 0


@gpu
@pytest.mark.parametrize("fft_impl", OURS)
def test_fir_of_an_empty_signal_is_empty(fft_impl):
    x = torch.zeros(3, 0, dtype=torch.complex64, device="cuda")
    assert rf.fir(x, torch.ones(5, device="cuda"), fft_impl=fft_impl).shape == (3, 0)


@gpu
@pytest.mark.parametrize("fft_impl", OURS)
@pytest.mark.parametrize("nfft", [2, 4, 16, 64, 256, 4096, 16384])
@pytest.mark.parametrize("complex_taps", [False, True])
def test_filter_spectrum_is_the_fft_of_the_padded_taps(rng, fft_impl, nfft, complex_taps):
    # rf_fir_spectrum reads the taps as they are (float32 or complex64) and zero-pads them in its
    # load: the nfft-point FFT of the taps followed by zeros (rf.py:145-147 of the reference).
    from oracle.tolerance import fft_tolerance

    for m in sorted({1, nfft // 2 + 1, nfft}):
        taps = random_complex(rng, m) if complex_taps else random_real(rng, m)
        h = torch.ops.spectral.rf_fir_spectrum(cuda(taps), nfft, fft_impl)
        padded = np.zeros(nfft, dtype=np.complex128)
        padded[:m] = taps
        assert h.shape == (nfft,) and h.dtype == torch.complex64
        assert relative_error(h.cpu().numpy(), np.fft.fft(padded)) < fft_tolerance(nfft)


@gpu
@pytest.mark.parametrize("fft_impl", OURS)
def test_fir_converts_other_tap_types(rng, fft_impl):
    x = random_complex(rng, 3000)
    taps = random_real(rng, 63).astype(np.float64)
    expected = scipy.signal.lfilter(taps, 1.0, x.astype(np.complex128))
    for t in (cuda(taps), cuda(taps).to(torch.complex128), torch.from_numpy(taps)):
        y = rf.fir(cuda(x), t, fft_impl=fft_impl)
        assert relative_error(y.cpu().numpy(), expected) < 2e-5


@gpu
def test_filter_spectrum_rejects_bad_arguments():
    taps = torch.ones(65, device="cuda")
    with pytest.raises(ValueError, match="at least len\\(taps\\) = 65"):
        torch.ops.spectral.rf_fir_spectrum(taps, 64, "stockham_r8")
    with pytest.raises(ValueError, match="float32 or complex64"):
        torch.ops.spectral.rf_fir_spectrum(taps.double(), 64, "stockham_r8")
    with pytest.raises(ValueError, match="no fused radio kernels"):
        torch.ops.spectral.rf_fir_spectrum(taps, 128, "naive")


@gpu
def test_fir_rejects_a_block_shorter_than_the_filter():
    x = torch.zeros(100, dtype=torch.complex64, device="cuda")
    with pytest.raises(ValueError, match="at least len\\(taps\\) = 65"):
        rf.fir(x, torch.ones(65, device="cuda"), nfft=64)


@gpu
def test_operators_reject_bad_arguments():
    x = torch.zeros(100, dtype=torch.complex64, device="cuda")
    with pytest.raises(ValueError, match="no fused radio kernels"):
        torch.ops.spectral.rf_spectrum(x, None, 64, "naive")
    with pytest.raises(ValueError, match="power of two from 2"):
        torch.ops.spectral.rf_spectrum(x, None, 48, "stockham_r8")
    with pytest.raises(RuntimeError, match="window must be"):
        torch.ops.spectral.rf_spectrum(x, torch.ones(32, device="cuda"), 64, "stockham_r8")
    with pytest.raises(ValueError, match="nfft = 64 point spectrum"):
        torch.ops.spectral.rf_fir(x, x[:32], 5, 64, "stockham_r8")


# --- Recordings -------------------------------------------------------------------------------


@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
def test_chirp_spectrum_peak_follows_the_sweep(fft_impl):
    x, meta = load_fixture("chirp")
    nfft = 256
    spec = rf.spectrum(cuda(x), nfft, window_name="hann", fft_impl=fft_impl).abs().cpu().numpy()
    peaks = np.fft.fftfreq(nfft)[np.argmax(spec, axis=-1)] * meta["sample_rate"]
    centers = (np.arange(len(peaks)) + 0.5) * nfft
    expected = meta["f0_hz"] + (meta["f1_hz"] - meta["f0_hz"]) * centers / len(x)
    assert np.max(np.abs(peaks - expected)) <= 2 * meta["sample_rate"] / nfft


def decode(name: str, fft_impl: str) -> tuple[np.ndarray, dict]:
    """Matched filter on the GPU, then one sample per symbol."""
    x, meta = load_fixture(name)
    taps = rf.read_f32(FIXTURES / meta["pulse"])
    y = rf.fir(cuda(x), cuda(taps), fft_impl=fft_impl).cpu().numpy()
    first, sps = meta["first_symbol_after_matched_filter"], meta["samples_per_symbol"]
    return y[first::sps], meta


@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
def test_bpsk_bits_are_recovered(fft_impl):
    samples, meta = decode("bpsk", fft_impl)
    bits = np.array(meta["bits"])[: len(samples)]
    assert np.array_equal((samples.real > 0).astype(int), bits)


@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
def test_qpsk_symbols_are_recovered(fft_impl):
    samples, meta = decode("qpsk", fft_impl)
    symbols = np.array(meta["symbols"])[: len(samples)]
    decided = (samples.real < 0).astype(int) + 2 * (samples.imag < 0).astype(int)  # Gray map
    assert np.array_equal(decided, symbols)


# --- Command line -----------------------------------------------------------------------------


@gpu
def test_command_line_fir_matches_the_api(tmp_path):
    out = tmp_path / "y.cf32"
    args = ["fir", "--in", str(FIXTURES / "bpsk.cf32"), "--taps", str(FIXTURES / "rrc.f32")]
    assert rf.main([*args, "--out", str(out), "--fft-impl", "stockham_r8"]) == 0
    x, _ = load_fixture("bpsk")
    expected = rf.fir(cuda(x), cuda(rf.read_f32(FIXTURES / "rrc.f32")), fft_impl="stockham_r8")
    np.testing.assert_array_equal(rf.read_cf32(out), expected.cpu().numpy())


@gpu
def test_command_line_spectrum(tmp_path):
    out = tmp_path / "s.cf32"
    args = ["spectrum", "--in", str(FIXTURES / "chirp.cf32"), "--out", str(out)]
    assert rf.main([*args, "--nfft", "512", "--window", "hann", "--fft-impl", "stockham_r4"]) == 0
    assert rf.read_cf32(out).size == 16384
