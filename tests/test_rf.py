"""The radio callers, spectral.rf (reference tests/test_rf.py covers the same ground): periodic
windows, the spectrum of back-to-back frames, FIR filtering by overlap-save, the command line,
and the chirp / BPSK / QPSK recordings the reference ships (kept as data in tests/golden/rf).
Every GPU check runs with the torch.fft backend and with each of this stack's implementations:
the Stockham ones take the one-launch kernels (torch.ops.spectral.rf_spectrum / rf_fir), "naive"
the composed path. Expected values are float64 restatements on the CPU: windows from their cosine
sums, spectra from numpy.fft of explicit frames, filters from the convolution sum."""

import ctypes
import json
from pathlib import Path

import numpy as np
import pytest
import scipy.signal
import torch

from oracle.tolerance import fft_tolerance, random_complex, random_real
from spectral import rf

GOLDEN_RF = Path(__file__).resolve().parent / "golden" / "rf"
LIBRARY = (Path(__file__).resolve().parents[1] / "gpu-spectral-stack_amd" / "python"
           / "spectral" / "libspectral_hip.so")
BACKENDS = rf.FFT_BACKENDS
ONE_LAUNCH = [b for b in BACKENDS if b.startswith("stockham")]

gpu = pytest.mark.gpu


def on_gpu(x) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def rel_l2(actual, expected) -> float:
    a = np.asarray(actual.cpu() if hasattr(actual, "cpu") else actual, np.complex128)
    e = np.asarray(expected, np.complex128)
    assert a.shape == e.shape, (a.shape, e.shape)
    return float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-300))


def recording(name: str) -> tuple[np.ndarray, dict]:
    meta = json.loads((GOLDEN_RF / f"{name}.json").read_text())
    return rf.read_cf32(GOLDEN_RF / f"{name}.cf32"), meta


COSINE_SUMS = {"rect": [1.0], "hann": [0.5, -0.5], "hamming": [0.54, -0.46],
               "blackman": [0.42, -0.5, 0.08]}


def periodic_window(name: str, n: int) -> np.ndarray:
    """sum_j a_j cos(2 pi j k / n) over k = 0 .. n-1, float64; [1] for one point."""
    if n == 1:
        return np.ones(1)
    k = np.arange(n)
    return sum(a * np.cos(2 * np.pi * j * k / n) for j, a in enumerate(COSINE_SUMS[name]))


def framed_spectrum(x: np.ndarray, nfft: int, window_name: str) -> np.ndarray:
    """numpy.fft of every nfft-sample frame of each row (the last completed with zeros) times
    the window, in float64."""
    n = x.shape[-1]
    count = max(1, -(-n // nfft))
    frames = np.zeros((*x.shape[:-1], count, nfft), np.complex128)
    for f in range(count):
        part = x[..., f * nfft:(f + 1) * nfft]
        frames[..., f, :part.shape[-1]] = part
    return np.fft.fft(frames * periodic_window(window_name, nfft), axis=-1)


def filtered(x: np.ndarray, taps: np.ndarray) -> np.ndarray:
    """y[n] = sum_k taps[k] x[n - k] with zero initial state, row by row, float64."""
    rows = np.atleast_2d(x).astype(np.complex128)
    out = np.stack([np.convolve(row, taps.astype(np.complex128))[:rows.shape[-1]]
                    for row in rows])
    return out.reshape(x.shape)


# --- windows, block sizes, backends (CPU) ----------------------------------------------------

@pytest.mark.parametrize("name", ["hann", "hamming", "blackman"])
@pytest.mark.parametrize("n", [1, 2, 7, 64, 1024])
def test_window_is_its_periodic_cosine_sum(name, n):
    w = rf.window(name, n).numpy()
    assert w.dtype == np.float32 and w.shape == (n,)
    assert np.max(np.abs(w - periodic_window(name, n))) <= 1e-7
    # scipy's periodic (fftbins) window agrees: the convention is the reference's.
    assert np.max(np.abs(w - scipy.signal.get_window(name, n, fftbins=True))) <= 1e-7


def test_rect_window_and_one_point_windows_are_ones():
    assert torch.equal(rf.window("rect", 5), torch.ones(5))
    for name in rf.WINDOWS:
        assert torch.equal(rf.window(name, 1), torch.ones(1)), name


@pytest.mark.parametrize(("call", "message"), [
    (lambda: rf.window("kaiser", 8), "unknown window"),
    (lambda: rf.window("hann", 0), "at least one point"),
    (lambda: rf.default_nfft(0), "at least one tap"),
    (lambda: rf.fft(torch.zeros(4, dtype=torch.complex64), fft_impl="fftw"), "unknown fft_impl"),
], ids=["window-name", "window-length", "no-taps", "backend"])
def test_bad_radio_requests_are_refused(call, message):
    with pytest.raises(ValueError, match=message):
        call()


@pytest.mark.parametrize("taps", [1, 2, 15, 16, 17, 63, 64, 500, 1024, 1025, 3000, 4096, 5000,
                                  9000])
def test_fir_block_size_is_a_power_of_two_about_four_times_the_filter(taps):
    nfft = rf.default_nfft(taps)
    assert nfft & (nfft - 1) == 0 and nfft >= max(64, taps)
    if 4 * taps <= 4096:
        assert 4 * taps <= nfft < max(128, 8 * taps)  # the nearest power of two above 4 taps
    else:
        assert nfft == max(4096, 1 << (taps - 1).bit_length())  # capped, unless taps need more


def test_reference_block_sizes():
    assert [rf.default_nfft(m) for m in (1, 63, 1025, 5000)] == [64, 256, 4096, 8192]


def test_backends_are_torch_fft_then_every_implementation():
    import spectral

    assert BACKENDS[:2] == ("rocfft", "cufft")
    assert list(BACKENDS[2:]) == list(spectral.FFT_IMPLS)


# --- the recordings (CPU) --------------------------------------------------------------------

def test_recordings_are_small_and_described():
    names = sorted(p.stem for p in GOLDEN_RF.glob("*.cf32"))
    assert names == ["bpsk", "chirp", "qpsk"]
    for name in names:
        samples, meta = recording(name)
        assert (GOLDEN_RF / f"{name}.cf32").stat().st_size < 1 << 20
        assert len(samples) == meta["num_samples"]
        assert {"sample_rate", "generator", "seed"} <= set(meta)


def test_chirp_sweeps_linearly_from_f0_to_f1():
    samples, meta = recording("chirp")
    fs = meta["sample_rate"]
    hz = np.angle(samples[1:] / samples[:-1]) * fs / (2 * np.pi)  # phase step per sample
    t = np.arange(len(samples) - 1) / len(samples)
    assert np.max(np.abs(hz - (meta["f0_hz"] + (meta["f1_hz"] - meta["f0_hz"]) * t))) < 0.002 * fs


def matched_filter_decisions(name: str, y: np.ndarray):
    """The symbol decisions of a matched-filter output and the ones the recording carries."""
    _, meta = recording(name)
    picked = y[meta["first_symbol_after_matched_filter"]::meta["samples_per_symbol"]]
    if name == "bpsk":
        return (picked.real > 0).astype(int), np.array(meta["bits"])[:len(picked)]
    gray = (picked.real < 0).astype(int) + 2 * (picked.imag < 0).astype(int)
    return gray, np.array(meta["symbols"])[:len(picked)]


@pytest.mark.parametrize("name", ["bpsk", "qpsk"])
def test_recordings_decode_through_a_float64_matched_filter(name):
    samples, meta = recording(name)
    taps = rf.read_f32(GOLDEN_RF / meta["pulse"])
    decided, sent = matched_filter_decisions(name, filtered(samples, taps))
    assert len(decided) > 100 and np.array_equal(decided, sent)


def test_c_abi_checks_radio_arguments_on_the_host():
    import spectral  # noqa: F401  # maps the library the way the package does

    lib = ctypes.CDLL(str(LIBRARY))
    lib.spx_last_error.restype = ctypes.c_char_p
    n64, one = ctypes.c_longlong(100), ctypes.c_longlong(1)
    src, dst = ctypes.c_void_p(0x1000), ctypes.c_void_p(0x100000)
    assert lib.spx_rf_max_nfft(0) == 0  # naive: the composed path only
    assert lib.spx_rf_max_nfft(3) == 16384
    for nfft in (3, 32768):
        assert lib.spx_rf_spectrum(3, src, None, dst, n64, nfft, one, None) == 1
        assert b"power of two from 2 to 16384" in lib.spx_last_error()
    assert lib.spx_rf_fir(3, src, src, dst, n64, 65, 64, one, None) == 1
    assert b"at least len(taps) = 65" in lib.spx_last_error()
    assert lib.spx_rf_fir(0, src, src, dst, n64, 3, 64, one, None) == 1
    assert b"no fused radio kernels" in lib.spx_last_error()


# --- spectrum (GPU) --------------------------------------------------------------------------

@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
@pytest.mark.parametrize("window_name", ["rect", "hann", "blackman"])
@pytest.mark.parametrize("n", [1, 1000, 4096])
def test_spectrum_parity(rng, n, window_name, fft_impl):
    x = random_complex(rng, n)
    y = rf.spectrum(on_gpu(x), 256, window_name=window_name, fft_impl=fft_impl)
    assert rel_l2(y, framed_spectrum(x, 256, window_name)) < 1e-5


@gpu
@pytest.mark.parametrize("fft_impl", ONE_LAUNCH)
@pytest.mark.parametrize("nfft", [2, 4, 8, 16, 32, 64, 128, 512, 1024, 2048, 4096, 8192, 16384])
def test_one_launch_spectrum_at_every_frame_size(rng, fft_impl, nfft):
    # Rows whose length leaves the last frame partly filled.
    x = random_complex(rng, (3, 2 * nfft + nfft // 2 + 1))
    y = rf.spectrum(on_gpu(x), nfft, window_name="hamming", fft_impl=fft_impl)
    assert tuple(y.shape) == (3, 3, nfft)
    assert rel_l2(y, framed_spectrum(x, nfft, "hamming")) < 1e-5 * max(1.0, np.log2(nfft) / 8)


@gpu
@pytest.mark.parametrize("fft_impl", ONE_LAUNCH)
def test_spectrum_of_many_frames_and_of_no_samples(rng, fft_impl):
    x = random_complex(rng, (2, 300_001))
    y = rf.spectrum(on_gpu(x), 1024, window_name="hann", fft_impl=fft_impl)
    assert rel_l2(y, framed_spectrum(x, 1024, "hann")) < 1e-5
    nothing = rf.spectrum(torch.zeros(2, 0, dtype=torch.complex64, device="cuda"), 64,
                          fft_impl=fft_impl)
    assert tuple(nothing.shape) == (2, 1, 64) and not bool(nothing.abs().max() > 0)


# --- FIR by overlap-save (GPU) ---------------------------------------------------------------

# (signal length, taps): one tap, a signal shorter than the filter, lengths that do not fill the
# last block, a filter past a quarter of the default block, and long filters (4096 taps take
# 16384-sample blocks).
FIR_CASES = [(1000, 1), (5, 63), (63, 63), (1000, 63), (4097, 64), (10_000, 1025), (3000, 4096)]


@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
@pytest.mark.parametrize(("n", "m"), FIR_CASES)
def test_fir_parity(rng, n, m, fft_impl):
    x, taps = random_complex(rng, n), random_real(rng, m)
    y = rf.fir(on_gpu(x), on_gpu(taps), fft_impl=fft_impl)
    assert tuple(y.shape) == (n,)
    assert rel_l2(y, filtered(x, taps)) < 2e-5


@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
def test_fir_of_rows_with_complex_taps_and_a_given_block(rng, fft_impl):
    x, taps = random_complex(rng, (3, 777)), random_complex(rng, 31)
    y = rf.fir(on_gpu(x), on_gpu(taps), nfft=64, fft_impl=fft_impl)
    assert rel_l2(y, filtered(x, taps)) < 2e-5
    # scipy's direct-form filter, the reference's oracle, agrees with the convolution sum.
    assert rel_l2(filtered(x, taps), scipy.signal.lfilter(taps, 1.0, x.astype(np.complex128))) \
        < 1e-12


@gpu
@pytest.mark.parametrize("fft_impl", ONE_LAUNCH)
@pytest.mark.parametrize("nfft", [2, 8, 32, 128, 1024, 8192])
def test_one_launch_fir_at_every_block_size(rng, fft_impl, nfft):
    x, taps = random_complex(rng, (2, 5 * nfft + 7)), random_real(rng, max(1, nfft // 3))
    y = rf.fir(on_gpu(x), on_gpu(taps), nfft=nfft, fft_impl=fft_impl)
    assert rel_l2(y, filtered(x, taps)) < 2e-5


@gpu
@pytest.mark.parametrize("fft_impl", ONE_LAUNCH)
def test_one_launch_fir_agrees_with_the_composed_path(rng, fft_impl):
    x, taps = on_gpu(random_complex(rng, (4, 50_000))), on_gpu(random_real(rng, 63))
    ours, composed = rf.fir(x, taps, fft_impl=fft_impl), rf.fir(x, taps, fft_impl="rocfft")
    assert rel_l2(ours, composed.cpu().numpy()) < 1e-5


@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
def test_fir_of_silence_is_silence(fft_impl):
    y = rf.fir(torch.zeros(500, dtype=torch.complex64, device="cuda"),
               torch.ones(17, device="cuda"), fft_impl=fft_impl)
    assert not bool(y.abs().max() > 0)


@gpu
@pytest.mark.parametrize("fft_impl", ONE_LAUNCH)
def test_fir_of_no_samples_is_empty(fft_impl):
    y = rf.fir(torch.zeros(3, 0, dtype=torch.complex64, device="cuda"),
               torch.ones(5, device="cuda"), fft_impl=fft_impl)
    assert tuple(y.shape) == (3, 0)


@gpu
@pytest.mark.parametrize("fft_impl", ONE_LAUNCH)
@pytest.mark.parametrize("nfft", [2, 4, 16, 64, 256, 4096, 16384])
@pytest.mark.parametrize("complex_taps", [False, True])
def test_filter_spectrum_is_the_fft_of_the_zero_padded_taps(rng, fft_impl, nfft, complex_taps):
    # rf_fir_spectrum reads float32 or complex64 taps as they are and pads them with zeros in
    # its load (the reference pads first, rf.py:145-147).
    for m in sorted({1, nfft // 2 + 1, nfft}):
        taps = random_complex(rng, m) if complex_taps else random_real(rng, m)
        h = torch.ops.spectral.rf_fir_spectrum(on_gpu(taps), nfft, fft_impl)
        assert tuple(h.shape) == (nfft,) and h.dtype == torch.complex64
        assert rel_l2(h, np.fft.fft(taps.astype(np.complex128), n=nfft)) < fft_tolerance(nfft)


@gpu
@pytest.mark.parametrize("fft_impl", ONE_LAUNCH)
def test_fir_takes_taps_of_other_types_and_devices(rng, fft_impl):
    x = random_complex(rng, 3000)
    taps = random_real(rng, 63).astype(np.float64)
    expected = filtered(x, taps)
    for t in (on_gpu(taps), on_gpu(taps).to(torch.complex128), torch.from_numpy(taps)):
        assert rel_l2(rf.fir(on_gpu(x), t, fft_impl=fft_impl), expected) < 2e-5


@gpu
@pytest.mark.parametrize(("call", "error", "message"), [
    (lambda: torch.ops.spectral.rf_fir_spectrum(torch.ones(65, device="cuda"), 64,
                                                "stockham_r8"), ValueError,
     r"at least len\(taps\) = 65"),
    (lambda: torch.ops.spectral.rf_fir_spectrum(torch.ones(65, device="cuda").double(), 128,
                                                "stockham_r8"), ValueError, "float32 or complex64"),
    (lambda: torch.ops.spectral.rf_fir_spectrum(torch.ones(65, device="cuda"), 128, "naive"),
     ValueError, "no fused radio kernels"),
    (lambda: rf.fir(torch.zeros(100, dtype=torch.complex64, device="cuda"),
                    torch.ones(65, device="cuda"), nfft=64), ValueError,
     r"at least len\(taps\) = 65"),
    (lambda: torch.ops.spectral.rf_spectrum(torch.zeros(100, dtype=torch.complex64,
                                                        device="cuda"), None, 64, "naive"),
     ValueError, "no fused radio kernels"),
    (lambda: torch.ops.spectral.rf_spectrum(torch.zeros(100, dtype=torch.complex64,
                                                        device="cuda"), None, 48, "stockham_r8"),
     ValueError, "power of two from 2"),
    (lambda: torch.ops.spectral.rf_spectrum(torch.zeros(100, dtype=torch.complex64,
                                                        device="cuda"),
                                            torch.ones(32, device="cuda"), 64, "stockham_r8"),
     RuntimeError, "window must be"),
    (lambda: torch.ops.spectral.rf_fir(torch.zeros(100, dtype=torch.complex64, device="cuda"),
                                       torch.zeros(32, dtype=torch.complex64, device="cuda"),
                                       5, 64, "stockham_r8"),
     ValueError, "nfft = 64 point spectrum"),
], ids=["taps-past-block", "tap-type", "naive-spectrum-of-taps", "fir-block", "naive-spectrum",
        "frame-size", "window-length", "filter-spectrum-length"])
def test_bad_radio_operator_calls_are_refused(call, error, message):
    with pytest.raises(error, match=message):
        call()


# --- the recordings through the GPU paths ----------------------------------------------------

@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
def test_chirp_spectrum_peaks_follow_the_sweep(fft_impl):
    samples, meta = recording("chirp")
    nfft, fs = 256, meta["sample_rate"]
    power = rf.spectrum(on_gpu(samples), nfft, window_name="hann", fft_impl=fft_impl).abs()
    peak_hz = np.fft.fftfreq(nfft, d=1 / fs)[power.argmax(dim=-1).cpu().numpy()]
    middle = (np.arange(peak_hz.size) * nfft + nfft / 2) / len(samples)  # frame centres, 0..1
    swept = meta["f0_hz"] + (meta["f1_hz"] - meta["f0_hz"]) * middle
    assert np.max(np.abs(peak_hz - swept)) <= 2 * fs / nfft  # within two bins


@gpu
@pytest.mark.parametrize("fft_impl", BACKENDS)
@pytest.mark.parametrize("name", ["bpsk", "qpsk"])
def test_recordings_decode_through_the_gpu_filter(name, fft_impl):
    samples, meta = recording(name)
    taps = rf.read_f32(GOLDEN_RF / meta["pulse"])
    y = rf.fir(on_gpu(samples), on_gpu(taps), fft_impl=fft_impl).cpu().numpy()
    decided, sent = matched_filter_decisions(name, y)
    assert np.array_equal(decided, sent)


# --- the command line ------------------------------------------------------------------------

@gpu
def test_command_line_fir_writes_what_the_api_returns(tmp_path):
    out = tmp_path / "filtered.cf32"
    status = rf.main(["fir", "--in", str(GOLDEN_RF / "bpsk.cf32"), "--taps",
                      str(GOLDEN_RF / "rrc.f32"), "--out", str(out), "--fft-impl", "stockham_r8"])
    assert status == 0
    samples, _ = recording("bpsk")
    direct = rf.fir(on_gpu(samples), on_gpu(rf.read_f32(GOLDEN_RF / "rrc.f32")),
                    fft_impl="stockham_r8")
    assert np.array_equal(rf.read_cf32(out), direct.cpu().numpy())


@gpu
def test_command_line_spectrum_writes_every_frame(tmp_path):
    out = tmp_path / "frames.cf32"
    status = rf.main(["spectrum", "--in", str(GOLDEN_RF / "chirp.cf32"), "--out", str(out),
                      "--nfft", "512", "--window", "hann", "--fft-impl", "stockham_r4"])
    assert status == 0
    samples, _ = recording("chirp")
    written = rf.read_cf32(out).reshape(-1, 512)
    assert written.shape[0] == -(-len(samples) // 512)
    assert rel_l2(written, framed_spectrum(samples, 512, "hann")) < 1e-5
