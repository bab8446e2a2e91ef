"""Parity with the float64 oracle over a fixed, seeded sample of random cases: every operator,
with sizes, batch counts, implementations and column methods drawn at random within the API's
limits. The hand-picked tests elsewhere pin each kernel's edges; this sample reaches the
combinations between them (odd batch counts against each plan's transforms per workgroup and
the persistent kernels' resident grid, flat and tall 2D shapes, pruned bounds), as a guard
against a case that none of them names. The radio callers and the Navier-Stokes many-step launch
(random grid, field count across several workgroups per compute unit, step count, shared or
per-field viscosity; against a stage per launch) get samples of their own. Every sample is drawn
once at collection from a fixed seed, so every run checks the same cases, each under its own
test id."""

import numpy as np
import pytest
import torch

import spectral
from spectral import rf
from oracle import reference as ref
from oracle.tolerance import (
    assert_transform_close,
    fft_tolerance,
    random_complex,
    random_real,
    to_numpy,
)

STOCKHAM = [impl for impl in spectral.FFT_IMPLS if impl.startswith("stockham")]
MAX_POINTS = 1 << 20  # values per case, so the float64 oracle stays quick
CASES_PER_OP = 100


def _pow2(draw, lo: int, hi: int) -> int:
    return 1 << int(draw.integers(lo, hi + 1))


def _batch(draw, points_per_item: int, cap: int) -> int:
    # Small counts half the time, else anything up to the size budget.
    top = max(1, min(cap, MAX_POINTS // points_per_item))
    return int(draw.integers(1, min(top, 8) + 1)) if draw.random() < 0.5 else \
        int(draw.integers(1, top + 1))


def _impl(draw, n_max: int) -> str:
    # naive is a direct DFT: keep it to small transforms.
    pool = STOCKHAM + (["naive"] if n_max <= 256 else [])
    return str(pool[int(draw.integers(len(pool)))])


def _columns(draw, impl: str) -> str:
    options = ["transpose", "auto"] + (["strided"] if impl != "naive" else [])
    return str(options[int(draw.integers(len(options)))])


def _draw_cases() -> list[tuple]:
    draw = np.random.default_rng(20261202)
    cases = []
    for _ in range(CASES_PER_OP):
        n = _pow2(draw, 1, 18)
        impl = _impl(draw, n) if n <= 4096 else str(STOCKHAM[int(draw.integers(len(STOCKHAM)))])
        cases.append(("c2c", impl, "", (n,), _batch(draw, n, 5000), bool(draw.integers(2))))
    for _ in range(CASES_PER_OP):
        n = _pow2(draw, 1, 13)
        cases.append(("real", _impl(draw, n), "", (n,), _batch(draw, n, 5000),
                      bool(draw.integers(2))))
    for _ in range(CASES_PER_OP):
        n = _pow2(draw, 1, 12)
        keep = int(draw.integers(1, n + 1))
        cases.append(("pruned1d", _impl(draw, n), "", (n, keep), _batch(draw, n, 3000),
                      bool(draw.integers(2))))
    for _ in range(CASES_PER_OP):
        while True:
            n1, n2 = _pow2(draw, 0, 12), _pow2(draw, 0, 12)
            if n1 * n2 <= 1 << 18:
                break
        impl = _impl(draw, max(n1, n2))
        cases.append(("fft2", impl, _columns(draw, impl), (n1, n2), _batch(draw, n1 * n2, 64),
                      bool(draw.integers(2))))
    for _ in range(CASES_PER_OP):
        while True:
            n1, n2 = _pow2(draw, 0, 12), _pow2(draw, 1, 13)
            if n1 * n2 <= 1 << 18:
                break
        impl = _impl(draw, max(n1, n2))
        cases.append(("real2", impl, _columns(draw, impl), (n1, n2), _batch(draw, n1 * n2, 64),
                      bool(draw.integers(2))))
    for _ in range(CASES_PER_OP):
        while True:
            n1, n2 = _pow2(draw, 1, 10), _pow2(draw, 1, 10)
            if n1 * n2 <= 1 << 18:
                break
        m1 = int(draw.integers(1, n1 // 2 + 1))
        m2 = int(draw.integers(1, n2 // 2 + 2))
        cases.append(("modes2d", _impl(draw, max(n1, n2)), "", (n1, n2, m1, m2),
                      _batch(draw, n1 * n2, 64), bool(draw.integers(2))))
    return cases


CASES = _draw_cases()


def _case_id(case) -> str:
    op, impl, columns, shape, batch, inverse = case
    dims = "x".join(str(s) for s in shape)
    method = f"-{columns}" if columns else ""
    return f"{op}-{impl}{method}-{dims}-b{batch}-{'inv' if inverse else 'fwd'}"


def dev(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(x).cuda()


def assert_kept_modes_close(actual, expected, full, n: int, axes: tuple[int, ...]) -> None:
    """A truncated forward transform against the oracle, its error measured against the norm of
    the whole transform: a few kept modes can cancel to almost nothing (a kept DC value of 0.007
    from inputs of norm 1.7), so their own norm would ask float32 arithmetic for more digits
    than the inputs carry. The tolerance is the whole transform's."""
    a = to_numpy(actual).astype(np.complex128)
    assert a.shape == expected.shape
    err = np.sqrt(np.sum(np.abs(a - expected) ** 2, axis=axes))
    norm = np.sqrt(np.sum(np.abs(full) ** 2, axis=axes))
    worst = float(np.max(err / np.maximum(norm, np.finfo(np.float64).tiny)))
    assert worst <= fft_tolerance(n), f"relative L2 error {worst:.3e} (n = {n})"


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[_case_id(c) for c in CASES])
def test_random_case_matches_the_oracle(rng, case):
    op, impl, columns, shape, batch, inverse = case
    if op == "c2c":
        (n,) = shape
        x = random_complex(rng, (batch, n))
        y = spectral.fft_c2c(dev(x), inverse=inverse, impl=impl)
        assert_transform_close(y, ref.ifft(x) if inverse else ref.fft(x), n)
    elif op == "real":
        (n,) = shape
        if inverse:
            half = ref.rfft(random_real(rng, (batch, n))).astype(np.complex64)
            y = spectral.irfft(dev(half), n, impl=impl)
            assert_transform_close(y, ref.irfft(half, n), n)
        else:
            x = random_real(rng, (batch, n))
            assert_transform_close(spectral.rfft(dev(x), impl=impl), ref.rfft(x), n)
    elif op == "pruned1d":
        n, keep = shape
        if inverse:
            modes = random_complex(rng, (batch, keep))
            y = spectral.ifft_from_modes(dev(modes), n, impl=impl)
            assert_transform_close(y, ref.ifft_from_modes(modes, n), n)
        else:
            x = random_complex(rng, (batch, n))
            y = spectral.fft_truncated(dev(x), keep, impl=impl)
            assert_kept_modes_close(y, ref.fft_truncate(x, keep), ref.fft(x), n, (-1,))
    elif op == "fft2":
        n1, n2 = shape
        x = random_complex(rng, (batch, n1, n2))
        y = spectral.fft2(dev(x), inverse=inverse, impl=impl, columns=columns)
        expected = ref.ifft2(x) if inverse else ref.fft2(x)
        assert_transform_close(y, expected, n1 * n2, axes=(-2, -1))
    elif op == "real2":
        n1, n2 = shape
        field = random_real(rng, (batch, n1, n2))
        if inverse:
            half = ref.rfft2(field).astype(np.complex64)
            y = spectral.irfft2(dev(half), n2, impl=impl, columns=columns)
            expected = ref.irfft2(half, (n1, n2))
        else:
            y = spectral.rfft2(dev(field), impl=impl, columns=columns)
            expected = ref.rfft2(field)
        assert_transform_close(y, expected, n1 * n2, axes=(-2, -1))
    else:
        n1, n2, m1, m2 = shape
        if inverse:
            modes = random_complex(rng, (batch, 2 * m1, m2))
            y = spectral.irfft2_from_modes(dev(modes), (n1, n2), impl=impl)
            expected = ref.irfft2_from_modes(modes, (n1, n2))
        else:
            field = random_real(rng, (batch, n1, n2))
            y = spectral.rfft2_truncated(dev(field), m1, m2, impl=impl)
            assert_kept_modes_close(y, ref.rfft2_truncate(field, m1, m2), ref.rfft2(field),
                                    n1 * n2, (-2, -1))
            return
        assert_transform_close(y, expected, n1 * n2, axes=(-2, -1))


# --- the radio callers: rf.spectrum and rf.fir --------------------------------------------

def _draw_radio_cases() -> list[tuple]:
    draw = np.random.default_rng(20261203)
    one_launch = [b for b in rf.FFT_BACKENDS if b.startswith("stockham")]
    cases = []
    for _ in range(CASES_PER_OP // 2):
        nfft = _pow2(draw, 1, 14)
        rows = int(draw.integers(1, 4))
        n = int(draw.integers(0, (1 << 18) // rows + 1))
        window = ["rect", "hann", "hamming", "blackman"][int(draw.integers(4))]
        cases.append(("spectrum", one_launch[int(draw.integers(len(one_launch)))], rows, n,
                      nfft, window))
    for _ in range(CASES_PER_OP // 2):
        taps = int(draw.integers(1, 5001))
        rows = int(draw.integers(1, 4))
        n = int(draw.integers(1, (1 << 16) // rows + 1))
        low = max(1, (taps - 1).bit_length())  # the smallest block that holds the filter
        nfft = None if draw.random() < 0.5 else _pow2(draw, low, max(low, 14))
        complex_taps = bool(draw.integers(2))
        cases.append(("fir", one_launch[int(draw.integers(len(one_launch)))], rows, n,
                      (taps, nfft, complex_taps), ""))
    return cases


RADIO_CASES = _draw_radio_cases()


def _radio_id(case) -> str:
    kind, impl, rows, n, shape, window = case
    if kind == "spectrum":
        return f"spectrum-{impl}-{rows}x{n}-nfft{shape}-{window}"
    taps, nfft, complex_taps = shape
    return (f"fir-{impl}-{rows}x{n}-taps{taps}{'c' if complex_taps else ''}"
            f"-nfft{nfft if nfft else 'default'}")


@pytest.mark.gpu
@pytest.mark.parametrize("case", RADIO_CASES, ids=[_radio_id(c) for c in RADIO_CASES])
def test_random_radio_case_matches_the_oracle(rng, case):
    from test_rf import filtered, framed_spectrum, rel_l2

    kind, impl, rows, n, shape, window = case
    x = random_complex(rng, (rows, n))
    if kind == "spectrum":
        nfft = shape
        y = rf.spectrum(dev(x), nfft, window_name=window, fft_impl=impl)
        assert rel_l2(y, framed_spectrum(x, nfft, window)) < 1e-5 * max(1.0, np.log2(nfft) / 8)
    else:
        taps_count, nfft, complex_taps = shape
        taps = (random_complex(rng, taps_count) if complex_taps
                else random_real(rng, taps_count))
        y = rf.fir(dev(x), dev(taps), nfft=nfft, fft_impl=impl)
        assert tuple(y.shape) == (rows, n)
        assert rel_l2(y, filtered(x, taps)) < 2e-5


# --- the Navier-Stokes caller: many steps per launch -------------------------------------------

def _draw_flow_cases() -> list[tuple]:
    draw = np.random.default_rng(20261204)
    cases = []
    for _ in range(12):
        n = [64, 128][int(draw.integers(2))]
        batch = int(draw.integers(1, 600))  # up to more than two workgroups per compute unit
        steps = int(draw.integers(0, 6))
        shared = bool(draw.integers(2))
        cases.append((n, batch, steps, shared))
    return cases


FLOW_CASES = _draw_flow_cases()


@pytest.mark.gpu
@pytest.mark.parametrize("case", FLOW_CASES,
                         ids=[f"ns{n}-b{b}-s{k}-{'shared' if sh else 'per-field'}"
                              for n, b, k, sh in FLOW_CASES])
def test_random_flow_case_matches_the_stages(rng, case):
    # Flow() defaults to drag 0.1, the value passed to the stage operators below.
    from spectral.flow import Flow
    from spectral.flow.gpu import GpuSolver

    n, batch, steps, shared = case
    viscosity = 2e-3 if shared else rng.uniform(1e-3, 5e-3, batch)
    solver = GpuSolver(n, Flow(viscosity=viscosity), 2.5e-3, pruned=True, fused=True)
    w = solver.to_spectral(dev(random_real(rng, (batch, n, n))))
    expected = w  # a stage per launch
    for _ in range(steps):
        f0, predicted = torch.ops.spectral.ns_predict(expected, solver.forcing_hat, solver.nu,
                                                      0.1, 2.5e-3, n)
        expected = torch.ops.spectral.ns_correct(predicted, expected, f0, solver.forcing_hat,
                                                 solver.nu, 0.1, 2.5e-3, n)
    got = solver.advance(w, steps)
    if steps == 0:
        assert torch.equal(got, w)
    else:
        err = torch.linalg.vector_norm(got - expected) / torch.linalg.vector_norm(expected)
        assert float(err) < 1e-5


def test_the_sample_covers_every_operator_and_implementation():
    ops = {c[0] for c in CASES}
    impls = {c[1] for c in CASES}
    assert ops == {"c2c", "real", "pruned1d", "fft2", "real2", "modes2d"}
    assert set(STOCKHAM) <= impls and "naive" in impls
    assert all(c[2] in ("strided", "transpose", "auto") for c in CASES if c[0] in ("fft2", "real2"))
    assert {c[0] for c in RADIO_CASES} == {"spectrum", "fir"}
    assert {c[0] for c in FLOW_CASES} == {64, 128} and max(c[1] for c in FLOW_CASES) > 512
    assert {c[2] for c in FLOW_CASES} >= {0, 1} and {c[3] for c in FLOW_CASES} == {True, False}
