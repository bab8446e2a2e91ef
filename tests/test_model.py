"""The NumPy model of the kernels' schedule (oracle/model.py) against the mathematics: the
Stockham index maps of every plan the kernels compile, the conjugate-pair real combine and
prepare, and the pruned index maps. A wrong index, twiddle or sign here is an O(1) error."""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import model
from oracle import reference as ref
from oracle.tolerance import random_complex, random_real

SIZES = [2**p for p in range(1, 13)]
RADICES = [2, 4, 8, 16]


@pytest.mark.parametrize("radix", RADICES)
@pytest.mark.parametrize("n", SIZES)
def test_stockham_schedule_is_the_dft(rng, n, radix):
    x = random_complex(rng, (2, n)).astype(np.complex128)
    np.testing.assert_allclose(model.stockham(x, radix), ref.fft(x), rtol=0, atol=1e-9 * n)
    np.testing.assert_allclose(model.stockham(x, radix, inverse=True) / n, ref.ifft(x), rtol=0,
                               atol=1e-9)


@pytest.mark.parametrize("e", [2, 4, 8, 16, 32])
def test_lane_split_does_not_change_the_result(rng, e):
    n = 64
    x = random_complex(rng, (1, n)).astype(np.complex128)
    for radix in [2, 4, 8]:
        if radix <= e:
            np.testing.assert_allclose(model.stockham(x, radix, e=e), ref.dft(x), atol=1e-10)


@pytest.mark.parametrize("radix", RADICES)
@pytest.mark.parametrize("n", SIZES)
def test_plan_shapes(n, radix):
    p = model.plan(n, radix)
    assert int(np.prod(p["radices"])) == n
    assert p["lanes"] * p["e"] == n and p["lanes"] * p["transforms"] == model.BLOCK
    # every stage's butterflies are split evenly over the lanes
    for rad in p["radices"]:
        assert (n // rad) % p["lanes"] == 0


@pytest.mark.parametrize("n", SIZES)
def test_direct_store_indices_cover_the_transform(n):
    p = model.plan(n, 8)
    rl = p["radices"][-1]
    seen = sorted(model.direct_output_index(n, 8, lane, b, r)
                  for lane in range(p["lanes"]) for b in range(p["e"] // rl) for r in range(rl))
    assert seen == list(range(n))


@pytest.mark.parametrize("n", SIZES)
def test_lds_padding_is_injective_and_fits(n):
    pos = model.pad(np.arange(n + 1))
    assert len(set(pos.tolist())) == n + 1
    assert pos.max() < model.stride(n)
    assert model.stride(n) % 2 == 1


@pytest.mark.parametrize("n", [2, 4, 8, 16, 64, 1024, 8192])
def test_real_forward_by_pairs(rng, n):
    m = n // 2
    x = random_real(rng, (3, n)).astype(np.float64)
    z = x[..., 0::2] + 1j * x[..., 1::2]
    np.testing.assert_allclose(model.r2c_from_half(np.fft.fft(z, axis=-1)), ref.rfft(x),
                               rtol=0, atol=1e-9 * n)
    keep = max(1, m // 3)
    np.testing.assert_allclose(model.r2c_from_half(np.fft.fft(z, axis=-1), keep),
                               ref.rfft(x)[..., :keep], rtol=0, atol=1e-9 * n)


@pytest.mark.parametrize("n", [2, 4, 8, 16, 64, 1024, 8192])
def test_real_inverse_by_pairs(rng, n):
    m = n // 2
    spec = random_complex(rng, (3, m + 1)).astype(np.complex128)  # not Hermitian on purpose
    z = model.c2r_to_half(spec, m)
    y = np.fft.ifft(z, axis=-1)  # includes the 1/m
    back = np.empty(spec.shape[:-1] + (n,))
    back[..., 0::2] = y.real
    back[..., 1::2] = y.imag
    np.testing.assert_allclose(back, ref.irfft(spec, n), rtol=0, atol=1e-12)
    keep = max(1, m // 4)
    z = model.c2r_to_half(spec[..., :keep], m)
    y = np.fft.ifft(z, axis=-1)
    back[..., 0::2] = y.real
    back[..., 1::2] = y.imag
    trunc = np.zeros_like(spec)
    trunc[..., :keep] = spec[..., :keep]
    np.testing.assert_allclose(back, ref.irfft(trunc, n), rtol=0, atol=1e-12)


@pytest.mark.parametrize(("n", "m1"), [(8, 0), (8, 2), (8, 4), (128, 16), (128, 43)])
def test_strided_row_map_by_frequency(n, m1):
    for i in range(n):
        row = model.strided_row(i, n, m1)
        if m1 == 0:
            assert row == i
            continue
        signed = i if i < n // 2 else i - n  # frequency i as a signed frequency
        kept = -m1 <= signed < m1
        assert (row >= 0) == kept
        if kept:
            assert row == (signed if signed >= 0 else signed + 2 * m1)


def test_full_index_matches_the_golden_fixture():
    data = json.loads((Path(__file__).parent / "golden" / "modes_index.json").read_text())
    assert len(data) >= 5
    for case in data:
        n1, n2, m1, m2 = case["n1"], case["n2"], case["m1"], case["m2"]
        w = n2 // 2 + 1
        got = [model.full_index(e, n1, w, m1, m2) for e in range(2 * m1 * m2)]
        assert got == case["positions"], case
        # two arrays: the second array's modes sit one full array further on
        got2 = [model.full_index(e, n1, w, m1, m2) for e in range(2 * m1 * m2, 4 * m1 * m2)]
        assert got2 == [p + n1 * w for p in case["positions"]]


def test_golden_fixture_agrees_with_the_reference_layout(rng):
    data = json.loads((Path(__file__).parent / "golden" / "modes_index.json").read_text())
    for case in data[:5]:
        n1, n2, m1, m2 = case["n1"], case["n2"], case["m1"], case["m2"]
        x = random_real(rng, (n1, n2))
        full = ref.rfft2(x).reshape(-1)
        modes = ref.rfft2_truncate(x, m1, m2).reshape(-1)
        np.testing.assert_array_equal(modes, full[case["positions"]])
