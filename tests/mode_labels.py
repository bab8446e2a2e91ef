"""Labelled half spectra for the bit-exact mode-layout tests: distinct Gaussian integers at the
kept FNO-mode positions (tests/golden/modes_index.json) of the half spectrum of a real field, and
what a real inverse makes of columns 0 and n2/2. Shared by the GPU layout test (test_pruned.py)
and its CPU check (test_oracle.py)."""

import json
from pathlib import Path

import numpy as np

# Golden-fixture shapes with at least one column between DC and Nyquist; (16, 16, 8, 9) keeps the
# Nyquist column and every row (m1 = n1/2, so row n1/2 is kept and is its own partner).
LAYOUT_CASES = [(8, 8, 2, 3), (16, 16, 3, 4), (16, 16, 8, 9), (64, 32, 12, 12), (32, 128, 4, 20),
                (128, 128, 16, 16)]


def golden_positions(n1: int, n2: int, m1: int, m2: int) -> np.ndarray:
    data = json.loads((Path(__file__).parent / "golden" / "modes_index.json").read_text())
    case = next(c for c in data if (c["n1"], c["n2"], c["m1"], c["m2"]) == (n1, n2, m1, m2))
    return np.array(case["positions"])


def labelled_half_spectrum(n1: int, n2: int, m1: int, m2: int):
    """Distinct Gaussian integers at the kept positions of a half spectrum that is the spectrum of
    a real field: (full, kept). `full` is the half spectrum (2, n1, w); `kept` the mode block's
    labels (2, 2 m1 * m2), in the fixture's slot order. In columns 0 and n2/2 a real field ties
    row r to row -r (conjugates; rows 0 and n1/2 real), so labels there come in conjugate pairs,
    and a kept row whose partner is dropped (row n1 - m1) puts the conjugate into `full` only.
    Those labels are even, so the halves the inverse's Hermitian join makes are integers too."""
    w = n2 // 2 + 1
    pos = golden_positions(n1, n2, m1, m2)
    full = np.zeros((2, n1, w), np.complex128)
    counter = iter(range(1, 1 << 20))
    for a in range(2):
        for p in pos:
            r, c = divmod(int(p), w)
            if c in (0, n2 // 2):
                continue
            full[a, r, c] = next(counter) - 1j * next(counter)
        for c in sorted({0, n2 // 2} & set(range(m2))):
            rows = [int(p) // w for p in pos if int(p) % w == c]
            for r in rows:
                partner = (n1 - r) % n1
                if partner == r:
                    full[a, r, c] = 2 * next(counter)
                elif full[a, r, c] == 0:
                    full[a, r, c] = 2 * next(counter) - 2j * next(counter)
                    full[a, partner, c] = np.conj(full[a, r, c])
    kept = full.reshape(2, -1)[:, pos]
    return full, kept


def hermitian_join(half: np.ndarray, n2: int) -> np.ndarray:
    """What a real inverse keeps of columns 0 and n2/2: (X[r] + conj X[-r]) / 2."""
    out = half.copy()
    for c in {0, n2 // 2}:
        col = half[..., :, c]
        mirror = np.conj(np.roll(col[..., ::-1], 1, axis=-1))  # X[-r] at row r
        out[..., :, c] = (col + mirror) / 2
    return out


def rounded(z: np.ndarray) -> np.ndarray:
    return np.round(z.real) + 1j * np.round(z.imag)
