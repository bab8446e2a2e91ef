"""Writes tests/golden/modes_index.json: for a few (n1, n2, m1, m2) shapes, the position in the
full rfft2 half spectrum (flattened n1 x (n2//2 + 1)) of every kept FNO mode, row-major over the
(2 m1) x m2 mode block.

The positions come from the frequency semantics alone (by brute-force enumeration, not from any
formula under test): kept row r carries vertical frequency f = r for r < m1 and f = r - 2 m1
(negative) otherwise; a real 2D spectrum stores frequency f at row f mod n1; column c is
horizontal frequency c. The shapes include the reference's own pruned test cases
(tests/test_pruned.py:32, CASES_2D) and the FNO benchmark shape 128 x 128 with m1 = m2 = 16.

    python tests/golden/make_fixtures.py
"""

import json
from pathlib import Path

SHAPES = [(2, 2, 1, 1), (8, 8, 2, 3), (16, 16, 8, 9), (64, 32, 12, 12), (32, 128, 4, 20),
          (16, 16, 3, 4), (128, 128, 16, 16)]


def positions(n1: int, n2: int, m1: int, m2: int) -> list[int]:
    w = n2 // 2 + 1
    kept_freqs = list(range(0, m1)) + list(range(-m1, 0))  # the order an FNO stores them
    out = []
    for f in kept_freqs:
        row = f % n1
        for c in range(m2):
            out.append(row * w + c)
    return out


def main() -> None:
    data = [{"n1": n1, "n2": n2, "m1": m1, "m2": m2, "positions": positions(n1, n2, m1, m2)}
            for n1, n2, m1, m2 in SHAPES]
    path = Path(__file__).with_name("modes_index.json")
    path.write_text(json.dumps(data, separators=(",", ":")) + "\n")
    print(f"wrote {path} ({len(data)} shapes)")


if __name__ == "__main__":
    main()
