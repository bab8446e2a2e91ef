"""Benchmark bookkeeping: GPU timing, the work conventions behind "effective GB/s", and the result
CSVs that `bin/spectral_bench` writes and regression checks compare.

Interfaces kept from the reference (python/spectral/benchmark.py:18-120, csrc/common/
bench.cpp:48-135, tools/bench_compare.py): the nine CSV columns and the row key
(op, impl, n, batch); the work formulas; `time_cuda`'s warm-up / rounds / iterations and its
median, minimum and maximum per call; `compare`'s result (report lines, regressed?) with its
rule that only rows slower than old * (1 + threshold) fail and unmatched rows never do.

Own to this stack:
* time_gpu records one event between consecutive rounds (rounds + 1 events on the stream) and
  waits once, at the end, so no host synchronization sits between two rounds.
* Result rows carry two more columns, the effective GB/s as a percentage of MI355X's datasheet
  HBM peak (8 TB/s) and of a measured copy ceiling, when one is given.
* `python -m spectral.benchmark compare OLD.csv NEW.csv [--threshold 0.10]` is the regression
  check: exit status 1 when a matched row got slower.
"""

from __future__ import annotations

import argparse
import csv
import io
import math
import statistics
import sys
from collections.abc import Callable, Iterable, Iterator, Sequence
from dataclasses import dataclass
from pathlib import Path

# The reference's result schema (csrc/tools/spectral_bench.cpp:185), then this stack's two.
CSV_COLUMNS = ["op", "impl", "n", "batch", "time_ms", "min_ms", "max_ms", "gflops", "gbps"]
PEAK_COLUMNS = ["pct_peak_datasheet", "pct_peak_measured"]
DATASHEET_PEAK_GBPS = 8000.0  # MI355X HBM3E
UNSTABLE_SPREAD = 0.05        # rounds differing by more than this mark a row unstable

Key = tuple[str, str, int, int]  # (op, impl, n, batch)
_KEY_COLUMNS = ("op", "impl", "n", "batch")


@dataclass(frozen=True)
class Timing:
    """Per-call times of one measurement, in ms."""

    median_ms: float
    min_ms: float
    max_ms: float

    @classmethod
    def of(cls, per_call_ms: Sequence[float]) -> "Timing":
        if not per_call_ms:
            raise ValueError("a timing needs at least one round")
        return cls(statistics.median(per_call_ms), min(per_call_ms), max(per_call_ms))

    @property
    def spread(self) -> float:
        """Slowest over fastest round, minus one."""
        return self.max_ms / self.min_ms - 1.0 if self.min_ms > 0 else math.inf

    @property
    def unstable(self) -> bool:
        return self.spread > UNSTABLE_SPREAD


@dataclass(frozen=True)
class Result:
    op: str
    impl: str
    n: int
    batch: int
    timing: Timing
    flops: float
    nbytes: float

    @property
    def key(self) -> Key:
        return (self.op, self.impl, self.n, self.batch)

    @property
    def gflops(self) -> float:
        return self.flops / (self.timing.median_ms * 1e6)

    @property
    def gbps(self) -> float:
        return self.nbytes / (self.timing.median_ms * 1e6)


def time_gpu(fn: Callable[[], object], *, warmup: int = 3, rounds: int = 5, iters: int = 20,
             stream=None) -> Timing:
    """Per-call time of `fn`, which queues GPU work on `stream` (default: PyTorch's current
    stream, where the spectral operators launch): `warmup` untimed calls, then `rounds` rounds of
    `iters` calls each, timed by the events between them."""
    if warmup < 0 or rounds < 1 or iters < 1:
        raise ValueError(f"need warmup >= 0, rounds >= 1, iters >= 1 "
                         f"(got warmup={warmup}, rounds={rounds}, iters={iters})")
    import torch

    stream = torch.cuda.current_stream() if stream is None else stream
    for _ in range(warmup):
        fn()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(rounds + 1)]
    marks[0].record(stream)
    for mark in marks[1:]:
        for _ in range(iters):
            fn()
        mark.record(stream)
    marks[-1].synchronize()
    return Timing.of([a.elapsed_time(b) / iters for a, b in zip(marks, marks[1:])])


# The reference's name for it.
time_cuda = time_gpu


# --- work conventions (reference csrc/common/bench.cpp:93-135) -------------------------------
# Flops are the nominal 5 N log2 N of a complex transform (2.5 N log2 N for a real one); bytes are
# what an out-of-place transform must read and write once: complex64 is 8 bytes, float32 4.

def fft_c2c_work(n: int, batch: int) -> tuple[float, float]:
    """(flops, bytes) of `batch` complex transforms of n points."""
    flops = 5.0 * n * math.log2(n) * batch
    return flops, 2 * 8.0 * n * batch


def fft_real_work(n: int, batch: int) -> tuple[float, float]:
    """(flops, bytes) of `batch` real transforms of n points, either direction."""
    flops = 2.5 * n * math.log2(n) * batch
    return flops, (4.0 * n + 8.0 * (n / 2 + 1)) * batch


def fft2_real_work(n1: int, n2: int, batch: int) -> tuple[float, float]:
    """(flops, bytes) of `batch` real 2D transforms of n1 x n2 (half spectrum n1 x (n2/2 + 1))."""
    flops, _ = fft_real_work(n1 * n2, batch)
    return flops, (4.0 * n1 * n2 + 8.0 * n1 * (n2 / 2 + 1)) * batch


def fft2_modes_work(n1: int, n2: int, m1: int, m2: int, batch: int) -> tuple[float, float]:
    """(flops, bytes) of `batch` pruned 2D transforms: the full transform's flops; the real
    array and the 2 m1 x m2 complex64 modes."""
    flops, _ = fft2_real_work(n1, n2, batch)
    return flops, (4.0 * n1 * n2 + 8.0 * (2 * m1) * m2) * batch


# --- result files ----------------------------------------------------------------------------

def format_csv(results: Iterable[Result], comments: Iterable[str], *,
               measured_peak_gbps: float | None = None) -> str:
    """Result rows as CSV: '#' comment lines, the header, then one row per result. The
    percentage of the measured ceiling is left empty when none is given."""
    out = io.StringIO()
    for comment in comments:
        out.write(f"# {comment}\n")
    writer = csv.writer(out, lineterminator="\n")
    writer.writerow(CSV_COLUMNS + PEAK_COLUMNS)
    for r in results:
        t = r.timing
        measured = (f"{100.0 * r.gbps / measured_peak_gbps:.1f}"
                    if measured_peak_gbps else "")
        writer.writerow([r.op, r.impl, r.n, r.batch, f"{t.median_ms:.6f}", f"{t.min_ms:.6f}",
                         f"{t.max_ms:.6f}", f"{r.gflops:.1f}", f"{r.gbps:.1f}",
                         f"{100.0 * r.gbps / DATASHEET_PEAK_GBPS:.1f}", measured])
    return out.getvalue()


def _records(path: Path) -> Iterator[dict[str, str]]:
    """The data rows of a results CSV as dicts, '#' and blank lines skipped."""
    with Path(path).open(newline="") as f:
        body = [line for line in f if line.strip() and not line.lstrip().startswith("#")]
    reader = csv.DictReader(body)
    missing = [c for c in (*_KEY_COLUMNS, "time_ms") if c not in (reader.fieldnames or [])]
    if missing:
        raise ValueError(f"{path}: no column {', '.join(missing)} in the header")
    yield from reader


def read_results(path: Path) -> dict[Key, float]:
    """Median ms per (op, impl, n, batch) of a results CSV (a later row of the same key wins)."""
    table: dict[Key, float] = {}
    for row in _records(path):
        table[(row["op"], row["impl"], int(row["n"]), int(row["batch"]))] = float(row["time_ms"])
    return table


@dataclass(frozen=True)
class Change:
    key: Key
    old_ms: float
    new_ms: float

    @property
    def ratio(self) -> float:
        return self.new_ms / self.old_ms

    def verdict(self, threshold: float) -> str:
        if self.ratio > 1.0 + threshold:
            return "SLOWER"
        if self.ratio < 1.0 - threshold:
            return "faster"
        return ""


def compare(old: dict[Key, float], new: dict[Key, float],
            threshold: float) -> tuple[list[str], bool]:
    """Report lines for the rows of `new` against `old`, and whether any row matched in both got
    slower than old * (1 + threshold). A row in one table only is reported and never fails."""
    changes = [Change(key, old[key], new[key]) for key in sorted(old.keys() & new.keys())]
    report = [f"op impl n batch: old ms -> new ms, new/old (threshold {threshold:.0%})"]
    for c in changes:
        op, impl, n, batch = c.key
        report.append(f"{op} {impl} n={n} batch={batch}: {c.old_ms:.4f} -> {c.new_ms:.4f} ms, "
                      f"x{c.ratio:.3f} {c.verdict(threshold)}".rstrip())
    report += [f"only in old: {key}" for key in sorted(old.keys() - new.keys())]
    report += [f"only in new: {key}" for key in sorted(new.keys() - old.keys())]
    return report, any(c.verdict(threshold) == "SLOWER" for c in changes)


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(prog="python -m spectral.benchmark",
                                     description="regression check of two result CSVs")
    sub = parser.add_subparsers(dest="command", required=True)
    cmp = sub.add_parser("compare", help="exit 1 when a row of NEW is slower than OLD allows")
    cmp.add_argument("old", type=Path)
    cmp.add_argument("new", type=Path)
    cmp.add_argument("--threshold", type=float, default=0.10,
                     help="allowed slowdown as a fraction (default 0.10)")
    args = parser.parse_args(argv)
    lines, regressed = compare(read_results(args.old), read_results(args.new), args.threshold)
    print("\n".join(lines))
    if regressed:
        print(f"regression: a row is more than {args.threshold:.0%} slower than the baseline")
    return 1 if regressed else 0


if __name__ == "__main__":
    sys.exit(main())
