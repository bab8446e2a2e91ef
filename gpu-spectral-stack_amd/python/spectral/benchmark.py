"""Timing GPU work from Python, the work conventions behind "effective GB/s", and reading and
comparing result CSVs (reference python/spectral/benchmark.py:1-120, csrc/common/bench.cpp:48-135).

time_gpu() records HIP events on the stream the work is queued on (PyTorch's current stream,
which the spectral operators launch on): warm-up calls, then `rounds` measurements of `iters`
back-to-back calls, reporting the median, minimum and maximum time per call.
"""

from __future__ import annotations

import csv
import math
import statistics
from collections.abc import Callable, Iterable
from dataclasses import dataclass
from pathlib import Path

CSV_COLUMNS = ["op", "impl", "n", "batch", "time_ms", "min_ms", "max_ms", "gflops", "gbps"]

Key = tuple[str, str, int, int]  # (op, impl, n, batch)


@dataclass(frozen=True)
class Timing:
    median_ms: float  # all three per call
    min_ms: float
    max_ms: float

    @property
    def spread(self) -> float:
        """max / min - 1: above 0.05 the reference's harness flags a row as unstable."""
        return self.max_ms / self.min_ms - 1.0 if self.min_ms > 0 else math.inf


@dataclass(frozen=True)
class Result:
    op: str
    impl: str
    n: int
    batch: int
    timing: Timing
    flops: float
    nbytes: float


def time_gpu(fn: Callable[[], object], *, warmup: int = 3, rounds: int = 5, iters: int = 20,
             stream=None) -> Timing:
    """Median, min and max time per call of `fn`, which must queue GPU work on `stream`
    (default: PyTorch's current stream)."""
    if warmup < 0 or rounds < 1 or iters < 1:
        raise ValueError("need warmup >= 0, rounds >= 1, iters >= 1")
    import torch

    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream() if stream is None else stream
    per_call = []
    for _ in range(rounds):
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(iters):
            fn()
        stop.record(stream)
        stop.synchronize()
        per_call.append(start.elapsed_time(stop) / iters)
    return Timing(statistics.median(per_call), min(per_call), max(per_call))


# The reference's name for the same helper.
time_cuda = time_gpu


def fft_c2c_work(n: int, batch: int) -> tuple[float, float]:
    """(flops, bytes): 5 n log2 n flops per transform, one complex64 read and one written per
    point (16 bytes)."""
    points = n * batch
    return 5.0 * points * math.log2(n), 16.0 * points


def fft_real_work(n: int, batch: int) -> tuple[float, float]:
    """(flops, bytes) of real transforms, either direction: 2.5 n log2 n flops, n float32 values
    plus n/2 + 1 complex64 values per transform."""
    return 2.5 * n * batch * math.log2(n), batch * (4.0 * n + 8.0 * (n / 2 + 1))


def fft2_real_work(n1: int, n2: int, batch: int) -> tuple[float, float]:
    """(flops, bytes) of 2D real transforms: n1 n2 float32 values and n1 (n2/2 + 1) complex64."""
    points = n1 * n2
    return 2.5 * points * batch * math.log2(points), batch * (4.0 * points + 8.0 * n1 * (n2 / 2 + 1))


def fft2_modes_work(n1: int, n2: int, m1: int, m2: int, batch: int) -> tuple[float, float]:
    """(flops, bytes) of a pruned 2D transform: the full-transform flop count, and the real array
    plus the 2 m1 x m2 complex64 modes moved."""
    flops, _ = fft2_real_work(n1, n2, batch)
    return flops, batch * (4.0 * n1 * n2 + 16.0 * m1 * m2)


def format_csv(results: Iterable[Result], comments: Iterable[str]) -> str:
    lines = [f"# {c}" for c in comments]
    lines.append(",".join(CSV_COLUMNS))
    for r in results:
        t = r.timing
        lines.append(
            f"{r.op},{r.impl},{r.n},{r.batch},{t.median_ms:.6f},{t.min_ms:.6f},{t.max_ms:.6f},"
            f"{r.flops / (t.median_ms * 1e6):.1f},{r.nbytes / (t.median_ms * 1e6):.1f}"
        )
    return "\n".join(lines) + "\n"


def read_results(path: Path) -> dict[Key, float]:
    """Median ms per (op, impl, n, batch) in a results CSV; '#' lines are skipped."""
    with Path(path).open(newline="") as f:
        lines = [line for line in f if not line.startswith("#")]
    return {
        (row["op"], row["impl"], int(row["n"]), int(row["batch"])): float(row["time_ms"])
        for row in csv.DictReader(lines)
    }


def compare(
    old: dict[Key, float], new: dict[Key, float], threshold: float
) -> tuple[list[str], bool]:
    """A report line per matched row, and whether any row is slower than old * (1 + threshold).
    Rows present on one side only are listed and never fail."""
    lines = [f"{'op':<10} {'impl':<12} {'n':>7} {'batch':>9} {'old ms':>10} {'new ms':>10} ratio"]
    regressed = False
    for key in sorted(old.keys() & new.keys()):
        ratio = new[key] / old[key]
        flag = ""
        if ratio > 1 + threshold:
            flag, regressed = "  SLOWER", True
        elif ratio < 1 - threshold:
            flag = "  faster"
        op, impl, n, batch = key
        lines.append(
            f"{op:<10} {impl:<12} {n:>7} {batch:>9} {old[key]:>10.4f} {new[key]:>10.4f} "
            f"{ratio:5.2f}x{flag}"
        )
    lines += [f"only in old: {key}" for key in sorted(old.keys() - new.keys())]
    lines += [f"only in new: {key}" for key in sorted(new.keys() - old.keys())]
    return lines, regressed
