"""The benchmark harness (reference python/spectral/benchmark.py, tools/bench_compare.py,
csrc/tools/spectral_bench.cpp): the work conventions behind effective GB/s, checked against byte
counts of real numpy arrays of each transform's input and output; the result CSV round trip and
the regression comparison; the spectral_bench command line, whose flag errors are caught on the
host and whose rows, on a GPU, follow the reference's CSV schema."""

import math
import subprocess
from pathlib import Path

import numpy as np
import pytest

from spectral.benchmark import (
    CSV_COLUMNS,
    PEAK_COLUMNS,
    Result,
    Timing,
    compare,
    fft2_modes_work,
    fft2_real_work,
    fft_c2c_work,
    fft_real_work,
    format_csv,
    main,
    read_results,
    time_gpu,
)

REPO = Path(__file__).resolve().parents[1]
SPECTRAL_BENCH = REPO / "gpu-spectral-stack_amd" / "bin" / "spectral_bench"
BASELINE_CSV = REPO / "profiles" / "spectral_bench_sweep.csv"

# A percentage column and the GB/s it is checked against are both printed to 0.1, so they agree
# to the percentage's rounding (0.05) plus the GB/s rounding's share (0.05 GB/s of a 6300-8000
# GB/s peak: under 0.001).
PCT_ROUNDING = 0.051


def radix2_flops(n: int, batch: int) -> int:
    # n/2 butterflies per stage, log2 n stages, 10 real flops per butterfly (a complex product
    # is 6, the sum and difference 4): the convention's 5 n log2 n.
    return batch * (n // 2) * int(math.log2(n)) * 10


# --- work conventions ------------------------------------------------------------------------

@pytest.mark.parametrize("n,batch", [(2, 7), (64, 1), (1024, 3), (4096, 4096)])
def test_complex_work_reads_and_writes_each_point_once(n, batch):
    x = np.zeros((batch, n), np.complex64)
    flops, nbytes = fft_c2c_work(n, batch)
    assert nbytes == x.nbytes + np.fft.fft(x).astype(np.complex64).nbytes
    assert flops == radix2_flops(n, batch)


@pytest.mark.parametrize("n,batch", [(2, 5), (16, 3), (1024, 16384), (8192, 2)])
def test_real_work_counts_the_real_row_and_the_half_spectrum(n, batch):
    x = np.zeros((batch, n), np.float32)
    half = np.fft.rfft(x).astype(np.complex64)
    flops, nbytes = fft_real_work(n, batch)
    assert nbytes == x.nbytes + half.nbytes
    assert flops == radix2_flops(n, batch) / 2


@pytest.mark.parametrize("n1,n2,batch", [(4, 8, 3), (128, 128, 2), (512, 256, 1)])
def test_2d_real_work_counts_the_array_and_its_half_spectrum(n1, n2, batch):
    x = np.zeros((batch, n1, n2), np.float32)
    flops, nbytes = fft2_real_work(n1, n2, batch)
    assert nbytes == x.nbytes + np.fft.rfft2(x).astype(np.complex64).nbytes
    assert flops == radix2_flops(n1 * n2, batch) / 2


def test_pruned_work_counts_the_modes_not_the_spectrum():
    # [2, 128, 128] float32 and its modes [2, 2 * 16, 12] complex64; the flops stay those of the
    # full transform, as the reference counts them.
    x = np.zeros((2, 128, 128), np.float32)
    modes = np.zeros((2, 32, 12), np.complex64)
    flops, nbytes = fft2_modes_work(128, 128, 16, 12, 2)
    assert nbytes == x.nbytes + modes.nbytes
    assert flops == fft2_real_work(128, 128, 2)[0]


def test_config_byte_counts():
    # The algorithmic bytes of the benchmark configurations (BASELINE: C1..C4).
    assert fft_c2c_work(1024, 16384)[1] == 268_435_456
    assert fft_real_work(1024, 16384)[1] == 134_348_800
    assert fft_real_work(2, 1 << 23)[1] == 201_326_592
    assert fft_real_work(4096, 4096)[1] == 134_250_496
    assert fft2_real_work(128, 128, 1024)[1] == 135_266_304
    assert fft2_real_work(512, 512, 64)[1] == 134_479_872
    assert fft2_modes_work(128, 128, 16, 16, 2048)[1] == 142_606_336


# --- result files and the regression check ---------------------------------------------------

def _result(impl: str, n: int, ms: float) -> Result:
    flops, nbytes = fft_c2c_work(n, 1 << 14)
    return Result("fft_c2c", impl, n, 1 << 14, Timing.of([ms, ms * 1.02, ms * 0.99]), flops,
                  nbytes)


def test_csv_round_trip_keeps_the_key_and_the_median(tmp_path):
    rows = [_result("rocfft", 256, 0.0317), _result("stockham_r8", 256, 0.0212),
            _result("stockham_r8", 1024, 0.0461)]
    text = format_csv(rows, ["device: test box", "timing: made up"], measured_peak_gbps=6300.0)
    lines = text.splitlines()
    assert lines[:2] == ["# device: test box", "# timing: made up"]
    assert lines[2].split(",") == CSV_COLUMNS + PEAK_COLUMNS
    path = tmp_path / "rows.csv"
    path.write_text(text)
    back = read_results(path)
    assert back == {r.key: pytest.approx(r.timing.median_ms, abs=5e-7) for r in rows}
    # The datasheet and measured percentages come from gbps alone.
    gbps, datasheet, measured = (float(v) for v in lines[4].split(",")[8:11])
    assert datasheet == pytest.approx(100 * gbps / 8000, abs=PCT_ROUNDING)
    assert measured == pytest.approx(100 * gbps / 6300, abs=PCT_ROUNDING)


def test_read_results_takes_the_reference_layout_without_the_peak_columns(tmp_path):
    # Nine columns (or fewer: only the key and time_ms are needed), '#' and blank lines between.
    path = tmp_path / "old.csv"
    path.write_text("# device: a laptop\n\nop,impl,n,batch,time_ms,gbps\n"
                    "fft_r2c,cufft,8,2097152,0.125000,1000.0\n# trailing note\n")
    assert read_results(path) == {("fft_r2c", "cufft", 8, 2097152): 0.125}


def test_read_results_names_a_missing_column(tmp_path):
    path = tmp_path / "bad.csv"
    path.write_text("op,impl,n,batch,median\nfft_c2c,x,2,2,1.0\n")
    with pytest.raises(ValueError, match="time_ms"):
        read_results(path)


def test_compare_fails_only_beyond_the_threshold():
    old = {("fft_c2c", impl, 64, 8): 1.0 for impl in "pqrs"}
    new = {("fft_c2c", "p", 64, 8): 1.25,   # exactly at the threshold: allowed
           ("fft_c2c", "q", 64, 8): 1.5,    # slower
           ("fft_c2c", "r", 64, 8): 0.5,    # faster
           ("fft_c2c", "s", 64, 8): 1.0}
    lines, regressed = compare(old, new, threshold=0.25)
    assert regressed
    flagged = {line.split()[1]: line.split()[-1] for line in lines[1:]}
    assert flagged["q"] == "SLOWER" and flagged["r"] == "faster"
    assert flagged["p"] not in ("SLOWER", "faster") and flagged["s"] not in ("SLOWER", "faster")
    assert not compare(old, {k: v for k, v in new.items() if k[1] != "q"}, 0.25)[1]


def test_compare_reports_rows_on_one_side_and_never_fails_on_them():
    old = {("fft_c2r", "naive", 16, 4): 2.0, ("scale", "ours", 64, 1): 1.0}
    new = {("fft_c2r", "naive", 32, 2): 9.0, ("scale", "ours", 64, 1): 1.0}
    lines, regressed = compare(old, new, 0.05)
    assert not regressed
    assert [line for line in lines if line.startswith("only in old")] == \
        ["only in old: ('fft_c2r', 'naive', 16, 4)"]
    assert [line for line in lines if line.startswith("only in new")] == \
        ["only in new: ('fft_c2r', 'naive', 32, 2)"]


def test_compare_command_exit_status(tmp_path, capsys):
    base, slow = tmp_path / "base.csv", tmp_path / "slow.csv"
    base.write_text(format_csv([_result("stockham_r8", 1024, 0.046)], []))
    slow.write_text(format_csv([_result("stockham_r8", 1024, 0.060)], []))
    assert main(["compare", str(base), str(base)]) == 0
    assert main(["compare", str(base), str(slow), "--threshold", "0.10"]) == 1
    assert "regression" in capsys.readouterr().out
    assert main(["compare", str(base), str(slow), "--threshold", "0.5"]) == 0


def test_timing_statistics_and_bad_configurations():
    t = Timing.of([3.0, 1.0, 2.0, 10.0])
    assert (t.median_ms, t.min_ms, t.max_ms) == (2.5, 1.0, 10.0)
    assert t.unstable and not Timing.of([1.0, 1.04]).unstable
    with pytest.raises(ValueError):
        Timing.of([])
    with pytest.raises(ValueError, match="rounds"):
        time_gpu(lambda: None, rounds=0)
    with pytest.raises(ValueError, match="iters"):
        time_gpu(lambda: None, iters=0)


# --- the spectral_bench command line ---------------------------------------------------------

def _bench(*flags, timeout=60):
    if not SPECTRAL_BENCH.exists():
        pytest.fail(f"{SPECTRAL_BENCH} is not built: run __graft_entry__.build()")
    return subprocess.run([str(SPECTRAL_BENCH), *map(str, flags)], capture_output=True,
                          text=True, timeout=timeout)


@pytest.mark.parametrize("flags,named", [
    (["--sizes", "3"], "--sizes"),
    (["--sizes", "64,,128"], "--sizes"),
    (["--iters", "0"], "--iters"),
    (["--rounds", "2x"], "--rounds"),
    (["--impl", "cufft"], "--impl"),
    (["--op", "fft3"], "--op"),
    (["--copy-peak", "-1"], "--copy-peak"),
    (["--warmup"], "--warmup"),
    (["--frobnicate", "1"], "--frobnicate"),
])
def test_spectral_bench_rejects_bad_flags_before_using_the_gpu(flags, named):
    done = _bench(*flags)
    assert done.returncode == 1
    assert done.stderr.startswith(f"error: {named}: "), done.stderr
    assert "usage: spectral_bench" in done.stderr


def test_spectral_bench_help_lists_the_registry():
    done = _bench("--help")
    assert done.returncode == 0
    assert "our FFTs: naive, stockham_r2, stockham_r4, stockham_r8, stockham_r8_table" in \
        done.stdout


def test_committed_sweep_is_a_usable_baseline():
    # The sweep under profiles/ is the baseline `compare` checks new runs against: it parses, it
    # covers every implementation next to rocFFT for the 1D and 2D real operations, and it
    # compares clean against itself.
    rows = read_results(BASELINE_CSV)
    ops = {op for op, _, _, _ in rows}
    assert {"fft_c2c", "fft_r2c", "fft_c2r", "fft2_r2c", "fft2_c2r", "rfft2_modes",
            "irfft2_modes", "scale"} <= ops
    for op in ("fft_c2c", "fft_r2c", "fft_c2r"):
        impls = {impl for o, impl, n, _ in rows if o == op and n == 1024}
        assert {"rocfft", "naive", "stockham_r2", "stockham_r4", "stockham_r8",
                "stockham_r8_table"} <= impls, op
    assert not compare(rows, rows, 0.0)[1]
    header = next(line for line in BASELINE_CSV.read_text().splitlines()
                  if not line.startswith("#"))
    assert header.split(",") == CSV_COLUMNS + PEAK_COLUMNS


@pytest.mark.gpu
@pytest.mark.parametrize("op,size,batch,ours", [("fft_c2c", 1024, 16384, "stockham_r8"),
                                                ("fft2_r2c", 128, 1024, "stockham_r8/strided")])
def test_spectral_bench_rows_follow_the_reference_schema(tmp_path, op, size, batch, ours):
    out = tmp_path / "rows.csv"
    done = _bench("--op", op, "--impl", "rocfft,stockham_r8", "--sizes", size, "--warmup", 1,
                  "--rounds", 1, "--iters", 2, "--out", out, timeout=120)
    assert done.returncode == 0, done.stderr
    lines = out.read_text().splitlines()
    header = next(line for line in lines if not line.startswith("#"))
    assert header.split(",")[:9] == CSV_COLUMNS
    assert header.split(",")[9:] == PEAK_COLUMNS
    assert any(line.startswith("# pct_peak_datasheet") for line in lines)
    rows = {tuple(line.split(",")[:2]): line.split(",") for line in lines
            if not line.startswith("#") and line != header}
    assert (op, "rocfft") in rows
    gbps = float(rows[(op, ours)][8])
    assert 1000 < gbps < 8000, gbps
    assert float(rows[(op, ours)][9]) == pytest.approx(100 * gbps / 8000, abs=PCT_ROUNDING)
    assert 0 < float(rows[(op, ours)][10]) < 150
    assert set(read_results(out)) == {(op, impl, size, batch) for _, impl in rows}


@pytest.mark.gpu
def test_time_gpu_measures_real_kernel_time():
    import torch

    import spectral

    small = torch.randn(1 << 22, dtype=torch.complex64, device="cuda")
    large = torch.randn(1 << 25, dtype=torch.complex64, device="cuda")
    t_small = time_gpu(lambda: spectral.scale(small, 0.5))
    t_large = time_gpu(lambda: spectral.scale(large, 0.5))
    assert 0 < t_large.min_ms <= t_large.median_ms <= t_large.max_ms
    # 8 times the data takes several times longer, at a rate an MI355X can reach: a timer that
    # did not wait for the GPU would see launch overhead only.
    assert t_large.median_ms > 3 * t_small.median_ms
    gbps = 16 * (1 << 25) / (t_large.median_ms * 1e6)
    assert 1000 < gbps < 8000


def test_cpu_baseline_reports_its_sample_and_the_wider_rows():
    import bench

    cb = bench.cpu_baseline(0.2)
    assert cb["unit"] == "GB/s" and cb["kind"] == "port" and cb["cores"] == 1
    assert cb["value"] > 0 and cb["complex128_1_thread_gbps"] > 0
    assert "on 1 host thread" in cb["sample"]
    if "scipy_all_cores_gbps" in cb:
        assert cb["scipy_all_cores_gbps"] > 0 and cb["scipy_threads"] >= 1


def test_bench_row_groups_select_and_reject():
    import bench

    assert bench.parse_args([]).extra == list(bench.EXTRA_GROUPS)
    assert bench.parse_args(["--no-extra"]).extra == []
    assert bench.parse_args(["--extra", "ns,capi"]).extra == ["ns", "capi"]
    with pytest.raises(SystemExit):
        bench.parse_args(["--extra", "ns,bogus"])
