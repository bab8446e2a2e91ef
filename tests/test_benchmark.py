"""Benchmark helpers (reference tests/test_benchmark.py): the work conventions behind effective
GB/s, regression comparison, CSV reading, and (on a GPU) that time_gpu measures kernel time."""

import pytest
import torch

from spectral.benchmark import (
    compare,
    fft2_modes_work,
    fft2_real_work,
    fft_c2c_work,
    fft_real_work,
    read_results,
    time_gpu,
)


def test_fft_work_follows_the_5_n_log2_n_convention():
    flops, nbytes = fft_c2c_work(1024, 3)
    assert flops == 5 * 1024 * 10 * 3
    assert nbytes == 16 * 1024 * 3


def test_real_fft_work_is_half_the_flops_and_counts_both_sides():
    flops, nbytes = fft_real_work(1024, 3)
    assert flops == fft_c2c_work(1024, 3)[0] / 2
    assert nbytes == 3 * (4 * 1024 + 8 * 513)


def test_config_byte_counts():
    # The algorithmic bytes of the benchmark configurations (BASELINE: C1..C4).
    assert fft_c2c_work(1024, 16384)[1] == 268_435_456
    assert fft_real_work(1024, 16384)[1] == 134_348_800
    assert fft_real_work(2, 1 << 23)[1] == 201_326_592
    assert fft_real_work(4096, 4096)[1] == 134_250_496
    assert fft2_real_work(128, 128, 1024)[1] == 135_266_304
    assert fft2_real_work(512, 512, 64)[1] == 134_479_872
    assert fft2_modes_work(128, 128, 16, 16, 2048)[1] == 142_606_336


def test_compare_flags_only_changes_beyond_the_threshold():
    old = {("fft", "a", 64, 1): 1.0, ("fft", "b", 64, 1): 1.0, ("fft", "c", 64, 1): 1.0}
    new = {("fft", "a", 64, 1): 1.05, ("fft", "b", 64, 1): 1.2, ("fft", "c", 64, 1): 0.5}
    lines, regressed = compare(old, new, threshold=0.10)
    assert regressed
    assert [line.split()[1] for line in lines if "SLOWER" in line] == ["b"]
    assert [line.split()[1] for line in lines if "faster" in line] == ["c"]


def test_compare_lists_unmatched_rows_without_failing():
    lines, regressed = compare({("fft", "a", 64, 1): 1.0}, {("fft", "a", 128, 1): 1.0}, 0.10)
    assert not regressed
    assert any(line.startswith("only in old") for line in lines)
    assert any(line.startswith("only in new") for line in lines)


def test_read_results_skips_comment_lines(tmp_path):
    path = tmp_path / "bench.csv"
    path.write_text(
        "# device: test\n"
        "op,impl,n,batch,time_ms,min_ms,gflops,gbps\n"
        "fft_c2c,rocfft,64,262144,0.250000,0.240000,100.0,800.0\n"
    )
    assert read_results(path) == {("fft_c2c", "rocfft", 64, 262144): 0.25}


def test_time_gpu_rejects_a_bad_configuration():
    with pytest.raises(ValueError, match="rounds"):
        time_gpu(lambda: None, rounds=0)


@pytest.mark.gpu
def test_time_gpu_measures_real_kernel_time():
    import spectral

    x = torch.randn(1 << 24, dtype=torch.complex64, device="cuda")
    t = time_gpu(lambda: spectral.scale(x, 0.5))
    assert 0 < t.min_ms <= t.median_ms <= t.max_ms
    # 16 bytes per point at a believable MI355X rate (peak 8 TB/s; the 256 MiB working set can
    # partly hit the 256 MB Infinity Cache). A timing bug gives absurd rates.
    gbps = 16 * (1 << 24) / (t.median_ms * 1e6)
    assert 100 < gbps < 20000


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
