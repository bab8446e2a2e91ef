"""Benchmark of the batched-FFT hot path on one MI355X; prints ONE JSON line.

Workload ("C1"): batched complex64 C2C, n = 1024, batch = 16384
(2^24 points), real and imaginary parts U[-1, 1) from a fixed seed (synthetic data). One step is
a forward transform plus an inverse transform (impl "stockham_r8" unless --impl says otherwise),
called through the C ABI (libspectral_hip.so) on one HIP stream.

value        effective HBM GB/s of the step: algorithmic bytes (16 B per point per direction,
             reference csrc/common/bench.cpp:93-100) / wall time of the timed steps.
roofline     the forward C2C kernel alone: the same algorithmic bytes per launch / its average
             launch time inside the timed region (the K forward launches are queued back to back
             between two HIP events on the stream they run on); peak = 8000 GB/s.
             `traffic` (HBM bytes per launch from rocprof FETCH_SIZE + WRITE_SIZE) is filled in
             from profiles/ when a counter summary for this kernel has been committed.
cpu_baseline numpy.fft (pocketfft, single thread) on the same kind of complex64 input, forward +
             inverse, on a bounded sample of the workload, in the same GB/s convention.
extra        secondary rows of the metric, each with rocFFT (torch.fft) on the same shape: C2
             R2C / C2R at n = 1024, C3 rfft2 / irfft2 at 128^2 x 1024 and 512^2 x 64 (columns
             strided and transpose), C4 pruned rfft2 / irfft2 on [64, 32, 128, 128] with
             m1 = m2 = 16 (ms and effective GB/s);
             C5 the Navier-Stokes solver on 128^2 x 256 trajectories, 32 frames 40 steps apart,
             fused (this stack's default for the pruned layout) next to this stack's composed
             pruned path, rocFFT pruned and rocFFT full (ms per step and trajectory-steps / s);
             the radio callers (spectral.rf) on 2^22 samples as the reference's bench_rf.py
             times them: FIR of 63 and 1025 taps and the Hann spectrum of 1024-sample frames,
             this stack's single kernels next to the same operations on torch.fft.

Launches rotate over buffer sets totalling well over twice the 256 MB Infinity Cache, so a
launch cannot read what the previous one left in the cache.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--impl NAME] [--no-extra | --extra LIST]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "gpu-spectral-stack_amd" / "python"))

N = 1024
BATCH = 16384
POINTS = N * BATCH
BYTES_PER_DIRECTION = 16 * POINTS  # 268,435,456
PEAK_GBPS = 8000.0
MALL_BYTES = 256 << 20  # MI355X Infinity Cache


def rotation(input_bytes: int) -> int:
    """Buffer sets so that the inputs in rotation total at least twice the Infinity Cache: a
    launch then reads data that the launches since its set's last use have evicted."""
    return max(2, -(-2 * MALL_BYTES // int(input_bytes)))


SETS = rotation(BYTES_PER_DIRECTION // 2)  # 4 x (x, y, z) x 128 MiB = 1.5 GiB in rotation


# Secondary row groups, in the order they run: C-ABI timings of the 2D and pruned configurations,
# the C2 size sweep, the torch-operator rows (C2, C3, C4, large C2C), the Navier-Stokes solvers
# (C5) and the radio callers.
EXTRA_GROUPS = ("capi", "sweep", "secondary", "ns", "radio")


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--impl", default="stockham_r8")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="approximate CPU time spent on the numpy baseline sample")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary rows")
    ap.add_argument("--extra", default=",".join(EXTRA_GROUPS),
                    help="comma-separated groups of secondary rows to run (default: all of "
                         + ", ".join(EXTRA_GROUPS) + ")")
    args = ap.parse_args(argv)
    groups = [] if args.no_extra else [g for g in args.extra.split(",") if g]
    unknown = sorted(set(groups) - set(EXTRA_GROUPS))
    if unknown:
        ap.error(f"unknown --extra group(s) {', '.join(unknown)}")
    args.extra = groups
    return args


def load_capi():
    import torch  # noqa: F401  # PyTorch's HIP runtime first

    import spectral  # noqa: F401  # fails loudly when the extension is not built

    lib = ctypes.CDLL(str(REPO / "gpu-spectral-stack_amd" / "python" / "spectral"
                          / "libspectral_hip.so"))
    lib.spx_last_error.restype = ctypes.c_char_p
    lib.spx_impl_find.argtypes = [ctypes.c_char_p]
    return lib


def traffic_from_profiles(kernel_tag: str):
    """HBM bytes per launch of the dominant kernel, from a committed rocprof counter summary
    (profiles/*traffic*.json: {"kernel": ..., "fetch_bytes": ..., "write_bytes": ...}), or None."""
    for path in sorted((REPO / "profiles").glob("*traffic*.json")):
        try:
            data = json.loads(path.read_text())
        except (OSError, ValueError):
            continue
        if data.get("kernel_tag") == kernel_tag:
            return float(data["fetch_bytes"]) + float(data["write_bytes"])
    return None


def _host_cpu() -> str:
    """The host CPU's model name, from /proc/cpuinfo (empty when unreadable)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _time_rows(fn, seconds: float) -> tuple[int, float]:
    """Runs fn() (after one warm-up call) until `seconds` have passed: (calls, elapsed s)."""
    fn()
    reps = 0
    t0 = time.perf_counter()
    while True:
        fn()
        reps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            return reps, elapsed


def cpu_baseline(seconds: float) -> dict:
    """numpy.fft forward + inverse over complex64 rows of 1024 on one host thread (the reported
    value), then, in a quarter of that time each, the same work in complex128 on one thread and
    scipy.fft complex64 on every host core. Rates use the complex64 work convention (16 B per
    point per transform), so they compare directly with the GPU's."""
    import os

    import numpy as np

    rng = np.random.default_rng(1)
    rows = 2048
    x = (rng.uniform(-1, 1, (rows, N)) + 1j * rng.uniform(-1, 1, (rows, N))).astype(np.complex64)
    work = 2 * 16 * rows * N  # bytes per forward + inverse pass

    reps, elapsed = _time_rows(lambda: np.fft.ifft(np.fft.fft(x, axis=-1), axis=-1), seconds)
    gbps = work * reps / elapsed / 1e9
    out = {"value": round(gbps, 3), "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": f"numpy {np.__version__} pocketfft fft+ifft complex64, {rows} x {N} rows "
                     f"repeated {reps}x ({elapsed:.1f} s) on 1 host thread"}

    x64 = x.astype(np.complex128)
    reps, elapsed = _time_rows(lambda: np.fft.ifft(np.fft.fft(x64, axis=-1), axis=-1),
                               seconds / 4)
    out["complex128_1_thread_gbps"] = round(work * reps / elapsed / 1e9, 3)
    try:
        import scipy
        import scipy.fft

        threads = os.cpu_count() or 1
        reps, elapsed = _time_rows(
            lambda: scipy.fft.ifft(scipy.fft.fft(x, axis=-1, workers=threads), axis=-1,
                                   workers=threads),
            seconds / 4)
        out["scipy_all_cores_gbps"] = round(work * reps / elapsed / 1e9, 3)
        out["scipy_threads"] = threads
        out["scipy"] = scipy.__version__
    except ImportError:
        pass
    out["host_cpu"] = _host_cpu()
    return out


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the "
              "batched FFT shards over the batch axis with no exchange, so N GPUs would run N "
              "independent copies of this workload", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    lib = load_capi()
    impl = lib.spx_impl_find(args.impl.encode())
    if impl < 0:
        raise SystemExit(f"unknown --impl {args.impl}")
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    sptr = ctypes.c_void_p(stream.cuda_stream)

    rng = np.random.default_rng(0)
    xs, ys, zs = [], [], []
    for _ in range(SETS):
        re = torch.from_numpy(rng.uniform(-1, 1, POINTS).astype(np.float32))
        im = torch.from_numpy(rng.uniform(-1, 1, POINTS).astype(np.float32))
        xs.append(torch.complex(re, im).to(dev).view(BATCH, N))
        ys.append(torch.empty(BATCH, N, dtype=torch.complex64, device=dev))
        zs.append(torch.empty(BATCH, N, dtype=torch.complex64, device=dev))
    torch.cuda.synchronize()

    def call(src, dst, inverse):
        rc = lib.spx_c2c(impl, ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()),
                         N, BATCH, inverse, sptr)
        if rc != 0:
            raise RuntimeError(lib.spx_last_error().decode())

    def step(i):
        s = i % SETS
        call(xs[s], ys[s], 0)
        call(ys[(s + SETS // 2) % SETS], zs[s], 1)

    # The achievable streaming rate on the same buffers, measured before the warm-up (which it
    # extends): this stack's scale kernel as a copy (y = 1.0 x, 16 B moved per complex value),
    # rotating over the sets like the loop.
    lib.spx_scale.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float,
                              ctypes.c_void_p]
    copies = 60
    c0 = torch.cuda.Event(enable_timing=True)
    c1 = torch.cuda.Event(enable_timing=True)
    for i in range(copies + 6):
        if i == 6:
            c0.record(stream)
        src, dst = xs[i % SETS], zs[(i + 1) % SETS]
        if lib.spx_scale(src.data_ptr(), dst.data_ptr(), POINTS, 1.0, sptr) != 0:
            raise RuntimeError(lib.spx_last_error().decode())
    c1.record(stream)
    torch.cuda.synchronize()
    copy_gbps = 16 * POINTS * copies / (c0.elapsed_time(c1) * 1e6)

    for s in range(SETS):
        call(xs[s], ys[s], 0)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # Timed region: exactly K steps between two synchronizations, queued as the K forward
    # transforms back to back, then the K inverse transforms (inverse i reads a spectrum written
    # four launches earlier, so never one still in the cache). A HIP event between the two halves,
    # on the stream the kernels run on, gives the forward kernel's average launch duration from
    # the same region without events between launches.
    start = torch.cuda.Event(enable_timing=True)
    mid = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(args.steps):
        call(xs[i % SETS], ys[i % SETS], 0)
    mid.record(stream)
    for i in range(args.steps):
        call(ys[(args.steps + i) % SETS], zs[i % SETS], 1)
    stop.record(stream)
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(stop) / args.steps
    value = 2 * BYTES_PER_DIRECTION / (ms_per_step * 1e6)
    fwd_ms = start.elapsed_time(mid) / args.steps
    inv_ms = mid.elapsed_time(stop) / args.steps
    achieved = BYTES_PER_DIRECTION / (fwd_ms * 1e6)
    kernel_tag = f"c2c_fwd_{args.impl}_n{N}_b{BATCH}"
    traffic = traffic_from_profiles(kernel_tag)

    extra = {"fwd_ms": round(fwd_ms, 5), "inv_ms": round(inv_ms, 5),
             "fwd_gbps": round(achieved, 1), "wall_s_timed": round(wall_s, 3)}
    extra["copy_gbps"] = round(copy_gbps, 1)
    extra["c1_pct_of_copy"] = round(100 * value / copy_gbps, 1)
    if args.extra:
        # Every row of this stack first; rocFFT's (through torch.fft) after all of them: rocFFT's
        # kernels on random data slowed this stack's launches that followed them by 5-12 %.
        later = []
        groups = {
            "capi": lambda: capi_rows(lib, impl, dev, stream),
            "sweep": lambda: sweep_rows(lib, impl, dev, stream, later),
            "secondary": lambda: secondary_rows(args.impl, dev, later),
            "ns": lambda: navier_stokes_rows(args.impl, dev, later),
            "radio": lambda: radio_rows(args.impl, dev, later),
        }
        for name in EXTRA_GROUPS:
            if name in args.extra:
                extra.update(groups[name]())
        for rocfft_rows in later:
            extra.update(rocfft_rows())

    line = {
        "metric": "effective HBM GB/s (% of peak) batched fp32 C2C/R2C at 2^24 points; "
                  "pruned 2D ms",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "C1: batched C2C forward+inverse, complex64, n=1024, "
                               "batch=16384 (2^24 points)",
                   "impl": args.impl, "n": N, "batch": BATCH,
                   "pct_of_peak": round(100 * value / PEAK_GBPS, 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_GBPS, 4),
                     "traffic": traffic,
                     "kernel": f"fft_kernel<Plan<1024, R, E>, forward, C2cIo<false>> ({args.impl})",
                     "bytes_per_launch": BYTES_PER_DIRECTION},
        "cpu_baseline": cpu_baseline(args.cpu_seconds),
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


def secondary_rows(impl: str, dev, later: list) -> dict:
    """The other configurations of the metric, each next to rocFFT (through torch.fft) on the same
    shape: C2 real transforms at n = 1024, C3 rfft2 / irfft2 at 128^2 x 1024 and 512^2 x 64 (both
    column methods: strided, the default, and transpose), C4 pruned transforms on
    [64, 32, 128, 128] with m1 = m2 = 16, and rocFFT on the C1 shape. Inputs rotate over enough
    sets to total twice the Infinity Cache (rotation()), so no call reads what an earlier one
    left there. rocFFT's rows are timed by what this appends to `later`, after every row of this
    stack."""
    import torch

    import spectral
    from spectral.benchmark import (fft2_modes_work, fft2_real_work, fft_real_work, time_gpu)

    g = torch.Generator(device=dev).manual_seed(0)

    def timed(fn, inputs):
        k = [0]

        def call():
            k[0] += 1
            return fn(inputs[k[0] % len(inputs)])

        return time_gpu(call).median_ms

    ours = []    # (row name, bytes, fn, inputs, rocFFT row)
    theirs = {}  # rocFFT row -> (fn, inputs)

    def sets(make, one_bytes):
        return [make() for _ in range(rotation(one_bytes))]

    # C2: real transforms, n = 1024, 16384 rows.
    xr = sets(lambda: torch.randn(16384, 1024, device=dev, generator=g), 64 << 20)
    xh = [torch.fft.rfft(x) for x in xr]
    work = fft_real_work(1024, 16384)[1]
    ours.append(("c2_r2c_1024", work, lambda x: spectral.rfft(x, impl=impl), xr, "r2c"))
    ours.append(("c2_c2r_1024", work, lambda x: spectral.irfft(x, 1024, impl=impl), xh, "c2r"))
    theirs["r2c"] = (torch.fft.rfft, xr)
    theirs["c2r"] = (lambda x: torch.fft.irfft(x, 1024), xh)
    # C3: 2D real transforms, both column methods.
    for n, arrays in ((128, 1024), (512, 64)):
        xs = sets(lambda: torch.randn(arrays, n, n, device=dev, generator=g), 64 << 20)
        hs = [torch.fft.rfft2(x) for x in xs]
        work = fft2_real_work(n, n, arrays)[1]
        ours.append((f"c3_rfft2_{n}", work, lambda x: spectral.rfft2(x, impl=impl), xs,
                     f"rfft2_{n}"))
        ours.append((f"c3_irfft2_{n}", work, lambda x, n=n: spectral.irfft2(x, n, impl=impl), hs,
                     f"irfft2_{n}"))
        ours.append((f"c3_rfft2_{n}_transpose", work,
                     lambda x: spectral.rfft2(x, impl=impl, columns="transpose"), xs,
                     f"rfft2_{n}"))
        ours.append((f"c3_irfft2_{n}_transpose", work,
                     lambda x, n=n: spectral.irfft2(x, n, impl=impl, columns="transpose"), hs,
                     f"irfft2_{n}"))
        theirs[f"rfft2_{n}"] = (torch.fft.rfft2, xs)
        theirs[f"irfft2_{n}"] = (lambda x, n=n: torch.fft.irfft2(x, s=(n, n)), hs)
    # C4: FNO pruned transforms, [64, 32, 128, 128] <-> modes [64, 32, 32, 16].
    xp = sets(lambda: torch.randn(64, 32, 128, 128, device=dev, generator=g), 128 << 20)
    # The inverse's input is 8 MiB of modes: 64 sets of them.
    mp = sets(lambda: torch.randn(64, 32, 32, 16, dtype=torch.complex64, device=dev,
                                  generator=g), 8 << 20)
    work = fft2_modes_work(128, 128, 16, 16, 2048)[1]

    def rocfft_gather(x):
        full = torch.fft.rfft2(x)
        return torch.cat([full[..., :16, :16], full[..., 112:, :16]], dim=-2)

    def rocfft_scatter(m):
        full = torch.zeros(64, 32, 128, 65, dtype=torch.complex64, device=dev)
        full[..., :16, :16] = m[..., :16, :]
        full[..., 112:, :16] = m[..., 16:, :]
        return torch.fft.irfft2(full, s=(128, 128))

    ours.append(("c4_rfft2_modes_128_m16", work,
                 lambda x: spectral.rfft2_truncated(x, 16, 16, impl=impl), xp, "modes_f"))
    ours.append(("c4_irfft2_modes_128_m16", work,
                 lambda m: spectral.irfft2_from_modes(m, (128, 128), impl=impl), mp, "modes_i"))
    theirs["modes_f"] = (rocfft_gather, xp)
    theirs["modes_i"] = (rocfft_scatter, mp)
    # rocFFT (through torch.fft) on the C1 shape, forward.
    xc = sets(lambda: torch.randn(BATCH, N, dtype=torch.complex64, device=dev, generator=g),
              128 << 20)
    theirs["c1"] = (torch.fft.fft, xc)
    torch.cuda.synchronize()

    out = {}
    for name, nbytes, fn, inputs, _ in ours:
        ms = timed(fn, inputs)
        out[f"{name}_ms"] = round(ms, 5)
        out[f"{name}_gbps"] = round(nbytes / (ms * 1e6), 1)

    def rocfft_rows():
        roc = {key: timed(fn, inputs) for key, (fn, inputs) in theirs.items()}
        rows = {f"{name}_rocfft_ms": round(roc[key], 5) for name, _, _, _, key in ours}
        rows["c1_rocfft_c2c_1024_fwd_ms"] = round(roc["c1"], 5)
        return rows

    later.append(rocfft_rows)
    return out


def sweep_rows(lib, impl: int, dev, stream, later: list) -> dict:
    """BASELINE C2's sweep and C1's sizes: C2C, R2C and C2R at n = 2, 4, ..., 4096 with
    batch = 2^24 / n, through the C ABI on `stream`, next to rocFFT (torch.fft) on the same shapes.
    Eight buffer sets of 2^24 complex values each (1 GiB per side) serve every size: the real
    transforms' 64 MiB inputs then total 512 MiB in rotation, twice the Infinity Cache. The sizes are interleaved: each of 9 rounds times 20 launches of every (op, n),
    after 2 untimed ones, so a transient slowdown of the device lands in a round or two of each
    row instead of all of one row's; a row reports the median round. rocFFT's columns are added
    by what this appends to `later`. Rows are
    [n, us, % of 8 TB/s, rocFFT us, rocFFT %]; bytes follow the reference's convention (16 B per
    C2C point, 4n + 8(n/2 + 1) B per real row)."""
    import statistics

    import torch

    from spectral.benchmark import fft_c2c_work, fft_real_work

    sptr = ctypes.c_void_p(stream.cuda_stream)
    g = torch.Generator(device=dev).manual_seed(2)
    total = 1 << 24
    nsets = rotation(4 * total)  # the smallest input: 2^24 float32 values
    ins = [torch.randn(total, dtype=torch.complex64, device=dev, generator=g)
           for _ in range(nsets)]
    outs = [torch.empty(total, dtype=torch.complex64, device=dev) for _ in range(nsets)]
    torch.cuda.synchronize()
    vp = ctypes.c_void_p

    def check(rc):
        if rc != 0:
            raise RuntimeError(lib.spx_last_error().decode())

    rows = []  # (op, n, bytes, ours(i), theirs(i), [our us], [rocFFT us])
    n = 2
    while n <= 4096:
        batch = total // n
        half = n // 2 + 1
        as_c = [x.view(batch, n) for x in ins]
        as_r = [x.view(torch.float32)[:total].view(batch, n) for x in ins]
        as_h = [x[: batch * half].view(batch, half) for x in ins]

        def c2c(i, n=n, batch=batch):
            check(lib.spx_c2c(impl, vp(ins[i].data_ptr()), vp(outs[i].data_ptr()), n, batch, 0,
                              sptr))

        def r2c(i, n=n, batch=batch):
            check(lib.spx_r2c(impl, vp(ins[i].data_ptr()), vp(outs[i].data_ptr()), n, batch,
                              None, sptr))

        def c2r(i, n=n, batch=batch):
            check(lib.spx_c2r(impl, vp(ins[i].data_ptr()), vp(outs[i].data_ptr()), n, batch,
                              None, sptr))

        rows.append(("c2c", n, fft_c2c_work(n, batch)[1], c2c,
                     lambda i, a=as_c: torch.fft.fft(a[i]), [], []))
        rows.append(("r2c", n, fft_real_work(n, batch)[1], r2c,
                     lambda i, a=as_r: torch.fft.rfft(a[i]), [], []))
        rows.append(("c2r", n, fft_real_work(n, batch)[1], c2r,
                     lambda i, a=as_h, n=n: torch.fft.irfft(a[i], n), [], []))
        n *= 2

    def timed_us(run, on):
        for i in range(2):
            run(i)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(on)
        for i in range(20):
            run(i % nsets)
        b.record(on)
        b.synchronize()
        return a.elapsed_time(b) / 20 * 1e3

    # Ours over every row first, then rocFFT's: rocFFT's kernels on random data, timed between
    # ours, slowed the following launches of this stack's 1024- to 4096-point C2C by 5-12 %
    # (the same launches after rocFFT on zeros, or alone, were not slowed).
    for _ in range(9):
        for _, _, _, ours, _, us, _ in rows:
            us.append(timed_us(ours, stream))
    out = {"c2c": [], "r2c": [], "c2r": []}
    reported = []  # the output row of each entry of `rows`
    for op, n, nbytes, _, _, us, _ in rows:
        t = statistics.median(us)
        out[op].append([n, round(t, 2), round(100 * nbytes / (t * 1e3) / PEAK_GBPS, 1)])
        reported.append(out[op][-1])

    def rocfft_columns():
        current = torch.cuda.current_stream(dev)
        for _ in range(9):
            for _, _, _, _, theirs, _, roc in rows:
                roc.append(timed_us(theirs, current))
        for (_, _, nbytes, _, _, _, roc), row in zip(rows, reported):
            r = statistics.median(roc)
            row += [round(r, 2), round(100 * nbytes / (r * 1e3) / PEAK_GBPS, 1)]
        return {}

    later.append(rocfft_columns)
    return {"c2_sweep": out}


def capi_rows(lib, impl: int, dev, stream) -> dict:
    """C3 and C4 again through the C ABI alone, as C1 is measured: outputs and workspaces
    allocated once, launches on `stream` between HIP events, inputs rotating over three sets.
    The `extra` rows above go through the PyTorch operators, whose per-call Python, dispatcher
    and allocation work shows up when a kernel takes some 30 us."""
    import statistics

    import torch

    from spectral.benchmark import fft2_modes_work, fft2_real_work

    sptr = ctypes.c_void_p(stream.cuda_stream)
    g = torch.Generator(device=dev).manual_seed(1)
    out = {}
    vp = ctypes.c_void_p

    def check(rc):
        if rc != 0:
            raise RuntimeError(lib.spx_last_error().decode())

    def workspace(query, *args):
        count = ctypes.c_size_t(0)
        check(query(*args, ctypes.byref(count)))
        return torch.empty(max(1, count.value), dtype=torch.complex64, device=dev)

    def time_calls(call, k):
        for i in range(3):
            call(i % k)
        runs = []
        for _ in range(5):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for i in range(20):
                call(i % k)
            b.record(stream)
            b.synchronize()
            runs.append(a.elapsed_time(b) / 20)
        return statistics.median(runs)

    def record(name, ms, nbytes):
        out[f"{name}_capi_ms"] = round(ms, 5)
        out[f"{name}_capi_gbps"] = round(nbytes / (ms * 1e6), 1)

    strided = 1  # SPX_COLUMNS_STRIDED
    k = rotation(64 << 20)  # C3's inputs: 64 MiB fields, 64.5 MiB spectra
    for n, arrays in ((128, 1024), (512, 64)):
        xs = [torch.randn(arrays, n, n, device=dev, generator=g) for _ in range(k)]
        ys = [torch.empty(arrays, n, n // 2 + 1, dtype=torch.complex64, device=dev)
              for _ in range(k)]
        zs = [torch.empty(arrays, n, n, device=dev) for _ in range(k)]
        w_f = workspace(lib.spx_fft2_r2c_workspace, impl, strided, n, n, arrays)
        w_i = workspace(lib.spx_fft2_c2r_workspace, impl, strided, n, n, arrays)
        torch.cuda.synchronize()
        work = fft2_real_work(n, n, arrays)[1]
        record(f"c3_rfft2_{n}", time_calls(lambda i: check(lib.spx_fft2_r2c(
            impl, strided, vp(xs[i].data_ptr()), vp(ys[i].data_ptr()), n, n, arrays,
            vp(w_f.data_ptr()), sptr)), k), work)
        record(f"c3_irfft2_{n}", time_calls(lambda i: check(lib.spx_fft2_c2r(
            impl, strided, vp(ys[i].data_ptr()), vp(zs[i].data_ptr()), n, n, arrays,
            vp(w_i.data_ptr()), sptr)), k), work)
        del xs, ys, zs, w_f, w_i
    # C4: [64, 32, 128, 128] <-> modes [64, 32, 32, 16], m1 = m2 = 16.
    arrays = 2048
    kf, ki = rotation(128 << 20), rotation(8 << 20)  # 128 MiB fields, 8 MiB of modes
    xs = [torch.randn(arrays, 128, 128, device=dev, generator=g) for _ in range(kf)]
    ms = [torch.randn(arrays, 32, 16, dtype=torch.complex64, device=dev, generator=g)
          for _ in range(ki)]
    zs = [torch.empty(arrays, 128, 128, device=dev) for _ in range(kf)]
    w_f = workspace(lib.spx_rfft2_modes_workspace, impl, 128, 128, 16, 16, arrays)
    w_i = workspace(lib.spx_irfft2_modes_workspace, impl, 128, 128, 16, 16, arrays)
    torch.cuda.synchronize()
    work = fft2_modes_work(128, 128, 16, 16, arrays)[1]
    record("c4_rfft2_modes_128_m16", time_calls(lambda i: check(lib.spx_rfft2_modes(
        impl, vp(xs[i].data_ptr()), vp(ms[i % ki].data_ptr()), 128, 128, 16, 16, arrays,
        vp(w_f.data_ptr()), sptr)), kf), work)
    record("c4_irfft2_modes_128_m16", time_calls(lambda i: check(lib.spx_irfft2_modes(
        impl, vp(ms[i].data_ptr()), vp(zs[i % kf].data_ptr()), 128, 128, 16, 16, arrays,
        vp(w_i.data_ptr()), sptr)), ki), work)
    return out


def radio_rows(impl: str, dev, later: list) -> dict:
    """spectral.rf as the reference's bench/bench_rf.py times it: 2^22 complex64 samples from
    seed 0, FIR of 63 and 1025 random taps (default block sizes 256 and 4096), and the Hann
    spectrum of 1024-sample frames; effective GB/s counts 16 bytes per sample (each read and
    written once). One signal is 32 MiB, so the calls rotate over `rotation()` signals (512 MiB)
    and none reads a signal an earlier call left in the Infinity Cache. The same operations
    composed on torch.fft are timed by what this appends to `later`."""
    import torch

    from spectral import rf
    from spectral.benchmark import time_gpu

    g = torch.Generator(device=dev).manual_seed(0)
    n = 1 << 22
    xs = [torch.randn(n, dtype=torch.complex64, device=dev, generator=g)
          for _ in range(rotation(8 * n))]
    turn = [0]

    def signal():
        turn[0] += 1
        return xs[turn[0] % len(xs)]

    out = {}

    theirs = []

    def record(name, fn_ours, fn_torch):
        ms = time_gpu(fn_ours).median_ms
        out[f"{name}_ms"] = round(ms, 5)
        out[f"{name}_gbps"] = round(16.0 * n / (ms * 1e6), 1)
        theirs.append((f"{name}_rocfft_ms", fn_torch))

    for m in (63, 1025):
        taps = torch.randn(m, device=dev, generator=g)
        record(f"rf_fir{m}_2e22", lambda t=taps: rf.fir(signal(), t, fft_impl=impl),
               lambda t=taps: rf.fir(signal(), t, fft_impl="rocfft"))
    record("rf_spectrum1024_hann_2e22",
           lambda: rf.spectrum(signal(), 1024, window_name="hann", fft_impl=impl),
           lambda: rf.spectrum(signal(), 1024, window_name="hann", fft_impl="rocfft"))
    later.append(lambda: {key: round(time_gpu(fn).median_ms, 5) for key, fn in theirs})
    return out


def random_vorticity(rng, n: int, batch: int, slope: float = -3.0):
    """Gaussian random vorticity fields with power spectrum |k|^slope, zero mean, unit RMS."""
    import numpy as np

    kx = np.fft.rfftfreq(n, 1.0 / n)[None, :]
    ky = np.fft.fftfreq(n, 1.0 / n)[:, None]
    k = np.sqrt(kx**2 + ky**2)
    amplitude = np.where(k > 0, k, 1.0) ** (slope / 2) * (k > 0)
    w = np.fft.irfft2(np.fft.rfft2(rng.standard_normal((batch, n, n))) * amplitude, s=(n, n))
    return (w / w.std(axis=(-2, -1), keepdims=True)).astype(np.float32)


def navier_stokes_rows(impl: str, dev, later: list) -> dict:
    """C5: the pseudo-spectral Navier-Stokes solver (spectral.flow.gpu.GpuSolver) on 128^2 x 256
    trajectories, viscosity U[1e-3, 5e-3] per trajectory, Kolmogorov forcing sin(4y), dt 0.0025,
    a k^-3 Gaussian random initial vorticity from seed 0; one job = 32 physical frames 40 steps
    apart (1240 IMEX steps, frames kept on the GPU). Timed once per backend after 40 warm-up
    steps: the fused stages (impl, pruned; the 40 steps between frames as one launch), this
    stack's composed pruned path, and, appended to `later`, rocFFT pruned and rocFFT full (the
    reference's torch.fft comparison). GpuSolver.advance is step() repeated for the last three."""
    import numpy as np
    import torch

    from spectral.flow import Flow
    from spectral.flow.gpu import GpuSolver

    n, batch, dt, frames, every = 128, 256, 0.0025, 32, 40
    rng = np.random.default_rng(0)
    flow = Flow(viscosity=rng.uniform(1e-3, 5e-3, batch))
    w0 = torch.as_tensor(random_vorticity(rng, n, batch), device=dev)
    out = {}
    record = torch.empty(frames, batch, n, n, device=dev)

    def run(name, kwargs):
        solver = GpuSolver(n, flow, dt, device=dev, **kwargs)
        w_hat = solver.advance(solver.to_spectral(w0), every)
        w_hat = solver.to_spectral(w0)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        record[0] = solver.to_physical(w_hat)
        for f in range(1, frames):
            w_hat = solver.advance(w_hat, every)  # `every` calls of step()
            record[f] = solver.to_physical(w_hat)
        stop.record()
        stop.synchronize()
        seconds = start.elapsed_time(stop) / 1e3
        steps = (frames - 1) * every
        if not bool(torch.isfinite(record[-1]).all()):
            raise RuntimeError(f"C5 {name}: the solution is not finite")
        return {f"c5_ns128_{name}_ms_per_step": round(1e3 * seconds / steps, 5),
                f"c5_ns128_{name}_traj_steps_per_s": round(batch * steps / seconds)}

    out.update(run("fused", dict(fft_impl=impl, pruned=True, fused=True)))
    out.update(run("composed", dict(fft_impl=impl, pruned=True, fused=False)))
    later.append(lambda: {**run("rocfft_pruned", dict(fft_impl="rocfft", pruned=True)),
                          **run("rocfft_full", dict(fft_impl="rocfft", pruned=False))})
    return out


if __name__ == "__main__":
    sys.exit(main())
