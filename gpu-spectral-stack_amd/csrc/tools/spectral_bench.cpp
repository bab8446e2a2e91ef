// spectral_bench: times every implementation of every operation of libspectral_hip.so on one
// MI355X, next to rocFFT (through hipFFT), and writes one CSV row per (operation, implementation,
// size, batch). The flags and the first nine CSV columns are those of the reference's
// csrc/tools/spectral_bench.cpp:48-60 and :185, so its result files and regression checks
// (python -m spectral.benchmark compare) work on these rows; the baseline row is "rocfft" where
// the reference has "cufft".
//
// What differs, for this GPU:
// * Every row rotates over --rotate buffer sets (input, output), 8 by default. At the default
//   2^24 points a set's input is 64 MiB (real) to 128 MiB (complex), so the inputs in rotation
//   total at least 512 MiB, twice MI355X's 256 MB Infinity Cache: a launch reads data that the
//   launches since its set's last use have evicted, and the rates are HBM rates.
// * Two more columns: pct_peak_datasheet, gbps as a percentage of the 8 TB/s HBM peak, and
//   pct_peak_measured, of the copy ceiling measured at start-up (spx_scale streaming 1 GiB into
//   another 1 GiB, the header says the figure) or given with --copy-peak.
// * --impl takes a comma-separated list (e.g. rocfft,stockham_r8); --sizes takes powers of two.
//
// Each size runs batch = total / n transforms (2^24 points by default); 2D rows use n x n arrays,
// batch = total / n^2. Pruned 2D rows keep m1 = m2 = max(1, n/8) modes; rocFFT has no pruned
// transform, so its row is the full transform plus this library's gather (or scatter).
// Timing: --warmup launches, then --rounds measurements of --iters launches between two HIP
// events on one stream; the median per launch is reported, and a row whose rounds differ by
// more than 5 % gets a warning on stderr.
//
//   spectral_bench [--op NAME] [--impl LIST] [--sizes LIST] [--total N] [--batches LIST]
//                  [--warmup N] [--rounds N] [--iters N] [--rotate N] [--copy-peak GBPS]
//                  [--out FILE]

#include "spectral_hip.h"

#include <hip/hip_runtime.h>
#include <hipfft/hipfft.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <iostream>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

constexpr double kPeakGbps = 8000.0;      // MI355X HBM3E datasheet
constexpr double kUnstableSpread = 0.05;  // max / min - 1 above this gets a warning

const char* const kUsage =
    "usage: spectral_bench [options]\n"
    "  --op NAME         all (default), fft_c2c, fft_r2c, fft_c2r, fft2_c2c, fft2_r2c,\n"
    "                    fft2_c2r, rfft2_modes, irfft2_modes, scale, or ns_step (two rows:\n"
    "                    a step as two stage launches, and 40 steps per launch, ns_steps40)\n"
    "  --impl LIST       all (default), or a comma-separated list of rocfft, ours (the scale\n"
    "                    and ns_step kernels) and our FFTs\n"
    "  --sizes LIST      comma-separated transform sizes, powers of two (default: 2,4,...,4096)\n"
    "  --total N         points per row; batch = total / n (default: 16777216)\n"
    "  --batches LIST    comma-separated batch counts to run at every size instead of\n"
    "                    total / n (rows whose points exceed --total are skipped)\n"
    "  --warmup N        untimed launches (default: 3)\n"
    "  --rounds N        timed measurements; the median is reported (default: 5)\n"
    "  --iters N         launches per measurement (default: 20)\n"
    "  --rotate N        buffer sets the launches rotate over (default: 8)\n"
    "  --copy-peak GBPS  the copy ceiling for pct_peak_measured (default: measured)\n"
    "  --out FILE        write the CSV to FILE instead of standard output\n";

void hip_check(hipError_t err, const char* what)
{
    if (err != hipSuccess) {
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(err));
    }
}

void fft_check(hipfftResult r, const char* what)
{
    if (r != HIPFFT_SUCCESS) {
        throw std::runtime_error(std::string(what) + " failed with hipFFT status "
                                 + std::to_string(static_cast<int>(r)));
    }
}

void spx_check(int rc, const char* what)
{
    if (rc != SPX_OK) {
        throw std::runtime_error(std::string(what) + ": " + spx_last_error());
    }
}

struct Options {
    std::string op = "all";
    std::vector<std::string> impls;  // empty: all
    std::vector<long long> sizes;
    std::vector<long long> batches;
    long long total = 1LL << 24;
    int warmup = 3;
    int rounds = 5;
    int iters = 20;
    int rotate = 8;
    double copy_peak = 0;  // GB/s; 0: measure
    std::string out;

    bool wants(const std::string& name) const
    {
        return impls.empty() || std::find(impls.begin(), impls.end(), name) != impls.end();
    }
};

// A flag's value that cannot be used: the message names the flag, then the usage follows.
struct FlagError : std::invalid_argument {
    FlagError(const std::string& flag, const std::string& what)
        : std::invalid_argument(flag + ": " + what + "\n" + kUsage)
    {
    }
};

std::vector<std::string> split_commas(const std::string& text)
{
    std::vector<std::string> items;
    std::size_t from = 0;
    while (from <= text.size()) {
        const std::size_t comma = std::min(text.find(',', from), text.size());
        items.push_back(text.substr(from, comma - from));
        from = comma + 1;
    }
    return items;
}

// A whole decimal integer >= lowest (strtoll must consume every character).
long long to_count(const std::string& text, const std::string& flag, long long lowest)
{
    if (text.empty()) {
        throw FlagError(flag, "empty value");
    }
    errno = 0;
    char* end = nullptr;
    const long long v = std::strtoll(text.c_str(), &end, 10);
    if (errno != 0 || end != text.c_str() + text.size()) {
        throw FlagError(flag, "'" + text + "' is not an integer");
    }
    if (v < lowest) {
        throw FlagError(flag, "'" + text + "' is below the least allowed value "
                                  + std::to_string(lowest));
    }
    return v;
}

std::vector<long long> to_counts(const std::string& text, const std::string& flag,
                                 bool powers_of_two)
{
    std::vector<long long> values;
    for (const std::string& item : split_commas(text)) {
        const long long v = to_count(item, flag, 1);
        if (powers_of_two && (v & (v - 1)) != 0) {
            throw FlagError(flag, "'" + item + "' is not a power of two");
        }
        values.push_back(v);
    }
    return values;
}

Options parse_options(int argc, char** argv)
{
    Options o;
    for (int i = 1; i < argc; ++i) {
        const std::string flag = argv[i];
        if (flag == "--help" || flag == "-h") {
            std::fputs(kUsage, stdout);
            std::printf("our FFTs: %s\n", spx_impl_names());
            std::exit(0);
        }
        if (i + 1 >= argc) {
            throw FlagError(flag, "needs a value");
        }
        const std::string v = argv[++i];
        if (flag == "--op") {
            static const char* const ops[] = {
                "all",      "fft_c2c",     "fft_r2c",      "fft_c2r", "fft2_c2c", "fft2_r2c",
                "fft2_c2r", "rfft2_modes", "irfft2_modes", "scale",   "ns_step"};
            if (std::find(std::begin(ops), std::end(ops), v) == std::end(ops)) {
                throw FlagError(flag, "unknown operation '" + v + "'");
            }
            o.op = v;
        } else if (flag == "--impl") {
            o.impls.clear();
            if (v != "all") {
                for (const std::string& name : split_commas(v)) {
                    if (name != "rocfft" && name != "ours" && spx_impl_find(name.c_str()) < 0) {
                        throw FlagError(flag, "unknown implementation '" + name
                                                  + "' (our FFTs: " + spx_impl_names() + ")");
                    }
                    o.impls.push_back(name);
                }
            }
        } else if (flag == "--sizes") {
            o.sizes = to_counts(v, flag, true);
        } else if (flag == "--batches") {
            o.batches = to_counts(v, flag, false);
        } else if (flag == "--total") {
            o.total = to_count(v, flag, 1);
        } else if (flag == "--warmup") {
            o.warmup = static_cast<int>(std::min(to_count(v, flag, 0), 1LL << 20));
        } else if (flag == "--rounds") {
            o.rounds = static_cast<int>(std::min(to_count(v, flag, 1), 1LL << 20));
        } else if (flag == "--iters") {
            o.iters = static_cast<int>(std::min(to_count(v, flag, 1), 1LL << 20));
        } else if (flag == "--rotate") {
            o.rotate = static_cast<int>(std::min(to_count(v, flag, 1), 64LL));
        } else if (flag == "--copy-peak") {
            char* end = nullptr;
            o.copy_peak = std::strtod(v.c_str(), &end);
            if (v.empty() || end != v.c_str() + v.size() || !(o.copy_peak > 0)) {
                throw FlagError(flag, "'" + v + "' is not a positive rate in GB/s");
            }
        } else if (flag == "--out") {
            o.out = v;
        } else {
            throw FlagError(flag, "unknown option");
        }
    }
    if (o.sizes.empty()) {
        for (long long n = 2; n <= 4096; n *= 2) {
            o.sizes.push_back(n);
        }
    }
    return o;
}

// --- timing ---------------------------------------------------------------------------------

struct Timing {
    double median_ms = 0;
    double min_ms = 0;
    double max_ms = 0;
};

// launch(set, stream) queues one launch on buffer set `set`.
Timing time_launches(const std::function<void(int, hipStream_t)>& launch, hipStream_t stream,
                     const Options& o)
{
    int k = 0;
    for (int i = 0; i < o.warmup; ++i) {
        launch(k++ % o.rotate, stream);
    }
    hipEvent_t start, stop;
    hip_check(hipEventCreate(&start), "hipEventCreate");
    hip_check(hipEventCreate(&stop), "hipEventCreate");
    std::vector<double> per;
    for (int r = 0; r < o.rounds; ++r) {
        hip_check(hipEventRecord(start, stream), "hipEventRecord");
        for (int i = 0; i < o.iters; ++i) {
            launch(k++ % o.rotate, stream);
        }
        hip_check(hipEventRecord(stop, stream), "hipEventRecord");
        hip_check(hipEventSynchronize(stop), "hipEventSynchronize");
        float ms = 0;
        hip_check(hipEventElapsedTime(&ms, start, stop), "hipEventElapsedTime");
        per.push_back(ms / o.iters);
    }
    hip_check(hipGetLastError(), "launch");
    hip_check(hipEventDestroy(start), "hipEventDestroy");
    hip_check(hipEventDestroy(stop), "hipEventDestroy");
    std::sort(per.begin(), per.end());
    const std::size_t n = per.size();
    Timing t;
    t.min_ms = per.front();
    t.max_ms = per.back();
    t.median_ms = n % 2 ? per[n / 2] : 0.5 * (per[n / 2 - 1] + per[n / 2]);
    return t;
}

// --- work conventions (reference csrc/common/bench.cpp:93-135) -------------------------------

struct Work {
    double flops = 0;
    double bytes = 0;
};

Work c2c_work(double n, double batch)
{
    return {5.0 * n * batch * std::log2(n), 16.0 * n * batch};
}

Work real_work(double n, double batch)
{
    return {2.5 * n * batch * std::log2(n), batch * (4.0 * n + 8.0 * (n / 2.0 + 1.0))};
}

Work real2_work(double n1, double n2, double batch)
{
    const double p = n1 * n2;
    return {2.5 * p * batch * std::log2(p), batch * (4.0 * p + 8.0 * n1 * (n2 / 2.0 + 1.0))};
}

Work modes_work(double n1, double n2, double m1, double m2, double batch)
{
    Work w = real2_work(n1, n2, batch);
    w.bytes = batch * (4.0 * n1 * n2 + 16.0 * m1 * m2);
    return w;
}

// --- output ---------------------------------------------------------------------------------

int unstable_rows = 0;
double copy_peak_gbps = 0;  // the measured (or given) copy ceiling of pct_peak_measured

void write_row(std::ostream& os, const std::string& op, const std::string& impl, long long n,
               long long batch, const Timing& t, const Work& w, bool progress)
{
    const double gflops = w.flops / (t.median_ms * 1e6);
    const double gbps = w.bytes / (t.median_ms * 1e6);
    char line[384];
    std::snprintf(line, sizeof line, "%s,%s,%lld,%lld,%.6f,%.6f,%.6f,%.1f,%.1f,%.1f,%.1f\n",
                  op.c_str(), impl.c_str(), n, batch, t.median_ms, t.min_ms, t.max_ms, gflops,
                  gbps, 100.0 * gbps / kPeakGbps, 100.0 * gbps / copy_peak_gbps);
    os << line << std::flush;
    if (progress) {
        std::fprintf(stderr, "%-12s %-22s n=%-6lld batch=%-9lld %9.4f ms %8.1f GB/s %5.1f %%\n",
                     op.c_str(), impl.c_str(), n, batch, t.median_ms, gbps,
                     100.0 * gbps / kPeakGbps);
    }
    if (t.max_ms / t.min_ms - 1.0 > kUnstableSpread) {
        ++unstable_rows;
        std::fprintf(stderr, "warning: %s %s n=%lld: rounds differ by %.0f %%\n", op.c_str(),
                     impl.c_str(), n, 100.0 * (t.max_ms / t.min_ms - 1.0));
    }
}

void write_header(std::ostream& os, const Options& o, bool measured)
{
    int device = 0;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    hipDeviceProp_t prop{};
    hip_check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    int runtime = 0;
    int driver = 0;
    hip_check(hipRuntimeGetVersion(&runtime), "hipRuntimeGetVersion");
    hip_check(hipDriverGetVersion(&driver), "hipDriverGetVersion");
    int fftver = 0;
    fft_check(hipfftGetVersion(&fftver), "hipfftGetVersion");
    char peak[160];
    std::snprintf(peak, sizeof peak, "%.1f GB/s (%s)", copy_peak_gbps,
                  measured ? "spx_scale, 1 GiB -> 1 GiB, median of 5 rounds" : "--copy-peak");
    os << "# device: " << prop.name << " (" << prop.gcnArchName << "), "
       << prop.multiProcessorCount << " CUs\n"
       << "# HIP runtime " << runtime << ", driver " << driver << ", hipFFT " << fftver << '\n'
       << "# timing: " << o.warmup << " warm-up launches, then the median over " << o.rounds
       << " rounds of " << o.iters << " launches rotating over " << o.rotate
       << " buffer sets; times are per launch\n"
       << "# pct_peak_datasheet = gbps / 8000; pct_peak_measured = gbps / copy ceiling " << peak
       << '\n'
       << "op,impl,n,batch,time_ms,min_ms,max_ms,gflops,gbps,pct_peak_datasheet,"
          "pct_peak_measured\n";
}

// --- buffers --------------------------------------------------------------------------------

struct Buffers {
    std::vector<void*> x;  // inputs, random
    std::vector<void*> y;  // outputs
    std::size_t bytes = 0;

    // Every set holds the same standard-normal values: the caches see distinct addresses,
    // whatever the values.
    Buffers(int sets, std::size_t nbytes) : bytes(nbytes)
    {
        std::mt19937 gen(12345);
        std::normal_distribution<float> normal(0.0f, 1.0f);
        std::vector<float> host(nbytes / sizeof(float));
        for (float& v : host) {
            v = normal(gen);
        }
        for (int s = 0; s < sets; ++s) {
            void* a = nullptr;
            void* b = nullptr;
            hip_check(hipMalloc(&a, nbytes), "hipMalloc");
            x.push_back(a);
            hip_check(hipMalloc(&b, nbytes), "hipMalloc");
            y.push_back(b);
            hip_check(hipMemcpy(a, host.data(), nbytes, hipMemcpyHostToDevice), "hipMemcpy");
        }
    }
    ~Buffers()
    {
        for (void* p : x) {
            (void)hipFree(p);
        }
        for (void* p : y) {
            (void)hipFree(p);
        }
    }
    Buffers(const Buffers&) = delete;
    Buffers& operator=(const Buffers&) = delete;
};

struct Scratch {
    void* p = nullptr;
    explicit Scratch(std::size_t bytes)
    {
        if (bytes > 0) {
            hip_check(hipMalloc(&p, bytes), "hipMalloc");
        }
    }
    ~Scratch() { (void)hipFree(p); }
    Scratch(const Scratch&) = delete;
    Scratch& operator=(const Scratch&) = delete;
};

// The copy ceiling: spx_scale (one dwordx4 load and store per lane) streaming 1 GiB into another
// 1 GiB, 8 times the Infinity Cache, so each launch reads HBM. Bytes: both sides.
double measure_copy_peak(hipStream_t stream)
{
    constexpr std::size_t kValues = std::size_t(1) << 27;  // cf32: 1 GiB
    Scratch src(kValues * 8);
    Scratch dst(kValues * 8);
    hip_check(hipMemsetAsync(src.p, 0, kValues * 8, stream), "hipMemsetAsync");
    Options copy;
    copy.warmup = 2;
    copy.rounds = 5;
    copy.iters = 5;
    copy.rotate = 1;
    const Timing t = time_launches(
        [&](int, hipStream_t st) { spx_check(spx_scale(src.p, dst.p, kValues, 1.0f, st), "scale"); },
        stream, copy);
    return 2.0 * kValues * 8 / (t.median_ms * 1e6);
}

struct Plan {
    hipfftHandle h{};
    Plan(int rank, int* dims, int batch, hipfftType type)
    {
        fft_check(hipfftPlanMany(&h, rank, dims, nullptr, 1, 0, nullptr, 1, 0, type, batch),
                  "hipfftPlanMany");
    }
    ~Plan() { (void)hipfftDestroy(h); }
    Plan(const Plan&) = delete;
    Plan& operator=(const Plan&) = delete;
};

struct Case {
    long long n;
    long long batch;
};

std::vector<Case> cases(const Options& o, int dims)
{
    std::vector<Case> out;
    for (const long long n : o.sizes) {
        const long long points = dims == 1 ? n : n * n;
        if (o.batches.empty()) {
            if (points <= o.total) {
                out.push_back({n, o.total / points});
            }
            continue;
        }
        for (const long long b : o.batches) {
            if (points * b <= o.total) {
                out.push_back({n, b});
            }
        }
    }
    return out;
}

std::vector<int> our_impls(const Options& o)
{
    std::vector<int> out;
    for (int i = 0; i < spx_impl_count(); ++i) {
        if (o.wants(spx_impl_name(i))) {
            out.push_back(i);
        }
    }
    return out;
}

// --- the benchmarks -------------------------------------------------------------------------

void bench_c2c(const Options& o, Buffers& b, hipStream_t s, std::ostream& os, bool progress)
{
    for (const Case& c : cases(o, 1)) {
        const int n = static_cast<int>(c.n);
        const int batch = static_cast<int>(c.batch);
        const Work w = c2c_work(c.n, c.batch);
        if (o.wants("rocfft")) {
            Plan plan(1, const_cast<int*>(&n), batch, HIPFFT_C2C);
            fft_check(hipfftSetStream(plan.h, s), "hipfftSetStream");
            const Timing t = time_launches(
                [&](int k, hipStream_t) {
                    fft_check(hipfftExecC2C(plan.h, static_cast<hipfftComplex*>(b.x[k]),
                                            static_cast<hipfftComplex*>(b.y[k]), HIPFFT_FORWARD),
                              "hipfftExecC2C");
                },
                s, o);
            write_row(os, "fft_c2c", "rocfft", c.n, c.batch, t, w, progress);
        }
        for (const int impl : our_impls(o)) {
            spx_impl_info info{};
            spx_impl_get_info(impl, &info);
            if (c.n > info.max_c2c_n) {
                continue;
            }
            const Timing t = time_launches(
                [&](int k, hipStream_t st) {
                    spx_check(spx_c2c(impl, b.x[k], b.y[k], n, batch, 0, st), "spx_c2c");
                },
                s, o);
            write_row(os, "fft_c2c", info.name, c.n, c.batch, t, w, progress);
        }
    }
}

void bench_real(const Options& o, const std::string& op, Buffers& b, hipStream_t s,
                std::ostream& os, bool progress)
{
    const bool forward = op == "fft_r2c";
    for (const Case& c : cases(o, 1)) {
        if (c.n < 2) {
            continue;
        }
        const int n = static_cast<int>(c.n);
        const int batch = static_cast<int>(c.batch);
        const Work w = real_work(c.n, c.batch);
        if (o.wants("rocfft")) {
            Plan plan(1, const_cast<int*>(&n), batch, forward ? HIPFFT_R2C : HIPFFT_C2R);
            fft_check(hipfftSetStream(plan.h, s), "hipfftSetStream");
            const Timing t = time_launches(
                [&](int k, hipStream_t) {
                    if (forward) {
                        fft_check(hipfftExecR2C(plan.h, static_cast<hipfftReal*>(b.x[k]),
                                                static_cast<hipfftComplex*>(b.y[k])),
                                  "hipfftExecR2C");
                    } else {
                        fft_check(hipfftExecC2R(plan.h, static_cast<hipfftComplex*>(b.x[k]),
                                                static_cast<hipfftReal*>(b.y[k])),
                                  "hipfftExecC2R");
                    }
                },
                s, o);
            write_row(os, op, "rocfft", c.n, c.batch, t, w, progress);
        }
        for (const int impl : our_impls(o)) {
            spx_impl_info info{};
            spx_impl_get_info(impl, &info);
            if (c.n > info.max_real_n) {
                continue;
            }
            Scratch work(info.real_needs_work
                             ? static_cast<std::size_t>(c.batch) * (c.n / 2) * 8
                             : 0);
            const Timing t = time_launches(
                [&](int k, hipStream_t st) {
                    if (forward) {
                        spx_check(spx_r2c(impl, static_cast<const float*>(b.x[k]), b.y[k], n,
                                          batch, work.p, st),
                                  "spx_r2c");
                    } else {
                        spx_check(spx_c2r(impl, b.x[k], static_cast<float*>(b.y[k]), n, batch,
                                          work.p, st),
                                  "spx_c2r");
                    }
                },
                s, o);
            write_row(os, op, info.name, c.n, c.batch, t, w, progress);
        }
    }
}

void bench_fft2(const Options& o, const std::string& op, Buffers& b, hipStream_t s,
                std::ostream& os, bool progress)
{
    const bool c2c = op == "fft2_c2c";
    const bool r2c = op == "fft2_r2c";
    for (const Case& c : cases(o, 2)) {
        if (!c2c && c.n < 2) {
            continue;
        }
        const int n = static_cast<int>(c.n);
        const int batch = static_cast<int>(c.batch);
        const Work w = c2c ? c2c_work(c.n * c.n, c.batch) : real2_work(c.n, c.n, c.batch);
        if (o.wants("rocfft")) {
            int dims[2] = {n, n};
            Plan plan(2, dims, batch, c2c ? HIPFFT_C2C : (r2c ? HIPFFT_R2C : HIPFFT_C2R));
            fft_check(hipfftSetStream(plan.h, s), "hipfftSetStream");
            const Timing t = time_launches(
                [&](int k, hipStream_t) {
                    auto* xc = static_cast<hipfftComplex*>(b.x[k]);
                    if (c2c) {
                        fft_check(hipfftExecC2C(plan.h, xc, static_cast<hipfftComplex*>(b.y[k]),
                                                HIPFFT_FORWARD),
                                  "hipfftExecC2C");
                    } else if (r2c) {
                        fft_check(hipfftExecR2C(plan.h, static_cast<hipfftReal*>(b.x[k]),
                                                static_cast<hipfftComplex*>(b.y[k])),
                                  "hipfftExecR2C");
                    } else {
                        fft_check(hipfftExecC2R(plan.h, xc, static_cast<hipfftReal*>(b.y[k])),
                                  "hipfftExecC2R");
                    }
                },
                s, o);
            write_row(os, op, "rocfft", c.n, c.batch, t, w, progress);
        }
        for (const int impl : our_impls(o)) {
            spx_impl_info info{};
            spx_impl_get_info(impl, &info);
            if (c.n > info.max_n || (!c2c && c.n > info.max_real_n)) {
                continue;
            }
            for (const int method : {SPX_COLUMNS_STRIDED, SPX_COLUMNS_TRANSPOSE}) {
                if (method == SPX_COLUMNS_STRIDED && !info.has_columns) {
                    continue;
                }
                std::size_t need = 0;
                if (c2c) {
                    spx_check(spx_fft2_c2c_workspace(impl, method, n, n, batch, &need), "ws");
                } else if (r2c) {
                    spx_check(spx_fft2_r2c_workspace(impl, method, n, n, batch, &need), "ws");
                } else {
                    spx_check(spx_fft2_c2r_workspace(impl, method, n, n, batch, &need), "ws");
                }
                Scratch work(need * 8);
                const Timing t = time_launches(
                    [&](int k, hipStream_t st) {
                        if (c2c) {
                            spx_check(spx_fft2_c2c(impl, method, b.x[k], b.y[k], n, n, batch, 0,
                                                   work.p, st),
                                      "spx_fft2_c2c");
                        } else if (r2c) {
                            spx_check(spx_fft2_r2c(impl, method, static_cast<const float*>(b.x[k]),
                                                   b.y[k], n, n, batch, work.p, st),
                                      "spx_fft2_r2c");
                        } else {
                            spx_check(spx_fft2_c2r(impl, method, b.x[k],
                                                   static_cast<float*>(b.y[k]), n, n, batch,
                                                   work.p, st),
                                      "spx_fft2_c2r");
                        }
                    },
                    s, o);
                const std::string label = std::string(info.name)
                                          + (method == SPX_COLUMNS_STRIDED ? "/strided"
                                                                           : "/transpose");
                write_row(os, op, label, c.n, c.batch, t, w, progress);
            }
        }
    }
}

void bench_modes(const Options& o, const std::string& op, Buffers& b, hipStream_t s,
                 std::ostream& os, bool progress)
{
    const bool forward = op == "rfft2_modes";
    for (const Case& c : cases(o, 2)) {
        if (c.n < 2) {
            continue;
        }
        const int n = static_cast<int>(c.n);
        const int m = static_cast<int>(std::max(1LL, c.n / 8));
        const int batch = static_cast<int>(c.batch);
        const Work w = modes_work(c.n, c.n, m, m, c.batch);
        if (o.wants("rocfft")) {
            int dims[2] = {n, n};
            Plan plan(2, dims, batch, forward ? HIPFFT_R2C : HIPFFT_C2R);
            fft_check(hipfftSetStream(plan.h, s), "hipfftSetStream");
            const int half = n / 2 + 1;
            Scratch full(static_cast<std::size_t>(batch) * n * half * 8);
            const Timing t = time_launches(
                [&](int k, hipStream_t st) {
                    auto* f = static_cast<hipfftComplex*>(full.p);
                    if (forward) {
                        fft_check(hipfftExecR2C(plan.h, static_cast<hipfftReal*>(b.x[k]), f),
                                  "hipfftExecR2C");
                        spx_check(spx_gather_modes(full.p, b.y[k], n, half, m, m, batch, st),
                                  "spx_gather_modes");
                    } else {
                        spx_check(spx_scatter_modes(b.x[k], full.p, n, half, m, m, batch, st),
                                  "spx_scatter_modes");
                        fft_check(hipfftExecC2R(plan.h, f, static_cast<hipfftReal*>(b.y[k])),
                                  "hipfftExecC2R");
                    }
                },
                s, o);
            write_row(os, op, forward ? "rocfft+gather" : "rocfft+scatter", c.n, c.batch, t, w,
                      progress);
        }
        for (const int impl : our_impls(o)) {
            spx_impl_info info{};
            spx_impl_get_info(impl, &info);
            if (c.n > info.max_n) {
                continue;
            }
            std::size_t need = 0;
            if (forward) {
                spx_check(spx_rfft2_modes_workspace(impl, n, n, m, m, batch, &need), "ws");
            } else {
                spx_check(spx_irfft2_modes_workspace(impl, n, n, m, m, batch, &need), "ws");
            }
            Scratch work(need * 8);
            const Timing t = time_launches(
                [&](int k, hipStream_t st) {
                    if (forward) {
                        spx_check(spx_rfft2_modes(impl, static_cast<const float*>(b.x[k]), b.y[k],
                                                  n, n, m, m, batch, work.p, st),
                                  "spx_rfft2_modes");
                    } else {
                        spx_check(spx_irfft2_modes(impl, b.x[k], static_cast<float*>(b.y[k]), n,
                                                   n, m, m, batch, work.p, st),
                                  "spx_irfft2_modes");
                    }
                },
                s, o);
            write_row(os, op, info.name, c.n, c.batch, t, w, progress);
        }
    }
}

// One IMEX step of the fused Navier-Stokes solver, the predictor and the corrector launch of
// spx_ns_stage, on batch fields of n x n grids in the pruned layout (m = n/3 + 1 kept modes per
// axis; n with a kernel only). Work per step: the nominal flops of the transforms the composed
// solver runs (per stage four inverse and one forward real 2D transform, 2.5 n^2 log2 n^2 each)
// and the HBM bytes of the mode arrays (stage 0 reads the state and writes the tendency and the
// predictor; stage 1 reads the predictor, the state and the tendency and writes the new state;
// the forcing modes once per stage).
void bench_ns(const Options& o, Buffers& b, hipStream_t s, std::ostream& os, bool progress)
{
    for (const Case& c : cases(o, 2)) {
        if (c.n > 4096 || spx_ns_supports(static_cast<int>(c.n)) != 1) {
            continue;
        }
        const int n = static_cast<int>(c.n);
        const int batch = static_cast<int>(c.batch);
        const std::size_t m = static_cast<std::size_t>(n / 3 + 1);
        const std::size_t field = 2 * m * m * 8;  // bytes of one field's modes
        if (3 * field * c.batch > b.bytes) {
            continue;  // the output buffer holds the tendency, the predictor and the new state
        }
        Scratch forcing(field);
        hip_check(hipMemset(forcing.p, 0, field), "hipMemset");
        Scratch nu(static_cast<std::size_t>(batch) * sizeof(float));
        const std::vector<float> nu_host(static_cast<std::size_t>(batch), 2e-3f);
        hip_check(hipMemcpy(nu.p, nu_host.data(), nu_host.size() * sizeof(float),
                            hipMemcpyHostToDevice),
                  "hipMemcpy");
        const double points = static_cast<double>(n) * n;
        const Work w{2.0 * 5.0 * 2.5 * points * std::log2(points) * c.batch,
                     (7.0 * c.batch + 2.0) * static_cast<double>(field)};
        const auto* viscosity = static_cast<const float*>(nu.p);
        const Timing t = time_launches(
            [&](int k, hipStream_t st) {
                char* const y = static_cast<char*>(b.y[k]);
                void* const f = y;
                void* const p = y + field * c.batch;
                void* const out = y + 2 * field * c.batch;
                spx_check(spx_ns_stage(b.x[k], nullptr, nullptr, f, p, forcing.p, viscosity, 1,
                                       0.1f, 2.5e-3f, n, batch, 0, st),
                          "spx_ns_stage");
                spx_check(spx_ns_stage(p, b.x[k], f, nullptr, out, forcing.p, viscosity, 1,
                                       0.1f, 2.5e-3f, n, batch, 1, st),
                          "spx_ns_stage");
            },
            s, o);
        write_row(os, "ns_step", "ours", c.n, c.batch, t, w, progress);

        // The same steps kStepsPerLaunch to a launch (spx_ns_steps): one row per launch.
        constexpr int kStepsPerLaunch = 40;
        const Work w_many{w.flops * kStepsPerLaunch, w.bytes * kStepsPerLaunch};
        const Timing t_many = time_launches(
            [&](int k, hipStream_t st) {
                char* const y = static_cast<char*>(b.y[k]);
                void* const work = y;
                void* const out = y + 2 * field * c.batch;
                spx_check(spx_ns_steps(b.x[k], out, work, forcing.p, viscosity, 1, 0.1f, 2.5e-3f,
                                       n, batch, kStepsPerLaunch, st),
                          "spx_ns_steps");
            },
            s, o);
        write_row(os, "ns_steps40", "ours", c.n, c.batch, t_many, w_many, progress);
    }
}

void bench_scale(const Options& o, Buffers& b, hipStream_t s, std::ostream& os, bool progress)
{
    const auto n = static_cast<std::size_t>(o.total);
    const Timing t = time_launches(
        [&](int k, hipStream_t st) { spx_check(spx_scale(b.x[k], b.y[k], n, 0.5f, st), "scale"); },
        s, o);
    write_row(os, "scale", "ours", o.total, 1, t, {2.0 * n, 16.0 * n}, progress);
}

}  // namespace

int main(int argc, char** argv)
{
    try {
        const Options o = parse_options(argc, argv);
        long long capacity = o.total;
        for (const long long n : o.sizes) {
            capacity = std::max(capacity, n);
        }
        // Complex64 values per buffer: every op's input and output fit (real sides are smaller).
        Buffers buffers(o.rotate, static_cast<std::size_t>(capacity) * 8);
        hipStream_t stream = nullptr;
        hip_check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");

        std::ofstream file;
        if (!o.out.empty()) {
            file.open(o.out);
            if (!file) {
                throw std::runtime_error("cannot open " + o.out + " for writing");
            }
        }
        std::ostream& os = o.out.empty() ? std::cout : file;
        const bool progress = !o.out.empty();
        copy_peak_gbps = o.copy_peak > 0 ? o.copy_peak : measure_copy_peak(stream);
        write_header(os, o, !(o.copy_peak > 0));
        auto want = [&](const char* op) { return o.op == "all" || o.op == op; };
        if (want("fft_c2c")) {
            bench_c2c(o, buffers, stream, os, progress);
        }
        for (const char* op : {"fft_r2c", "fft_c2r"}) {
            if (want(op)) {
                bench_real(o, op, buffers, stream, os, progress);
            }
        }
        for (const char* op : {"fft2_c2c", "fft2_r2c", "fft2_c2r"}) {
            if (want(op)) {
                bench_fft2(o, op, buffers, stream, os, progress);
            }
        }
        for (const char* op : {"rfft2_modes", "irfft2_modes"}) {
            if (want(op)) {
                bench_modes(o, op, buffers, stream, os, progress);
            }
        }
        if (want("scale") && o.wants("ours")) {
            bench_scale(o, buffers, stream, os, progress);
        }
        if (want("ns_step") && o.wants("ours")) {
            bench_ns(o, buffers, stream, os, progress);
        }
        hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
        hip_check(hipStreamDestroy(stream), "hipStreamDestroy");
        if (unstable_rows > 0) {
            std::fprintf(stderr, "warning: %d unstable row(s)\n", unstable_rows);
        }
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
}
