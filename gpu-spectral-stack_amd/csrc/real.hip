// Argument checks shared by the variants, the twiddle table, and the real-FFT combine / prepare
// as stand-alone passes: for n = 2 (m = 1, where the complex transform is the identity) and for
// the generic path around any complex implementation (naive), which costs one extra HBM pass.
//
// Reference: real.cu:29-216 (the same formulas, evaluated here per conjugate pair so one twiddle
// serves bins k and m - k), twiddles.cu:17-46, stockham.cuh:489-583.

#include "stockham.hpp"
#include "variant.hpp"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

namespace spx {

void check_size(int n, const char* who)
{
    if (n < 1 || n > kStockhamMaxN || !is_pow2(n)) {
        throw InvalidArgument(std::string(who) + ": n must be a power of two from 1 to "
                              + str(kStockhamMaxN) + ", got " + str(n));
    }
}

void check_keep(int keep, int n, const char* who)
{
    if (keep < 1 || keep > n / 2 + 1) {
        throw InvalidArgument(std::string(who) + ": keep must be in [1, n/2 + 1 = "
                              + str(n / 2 + 1) + "], got " + str(keep));
    }
}

void check_real_arguments(const void* real_side, const void* complex_side, int n, int batch,
                          int complex_row, int max_n, const char* who)
{
    const std::string name(who);
    if (n < 2 || n > max_n || !is_pow2(n)) {
        throw InvalidArgument(name + ": n must be a power of two from 2 to " + str(max_n)
                              + ", got " + str(n));
    }
    if (batch < 1) {
        throw InvalidArgument(name + ": batch must be at least 1, got " + str(batch));
    }
    const auto rows = static_cast<std::size_t>(batch);
    const auto* r = static_cast<const char*>(real_side);
    const auto* c = static_cast<const char*>(complex_side);
    const std::size_t real_bytes = rows * static_cast<std::size_t>(n) * sizeof(float);
    const std::size_t complex_bytes = rows * static_cast<std::size_t>(complex_row) * sizeof(cf32);
    if (r < c + complex_bytes && c < r + real_bytes) {
        throw InvalidArgument(name + ": input and output must not overlap");
    }
}

const cf32* twiddle_table()
{
    static std::mutex mutex;
    static std::vector<cf32*> tables;  // per device, kept until the process exits

    int device = 0;
    SPX_HIP_CHECK(hipGetDevice(&device));
    const std::lock_guard<std::mutex> lock(mutex);
    if (tables.size() <= static_cast<std::size_t>(device)) {
        tables.resize(static_cast<std::size_t>(device) + 1, nullptr);
    }
    cf32*& table = tables[static_cast<std::size_t>(device)];
    if (table == nullptr) {
        std::vector<cf32> host(dev::kTableN);
        for (int m = 0; m < dev::kTableN; ++m) {
            // exp(-2 pi i m / N) in double, rounded once; sin/cos of pi * (2m/N) by octant would
            // not change the float result.
            const double a = -2.0 * M_PI * static_cast<double>(m) / dev::kTableN;
            host[static_cast<std::size_t>(m)] =
                cf32{static_cast<float>(std::cos(a)), static_cast<float>(std::sin(a))};
        }
        cf32* device_table = nullptr;
        SPX_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&device_table),
                                host.size() * sizeof(cf32)));
        // Synchronous, so the table is complete before any kernel reads it.
        SPX_HIP_CHECK(hipMemcpy(device_table, host.data(), host.size() * sizeof(cf32),
                                hipMemcpyHostToDevice));
        table = device_table;
    }
    return table;
}

namespace {

constexpr int kThreads = 256;

unsigned grid_for(std::size_t work)
{
    const std::size_t blocks = (work + kThreads - 1) / kThreads;
    return static_cast<unsigned>(std::min<std::size_t>(std::max<std::size_t>(blocks, 1), 65536));
}

// One lane per conjugate pair (k, m-k), k = 0 .. m/2, of each row: X[k] and X[m-k] from Z.
__global__ void __launch_bounds__(kThreads)
    r2c_post_kernel(const cf32* __restrict__ z, cf32* __restrict__ y, int m, int keep,
                    std::size_t pairs_total)
{
    using namespace dev;
    const int pairs = m / 2 + 1;
    for (std::size_t e = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x;
         e < pairs_total; e += static_cast<std::size_t>(gridDim.x) * kThreads) {
        const std::size_t t = e / static_cast<std::size_t>(pairs);
        const int k = static_cast<int>(e - t * pairs);
        const cf32* row = z + t * m;
        const cf32 zk = row[k & (m - 1)];
        const cf32 zm = row[(m - k) & (m - 1)];
        const cf32 ev{0.5f * (zk.re + zm.re), 0.5f * (zk.im - zm.im)};
        const cf32 od{0.5f * (zk.im + zm.im), -0.5f * (zk.re - zm.re)};
        const cf32 wo = cmul(cconj(expi_pi(static_cast<float>(k) / static_cast<float>(m))), od);
        cf32* out = y + t * keep;
        if (k < keep) {
            out[k] = cadd(ev, wo);
        }
        if (k < m - k && m - k < keep) {
            out[m - k] = cconj(csub(ev, wo));
        }
    }
}

// One lane per pair: Z[k] and Z[m-k] from X[k] and X[m-k] (rows of keep values, rest zero).
__global__ void __launch_bounds__(kThreads)
    c2r_pre_kernel(const cf32* __restrict__ x, cf32* __restrict__ z, int m, int keep,
                   std::size_t pairs_total)
{
    using namespace dev;
    const int pairs = m / 2 + 1;
    for (std::size_t e = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x;
         e < pairs_total; e += static_cast<std::size_t>(gridDim.x) * kThreads) {
        const std::size_t t = e / static_cast<std::size_t>(pairs);
        const int k = static_cast<int>(e - t * pairs);
        const cf32* row = x + t * keep;
        cf32 xk = k < keep ? row[k] : czero();
        cf32 xm = m - k < keep ? row[m - k] : czero();
        if (k == 0) {
            xk.im = 0.0f;
            xm.im = 0.0f;
        }
        const cf32 ev{0.5f * (xk.re + xm.re), 0.5f * (xk.im - xm.im)};
        const cf32 d{0.5f * (xk.re - xm.re), 0.5f * (xk.im + xm.im)};
        const cf32 od = cmul(d, expi_pi(static_cast<float>(k) / static_cast<float>(m)));
        const cf32 iod{-od.im, od.re};
        cf32* out = z + t * m;
        if (k < m) {
            out[k] = cadd(ev, iod);
        }
        if (k > 0 && k < m - k) {
            out[m - k] = cconj(csub(ev, iod));
        }
    }
}

}  // namespace

void r2c_postprocess(const cf32* z, cf32* y, int m, int batch, int keep, hipStream_t stream)
{
    const std::size_t total = static_cast<std::size_t>(batch) * (m / 2 + 1);
    hipLaunchKernelGGL(r2c_post_kernel, dim3(grid_for(total)), dim3(kThreads), 0, stream, z, y, m,
                       keep, total);
    SPX_LAUNCH_CHECK();
}

void c2r_preprocess(const cf32* x, cf32* z, int m, int batch, int keep, hipStream_t stream)
{
    const std::size_t total = static_cast<std::size_t>(batch) * (m / 2 + 1);
    hipLaunchKernelGGL(c2r_pre_kernel, dim3(grid_for(total)), dim3(kThreads), 0, stream, x, z, m,
                       keep, total);
    SPX_LAUNCH_CHECK();
}

void r2c_via_c2c(C2cFn c2c, const float* x, cf32* y, int n, int batch, cf32* work,
                 hipStream_t stream)
{
    check_real_arguments(x, y, n, batch, n / 2 + 1, 1 << 30, "r2c");
    if (work == nullptr) {
        throw InvalidArgument("r2c: this implementation needs a workspace");
    }
    const int m = n / 2;
    c2c(reinterpret_cast<const cf32*>(x), work, m, batch, Direction::Forward, stream);
    r2c_postprocess(work, y, m, batch, m + 1, stream);
}

void c2r_via_c2c(C2cFn c2c, const cf32* x, float* y, int n, int batch, cf32* work,
                 hipStream_t stream)
{
    check_real_arguments(y, x, n, batch, n / 2 + 1, 1 << 30, "c2r");
    if (work == nullptr) {
        throw InvalidArgument("c2r: this implementation needs a workspace");
    }
    const int m = n / 2;
    c2r_preprocess(x, work, m, batch, m + 1, stream);
    c2c(work, reinterpret_cast<cf32*>(y), m, batch, Direction::Inverse, stream);
}

void r2c_naive(const float* x, cf32* y, int n, int batch, cf32* work, hipStream_t stream)
{
    r2c_via_c2c(&c2c_naive, x, y, n, batch, work, stream);
}

void c2r_naive(const cf32* x, float* y, int n, int batch, cf32* work, hipStream_t stream)
{
    c2r_via_c2c(&c2c_naive, x, y, n, batch, work, stream);
}

}  // namespace spx
