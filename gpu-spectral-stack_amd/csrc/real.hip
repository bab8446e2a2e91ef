// Argument checks shared by the variants, the twiddle table, and the real-FFT combine / prepare
// as stand-alone passes: for n = 2 (m = 1, where the complex transform is the identity) and for
// the generic path around any complex implementation (naive), which costs one extra HBM pass.
//
// Reference: real.cu:29-216 (the same formulas, evaluated here per conjugate pair so one twiddle
// serves bins k and m - k), twiddles.cu:17-46, stockham.cuh:489-583.

#include "stockham.hpp"
#include "variant.hpp"

#include <algorithm>
#include <cstdint>
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

bool pool_retained()
{
    // Decided once per device: 1 retained, 2 no memory pools.
    static std::mutex mutex;
    static std::vector<unsigned char> state;

    int device = 0;
    SPX_HIP_CHECK(hipGetDevice(&device));
    const std::lock_guard<std::mutex> lock(mutex);
    if (state.size() <= static_cast<std::size_t>(device)) {
        state.resize(static_cast<std::size_t>(device) + 1, 0);
    }
    unsigned char& s = state[static_cast<std::size_t>(device)];
    if (s == 0) {
        int pools = 0;
        SPX_HIP_CHECK(hipDeviceGetAttribute(&pools, hipDeviceAttributeMemoryPoolsSupported,
                                            device));
        if (pools != 0) {
            hipMemPool_t pool = nullptr;
            SPX_HIP_CHECK(hipDeviceGetDefaultMemPool(&pool, device));
            std::uint64_t keep_everything = UINT64_MAX;
            SPX_HIP_CHECK(
                hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep_everything));
        }
        s = pools != 0 ? 1 : 2;
    }
    return s == 1;
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

// n = 2 (m = 1), one row per lane: X[0] = x0 + x1 and X[1] = x0 - x1 (both real), from one 8-byte
// load to one 16-byte store (8 bytes when keep = 1). The grid covers the rows once, so every lane
// moves exactly one row, the pattern that streams best.
using f2v = float __attribute__((ext_vector_type(2)));
using f4v = float __attribute__((ext_vector_type(4)));

template <bool Vec>
__global__ void __launch_bounds__(kThreads)
    r2c_n2_kernel(const f2v* __restrict__ x, cf32* __restrict__ y, int keep, std::size_t rows)
{
    const std::size_t row = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x;
    if (row >= rows) {
        return;
    }
    const f2v v = x[row];
    const float x0 = v.x + v.y;
    const float x1 = v.x - v.y;
    if (keep == 2) {
        if constexpr (Vec) {
            __builtin_nontemporal_store(f4v{x0, 0.0f, x1, 0.0f}, reinterpret_cast<f4v*>(y) + row);
        } else {
            __builtin_nontemporal_store(f2v{x0, 0.0f}, reinterpret_cast<f2v*>(y + 2 * row));
            __builtin_nontemporal_store(f2v{x1, 0.0f}, reinterpret_cast<f2v*>(y + 2 * row + 1));
        }
    } else {
        __builtin_nontemporal_store(f2v{x0, 0.0f}, reinterpret_cast<f2v*>(y + row));
    }
}

// The inverse for n = 2: y0 = (X[0] + X[1]) / 2, y1 = (X[0] - X[1]) / 2, real parts only (the
// imaginary parts of the DC and Nyquist bins are ignored; X[1] = 0 when keep = 1).
template <bool Vec>
__global__ void __launch_bounds__(kThreads)
    c2r_n2_kernel(const cf32* __restrict__ x, f2v* __restrict__ y, int keep, std::size_t rows)
{
    const std::size_t row = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x;
    if (row >= rows) {
        return;
    }
    float a = 0.0f;
    float b = 0.0f;
    if (keep == 2) {
        if constexpr (Vec) {
            const f4v v = reinterpret_cast<const f4v*>(x)[row];
            a = v.x;
            b = v.z;
        } else {
            a = x[2 * row].re;
            b = x[2 * row + 1].re;
        }
    } else {
        a = x[row].re;
    }
    __builtin_nontemporal_store(f2v{0.5f * (a + b), 0.5f * (a - b)}, y + row);
}

// The inverse for n = 4, one row per lane: from X[0], X[1] = p + iq, X[2] (the rest zero beyond
// keep; imaginary parts of X[0] and X[2] ignored), y[t] = (X0 + 2 Re(X1 i^t) + (-1)^t X2) / 4:
//   y0 = (a + 2p + c) / 4,  y1 = (a - 2q - c) / 4,  y2 = (a - 2p + c) / 4,  y3 = (a + 2q - c) / 4.
__global__ void __launch_bounds__(kThreads)
    c2r_n4_kernel(const cf32* __restrict__ x, f4v* __restrict__ y, int keep, std::size_t rows)
{
    const std::size_t row = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x;
    if (row >= rows) {
        return;
    }
    const cf32* in = x + row * static_cast<std::size_t>(keep);
    const float a = in[0].re;
    const cf32 x1 = keep > 1 ? in[1] : cf32{0.0f, 0.0f};
    const float c = keep > 2 ? in[2].re : 0.0f;
    const float ac = a + c;
    const float amc = a - c;
    const float p2 = 2.0f * x1.re;
    const float q2 = 2.0f * x1.im;
    __builtin_nontemporal_store(
        f4v{0.25f * (ac + p2), 0.25f * (amc - q2), 0.25f * (ac - p2), 0.25f * (amc + q2)},
        y + row);
}

// Full-width n = 2 and n = 4 inverses staged through LDS, so every global access is a 16-byte
// vector at unit stride across the lanes: rows of 2 complex (n = 2) or 3 complex (n = 4) values
// are read flat as float4s, each lane then takes its rows from LDS. The per-row kernels above
// store 8 bytes per lane (n = 2) or load three strided 8-byte values per lane (n = 4); measured
// 70.5 % and 68.8 % of peak at 2^24 points.
constexpr int kStagedRows2 = 2 * kThreads;  // n = 2: two rows per lane, one float4 out
constexpr int kStagedRows4 = kThreads;      // n = 4: one row per lane, one float4 out

__global__ void __launch_bounds__(kThreads)
    c2r_n2_staged_kernel(const f4v* __restrict__ x, f4v* __restrict__ y, std::size_t rows)
{
    __shared__ f4v lds[kStagedRows2];
    const std::size_t first = blockIdx.x * static_cast<std::size_t>(kStagedRows2);
    const int tid = threadIdx.x;
    const std::size_t left = rows - first;
    const int count = left < kStagedRows2 ? static_cast<int>(left) : kStagedRows2;
    f4v v[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int r = tid + k * kThreads;
        v[k] = r < count ? __builtin_nontemporal_load(x + first + r) : f4v{};
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        lds[tid + k * kThreads] = v[k];
    }
    __syncthreads();
    const int r = 2 * tid;
    if (r < count) {
        const f4v p = lds[r];
        const f4v q = lds[r + 1];  // beyond count: unused
        const f4v out{0.5f * (p.x + p.z), 0.5f * (p.x - p.z), 0.5f * (q.x + q.z),
                      0.5f * (q.x - q.z)};
        if (r + 1 < count) {
            __builtin_nontemporal_store(out, y + (first + r) / 2);
        } else {
            __builtin_nontemporal_store(f2v{out.x, out.y},
                                        reinterpret_cast<f2v*>(y) + first + r);
        }
    }
}

__global__ void __launch_bounds__(kThreads)
    c2r_n4_staged_kernel(const float* __restrict__ x, f4v* __restrict__ y, std::size_t rows)
{
    constexpr int kFloats = 6 * kStagedRows4;  // 3 complex values per row
    __shared__ float lds[kFloats];
    const std::size_t first = blockIdx.x * static_cast<std::size_t>(kStagedRows4);
    const int tid = threadIdx.x;
    const std::size_t left = rows - first;
    const int count = left < kStagedRows4 ? static_cast<int>(left) : kStagedRows4;
    const float* src = x + first * 6;
    if (count == kStagedRows4) {
        const f4v* src4 = reinterpret_cast<const f4v*>(src);  // 6 kThreads floats, 16-byte aligned
        f4v v[kFloats / 4 / kThreads + 1];
#pragma unroll
        for (int k = 0; k * kThreads < kFloats / 4; ++k) {
            const int i = tid + k * kThreads;
            v[k] = i < kFloats / 4 ? __builtin_nontemporal_load(src4 + i) : f4v{};
        }
#pragma unroll
        for (int k = 0; k * kThreads < kFloats / 4; ++k) {
            const int i = tid + k * kThreads;
            if (i < kFloats / 4) {
                reinterpret_cast<f4v*>(lds)[i] = v[k];
            }
        }
    } else {
        for (int i = tid; i < 6 * count; i += kThreads) {
            lds[i] = src[i];
        }
    }
    __syncthreads();
    if (tid < count) {
        const float* in = lds + 6 * tid;
        const float ac = in[0] + in[4];
        const float amc = in[0] - in[4];
        const float p2 = 2.0f * in[2];
        const float q2 = 2.0f * in[3];
        __builtin_nontemporal_store(
            f4v{0.25f * (ac + p2), 0.25f * (amc - q2), 0.25f * (ac - p2), 0.25f * (amc + q2)},
            y + first + tid);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15) == 0; }

}  // namespace

void r2c_n2(const float* x, cf32* y, int batch, int keep, hipStream_t stream)
{
    const auto rows = static_cast<std::size_t>(batch);
    const dim3 grid(static_cast<unsigned>((rows + kThreads - 1) / kThreads));
    const auto* xv = reinterpret_cast<const f2v*>(x);
    if (aligned16(y)) {
        hipLaunchKernelGGL(r2c_n2_kernel<true>, grid, dim3(kThreads), 0, stream, xv, y, keep, rows);
    } else {
        hipLaunchKernelGGL(r2c_n2_kernel<false>, grid, dim3(kThreads), 0, stream, xv, y, keep,
                           rows);
    }
    SPX_LAUNCH_CHECK();
}

void c2r_n2(const cf32* x, float* y, int batch, int keep, hipStream_t stream)
{
    const auto rows = static_cast<std::size_t>(batch);
    const dim3 grid(static_cast<unsigned>((rows + kThreads - 1) / kThreads));
    auto* yv = reinterpret_cast<f2v*>(y);
    if (keep == 2 && aligned16(x) && aligned16(y)) {
        const dim3 staged(static_cast<unsigned>((rows + kStagedRows2 - 1) / kStagedRows2));
        hipLaunchKernelGGL(c2r_n2_staged_kernel, staged, dim3(kThreads), 0, stream,
                           reinterpret_cast<const f4v*>(x), reinterpret_cast<f4v*>(y), rows);
        SPX_LAUNCH_CHECK();
        return;
    }
    if (aligned16(x)) {
        hipLaunchKernelGGL(c2r_n2_kernel<true>, grid, dim3(kThreads), 0, stream, x, yv, keep, rows);
    } else {
        hipLaunchKernelGGL(c2r_n2_kernel<false>, grid, dim3(kThreads), 0, stream, x, yv, keep,
                           rows);
    }
    SPX_LAUNCH_CHECK();
}

bool c2r_n4(const cf32* x, float* y, int batch, int keep, hipStream_t stream)
{
    if (!aligned16(y)) {
        return false;  // the caller runs the general kernel instead
    }
    const auto rows = static_cast<std::size_t>(batch);
    if (keep == 3 && aligned16(x)) {
        const dim3 staged(static_cast<unsigned>((rows + kStagedRows4 - 1) / kStagedRows4));
        hipLaunchKernelGGL(c2r_n4_staged_kernel, staged, dim3(kThreads), 0, stream,
                           reinterpret_cast<const float*>(x), reinterpret_cast<f4v*>(y), rows);
        SPX_LAUNCH_CHECK();
        return true;
    }
    const dim3 grid(static_cast<unsigned>((rows + kThreads - 1) / kThreads));
    hipLaunchKernelGGL(c2r_n4_kernel, grid, dim3(kThreads), 0, stream, x,
                       reinterpret_cast<f4v*>(y), keep, rows);
    SPX_LAUNCH_CHECK();
    return true;
}

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
