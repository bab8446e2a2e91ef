// Pruned transforms for the FNO mode layout (reference pruned.hpp:3-17, pruned.cu:17-209).
//
//   1D complex  forward keeps the first `keep` outputs; inverse reads `keep` inputs, the rest zero.
//   2D real     of rfft2's n1 x (n2/2 + 1) spectrum, rows 0 .. m1-1 then n1-m1 .. n1-1 and
//               columns 0 .. m2-1, as a (2 m1) x m2 block; the inverse zero-fills the rest.
//
// Implementations with in-kernel pruning run real rows that write only m2 columns, then columns
// over those m2 that write only the 2 m1 kept rows (inverse: mirrored). The others compute the full
// transform and gather (scatter into zeros, then invert), giving the same modes.

#include "fft_api.hpp"

#include <algorithm>
#include <climits>

namespace spx {
namespace {

constexpr int kThreads = 256;

unsigned grid_for(std::size_t work)
{
    const std::size_t blocks = (work + kThreads - 1) / kThreads;
    return static_cast<unsigned>(std::min<std::size_t>(std::max<std::size_t>(blocks, 1), 65536));
}

// Position in `full` (arrays of n1 x w) of mode e of `modes` (arrays of rows x m2, rows = 2 m1,
// or n1 when m1 = 0). Row r < m1 is frequency r; row r >= m1 is frequency r - 2 m1 + n1.
__device__ __forceinline__ std::size_t full_index(std::size_t e, int n1, int w, int m1, int m2)
{
    const int rows = m1 > 0 ? 2 * m1 : n1;
    const std::size_t per_array = static_cast<std::size_t>(rows) * static_cast<std::size_t>(m2);
    const std::size_t b = e / per_array;
    const auto rem = static_cast<int>(e - b * per_array);
    const int r = rem / m2;
    const int c = rem - r * m2;
    const int row = (m1 > 0 && r >= m1) ? r + (n1 - rows) : r;
    return (b * static_cast<std::size_t>(n1) + static_cast<std::size_t>(row))
               * static_cast<std::size_t>(w)
           + static_cast<std::size_t>(c);
}

__global__ void __launch_bounds__(kThreads)
    gather_kernel(const cf32* __restrict__ full, cf32* __restrict__ modes, int n1, int w, int m1,
                  int m2, std::size_t total)
{
    for (std::size_t e = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x; e < total;
         e += static_cast<std::size_t>(gridDim.x) * kThreads) {
        modes[e] = full[full_index(e, n1, w, m1, m2)];
    }
}

__global__ void __launch_bounds__(kThreads)
    scatter_kernel(const cf32* __restrict__ modes, cf32* __restrict__ full, int n1, int w, int m1,
                   int m2, std::size_t total)
{
    for (std::size_t e = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x; e < total;
         e += static_cast<std::size_t>(gridDim.x) * kThreads) {
        full[full_index(e, n1, w, m1, m2)] = modes[e];
    }
}

// Zero fill as a kernel (not hipMemsetAsync), so the call stays safe inside a captured graph.
__global__ void __launch_bounds__(kThreads) zero_kernel(cf32* __restrict__ p, std::size_t total)
{
    for (std::size_t e = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x; e < total;
         e += static_cast<std::size_t>(gridDim.x) * kThreads) {
        p[e] = cf32{0.0f, 0.0f};
    }
}

std::size_t mode_count(int n1, int m1, int m2, int batch)
{
    const int rows = m1 > 0 ? 2 * m1 : n1;
    return static_cast<std::size_t>(batch) * static_cast<std::size_t>(rows)
           * static_cast<std::size_t>(m2);
}

std::size_t count(int n1, int n2, int batch)
{
    return static_cast<std::size_t>(batch) * static_cast<std::size_t>(n1)
           * static_cast<std::size_t>(n2);
}

void check_1d(const FftImpl& impl, int n, int keep, int batch)
{
    if (!is_pow2(n) || n > impl.max_n) {
        throw InvalidArgument("fft_c2c_pruned: " + std::string(impl.name)
                              + " needs n to be a power of two up to " + str(impl.max_n)
                              + ", got " + str(n));
    }
    if (keep < 1 || keep > n) {
        throw InvalidArgument("fft_c2c_pruned: keep must be in [1, " + str(n) + "], got "
                              + str(keep));
    }
    if (batch < 1) {
        throw InvalidArgument("fft_c2c_pruned: batch must be at least 1");
    }
}

void check_2d(const FftImpl& impl, int n1, int n2, int m1, int m2, int batch)
{
    const std::string name = impl.name;
    if (!is_pow2(n1) || n1 > impl.max_n) {
        throw InvalidArgument("rfft2 modes: " + name + " needs n1 to be a power of two up to "
                              + str(impl.max_n) + ", got " + str(n1));
    }
    if (!is_pow2(n2) || n2 < 2 || n2 > impl.max_real_n) {
        throw InvalidArgument("rfft2 modes: " + name
                              + " needs n2 to be a power of two from 2 up to "
                              + str(impl.max_real_n) + ", got " + str(n2));
    }
    if (m1 < 1 || 2 * m1 > n1 || m2 < 1 || m2 > n2 / 2 + 1) {
        throw InvalidArgument("rfft2 modes: need 1 <= m1 <= n1/2 and 1 <= m2 <= n2/2 + 1, got m1 = "
                              + str(m1) + ", m2 = " + str(m2) + " for " + str(n1) + " x "
                              + str(n2));
    }
    if (batch < 1 || static_cast<long long>(batch) * std::max(n1, n2) > INT_MAX) {
        throw InvalidArgument("rfft2 modes: batch out of range");
    }
}

}  // namespace

void gather_modes(const cf32* full, cf32* modes, int n1, int w, int m1, int m2, int batch,
                  hipStream_t stream)
{
    const std::size_t total = mode_count(n1, m1, m2, batch);
    hipLaunchKernelGGL(gather_kernel, dim3(grid_for(total)), dim3(kThreads), 0, stream, full,
                       modes, n1, w, m1, m2, total);
    SPX_LAUNCH_CHECK();
}

void scatter_modes(const cf32* modes, cf32* full, int n1, int w, int m1, int m2, int batch,
                   hipStream_t stream)
{
    const std::size_t zeros = count(n1, w, batch);
    hipLaunchKernelGGL(zero_kernel, dim3(grid_for(zeros)), dim3(kThreads), 0, stream, full,
                       zeros);
    SPX_LAUNCH_CHECK();
    const std::size_t total = mode_count(n1, m1, m2, batch);
    hipLaunchKernelGGL(scatter_kernel, dim3(grid_for(total)), dim3(kThreads), 0, stream, modes,
                       full, n1, w, m1, m2, total);
    SPX_LAUNCH_CHECK();
}

std::size_t fft_c2c_pruned_workspace(const FftImpl& impl, int n, int, int batch)
{
    return impl.pruned != nullptr ? 0 : count(1, n, batch);
}

void fft_c2c_pruned(const FftImpl& impl, const cf32* x, cf32* y, int n, int keep, int batch,
                    Direction direction, cf32* work, hipStream_t stream)
{
    check_1d(impl, n, keep, batch);
    if (impl.pruned != nullptr) {
        impl.pruned->c2c(x, y, n, batch, keep, direction, stream);
        return;
    }
    // Each transform is an array of one row of n values; its first keep are the modes.
    if (direction == Direction::Forward) {
        impl.c2c(x, work, n, batch, direction, stream);
        gather_modes(work, y, 1, n, 0, keep, batch, stream);
    } else {
        scatter_modes(x, work, 1, n, 0, keep, batch, stream);
        impl.c2c(work, y, n, batch, direction, stream);
    }
}

namespace {

// One single-pass kernel when the implementation has one for the shape.
bool fused(const FftImpl& impl, int n1, int n2)
{
    return impl.fused != nullptr && impl.fused->supports(n1, n2);
}

}  // namespace

std::size_t rfft2_modes_workspace(const FftImpl& impl, int n1, int n2, int, int m2, int batch)
{
    if (fused(impl, n1, n2)) {
        return 0;  // one single-pass kernel
    }
    if (impl.pruned != nullptr) {
        return count(n1, m2, batch);  // the row transforms' m2 columns
    }
    return count(n1, n2 / 2 + 1, batch)
           + fft2_r2c_workspace(impl, Columns::Transpose, n1, n2, batch);
}

void rfft2_modes(const FftImpl& impl, const float* x, cf32* modes, int n1, int n2, int m1,
                 int m2, int batch, cf32* work, hipStream_t stream)
{
    check_2d(impl, n1, n2, m1, m2, batch);
    if (fused(impl, n1, n2)) {
        impl.fused->r2c(x, modes, n1, n2, m1, m2, batch, stream);
        return;
    }
    if (impl.pruned != nullptr) {
        impl.pruned->r2c_work(x, work, n2, batch * n1, m2, stream);  // n1 x m2 per array
        impl.pruned->columns(work, modes, n1, m2, batch, 0, m1, Direction::Forward, stream);
        return;
    }
    cf32* full = work;
    cf32* rest = work + count(n1, n2 / 2 + 1, batch);
    fft2_r2c(impl, Columns::Transpose, x, full, n1, n2, batch, rest, stream);
    gather_modes(full, modes, n1, n2 / 2 + 1, m1, m2, batch, stream);
}

std::size_t irfft2_modes_workspace(const FftImpl& impl, int n1, int n2, int, int m2, int batch)
{
    if (fused(impl, n1, n2)) {
        return 0;
    }
    if (impl.pruned != nullptr) {
        return count(n1, m2, batch);
    }
    return count(n1, n2 / 2 + 1, batch)
           + fft2_c2r_workspace(impl, Columns::Transpose, n1, n2, batch);
}

void irfft2_modes(const FftImpl& impl, const cf32* modes, float* y, int n1, int n2, int m1,
                  int m2, int batch, cf32* work, hipStream_t stream)
{
    check_2d(impl, n1, n2, m1, m2, batch);
    if (fused(impl, n1, n2)) {
        impl.fused->c2r(modes, y, n1, n2, m1, m2, batch, stream);
        return;
    }
    if (impl.pruned != nullptr) {
        impl.pruned->columns_work(modes, work, n1, m2, batch, m1, 0, Direction::Inverse, stream);
        impl.pruned->c2r(work, y, n2, batch * n1, m2, stream);  // columns m2.. are zero
        return;
    }
    cf32* full = work;
    cf32* rest = work + count(n1, n2 / 2 + 1, batch);
    scatter_modes(modes, full, n1, n2 / 2 + 1, m1, m2, batch, stream);
    fft2_c2r(impl, Columns::Transpose, full, y, n1, n2, batch, rest, stream);
}

}  // namespace spx
