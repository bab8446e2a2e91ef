// The "naive" implementation: iterative radix-2 Cooley-Tukey (decimation in time), one launch for
// the bit-reversal permutation, one per stage, and a scaling pass for the inverse. It is the
// registry's first row and the default `impl` of every operator (reference naive.cu:25-120,
// ops.cpp:450-460), so it must exist and be right; its speed is not a target (log2 n full HBM
// round trips).

#include "fft_api.hpp"
#include "stockham.hpp"

#include <algorithm>

namespace spx {
namespace {

constexpr int kThreads = 256;

unsigned grid_for(std::size_t work)
{
    const std::size_t blocks = (work + kThreads - 1) / kThreads;
    return static_cast<unsigned>(std::min<std::size_t>(std::max<std::size_t>(blocks, 1), 65536));
}

// y[base + i] = x[base + reverse(i)], reverse() mirroring the low log2n bits.
__global__ void __launch_bounds__(kThreads)
    bit_reverse_kernel(const cf32* __restrict__ x, cf32* __restrict__ y, std::size_t total,
                       int log2n)
{
    const std::size_t mask = (std::size_t{1} << log2n) - 1;
    for (std::size_t e = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x;
         e < total; e += static_cast<std::size_t>(gridDim.x) * kThreads) {
        const auto i = static_cast<unsigned>(e & mask);
        const unsigned r = __builtin_bitreverse32(i) >> (32 - log2n);
        y[e] = x[(e & ~mask) + r];
    }
}

// One radix-2 stage in place: blocks of 2h values, butterfly k of a block combines positions k
// and k + h with the twiddle exp(sign pi i k / h).
__global__ void __launch_bounds__(kThreads)
    radix2_kernel(cf32* y, std::size_t butterflies, int log2h, float sign)
{
    using namespace dev;
    const std::size_t h = std::size_t{1} << log2h;
    const float inv_h = 1.0f / static_cast<float>(h);
    for (std::size_t e = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x;
         e < butterflies; e += static_cast<std::size_t>(gridDim.x) * kThreads) {
        const std::size_t k = e & (h - 1);
        const std::size_t i0 = ((e >> log2h) << (log2h + 1)) | k;
        const std::size_t i1 = i0 + h;
        cf32 w = expi_pi(static_cast<float>(k) * inv_h);
        w.im *= sign;
        const cf32 a = y[i0];
        const cf32 b = cmul(y[i1], w);
        y[i0] = cadd(a, b);
        y[i1] = csub(a, b);
    }
}

}  // namespace

void c2c_naive(const cf32* x, cf32* y, int n, int batch, Direction direction,
               hipStream_t stream)
{
    if (n < 1 || !is_pow2(n)) {
        throw InvalidArgument("fft: n must be a power of two, got " + str(n));
    }
    if (batch < 1) {
        throw InvalidArgument("fft: batch must be at least 1, got " + str(batch));
    }
    const std::size_t total = static_cast<std::size_t>(n) * static_cast<std::size_t>(batch);
    if (x < y + total && y < x + total) {
        throw InvalidArgument("fft: x and y must not overlap (out-of-place only)");
    }
    if (n == 1) {
        SPX_HIP_CHECK(hipMemcpyAsync(y, x, total * sizeof(cf32), hipMemcpyDeviceToDevice, stream));
        return;
    }
    const int log2n = ilog2_host(n);
    hipLaunchKernelGGL(bit_reverse_kernel, dim3(grid_for(total)), dim3(kThreads), 0, stream, x, y,
                       total, log2n);
    SPX_LAUNCH_CHECK();
    const float sign = direction == Direction::Forward ? -1.0f : 1.0f;
    for (int s = 0; s < log2n; ++s) {
        hipLaunchKernelGGL(radix2_kernel, dim3(grid_for(total / 2)), dim3(kThreads), 0, stream,
                           y, total / 2, s, sign);
        SPX_LAUNCH_CHECK();
    }
    if (direction == Direction::Inverse) {
        scale_c2c(y, y, total, 1.0f / static_cast<float>(n), stream);  // exact: n = 2^k
    }
}

}  // namespace spx
