// y = alpha x over complex64 (reference ops/scale.cu:7-27): the `spectral::scale` operator, the
// extension's smoke op, and a copy-bound bandwidth yardstick. Each lane moves two complex values
// (16 bytes) per access when the pointers allow it. x == y is allowed (the naive inverse scales in
// place), so the pointers are not restrict.

#include "fft_api.hpp"

#include <algorithm>
#include <cstdint>

namespace spx {
namespace {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads)
    scale_pairs_kernel(const float4* x, float4* y, std::size_t pairs,
                       float alpha)
{
    for (std::size_t i = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x; i < pairs;
         i += static_cast<std::size_t>(gridDim.x) * kThreads) {
        const float4 v = x[i];
        y[i] = make_float4(alpha * v.x, alpha * v.y, alpha * v.z, alpha * v.w);
    }
}

__global__ void __launch_bounds__(kThreads)
    scale_kernel(const cf32* x, cf32* y, std::size_t n, float alpha)
{
    for (std::size_t i = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x; i < n;
         i += static_cast<std::size_t>(gridDim.x) * kThreads) {
        const cf32 v = x[i];
        y[i] = cf32{alpha * v.re, alpha * v.im};
    }
}

unsigned grid_for(std::size_t work)
{
    const std::size_t blocks = (work + kThreads - 1) / kThreads;
    return static_cast<unsigned>(std::min<std::size_t>(std::max<std::size_t>(blocks, 1), 8192));
}

}  // namespace

void scale_c2c(const cf32* x, cf32* y, std::size_t n, float alpha, hipStream_t stream)
{
    if (n == 0) {
        return;
    }
    const bool aligned = (reinterpret_cast<std::uintptr_t>(x) % 16 == 0)
                         && (reinterpret_cast<std::uintptr_t>(y) % 16 == 0) && n % 2 == 0;
    if (aligned) {
        const std::size_t pairs = n / 2;
        hipLaunchKernelGGL(scale_pairs_kernel, dim3(grid_for(pairs)), dim3(kThreads), 0, stream,
                           reinterpret_cast<const float4*>(x), reinterpret_cast<float4*>(y), pairs,
                           alpha);
    } else {
        hipLaunchKernelGGL(scale_kernel, dim3(grid_for(n)), dim3(kThreads), 0, stream, x, y, n,
                           alpha);
    }
    SPX_LAUNCH_CHECK();
}

}  // namespace spx
