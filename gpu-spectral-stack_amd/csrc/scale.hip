// y = alpha x over complex64 (reference ops/scale.cu:7-27): the `spectral::scale` operator, the
// extension's smoke op, and the copy-bound bandwidth yardstick of bench.py. Each lane moves two
// complex values (16 bytes) per access when the pointers allow it. x == y is allowed (the naive
// inverse scales in place), so the pointers are not restrict.

#include "fft_api.hpp"

#include <algorithm>
#include <cstdint>

namespace spx {
namespace {

constexpr int kThreads = 256;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

// One block streams kThreads x kPerLane consecutive vectors (V = f4: two complex values, or f2:
// one), 16 bytes per lane either way: every lane issues its nontemporal loads, then its stores. A
// lane writes only what it read, so x == y works. One 16-byte access per lane, nontemporal both
// ways, measured fastest on MI355X (6.3-6.5 TB/s over 128 MiB - 1 GiB); more accesses per lane
// measured slower (8 per lane: 4.0-4.3 TB/s).
template <class V, int kPerLane>
__global__ void __launch_bounds__(kThreads)
    scale_stream_kernel(const V* x, V* y, std::size_t count, float alpha)
{
    const std::size_t base =
        static_cast<std::size_t>(blockIdx.x) * kThreads * kPerLane + threadIdx.x;
    V v[kPerLane];
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
        const std::size_t i = base + static_cast<std::size_t>(k) * kThreads;
        if (i < count) {
            v[k] = __builtin_nontemporal_load(x + i);
        }
    }
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
        const std::size_t i = base + static_cast<std::size_t>(k) * kThreads;
        if (i < count) {
            __builtin_nontemporal_store(alpha * v[k], y + i);
        }
    }
}

template <class V>
void launch_stream(const void* x, void* y, std::size_t count, float alpha, hipStream_t stream)
{
    constexpr int kPerLane = 16 / static_cast<int>(sizeof(V));
    constexpr std::size_t kPerBlock = static_cast<std::size_t>(kThreads) * kPerLane;
    const std::size_t blocks = (count + kPerBlock - 1) / kPerBlock;
    hipLaunchKernelGGL((scale_stream_kernel<V, kPerLane>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kThreads), 0, stream, static_cast<const V*>(x), static_cast<V*>(y),
                       count, alpha);
}

}  // namespace

void scale_c2c(const cf32* x, cf32* y, std::size_t n, float alpha, hipStream_t stream)
{
    if (n == 0) {
        return;
    }
    if (n > (std::size_t{1} << 40)) {  // keeps the grid within 2^31 blocks
        throw InvalidArgument("scale: n too large");
    }
    const bool aligned = (reinterpret_cast<std::uintptr_t>(x) % 16 == 0)
                         && (reinterpret_cast<std::uintptr_t>(y) % 16 == 0) && n % 2 == 0;
    if (aligned) {
        launch_stream<f4>(x, y, n / 2, alpha, stream);
    } else {
        launch_stream<f2>(x, y, n, alpha, stream);
    }
    SPX_LAUNCH_CHECK();
}

}  // namespace spx
