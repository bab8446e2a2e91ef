#pragma once

// Types and error handling shared by every translation unit of libspectral_hip.so.
//
// Host code throws spx::InvalidArgument for rejected arguments and spx::HipError for runtime
// failures; the C ABI (capi.cpp) turns them into SPX_EINVAL / SPX_ERUNTIME and a thread-local
// message, so no exception ever crosses the library boundary.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <stdexcept>
#include <string>

namespace spx {

// One complex float32 value, interleaved (re, im): the layout of torch.complex64. Kept a plain
// aggregate so device code can use it freely; 8-byte aligned so a pair loads as one dwordx4.
struct __attribute__((aligned(8))) cf32 {
    float re;
    float im;
};
static_assert(sizeof(cf32) == 8, "cf32 must be two packed floats");

enum class Direction { Forward, Inverse };

struct InvalidArgument : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};

struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] inline void throw_hip(hipError_t err, const char* what, const char* file, int line)
{
    throw HipError(std::string(what) + " failed: " + hipGetErrorString(err) + " (" + file + ":"
                   + std::to_string(line) + ")");
}

#define SPX_HIP_CHECK(expr)                                    \
    do {                                                       \
        const hipError_t spx_err_ = (expr);                    \
        if (spx_err_ != hipSuccess) {                          \
            ::spx::throw_hip(spx_err_, #expr, __FILE__, __LINE__); \
        }                                                      \
    } while (0)

// After a kernel launch: launch-configuration errors surface here.
#define SPX_LAUNCH_CHECK() SPX_HIP_CHECK(hipGetLastError())

inline bool is_pow2(long long n) { return n >= 1 && (n & (n - 1)) == 0; }

inline int ilog2_host(long long n)
{
    int r = 0;
    while ((1LL << r) < n) {
        ++r;
    }
    return r;
}

inline std::string str(long long v) { return std::to_string(v); }

// Compute units of the current device, looked up once per device.
inline int device_cus()
{
    int device = 0;
    SPX_HIP_CHECK(hipGetDevice(&device));
    constexpr int kDevices = 64;
    static std::atomic<int> known[kDevices] = {};
    if (device < kDevices) {
        const int cus = known[device].load(std::memory_order_relaxed);
        if (cus > 0) {
            return cus;
        }
    }
    int cus = 0;
    SPX_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
    if (device < kDevices) {
        known[device].store(cus, std::memory_order_relaxed);
    }
    return cus;
}

}  // namespace spx
