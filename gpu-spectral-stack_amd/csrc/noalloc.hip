// c2c that allocates nothing, for callers that cannot allocate device memory (code being captured
// into a HIP graph, tight serving loops, harnesses that forbid hipMalloc). It runs the same kernels
// as c2c; the one difference is where the scratch of the large transforms (two and three passes,
// n > kSinglePassMaxN: one intermediate of n x batch values) lives: in `scratch` below, a static
// device array of kNoAllocScratchValues values (32 MiB) that every GPU the library runs on holds
// from the library's load until the process ends.
//
// Every call on a GPU shares that GPU's array, and the array keeps the last call's contents. The
// transforms write every scratch value they read before reading it, so nothing needs clearing.
// Calls that overlap on one GPU (two streams, or two host threads) race on the array.
//
// In host code `scratch` names a host-side stand-in, not device memory: its device address comes
// from hipGetSymbolAddress, once per device with that device current, and only that address is
// passed to kernels.

#include "fft_api.hpp"

#include <mutex>
#include <vector>

namespace spx {

static __device__ __align__(256) cf32 scratch[kNoAllocScratchValues];

namespace {

// The current device's address of `scratch`.
cf32* scratch_on_current_device()
{
    static std::mutex mutex;
    static std::vector<cf32*> addresses;  // per device

    int device = 0;
    SPX_HIP_CHECK(hipGetDevice(&device));
    const std::lock_guard<std::mutex> lock(mutex);
    if (addresses.size() <= static_cast<std::size_t>(device)) {
        addresses.resize(static_cast<std::size_t>(device) + 1, nullptr);
    }
    cf32*& address = addresses[static_cast<std::size_t>(device)];
    if (address == nullptr) {
        void* p = nullptr;
        SPX_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        address = static_cast<cf32*>(p);
    }
    return address;
}

}  // namespace

void c2c_noalloc(const FftImpl& impl, const cf32* x, cf32* y, int n, int batch,
                 Direction direction, hipStream_t stream)
{
    if (impl.lazy_table) {
        throw InvalidArgument("spx_c2c_noalloc: " + std::string(impl.name)
                              + " allocates its twiddle table on first use; use an "
                                "implementation with computed twiddles");
    }
    if (impl.c2c_work == nullptr) {
        impl.c2c(x, y, n, batch, direction, stream);  // no size of this implementation allocates
        return;
    }
    if (!is_pow2(n) || n > impl.max_c2c_n || batch < 1) {
        // Rejected by the transform's own argument checks, before it would allocate anything.
        impl.c2c_work(x, y, n, batch, direction, nullptr, stream);
        return;
    }
    const std::size_t need = c2c_scratch_values(impl, n, batch);
    if (need > kNoAllocScratchValues) {
        throw InvalidArgument("spx_c2c_noalloc: n * batch = " + str(static_cast<long long>(need))
                              + " needs more scratch than the static "
                              + str(static_cast<long long>(kNoAllocScratchValues))
                              + " values; split the batch");
    }
    impl.c2c_work(x, y, n, batch, direction, need > 0 ? scratch_on_current_device() : nullptr,
                  stream);
}

}  // namespace spx
