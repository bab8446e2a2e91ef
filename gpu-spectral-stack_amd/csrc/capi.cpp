// The C ABI of libspectral_hip.so (include/spectral_hip.h): argument decoding, dispatch through
// the registry, and exception-to-status translation. Nothing here launches work of its own.

#include "spectral_hip.h"

#include "fft_api.hpp"

#include <cstring>
#include <exception>
#include <new>
#include <string>

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* message)
{
    g_last_error = message;
    return code;
}

// Runs `body`, mapping the library's exceptions to status codes.
template <class Body>
int guarded(Body&& body)
{
    try {
        body();
        g_last_error.clear();
        return SPX_OK;
    } catch (const spx::InvalidArgument& e) {
        return fail(SPX_EINVAL, e.what());
    } catch (const spx::HipError& e) {
        return fail(SPX_ERUNTIME, e.what());
    } catch (const std::bad_alloc&) {
        return fail(SPX_ERUNTIME, "out of host memory");
    } catch (const std::exception& e) {
        return fail(SPX_ERUNTIME, e.what());
    } catch (...) {
        return fail(SPX_ERUNTIME, "unknown error");
    }
}

const spx::FftImpl& impl_at(int impl)
{
    if (impl < 0 || impl >= spx::impl_count()) {
        throw spx::InvalidArgument("unknown FFT implementation index " + std::to_string(impl));
    }
    return spx::impls()[impl];
}

spx::Direction dir(int inverse)
{
    return inverse ? spx::Direction::Inverse : spx::Direction::Forward;
}

spx::Columns columns_of(const spx::FftImpl& impl, int columns)
{
    if (columns == SPX_COLUMNS_STRIDED) {
        return spx::Columns::Strided;
    }
    if (columns == SPX_COLUMNS_TRANSPOSE) {
        return spx::Columns::Transpose;
    }
    (void)impl;
    throw spx::InvalidArgument("columns must be SPX_COLUMNS_TRANSPOSE or SPX_COLUMNS_STRIDED");
}

const spx::cf32* cc(const void* p) { return static_cast<const spx::cf32*>(p); }
spx::cf32* cm(void* p) { return static_cast<spx::cf32*>(p); }

const spx::PrunedFns& pruned_of(const spx::FftImpl& impl)
{
    if (impl.pruned == nullptr) {
        throw spx::InvalidArgument(std::string(impl.name) + " has no pruned kernels");
    }
    return *impl.pruned;
}

const spx::RfFns& rf_of(const spx::FftImpl& impl)
{
    if (impl.rf == nullptr) {
        throw spx::InvalidArgument(std::string(impl.name) + " has no fused radio kernels");
    }
    return *impl.rf;
}

std::string join_names()
{
    std::string names;
    for (int i = 0; i < spx::impl_count(); ++i) {
        names += names.empty() ? "" : ", ";
        names += spx::impls()[i].name;
    }
    return names;
}

}  // namespace

extern "C" {

int spx_impl_count(void) { return spx::impl_count(); }

const char* spx_impl_name(int impl)
{
    if (impl < 0 || impl >= spx::impl_count()) {
        return nullptr;
    }
    return spx::impls()[impl].name;
}

int spx_impl_find(const char* name)
{
    if (name == nullptr) {
        return -1;
    }
    for (int i = 0; i < spx::impl_count(); ++i) {
        if (std::strcmp(name, spx::impls()[i].name) == 0) {
            return i;
        }
    }
    return -1;
}

int spx_impl_get_info(int impl, spx_impl_info* out)
{
    return guarded([&] {
        const spx::FftImpl& i = impl_at(impl);
        if (out == nullptr) {
            throw spx::InvalidArgument("spx_impl_get_info: out is NULL");
        }
        out->name = i.name;
        out->has_columns = i.columns != nullptr;
        out->has_pruned = i.pruned != nullptr;
        out->max_n = i.max_n;
        out->max_c2c_n = i.max_c2c_n;
        out->max_real_n = i.max_real_n;
        out->real_needs_work = i.real_needs_work;
        out->lazy_table = i.lazy_table;
    });
}

const char* spx_impl_names(void)
{
    static const std::string names = join_names();
    return names.c_str();
}

const char* spx_last_error(void) { return g_last_error.c_str(); }

int spx_scale(const void* x, void* y, size_t n, float alpha, hipStream_t stream)
{
    return guarded([&] { spx::scale_c2c(cc(x), cm(y), n, alpha, stream); });
}

int spx_c2c(int impl, const void* x, void* y, int n, int batch, int inverse, hipStream_t stream)
{
    return guarded([&] { impl_at(impl).c2c(cc(x), cm(y), n, batch, dir(inverse), stream); });
}

int spx_c2c_noalloc(int impl, const void* x, void* y, int n, int batch, int inverse,
                    hipStream_t stream)
{
    static_assert(SPX_NOALLOC_SCRATCH_VALUES == spx::kNoAllocScratchValues,
                  "the header's scratch size must match the library's");
    return guarded(
        [&] { spx::c2c_noalloc(impl_at(impl), cc(x), cm(y), n, batch, dir(inverse), stream); });
}

int spx_r2c(int impl, const float* x, void* y, int n, int batch, void* work, hipStream_t stream)
{
    return guarded([&] { impl_at(impl).r2c(x, cm(y), n, batch, cm(work), stream); });
}

int spx_c2r(int impl, const void* x, float* y, int n, int batch, void* work, hipStream_t stream)
{
    return guarded([&] { impl_at(impl).c2r(cc(x), y, n, batch, cm(work), stream); });
}

int spx_columns(int impl, const void* x, void* y, int n, int cols, int slabs, int inverse,
                hipStream_t stream)
{
    return guarded([&] {
        const spx::FftImpl& i = impl_at(impl);
        if (i.columns == nullptr) {
            throw spx::InvalidArgument(std::string(i.name) + " has no strided column kernel");
        }
        i.columns(cc(x), cm(y), n, cols, slabs, dir(inverse), stream);
    });
}

int spx_pruned_c2c(int impl, const void* x, void* y, int n, int batch, int keep, int inverse,
                   hipStream_t stream)
{
    return guarded([&] {
        pruned_of(impl_at(impl)).c2c(cc(x), cm(y), n, batch, keep, dir(inverse), stream);
    });
}

int spx_pruned_r2c(int impl, const float* x, void* y, int n, int batch, int keep,
                   hipStream_t stream)
{
    return guarded([&] { pruned_of(impl_at(impl)).r2c(x, cm(y), n, batch, keep, stream); });
}

int spx_pruned_c2r(int impl, const void* x, float* y, int n, int batch, int keep,
                   hipStream_t stream)
{
    return guarded([&] { pruned_of(impl_at(impl)).c2r(cc(x), y, n, batch, keep, stream); });
}

int spx_pruned_columns(int impl, const void* x, void* y, int n, int cols, int slabs, int m1_in,
                       int m1_out, int inverse, hipStream_t stream)
{
    return guarded([&] {
        pruned_of(impl_at(impl)).columns(cc(x), cm(y), n, cols, slabs, m1_in, m1_out,
                                         dir(inverse), stream);
    });
}

int spx_fft2_c2c_workspace(int impl, int columns, int n1, int n2, int batch, size_t* count)
{
    return guarded([&] {
        const spx::FftImpl& i = impl_at(impl);
        *count = spx::fft2_c2c_workspace(i, columns_of(i, columns), n1, n2, batch);
    });
}

int spx_fft2_r2c_workspace(int impl, int columns, int n1, int n2, int batch, size_t* count)
{
    return guarded([&] {
        const spx::FftImpl& i = impl_at(impl);
        *count = spx::fft2_r2c_workspace(i, columns_of(i, columns), n1, n2, batch);
    });
}

int spx_fft2_c2r_workspace(int impl, int columns, int n1, int n2, int batch, size_t* count)
{
    return guarded([&] {
        const spx::FftImpl& i = impl_at(impl);
        *count = spx::fft2_c2r_workspace(i, columns_of(i, columns), n1, n2, batch);
    });
}

int spx_fft2_c2c(int impl, int columns, const void* x, void* y, int n1, int n2, int batch,
                 int inverse, void* work, hipStream_t stream)
{
    return guarded([&] {
        const spx::FftImpl& i = impl_at(impl);
        spx::fft2_c2c(i, columns_of(i, columns), cc(x), cm(y), n1, n2, batch, dir(inverse),
                      cm(work), stream);
    });
}

int spx_fft2_r2c(int impl, int columns, const float* x, void* y, int n1, int n2, int batch,
                 void* work, hipStream_t stream)
{
    return guarded([&] {
        const spx::FftImpl& i = impl_at(impl);
        spx::fft2_r2c(i, columns_of(i, columns), x, cm(y), n1, n2, batch, cm(work), stream);
    });
}

int spx_fft2_c2r(int impl, int columns, const void* x, float* y, int n1, int n2, int batch,
                 void* work, hipStream_t stream)
{
    return guarded([&] {
        const spx::FftImpl& i = impl_at(impl);
        spx::fft2_c2r(i, columns_of(i, columns), cc(x), y, n1, n2, batch, cm(work), stream);
    });
}

int spx_transpose(const void* x, void* y, int rows, int cols, int batch, hipStream_t stream)
{
    return guarded([&] { spx::transpose(cc(x), cm(y), rows, cols, batch, stream); });
}

int spx_fft_c2c_pruned_workspace(int impl, int n, int keep, int batch, size_t* count)
{
    return guarded(
        [&] { *count = spx::fft_c2c_pruned_workspace(impl_at(impl), n, keep, batch); });
}

int spx_rfft2_modes_workspace(int impl, int n1, int n2, int m1, int m2, int batch, size_t* count)
{
    return guarded(
        [&] { *count = spx::rfft2_modes_workspace(impl_at(impl), n1, n2, m1, m2, batch); });
}

int spx_irfft2_modes_workspace(int impl, int n1, int n2, int m1, int m2, int batch,
                               size_t* count)
{
    return guarded(
        [&] { *count = spx::irfft2_modes_workspace(impl_at(impl), n1, n2, m1, m2, batch); });
}

int spx_fft_c2c_pruned(int impl, const void* x, void* y, int n, int keep, int batch, int inverse,
                       void* work, hipStream_t stream)
{
    return guarded([&] {
        spx::fft_c2c_pruned(impl_at(impl), cc(x), cm(y), n, keep, batch, dir(inverse), cm(work),
                            stream);
    });
}

int spx_rfft2_modes(int impl, const float* x, void* modes, int n1, int n2, int m1, int m2,
                    int batch, void* work, hipStream_t stream)
{
    return guarded([&] {
        spx::rfft2_modes(impl_at(impl), x, cm(modes), n1, n2, m1, m2, batch, cm(work), stream);
    });
}

int spx_irfft2_modes(int impl, const void* modes, float* y, int n1, int n2, int m1, int m2,
                     int batch, void* work, hipStream_t stream)
{
    return guarded([&] {
        spx::irfft2_modes(impl_at(impl), cc(modes), y, n1, n2, m1, m2, batch, cm(work), stream);
    });
}

int spx_gather_modes(const void* full, void* modes, int n1, int w, int m1, int m2, int batch,
                     hipStream_t stream)
{
    return guarded(
        [&] { spx::gather_modes(cc(full), cm(modes), n1, w, m1, m2, batch, stream); });
}

int spx_scatter_modes(const void* modes, void* full, int n1, int w, int m1, int m2, int batch,
                      hipStream_t stream)
{
    return guarded(
        [&] { spx::scatter_modes(cc(modes), cm(full), n1, w, m1, m2, batch, stream); });
}


int spx_ns_supports(int n) { return spx::ns_supports(n) ? 1 : 0; }

int spx_ns_stage(const void* state, const void* w0, const void* f0, void* out_f, void* out_w,
                 const void* forcing_hat, const float* nu, int nu_stride, float drag, float dt,
                 int n, int batch, int stage, hipStream_t stream)
{
    return guarded([&] {
        spx::ns_stage(cc(state), cc(w0), cc(f0), cm(out_f), cm(out_w), cc(forcing_hat), nu,
                      nu_stride, drag, dt, n, batch, stage, stream);
    });
}

int spx_ns_steps(const void* w_in, void* w_out, void* work, const void* forcing_hat,
                 const float* nu, int nu_stride, float drag, float dt, int n, int batch,
                 int steps, hipStream_t stream)
{
    return guarded([&] {
        spx::ns_steps(cc(w_in), cm(w_out), cm(work), cc(forcing_hat), nu, nu_stride, drag, dt, n,
                      batch, steps, stream);
    });
}

int spx_rf_max_nfft(int impl)
{
    if (impl < 0 || impl >= spx::impl_count() || spx::impls()[impl].rf == nullptr) {
        return 0;
    }
    return spx::impls()[impl].rf->max_nfft;
}

int spx_rf_spectrum(int impl, const void* x, const float* window, void* y, long long n,
                    int nfft, long long rows, hipStream_t stream)
{
    return guarded([&] { rf_of(impl_at(impl)).spectrum(cc(x), window, cm(y), n, nfft, rows, stream); });
}

int spx_rf_fir(int impl, const void* x, const void* h, void* y, long long n, int taps, int nfft,
               long long rows, hipStream_t stream)
{
    return guarded([&] {
        rf_of(impl_at(impl)).fir(cc(x), cc(h), cm(y), n, taps, nfft, rows, stream);
    });
}

int spx_rf_fir_spectrum(int impl, const void* taps, int complex_taps, void* h, int count,
                        int nfft, hipStream_t stream)
{
    return guarded([&] {
        rf_of(impl_at(impl)).filter(taps, complex_taps != 0, cm(h), count, nfft, stream);
    });
}

}  // extern "C"
