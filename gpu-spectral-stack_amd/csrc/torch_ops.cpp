// PyTorch operators over the C ABI of libspectral_hip.so.
//
// The schema, defaults, argument checks and error messages are those of the reference's binding
// (csrc/torch/ops.cpp:47-475), so `torch.ops.spectral.*` and `spectral._C.fft_impls()` are a
// drop-in. ROCm tensors report the CUDA device type, so the operators are registered for the
// CUDA dispatch key and CPU tensors are refused by the dispatcher. Each operator checks its
// arguments, allocates outputs and workspace with torch on the input's device, and calls the C
// ABI on PyTorch's current HIP stream. Status codes map back to the reference's exception types:
// SPX_EINVAL (the reference's std::invalid_argument) -> ValueError, SPX_ERUNTIME -> RuntimeError.

#include <Python.h>

#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include "spectral_hip.h"

#include <climits>
#include <cstdint>
#include <optional>
#include <string>
#include <tuple>
#include <vector>

namespace {

static_assert(sizeof(c10::complex<float>) == 8, "complex64 must be two packed floats");

hipStream_t current_stream()
{
    return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
}

void check_status(int status)
{
    if (status == SPX_OK) {
        return;
    }
    const std::string message = spx_last_error();
    TORCH_CHECK_VALUE(status != SPX_EINVAL, message);
    TORCH_CHECK(false, message);
}

const void* cptr(const at::Tensor& t) { return t.const_data_ptr(); }
void* mptr(at::Tensor& t) { return t.mutable_data_ptr(); }
void* work_ptr(at::Tensor& w) { return w.numel() == 0 ? nullptr : w.mutable_data_ptr(); }

void check_complex64_cuda(const at::Tensor& t, const char* name)
{
    TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
    TORCH_CHECK(t.scalar_type() == at::kComplexFloat, name, " must be complex64, got ",
                t.scalar_type());
}

void check_float32_cuda(const at::Tensor& t)
{
    TORCH_CHECK(t.is_cuda(), "x must be a CUDA tensor");
    TORCH_CHECK(t.scalar_type() == at::kFloat, "x must be float32, got ", t.scalar_type());
}

struct Impl {
    int index;
    spx_impl_info info;
};

Impl find_impl(c10::string_view impl_name)
{
    const std::string name(impl_name.data(), impl_name.size());
    const int index = spx_impl_find(name.c_str());
    TORCH_CHECK(index >= 0, "unknown FFT implementation '", name, "' (available: ",
                spx_impl_names(), ")");
    Impl impl{index, {}};
    check_status(spx_impl_get_info(index, &impl.info));
    return impl;
}

int batch_of(const at::Tensor& x, int64_t row, const char* op)
{
    const int64_t batch = x.numel() / row;
    TORCH_CHECK(batch <= INT_MAX, op, ": too many transforms");
    return static_cast<int>(batch);
}

at::Tensor workspace(std::size_t count, const at::Tensor& like)
{
    return at::empty({static_cast<int64_t>(count)}, like.options().dtype(at::kComplexFloat));
}

at::Tensor scale_op(const at::Tensor& x, double alpha)
{
    check_complex64_cuda(x, "x");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const at::Tensor xc = x.contiguous();
    at::Tensor y = at::empty_like(xc);
    check_status(spx_scale(cptr(xc), mptr(y), static_cast<size_t>(xc.numel()),
                           static_cast<float>(alpha), current_stream()));
    return y;
}

at::Tensor fft_c2c_op(const at::Tensor& x, bool inverse, c10::string_view impl_name)
{
    check_complex64_cuda(x, "x");
    TORCH_CHECK(x.dim() >= 1, "fft_c2c: x needs at least one dimension");
    const Impl impl = find_impl(impl_name);
    if (x.numel() == 0) {
        return at::empty_like(x, at::MemoryFormat::Contiguous);
    }
    const int64_t n = x.size(-1);
    TORCH_CHECK((n & (n - 1)) == 0, "fft_c2c: the last dimension must be a power of two, got ",
                n);
    TORCH_CHECK(n <= impl.info.max_c2c_n, "fft_c2c: ", impl.info.name, " supports sizes up to ",
                impl.info.max_c2c_n, ", got ", n);
    const int batch = batch_of(x, n, "fft_c2c");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const at::Tensor xc = x.contiguous();
    at::Tensor y = at::empty_like(xc);
    check_status(spx_c2c(impl.index, cptr(xc), mptr(y), static_cast<int>(n), batch,
                         inverse ? 1 : 0, current_stream()));
    return y;
}

void check_real_size(int64_t n, const Impl& impl, const char* op)
{
    TORCH_CHECK(n >= 2 && (n & (n - 1)) == 0, op,
                ": the real transform size must be a power of two of at least 2, got ", n);
    TORCH_CHECK(n <= impl.info.max_real_n, op, ": ", impl.info.name, " supports real sizes up to ",
                impl.info.max_real_n, ", got ", n);
}

at::Tensor real_workspace(const Impl& impl, int64_t n, int batch, const at::Tensor& like)
{
    const int64_t count = impl.info.real_needs_work ? static_cast<int64_t>(batch) * (n / 2) : 0;
    return at::empty({count}, like.options().dtype(at::kComplexFloat));
}

at::Tensor fft_r2c_op(const at::Tensor& x, c10::string_view impl_name)
{
    check_float32_cuda(x);
    TORCH_CHECK(x.dim() >= 1, "fft_r2c: x needs at least one dimension");
    const Impl impl = find_impl(impl_name);
    const int64_t n = x.size(-1);
    check_real_size(n, impl, "fft_r2c");
    std::vector<int64_t> shape = x.sizes().vec();
    shape.back() = n / 2 + 1;
    at::Tensor y = at::empty(shape, x.options().dtype(at::kComplexFloat));
    if (x.numel() == 0) {
        return y;
    }
    const int batch = batch_of(x, n, "fft_r2c");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const at::Tensor xc = x.contiguous();
    at::Tensor work = real_workspace(impl, n, batch, x);
    check_status(spx_r2c(impl.index, xc.const_data_ptr<float>(), mptr(y), static_cast<int>(n),
                         batch, work_ptr(work), current_stream()));
    return y;
}

at::Tensor fft_c2r_op(const at::Tensor& x, int64_t n, c10::string_view impl_name)
{
    check_complex64_cuda(x, "x");
    TORCH_CHECK(x.dim() >= 1, "fft_c2r: x needs at least one dimension");
    const Impl impl = find_impl(impl_name);
    check_real_size(n, impl, "fft_c2r");
    TORCH_CHECK(x.size(-1) == n / 2 + 1, "fft_c2r: an output of ", n, " points needs n/2 + 1 = ",
                n / 2 + 1, " inputs per transform, got ", x.size(-1));
    std::vector<int64_t> shape = x.sizes().vec();
    shape.back() = n;
    at::Tensor y = at::empty(shape, x.options().dtype(at::kFloat));
    if (x.numel() == 0) {
        return y;
    }
    const int batch = batch_of(x, n / 2 + 1, "fft_c2r");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const at::Tensor xc = x.contiguous();
    at::Tensor work = real_workspace(impl, n, batch, x);
    check_status(spx_c2r(impl.index, cptr(xc), y.mutable_data_ptr<float>(), static_cast<int>(n),
                         batch, work_ptr(work), current_stream()));
    return y;
}

// "auto" picks the strided column kernel when the implementation has one.
int parse_columns(c10::string_view text, const Impl& impl)
{
    const std::string s(text.data(), text.size());
    if (s == "auto") {
        return impl.info.has_columns ? SPX_COLUMNS_STRIDED : SPX_COLUMNS_TRANSPOSE;
    }
    if (s == "strided") {
        TORCH_CHECK(impl.info.has_columns, impl.info.name,
                    " has no strided column kernel; use columns=\"transpose\"");
        return SPX_COLUMNS_STRIDED;
    }
    TORCH_CHECK(s == "transpose", "columns must be \"auto\", \"strided\", or \"transpose\", got '",
                s, "'");
    return SPX_COLUMNS_TRANSPOSE;
}

struct Shape2d {
    int64_t n1;
    int64_t n2;
    int batch;
};

Shape2d shape2d(const at::Tensor& x, int64_t n2, int64_t n2_stored, const char* op)
{
    TORCH_CHECK(x.dim() >= 2, op, ": x needs at least two dimensions");
    const int64_t n1 = x.size(-2);
    TORCH_CHECK(n1 >= 1 && n2 >= 1, op, ": empty transform dimensions");
    return {n1, n2, batch_of(x, n1 * n2_stored, op)};
}

at::Tensor fft2_c2c_op(const at::Tensor& x, bool inverse, c10::string_view impl_name,
                       c10::string_view columns)
{
    check_complex64_cuda(x, "x");
    const Impl impl = find_impl(impl_name);
    const int method = parse_columns(columns, impl);
    TORCH_CHECK(x.dim() >= 2, "fft2_c2c: x needs at least two dimensions");
    if (x.numel() == 0) {
        return at::empty_like(x, at::MemoryFormat::Contiguous);
    }
    const Shape2d s = shape2d(x, x.size(-1), x.size(-1), "fft2_c2c");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const at::Tensor xc = x.contiguous();
    at::Tensor y = at::empty_like(xc);
    const auto n1 = static_cast<int>(s.n1);
    const auto n2 = static_cast<int>(s.n2);
    size_t count = 0;
    check_status(spx_fft2_c2c_workspace(impl.index, method, n1, n2, s.batch, &count));
    at::Tensor work = workspace(count, x);
    check_status(spx_fft2_c2c(impl.index, method, cptr(xc), mptr(y), n1, n2, s.batch,
                              inverse ? 1 : 0, work_ptr(work), current_stream()));
    return y;
}

at::Tensor fft2_r2c_op(const at::Tensor& x, c10::string_view impl_name, c10::string_view columns)
{
    check_float32_cuda(x);
    const Impl impl = find_impl(impl_name);
    const int method = parse_columns(columns, impl);
    TORCH_CHECK(x.dim() >= 2, "fft2_r2c: x needs at least two dimensions");
    const int64_t n2 = x.size(-1);
    check_real_size(n2, impl, "fft2_r2c");
    std::vector<int64_t> shape = x.sizes().vec();
    shape.back() = n2 / 2 + 1;
    at::Tensor y = at::empty(shape, x.options().dtype(at::kComplexFloat));
    if (x.numel() == 0) {
        return y;
    }
    const Shape2d s = shape2d(x, n2, n2, "fft2_r2c");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const at::Tensor xc = x.contiguous();
    const auto n1 = static_cast<int>(s.n1);
    size_t count = 0;
    check_status(spx_fft2_r2c_workspace(impl.index, method, n1, static_cast<int>(n2), s.batch,
                                        &count));
    at::Tensor work = workspace(count, x);
    check_status(spx_fft2_r2c(impl.index, method, xc.const_data_ptr<float>(), mptr(y), n1,
                              static_cast<int>(n2), s.batch, work_ptr(work), current_stream()));
    return y;
}

at::Tensor fft2_c2r_op(const at::Tensor& x, int64_t n2, c10::string_view impl_name,
                       c10::string_view columns)
{
    check_complex64_cuda(x, "x");
    const Impl impl = find_impl(impl_name);
    const int method = parse_columns(columns, impl);
    TORCH_CHECK(x.dim() >= 2, "fft2_c2r: x needs at least two dimensions");
    check_real_size(n2, impl, "fft2_c2r");
    TORCH_CHECK(x.size(-1) == n2 / 2 + 1, "fft2_c2r: an output of ", n2,
                " columns needs n2/2 + 1 = ", n2 / 2 + 1, " input columns, got ", x.size(-1));
    std::vector<int64_t> shape = x.sizes().vec();
    shape.back() = n2;
    at::Tensor y = at::empty(shape, x.options().dtype(at::kFloat));
    if (x.numel() == 0) {
        return y;
    }
    const Shape2d s = shape2d(x, n2, n2 / 2 + 1, "fft2_c2r");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const at::Tensor xc = x.contiguous();
    const auto n1 = static_cast<int>(s.n1);
    size_t count = 0;
    check_status(spx_fft2_c2r_workspace(impl.index, method, n1, static_cast<int>(n2), s.batch,
                                        &count));
    at::Tensor work = workspace(count, x);
    check_status(spx_fft2_c2r(impl.index, method, cptr(xc), y.mutable_data_ptr<float>(), n1,
                              static_cast<int>(n2), s.batch, work_ptr(work), current_stream()));
    return y;
}

at::Tensor fft_c2c_pruned_op(const at::Tensor& x, int64_t n, int64_t keep, bool inverse,
                             c10::string_view impl_name)
{
    check_complex64_cuda(x, "x");
    TORCH_CHECK(x.dim() >= 1, "fft_c2c_pruned: x needs at least one dimension");
    const Impl impl = find_impl(impl_name);
    TORCH_CHECK(n >= 1 && n <= INT_MAX && keep >= 1 && keep <= n,
                "fft_c2c_pruned: need 1 <= keep <= n, got keep = ", keep, ", n = ", n);
    const int64_t row_in = inverse ? keep : n;
    TORCH_CHECK(x.size(-1) == row_in, "fft_c2c_pruned: expected ", row_in,
                " values in the last dimension, got ", x.size(-1));
    std::vector<int64_t> shape = x.sizes().vec();
    shape.back() = inverse ? n : keep;
    at::Tensor y = at::empty(shape, x.options());
    if (x.numel() == 0) {
        return y;
    }
    const int batch = batch_of(x, row_in, "fft_c2c_pruned");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const at::Tensor xc = x.contiguous();
    const auto ni = static_cast<int>(n);
    const auto ki = static_cast<int>(keep);
    size_t count = 0;
    check_status(spx_fft_c2c_pruned_workspace(impl.index, ni, ki, batch, &count));
    at::Tensor work = workspace(count, x);
    check_status(spx_fft_c2c_pruned(impl.index, cptr(xc), mptr(y), ni, ki, batch,
                                    inverse ? 1 : 0, work_ptr(work), current_stream()));
    return y;
}

at::Tensor rfft2_modes_op(const at::Tensor& x, int64_t m1, int64_t m2, c10::string_view impl_name)
{
    check_float32_cuda(x);
    TORCH_CHECK(x.dim() >= 2, "rfft2_modes: x needs at least two dimensions");
    const Impl impl = find_impl(impl_name);
    const int64_t n1 = x.size(-2);
    const int64_t n2 = x.size(-1);
    TORCH_CHECK(m1 >= 1 && 2 * m1 <= n1 && m2 >= 1 && m2 <= n2 / 2 + 1,
                "rfft2_modes: need 1 <= m1 <= n1/2 and 1 <= m2 <= n2/2 + 1, got m1 = ", m1,
                ", m2 = ", m2, " for ", n1, " x ", n2);
    std::vector<int64_t> shape = x.sizes().vec();
    shape[shape.size() - 2] = 2 * m1;
    shape.back() = m2;
    at::Tensor y = at::empty(shape, x.options().dtype(at::kComplexFloat));
    if (x.numel() == 0) {
        return y;
    }
    const int batch = batch_of(x, n1 * n2, "rfft2_modes");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const at::Tensor xc = x.contiguous();
    const int a = static_cast<int>(n1);
    const int b = static_cast<int>(n2);
    const int p = static_cast<int>(m1);
    const int q = static_cast<int>(m2);
    size_t count = 0;
    check_status(spx_rfft2_modes_workspace(impl.index, a, b, p, q, batch, &count));
    at::Tensor work = workspace(count, x);
    check_status(spx_rfft2_modes(impl.index, xc.const_data_ptr<float>(), mptr(y), a, b, p, q,
                                 batch, work_ptr(work), current_stream()));
    return y;
}

at::Tensor irfft2_modes_op(const at::Tensor& modes, int64_t n1, int64_t n2,
                           c10::string_view impl_name)
{
    check_complex64_cuda(modes, "modes");
    TORCH_CHECK(modes.dim() >= 2, "irfft2_modes: modes needs at least two dimensions");
    const Impl impl = find_impl(impl_name);
    const int64_t two_m1 = modes.size(-2);
    const int64_t m2 = modes.size(-1);
    TORCH_CHECK(two_m1 % 2 == 0 && two_m1 >= 2 && two_m1 <= n1 && m2 >= 1 && m2 <= n2 / 2 + 1,
                "irfft2_modes: modes of shape (", two_m1, ", ", m2, ") do not fit an output of ",
                n1, " x ", n2);
    std::vector<int64_t> shape = modes.sizes().vec();
    shape[shape.size() - 2] = n1;
    shape.back() = n2;
    at::Tensor y = at::empty(shape, modes.options().dtype(at::kFloat));
    if (modes.numel() == 0) {
        return y;
    }
    const int batch = batch_of(modes, two_m1 * m2, "irfft2_modes");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(modes.device());
    const at::Tensor mc = modes.contiguous();
    const int a = static_cast<int>(n1);
    const int b = static_cast<int>(n2);
    const int p = static_cast<int>(two_m1 / 2);
    const int q = static_cast<int>(m2);
    size_t count = 0;
    check_status(spx_irfft2_modes_workspace(impl.index, a, b, p, q, batch, &count));
    at::Tensor work = workspace(count, modes);
    check_status(spx_irfft2_modes(impl.index, cptr(mc), y.mutable_data_ptr<float>(), a, b, p, q,
                                  batch, work_ptr(work), current_stream()));
    return y;
}

// --- the radio callers: windowed framed spectrum and overlap-save FIR, one kernel each (no
// reference operator; the reference's rf.py composes fft_c2c with torch ops) ----------------

at::Tensor rf_spectrum_op(const at::Tensor& x, const std::optional<at::Tensor>& window,
                          int64_t nfft, c10::string_view impl_name)
{
    check_complex64_cuda(x, "x");
    TORCH_CHECK(x.dim() >= 1, "rf_spectrum: x needs at least one dimension");
    const Impl impl = find_impl(impl_name);
    TORCH_CHECK_VALUE(spx_rf_max_nfft(impl.index) > 0, impl.info.name,
                      " has no fused radio kernels");
    TORCH_CHECK_VALUE(nfft >= 2 && nfft <= spx_rf_max_nfft(impl.index) && (nfft & (nfft - 1)) == 0,
                      "rf_spectrum: nfft must be a power of two from 2 to ",
                      spx_rf_max_nfft(impl.index), ", got ", nfft);
    const int64_t n = x.size(-1);
    const int64_t frames = n > nfft ? (n + nfft - 1) / nfft : 1;
    std::vector<int64_t> shape = x.sizes().vec();
    shape.back() = frames;
    shape.push_back(nfft);
    at::Tensor y = at::empty(shape, x.options());
    const int64_t rows = n > 0 ? x.numel() / n : (x.numel() == 0 ? y.numel() / (frames * nfft) : 0);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const at::Tensor xc = x.contiguous();
    at::Tensor w;
    const float* wp = nullptr;
    if (window.has_value()) {
        w = window->contiguous();
        TORCH_CHECK(w.is_cuda() && w.scalar_type() == at::kFloat && w.numel() == nfft,
                    "rf_spectrum: window must be a float32 CUDA tensor of nfft values");
        wp = w.const_data_ptr<float>();
    }
    if (y.numel() > 0) {
        check_status(spx_rf_spectrum(impl.index, n > 0 ? cptr(xc) : nullptr, wp, mptr(y), n,
                                     static_cast<int>(nfft), rows, current_stream()));
    }
    return y;
}

at::Tensor rf_fir_op(const at::Tensor& x, const at::Tensor& h, int64_t taps, int64_t nfft,
                     c10::string_view impl_name)
{
    check_complex64_cuda(x, "x");
    check_complex64_cuda(h, "h");
    TORCH_CHECK(x.dim() >= 1, "rf_fir: x needs at least one dimension");
    const Impl impl = find_impl(impl_name);
    TORCH_CHECK_VALUE(spx_rf_max_nfft(impl.index) > 0, impl.info.name,
                      " has no fused radio kernels");
    TORCH_CHECK_VALUE(h.numel() == nfft, "rf_fir: h must hold the nfft = ", nfft,
                      " point spectrum of the taps");
    at::Tensor y = at::empty(x.sizes(), x.options());
    const int64_t n = x.size(-1);
    if (x.numel() == 0) {
        return y;
    }
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const at::Tensor xc = x.contiguous();
    const at::Tensor hc = h.contiguous();
    check_status(spx_rf_fir(impl.index, cptr(xc), cptr(hc), mptr(y), n, static_cast<int>(taps),
                            static_cast<int>(nfft), x.numel() / n, current_stream()));
    return y;
}

// The FIR's filter spectrum from its taps (float32 or complex64, on the device), one launch.
at::Tensor rf_fir_spectrum_op(const at::Tensor& taps, int64_t nfft, c10::string_view impl_name)
{
    TORCH_CHECK_VALUE(taps.is_cuda() && (taps.scalar_type() == at::kFloat
                                         || taps.scalar_type() == at::kComplexFloat),
                      "taps must be a float32 or complex64 CUDA tensor, got ", taps.scalar_type(),
                      " on ", taps.device());
    TORCH_CHECK_VALUE(taps.dim() == 1 && taps.numel() >= 1, "taps must be a non-empty 1D tensor");
    const Impl impl = find_impl(impl_name);
    TORCH_CHECK_VALUE(spx_rf_max_nfft(impl.index) > 0, impl.info.name,
                      " has no fused radio kernels");
    at::Tensor h = at::empty({nfft}, taps.options().dtype(at::kComplexFloat));
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(taps.device());
    const at::Tensor tc = taps.contiguous();
    check_status(spx_rf_fir_spectrum(impl.index, tc.data_ptr(),
                                     taps.scalar_type() == at::kComplexFloat ? 1 : 0, mptr(h),
                                     static_cast<int>(taps.numel()), static_cast<int>(nfft),
                                     current_stream()));
    return h;
}

// --- the Navier-Stokes caller: one fused IMEX stage per field (no reference operator; the
// reference's GpuSolver composes its transforms with torch elementwise ops instead) ----------

void check_ns(const at::Tensor& state, const at::Tensor& forcing_hat, const at::Tensor& nu,
              int64_t n)
{
    check_complex64_cuda(state, "state");
    check_complex64_cuda(forcing_hat, "forcing_hat");
    TORCH_CHECK(spx_ns_supports(static_cast<int>(n)) == 1,
                "ns: the fused Navier-Stokes stage supports n = 64 and 128, got ", n);
    const int64_t m = n / 3 + 1;
    TORCH_CHECK(state.dim() >= 2 && state.size(-2) == 2 * m && state.size(-1) == m,
                "ns: state must hold (..., ", 2 * m, ", ", m, ") modes for n = ", n);
    TORCH_CHECK(forcing_hat.numel() == 2 * m * m, "ns: forcing_hat must hold ", 2 * m, " x ", m,
                " modes");
    TORCH_CHECK(nu.is_cuda() && nu.scalar_type() == at::kFloat,
                "ns: nu must be a float32 CUDA tensor");
    const int64_t fields = state.numel() / (2 * m * m);
    TORCH_CHECK(nu.numel() == 1 || nu.numel() == fields,
                "ns: nu must hold one viscosity or one per field");
}

std::tuple<at::Tensor, at::Tensor> ns_predict_op(const at::Tensor& w_hat,
                                                 const at::Tensor& forcing_hat,
                                                 const at::Tensor& nu, double drag, double dt,
                                                 int64_t n)
{
    check_ns(w_hat, forcing_hat, nu, n);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(w_hat.device());
    const at::Tensor w = w_hat.contiguous();
    const at::Tensor fh = forcing_hat.contiguous();
    const at::Tensor nc = nu.contiguous();
    at::Tensor f0 = at::empty_like(w);
    at::Tensor predicted = at::empty_like(w);
    const int64_t m = n / 3 + 1;
    const int batch = batch_of(w, 2 * m * m, "ns_predict");
    if (batch > 0) {
        check_status(spx_ns_stage(cptr(w), nullptr, nullptr, mptr(f0), mptr(predicted),
                                  cptr(fh), nc.const_data_ptr<float>(), nc.numel() == 1 ? 0 : 1,
                                  static_cast<float>(drag), static_cast<float>(dt),
                                  static_cast<int>(n), batch, 0, current_stream()));
    }
    return {f0, predicted};
}

at::Tensor ns_correct_op(const at::Tensor& predicted, const at::Tensor& w_hat,
                         const at::Tensor& f0, const at::Tensor& forcing_hat,
                         const at::Tensor& nu, double drag, double dt, int64_t n)
{
    check_ns(predicted, forcing_hat, nu, n);
    TORCH_CHECK(w_hat.sizes() == predicted.sizes() && f0.sizes() == predicted.sizes(),
                "ns_correct: w_hat, f0 and predicted must have the same shape");
    check_complex64_cuda(w_hat, "w_hat");
    check_complex64_cuda(f0, "f0");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(predicted.device());
    const at::Tensor p = predicted.contiguous();
    const at::Tensor w = w_hat.contiguous();
    const at::Tensor f = f0.contiguous();
    const at::Tensor fh = forcing_hat.contiguous();
    const at::Tensor nc = nu.contiguous();
    at::Tensor out = at::empty_like(p);
    const int64_t m = n / 3 + 1;
    const int batch = batch_of(p, 2 * m * m, "ns_correct");
    if (batch > 0) {
        check_status(spx_ns_stage(cptr(p), cptr(w), cptr(f), nullptr, mptr(out), cptr(fh),
                                  nc.const_data_ptr<float>(), nc.numel() == 1 ? 0 : 1,
                                  static_cast<float>(drag), static_cast<float>(dt),
                                  static_cast<int>(n), batch, 1, current_stream()));
    }
    return out;
}

// `steps` whole steps in one launch into a new tensor (the input is left as it is).
at::Tensor ns_advance_op(const at::Tensor& w_hat, const at::Tensor& forcing_hat,
                         const at::Tensor& nu, double drag, double dt, int64_t n, int64_t steps)
{
    check_ns(w_hat, forcing_hat, nu, n);
    TORCH_CHECK(steps >= 0 && steps < (int64_t{1} << 31),
                "ns_advance: steps must be >= 0 and below 2^31, got ", steps);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(w_hat.device());
    const at::Tensor w = w_hat.contiguous();
    const at::Tensor fh = forcing_hat.contiguous();
    const at::Tensor nc = nu.contiguous();
    at::Tensor out = at::empty_like(w);
    const int64_t m = n / 3 + 1;
    const int batch = batch_of(w, 2 * m * m, "ns_advance");
    if (batch > 0) {
        at::Tensor work = at::empty({2, w.numel()}, w.options());
        check_status(spx_ns_steps(cptr(w), mptr(out), mptr(work), cptr(fh),
                                  nc.const_data_ptr<float>(), nc.numel() == 1 ? 0 : 1,
                                  static_cast<float>(drag), static_cast<float>(dt),
                                  static_cast<int>(n), batch, static_cast<int>(steps),
                                  current_stream()));
    }
    return out;
}

// spectral._C.fft_impls(): the registry's names, in order, as a tuple of str.
PyObject* py_fft_impls(PyObject*, PyObject*)
{
    const int count = spx_impl_count();
    PyObject* names = PyTuple_New(count);
    if (names == nullptr) {
        return nullptr;
    }
    for (int i = 0; i < count; ++i) {
        PyObject* name = PyUnicode_FromString(spx_impl_name(i));
        if (name == nullptr) {
            Py_DECREF(names);
            return nullptr;
        }
        PyTuple_SET_ITEM(names, i, name);  // steals the reference
    }
    return names;
}

// spectral._C.ns_supports(n): whether the fused Navier-Stokes stage has a kernel for an n x n grid.
PyObject* py_ns_supports(PyObject*, PyObject* arg)
{
    const long n = PyLong_AsLong(arg);
    if (n == -1 && PyErr_Occurred() != nullptr) {
        return nullptr;
    }
    return PyBool_FromLong(n > 0 && n < (1L << 30) && spx_ns_supports(static_cast<int>(n)) == 1);
}

PyMethodDef module_methods[] = {
    {"fft_impls", py_fft_impls, METH_NOARGS, "Names of the FFT implementations, in order."},
    {"ns_supports", py_ns_supports, METH_O,
     "Whether the fused Navier-Stokes stage has a kernel for an n x n grid."},
    {nullptr, nullptr, 0, nullptr},
};

}  // namespace

TORCH_LIBRARY(spectral, m)
{
    m.def("scale(Tensor x, float alpha) -> Tensor");
    m.def("fft_c2c(Tensor x, bool inverse=False, str impl=\"naive\") -> Tensor");
    m.def("fft_r2c(Tensor x, str impl=\"naive\") -> Tensor");
    m.def("fft_c2r(Tensor x, int n, str impl=\"naive\") -> Tensor");
    m.def("fft2_c2c(Tensor x, bool inverse=False, str impl=\"naive\", str columns=\"auto\")"
          " -> Tensor");
    m.def("fft2_r2c(Tensor x, str impl=\"naive\", str columns=\"auto\") -> Tensor");
    m.def("fft2_c2r(Tensor x, int n2, str impl=\"naive\", str columns=\"auto\") -> Tensor");
    m.def("fft_c2c_pruned(Tensor x, int n, int keep, bool inverse=False, str impl=\"naive\")"
          " -> Tensor");
    m.def("rfft2_modes(Tensor x, int m1, int m2, str impl=\"naive\") -> Tensor");
    m.def("irfft2_modes(Tensor modes, int n1, int n2, str impl=\"naive\") -> Tensor");
    // The radio callers' fused kernels (no reference operator).
    m.def("rf_spectrum(Tensor x, Tensor? window, int nfft, str impl) -> Tensor");
    m.def("rf_fir(Tensor x, Tensor h, int taps, int nfft, str impl) -> Tensor");
    m.def("rf_fir_spectrum(Tensor taps, int nfft, str impl) -> Tensor");
    // The Navier-Stokes caller's fused stages (no reference operator).
    m.def("ns_predict(Tensor w_hat, Tensor forcing_hat, Tensor nu, float drag, float dt, int n)"
          " -> (Tensor, Tensor)");
    m.def("ns_correct(Tensor predicted, Tensor w_hat, Tensor f0, Tensor forcing_hat, Tensor nu,"
          " float drag, float dt, int n) -> Tensor");
    m.def("ns_advance(Tensor w_hat, Tensor forcing_hat, Tensor nu, float drag, float dt, int n,"
          " int steps) -> Tensor");
}

TORCH_LIBRARY_IMPL(spectral, CUDA, m)
{
    m.impl("scale", &scale_op);
    m.impl("fft_c2c", &fft_c2c_op);
    m.impl("fft_r2c", &fft_r2c_op);
    m.impl("fft_c2r", &fft_c2r_op);
    m.impl("fft2_c2c", &fft2_c2c_op);
    m.impl("fft2_r2c", &fft2_r2c_op);
    m.impl("fft2_c2r", &fft2_c2r_op);
    m.impl("fft_c2c_pruned", &fft_c2c_pruned_op);
    m.impl("rfft2_modes", &rfft2_modes_op);
    m.impl("irfft2_modes", &irfft2_modes_op);
    m.impl("rf_spectrum", &rf_spectrum_op);
    m.impl("rf_fir", &rf_fir_op);
    m.impl("rf_fir_spectrum", &rf_fir_spectrum_op);
    m.impl("ns_predict", &ns_predict_op);
    m.impl("ns_correct", &ns_correct_op);
    m.impl("ns_advance", &ns_advance_op);
}

// Importing spectral._C runs the TORCH_LIBRARY blocks (registering torch.ops.spectral) and
// returns a module holding fft_impls().
PyMODINIT_FUNC PyInit__C(void)
{
    static PyModuleDef module_def = {
        PyModuleDef_HEAD_INIT, "_C", nullptr, -1, module_methods,
    };
    return PyModule_Create(&module_def);
}
