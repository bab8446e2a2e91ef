/*
 * spectral_hip.h: the C ABI of libspectral_hip.so, the MI355X (gfx950) FFT kernels.
 *
 * Every entry point is `extern "C"`, takes plain device pointers, sizes and an explicit HIP
 * stream, returns a status code and throws nothing. Complex data is interleaved float32
 * (re, im), 8 bytes per value: the layout of torch.complex64, std::complex<float> and
 * hipfftComplex. Transforms are batched and out of place, with the transforms of a batch stored
 * back to back; forward transforms are unnormalized and inverse ones divide by n (by n1 * n2 in
 * 2D), the numpy.fft / torch.fft convention.
 *
 * Status codes:
 *   SPX_OK        success; the work is queued on `stream`
 *   SPX_EINVAL    an argument was rejected before anything was queued (the reference raises
 *                 std::invalid_argument there, which PyTorch reports as ValueError)
 *   SPX_ERUNTIME  the HIP runtime reported an error (RuntimeError)
 * spx_last_error() returns the message of the last failure on the calling thread.
 *
 * Implementations are addressed by index into the registry (spx_impl_count / spx_impl_name /
 * spx_impl_find), in the order of the reference's table, csrc/fft/registry.hpp:28-40.
 *
 * Each declaration names the reference interface it replaces (file:line in
 * Jeanm2005/gpu-spectral-stack).
 */
#ifndef SPECTRAL_HIP_H
#define SPECTRAL_HIP_H

#include <stddef.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    SPX_OK = 0,
    SPX_EINVAL = 1,
    SPX_ERUNTIME = 2,
};

/* Column method of the 2D transforms; fft2d.hpp:24 (enum class Columns). */
enum {
    SPX_COLUMNS_TRANSPOSE = 0,
    SPX_COLUMNS_STRIDED = 1,
};

/* One row of the registry; registry.hpp:14-25 (struct FftImpl). Function pointers become
 * has_columns / has_pruned flags: the entry points below dispatch on the index. */
typedef struct spx_impl_info {
    const char* name;
    int has_columns;      /* a strided column kernel exists (FftImpl::columns != nullptr) */
    int has_pruned;       /* pruning inside the kernels (FftImpl::pruned != nullptr) */
    int max_n;            /* largest complex transform in one kernel (2D, pruned) */
    int max_c2c_n;        /* largest 1D complex transform */
    int max_real_n;       /* largest real transform */
    int real_needs_work;  /* r2c / c2r need the `work` buffer */
    int lazy_table;       /* the first call on a device allocates a table (no reference field:
                             spx_c2c_noalloc refuses these) */
} spx_impl_info;

/* --- registry: registry.hpp:28-62 (kFftImpls, find_impl, impl_names), ops.cpp:422-443 ------ */
int spx_impl_count(void);
const char* spx_impl_name(int impl);                  /* NULL when impl is out of range */
int spx_impl_find(const char* name);                  /* index, or -1 */
int spx_impl_get_info(int impl, spx_impl_info* out);
const char* spx_impl_names(void);                     /* "naive, stockham_r2, ..." */

/* Message of the last failed call on this thread ("" if none). */
const char* spx_last_error(void);

/* --- scale: ops/scale.hpp:7 (scale_c2c) ------------------------------------------------------
 * y[i] = alpha * x[i] for n complex values. */
int spx_scale(const void* x, void* y, size_t n, float alpha, hipStream_t stream);

/* --- 1D: fft.hpp:14-16 (C2cFn), :36-39 (R2cFn, C2rFn), :59-60 (ColumnsFn) --------------------
 * c2c: batch transforms of n points (n a power of two up to max_c2c_n).
 * r2c: batch transforms of n reals -> n/2 + 1 complex values; c2r the inverse (divided by n).
 *      `work` holds batch * n/2 complex values when real_needs_work, else may be NULL.
 * columns: slabs row-major arrays of n rows by cols columns; transforms every column, in place
 *      when x == y. Only implementations with has_columns. */
int spx_c2c(int impl, const void* x, void* y, int n, int batch, int inverse, hipStream_t stream);

/* --- c2c without allocation: no counterpart in the reference ----------------------------------
 * For callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments, kernels and results as spx_c2c, but
 * the scratch of the large transforms (n > 16384: n * batch complex values) lives in a static
 * per-device array of SPX_NOALLOC_SCRATCH_VALUES complex values (32 MiB, held by every GPU the
 * library runs on until the process ends), and the call makes no hipMalloc, hipMallocAsync or
 * hipFree. Returns SPX_EINVAL when n * batch exceeds that array (n > 16384), and for
 * stockham_r8_table (its twiddle table is allocated on first use). Calls that overlap on one GPU
 * race on the shared array. */
#define SPX_NOALLOC_SCRATCH_VALUES (1u << 22)
int spx_c2c_noalloc(int impl, const void* x, void* y, int n, int batch, int inverse,
                    hipStream_t stream);
int spx_r2c(int impl, const float* x, void* y, int n, int batch, void* work, hipStream_t stream);
int spx_c2r(int impl, const void* x, float* y, int n, int batch, void* work, hipStream_t stream);
int spx_columns(int impl, const void* x, void* y, int n, int cols, int slabs, int inverse,
                hipStream_t stream);

/* --- pruned kernels of one implementation: fft.hpp:62-76 (struct PrunedFns) ------------------
 * c2c: forward writes the first keep outputs per transform; inverse reads keep inputs per
 *      transform (the rest zero). r2c writes keep of the n/2 + 1 outputs; c2r reads keep of
 *      them (the rest zero). columns: m1_in / m1_out > 0 keep only rows 0 .. m1-1 and
 *      n-m1 .. n-1 on that side; never in place when pruned. Only implementations with
 *      has_pruned. */
int spx_pruned_c2c(int impl, const void* x, void* y, int n, int batch, int keep, int inverse,
                   hipStream_t stream);
int spx_pruned_r2c(int impl, const float* x, void* y, int n, int batch, int keep,
                   hipStream_t stream);
int spx_pruned_c2r(int impl, const void* x, float* y, int n, int batch, int keep,
                   hipStream_t stream);
int spx_pruned_columns(int impl, const void* x, void* y, int n, int cols, int slabs, int m1_in,
                       int m1_out, int inverse, hipStream_t stream);

/* --- 2D: fft2d.hpp:27-39 -------------------------------------------------------------------
 * batch row-major arrays of n1 x n2 (complex side of a real transform: n1 x (n2/2 + 1)).
 * The *_workspace queries give the complex values `work` must hold (0: work may be NULL). */
int spx_fft2_c2c_workspace(int impl, int columns, int n1, int n2, int batch, size_t* count);
int spx_fft2_r2c_workspace(int impl, int columns, int n1, int n2, int batch, size_t* count);
int spx_fft2_c2r_workspace(int impl, int columns, int n1, int n2, int batch, size_t* count);
int spx_fft2_c2c(int impl, int columns, const void* x, void* y, int n1, int n2, int batch,
                 int inverse, void* work, hipStream_t stream);
int spx_fft2_r2c(int impl, int columns, const float* x, void* y, int n1, int n2, int batch,
                 void* work, hipStream_t stream);
int spx_fft2_c2r(int impl, int columns, const void* x, float* y, int n1, int n2, int batch,
                 void* work, hipStream_t stream);
/* y = the transpose of x for batch row-major rows x cols complex arrays; fft2d.hpp:39. */
int spx_transpose(const void* x, void* y, int rows, int cols, int batch, hipStream_t stream);

/* --- pruned drivers: pruned.hpp:26-43 --------------------------------------------------------
 * fft_c2c_pruned: forward (batch, n) -> (batch, keep); inverse (batch, keep) -> (batch, n).
 * rfft2_modes: (batch, n1, n2) real -> (batch, 2 m1, m2) modes, rows 0 .. m1-1 then
 *      n1-m1 .. n1-1 of rfft2, columns 0 .. m2-1. irfft2_modes is its inverse (other modes 0).
 * gather_modes / scatter_modes copy those modes out of / into full n1 x w arrays (m1 = 0: all
 *      n1 rows); scatter zeroes `full` first. */
int spx_fft_c2c_pruned_workspace(int impl, int n, int keep, int batch, size_t* count);
int spx_rfft2_modes_workspace(int impl, int n1, int n2, int m1, int m2, int batch,
                              size_t* count);
int spx_irfft2_modes_workspace(int impl, int n1, int n2, int m1, int m2, int batch,
                               size_t* count);
int spx_fft_c2c_pruned(int impl, const void* x, void* y, int n, int keep, int batch,
                       int inverse, void* work, hipStream_t stream);
int spx_rfft2_modes(int impl, const float* x, void* modes, int n1, int n2, int m1, int m2,
                    int batch, void* work, hipStream_t stream);
int spx_irfft2_modes(int impl, const void* modes, float* y, int n1, int n2, int m1, int m2,
                     int batch, void* work, hipStream_t stream);
int spx_gather_modes(const void* full, void* modes, int n1, int w, int m1, int m2, int batch,
                     hipStream_t stream);
int spx_scatter_modes(const void* modes, void* full, int n1, int w, int m1, int m2, int batch,
                      hipStream_t stream);

/* --- the Navier-Stokes caller -------------------------------------------------------------
 * No counterpart in the reference's FFI: its GpuSolver (python/spectral/flow/gpu.py:115-129)
 * composes the transforms above with torch elementwise kernels. This entry runs one IMEX
 * Crank-Nicolson / Heun stage of that solver per field as a single kernel, for the pruned
 * layout with m = n/3 + 1 ((2m) x m complex modes per field, rows ky = 0 .. m-1 then -m .. -1):
 *   stage 0: out_f = F(state) = f_hat - mask N_hat(state), out_w = (e state + dt F) i
 *   stage 1: out_w = (e w0 + dt/2 (f0 + F(state))) i
 * with e = 1 + dt/2 L, i = 1 / (1 - dt/2 L), L = -nu |k|^2 - drag, nu = nu[field * nu_stride]
 * (nu_stride 0: one viscosity for all fields). forcing_hat: (2m) x m modes shared by all fields.
 * spx_ns_supports(n) is 1 for the grid sizes with a kernel (64, 128). */
int spx_ns_supports(int n);
int spx_ns_stage(const void* state, const void* w0, const void* f0, void* out_f, void* out_w,
                 const void* forcing_hat, const float* nu, int nu_stride, float drag, float dt,
                 int n, int batch, int stage, hipStream_t stream);
/* spx_ns_steps: `steps` whole steps (stage 0, then stage 1, as spx_ns_stage computes them) of
 * every field in one launch, to float32 rounding the arithmetic of alternating spx_ns_stage
 * calls. The first step reads w_in and writes w_out; later steps advance w_out in place. w_in and
 * w_out ((2m) x m modes per field) are the same array or do not overlap. `work` holds
 * 2 * batch * (2m) * m complex values (each field's tendency and predictor; after the call, the
 * last step's) and overlaps neither, nor forcing_hat. steps = 0 copies w_in to w_out. No
 * counterpart in the reference: its solver launches every step's kernels from Python
 * (python/spectral/flow/gpu.py:125-142). */
int spx_ns_steps(const void* w_in, void* w_out, void* work, const void* forcing_hat,
                 const float* nu, int nu_stride, float drag, float dt, int n, int batch,
                 int steps, hipStream_t stream);

/* --- the radio callers -------------------------------------------------------------------
 * No counterpart in the reference's FFI: its rf.spectrum and rf.fir (python/spectral/rf.py:94-153)
 * compose fft_c2c with torch ops. These run each as one kernel on rows of n complex samples, for
 * the implementations with such kernels (spx_rf_max_nfft(impl) > 0: the Stockham variants), nfft
 * a power of two from 2 to spx_rf_max_nfft(impl).
 *   spx_rf_spectrum  y (rows, F, nfft), F = ceil(n / nfft) (1 when n <= nfft): the FFT of frame f
 *                    of each row, x[f nfft .. f nfft + nfft) zero-padded past n, times window
 *                    (nfft floats; NULL for the rectangular window).
 *   spx_rf_fir       y (rows, n): x filtered by a causal FIR of `taps` taps (1 <= taps <= nfft)
 *                    with zero initial state, by overlap-save in blocks of nfft; h is the nfft-point
 *                    forward FFT of the taps zero-padded to nfft (complex64).
 *   spx_rf_fir_spectrum  that h from `count` taps (float32, or complex64 when complex_taps != 0),
 *                    1 <= count <= nfft, in one launch; it replaces rf.py:145-147 (zeros, a copy
 *                    of the converted taps, fft). */
int spx_rf_max_nfft(int impl);
int spx_rf_spectrum(int impl, const void* x, const float* window, void* y, long long n, int nfft,
                    long long rows, hipStream_t stream);
int spx_rf_fir(int impl, const void* x, const void* h, void* y, long long n, int taps, int nfft,
               long long rows, hipStream_t stream);
int spx_rf_fir_spectrum(int impl, const void* taps, int complex_taps, void* h, int count,
                        int nfft, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SPECTRAL_HIP_H */
