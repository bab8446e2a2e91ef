#pragma once

// The library's internal C++ interface: entry-point contracts, the registry row, and the 2D and
// pruned drivers. The C ABI (capi.cpp, include/spectral_hip.h) is a thin layer over this.
//
// Conventions, as numpy.fft and torch.fft (reference fft.hpp:1-5): batched and out of place,
// transforms of a batch back to back, forward unnormalized, inverse divided by n.

#include "spx_common.hpp"

#include <cstddef>

namespace spx {

constexpr int kStockhamMaxN = 4096;                          // one kernel, LDS-resident
constexpr int kFourStepMaxN = kStockhamMaxN * kStockhamMaxN;  // 2^24 (reference fft.hpp:18-21)
// C2C sizes above kStockhamMaxN that still run as one kernel per transform (the whole transform
// in one workgroup's LDS); the multi-pass splits take over beyond.
constexpr int kSinglePassMaxN = 16384;
// Above that, up to kTwoPassMaxN, a column pass and a row pass that stores transposed; beyond,
// the column pass itself runs as two. SPX_TWO_PASS_MAX_LOG2 overrides it in a variant build,
// to measure the three-pass split at sizes the two-pass one serves.
#ifndef SPX_TWO_PASS_MAX_LOG2
#define SPX_TWO_PASS_MAX_LOG2 20
#endif
constexpr int kTwoPassMaxN = 1 << SPX_TWO_PASS_MAX_LOG2;

// reference fft.hpp:14-15, 36-39, 59-60
using C2cFn = void (*)(const cf32* x, cf32* y, int n, int batch, Direction direction,
                       hipStream_t stream);
using R2cFn = void (*)(const float* x, cf32* y, int n, int batch, cf32* work,
                       hipStream_t stream);
using C2rFn = void (*)(const cf32* x, float* y, int n, int batch, cf32* work,
                       hipStream_t stream);
using ColumnsFn = void (*)(const cf32* x, cf32* y, int n, int cols, int slabs,
                           Direction direction, hipStream_t stream);
using C2cWorkFn = void (*)(const cf32* x, cf32* y, int n, int batch, Direction direction,
                           cf32* work, hipStream_t stream);

// reference fft.hpp:62-72
struct PrunedFns {
    void (*c2c)(const cf32* x, cf32* y, int n, int batch, int keep, Direction direction,
                hipStream_t stream);
    void (*r2c)(const float* x, cf32* y, int n, int batch, int keep, hipStream_t stream);
    void (*c2r)(const cf32* x, float* y, int n, int batch, int keep, hipStream_t stream);
    void (*columns)(const cf32* x, cf32* y, int n, int cols, int slabs, int m1_in, int m1_out,
                    Direction direction, hipStream_t stream);
    // r2c and columns into a workspace that the next pass reads (plain stores): the two-pass
    // rfft2_modes / irfft2_modes.
    void (*r2c_work)(const float* x, cf32* y, int n, int batch, int keep, hipStream_t stream);
    void (*columns_work)(const cf32* x, cf32* y, int n, int cols, int slabs, int m1_in,
                         int m1_out, Direction direction, hipStream_t stream);
};

// Single-pass 2D real transforms for the shapes whose half spectrum fits in LDS (fft2_fused.hpp):
// one kernel and one HBM round trip instead of a row pass and a column pass. They keep rows 0 ..
// n1-1 (m1 = 0) or 0 .. m1-1 and n1-m1 .. n1-1 (m1 > 0), and columns 0 .. w-1 of the half
// spectrum; the inverse reads that layout with every other frequency zero.
struct Fused2dFns {
    bool (*supports)(int n1, int n2);
    void (*r2c)(const float* x, cf32* y, int n1, int n2, int m1, int w, int batch,
                hipStream_t stream);
    void (*c2r)(const cf32* x, float* y, int n1, int n2, int m1, int w, int batch,
                hipStream_t stream);
    // The column-first forward's column pass: x (batch x n1 x m packed real rows) -> z, the
    // workspace the row-pair pass reads (kept in the caches where it can be).
    void (*r2c_columns)(const cf32* x, cf32* z, int n1, int m, int batch, hipStream_t stream);
    // Row-pair passes of the column-first 2D real transforms (fft2_pairs.hpp), m = n2 / 2 from
    // 16 to 4096: z (batch x n1 x m, column-transformed packed rows) -> y (batch x n1 x (m + 1)),
    // and x (batch x n1 x (m + 1)) -> z (prepared, row-inverted, scaled by 1 / m).
    void (*r2c_rows)(const cf32* z, cf32* y, int n1, int m, int batch, hipStream_t stream);
    void (*c2r_rows)(const cf32* x, cf32* z, int n1, int m, int batch, hipStream_t stream);
    // Single-pass complex 2D (batch arrays of n1 x n2) where c2c_supports(n1, n2).
    bool (*c2c_supports)(int n1, int n2);
    void (*c2c)(const cf32* x, cf32* y, int n1, int n2, int batch, Direction direction,
                hipStream_t stream);
    // The row pass of the row-then-column complex 2D (batch rows of n), into y, which the column
    // pass then transforms in place (plain stores).
    void (*c2c_rows)(const cf32* x, cf32* y, int n, int batch, Direction direction,
                     hipStream_t stream);
    // The "transpose" column method in two passes that transpose through their LDS tiles
    // (fft2_transposed.hpp), n1 >= 2 and n2 >= 2 (complex) or 4 (real): work holds batch arrays
    // of n2 x n1 (complex) or (n2/2 + 1) x n1 (real) values.
    void (*c2c_transposed)(const cf32* x, cf32* y, cf32* work, int n1, int n2, int batch,
                           Direction direction, hipStream_t stream);
    void (*r2c_transposed)(const float* x, cf32* y, cf32* work, int n1, int n2, int batch,
                           hipStream_t stream);
    void (*c2r_transposed)(const cf32* x, float* y, cf32* work, int n1, int n2, int batch,
                           hipStream_t stream);
};

// The radio callers (rf.hpp): windowed spectrum of back-to-back frames, and overlap-save FIR.
// Rows of n complex samples; nfft a power of two from 2 to max_nfft.
struct RfFns {
    // y (rows, ceil(n / nfft) or 1, nfft) = FFT of each frame of x times window (nullptr: rect).
    void (*spectrum)(const cf32* x, const float* window, cf32* y, long long n, int nfft,
                     long long rows, hipStream_t stream);
    // y (rows, n) = x filtered by the taps whose nfft-point spectrum is h (taps <= nfft).
    void (*fir)(const cf32* x, const cf32* h, cf32* y, long long n, int taps, int nfft,
                long long rows, hipStream_t stream);
    // h (nfft) = FFT of the taps (float32, or complex64 when complex_taps) zero-padded to nfft.
    void (*filter)(const void* taps, bool complex_taps, cf32* h, int count, int nfft,
                   hipStream_t stream);
    int max_nfft;
};

// One implementation, by name (reference registry.hpp:14-25).
struct FftImpl {
    const char* name;
    C2cFn c2c;
    R2cFn r2c;
    C2rFn c2r;
    ColumnsFn columns;        // strided column transforms, or nullptr (2D then transposes)
    const PrunedFns* pruned;  // pruning inside the kernels, or nullptr (gather / scatter)
    int max_n;                // largest complex transform in one kernel (2D, pruned)
    int max_c2c_n;            // largest 1D complex transform
    int max_real_n;           // largest real transform
    bool real_needs_work;     // r2c and c2r use the work buffer
    const Fused2dFns* fused;  // single-pass 2D kernels, or nullptr
    const RfFns* rf;          // the radio callers' fused kernels, or nullptr
    // c2c with the caller's scratch for the sizes that need one (c2c_scratch_values), instead
    // of scratch allocated on the stream; nullptr when no size needs scratch.
    C2cWorkFn c2c_work;
    // The first call on a device allocates a per-device table (twiddle_table), so the entry
    // points that promise no allocation refuse this implementation.
    bool lazy_table;
};

// Scratch values c2c_work needs for batch transforms of n points: n x batch beyond the
// single-pass sizes (the two- and three-pass intermediates), none up to kSinglePassMaxN.
std::size_t c2c_scratch_values(const FftImpl& impl, int n, int batch);

// c2c that allocates nothing (noalloc.hip): large transforms use a static per-device scratch of
// kNoAllocScratchValues values. Throws InvalidArgument past that, or for an implementation whose
// first call allocates a table.
constexpr std::size_t kNoAllocScratchValues = std::size_t(1) << 22;  // 32 MiB of cf32
void c2c_noalloc(const FftImpl& impl, const cf32* x, cf32* y, int n, int batch,
                 Direction direction, hipStream_t stream);

// The registry, in the reference's order (registry.hpp:28-40).
const FftImpl* impls();
int impl_count();

// --- naive radix-2 and the generic real path (naive.hip, real.hip) -------------------------
void c2c_naive(const cf32* x, cf32* y, int n, int batch, Direction direction,
               hipStream_t stream);
void r2c_naive(const float* x, cf32* y, int n, int batch, cf32* work, hipStream_t stream);
void c2r_naive(const cf32* x, float* y, int n, int batch, cf32* work, hipStream_t stream);
void r2c_via_c2c(C2cFn c2c, const float* x, cf32* y, int n, int batch, cf32* work,
                 hipStream_t stream);
void c2r_via_c2c(C2cFn c2c, const cf32* x, float* y, int n, int batch, cf32* work,
                 hipStream_t stream);

// --- scale (scale.hip) ----------------------------------------------------------------------
void scale_c2c(const cf32* x, cf32* y, std::size_t n, float alpha, hipStream_t stream);

// --- index remaps (remap.hip): transposes, mode gathers and mode scatters ---------------------
//
// Where output index i along one axis reads along the input axis, or -1 for a zero:
//   Identity  i -> i while i < limit
//   Keep      kept position -> full position, the FNO rows: i < m1 ? i : i + n - 2 m1
//             (m1 = 0 keeps every position: i -> i while i < n)
//   Spread    full position -> kept position, the inverse of Keep (-1 for a dropped one),
//             and -1 past `limit` kept positions when the axis is narrowed
struct AxisMap {
    enum Kind : int { Identity, Keep, Spread };
    Kind kind;
    int n;
    int m1;
    int limit;

    static AxisMap identity(int limit) { return {Identity, limit, 0, limit}; }
    static AxisMap keep(int n, int m1) { return {Keep, n, m1, m1 > 0 ? 2 * m1 : n}; }
    static AxisMap spread(int n, int m1) { return {Spread, n, m1, n}; }

    __host__ __device__ int operator()(int i) const
    {
        if (kind == Identity) {
            return i < limit ? i : -1;
        }
        if (kind == Keep) {
            return m1 == 0 || i < m1 ? i : i + n - 2 * m1;
        }
        if (m1 == 0 || i < m1) {
            return i < limit ? i : -1;
        }
        return i >= n - m1 ? i - n + 2 * m1 : -1;
    }
};

// batch arrays: y (y_rows x y_cols per array, dense) from x (x_array values per array, rows of
// x_pitch). Not transposed: y[q][p] = x[rows(q)][cols(p)]. Transposed: y[q][p] = x[rows(p)][cols(q)].
// A -1 from either map writes a zero, so a scatter fills the whole output in the same pass.
struct Remap {
    int y_rows;
    int y_cols;
    long long x_pitch;
    long long x_array;
    int batch;
    AxisMap rows;
    AxisMap cols;
};
void remap(const cf32* x, cf32* y, const Remap& r, bool transposed, hipStream_t stream);

// --- 2D (fft2d.hip), reference fft2d.hpp:24-39 -----------------------------------------------
enum class Columns { Transpose, Strided };

std::size_t fft2_c2c_workspace(const FftImpl& impl, Columns columns, int n1, int n2, int batch);
std::size_t fft2_r2c_workspace(const FftImpl& impl, Columns columns, int n1, int n2, int batch);
std::size_t fft2_c2r_workspace(const FftImpl& impl, Columns columns, int n1, int n2, int batch);
void fft2_c2c(const FftImpl& impl, Columns columns, const cf32* x, cf32* y, int n1, int n2,
              int batch, Direction direction, cf32* work, hipStream_t stream);
void fft2_r2c(const FftImpl& impl, Columns columns, const float* x, cf32* y, int n1, int n2,
              int batch, cf32* work, hipStream_t stream);
void fft2_c2r(const FftImpl& impl, Columns columns, const cf32* x, float* y, int n1, int n2,
              int batch, cf32* work, hipStream_t stream);
void transpose(const cf32* x, cf32* y, int rows, int cols, int batch, hipStream_t stream);

// --- pruned (pruned.hip), reference pruned.hpp:26-43 -----------------------------------------
std::size_t fft_c2c_pruned_workspace(const FftImpl& impl, int n, int keep, int batch);
std::size_t rfft2_modes_workspace(const FftImpl& impl, int n1, int n2, int m1, int m2, int batch);
std::size_t irfft2_modes_workspace(const FftImpl& impl, int n1, int n2, int m1, int m2,
                                   int batch);
void fft_c2c_pruned(const FftImpl& impl, const cf32* x, cf32* y, int n, int keep, int batch,
                    Direction direction, cf32* work, hipStream_t stream);
void rfft2_modes(const FftImpl& impl, const float* x, cf32* modes, int n1, int n2, int m1,
                 int m2, int batch, cf32* work, hipStream_t stream);
void irfft2_modes(const FftImpl& impl, const cf32* modes, float* y, int n1, int n2, int m1,
                  int m2, int batch, cf32* work, hipStream_t stream);
void gather_modes(const cf32* full, cf32* modes, int n1, int w, int m1, int m2, int batch,
                  hipStream_t stream);
void scatter_modes(const cf32* modes, cf32* full, int n1, int w, int m1, int m2, int batch,
                   hipStream_t stream);

// --- the Navier-Stokes caller (ns.hip): one fused IMEX stage per field ----------------------
// Modes in the FNO layout with m = n/3 + 1 ((2m) x m per field). stage 0: out_f = F(state),
// out_w = the predictor; stage 1: out_w = the corrector from w0, f0 and F(state).
bool ns_supports(int n);
void ns_stage(const cf32* state, const cf32* w0, const cf32* f0, cf32* out_f, cf32* out_w,
              const cf32* forcing_hat, const float* nu, int nu_stride, float drag, float dt,
              int n, int batch, int stage, hipStream_t stream);
// `steps` whole steps in one launch from w_in to w_out (the same array, or disjoint ones); work
// holds 2 batch (2m) m values (each field's tendency and predictor).
void ns_steps(const cf32* w_in, cf32* w_out, cf32* work, const cf32* forcing_hat,
              const float* nu, int nu_stride, float drag, float dt, int n, int batch, int steps,
              hipStream_t stream);

}  // namespace spx

// --- the Stockham variants (stockham_*.hip) ---------------------------------------------------
#define SPX_DECLARE_VARIANT(NAME)                                                               \
    void c2c_##NAME(const cf32* x, cf32* y, int n, int batch, Direction direction,             \
                    hipStream_t stream);                                                        \
    void c2c_work_##NAME(const cf32* x, cf32* y, int n, int batch, Direction direction,        \
                         cf32* work, hipStream_t stream);                                       \
    void r2c_##NAME(const float* x, cf32* y, int n, int batch, cf32* work, hipStream_t stream); \
    void c2r_##NAME(const cf32* x, float* y, int n, int batch, cf32* work, hipStream_t stream); \
    void columns_##NAME(const cf32* x, cf32* y, int n, int cols, int slabs,                    \
                        Direction direction, hipStream_t stream);                               \
    extern const PrunedFns pruned_##NAME;                                                      \
    extern const Fused2dFns fused_##NAME;                                                      \
    extern const RfFns rf_##NAME;

namespace spx {
SPX_DECLARE_VARIANT(stockham_r2)
SPX_DECLARE_VARIANT(stockham_r4)
SPX_DECLARE_VARIANT(stockham_r8)
SPX_DECLARE_VARIANT(stockham_r8_table)
}  // namespace spx
