// Two-dimensional FFTs over the last two axes of batch arrays of n1 x n2 (the contract of
// reference fft2d.hpp:3-16: rows then columns, real transforms keep n2/2 + 1 columns on the
// complex side, forward unnormalized, inverse divided by n1 n2).
//
// A request is planned once (plan_2d): the route it takes and the workspace that route needs.
// The workspace queries return the plan's size and the transforms run the plan's route, so the
// two agree by construction. Routes, best first for the strided method:
//
//   SinglePass        the whole array in one workgroup's LDS, one kernel (fft2_fused.hpp)
//   ColumnFirst       real transforms from n2 = 32: columns of the real array read as complex,
//                     then one pass over row pairs (k1, -k1) (fft2_pairs.hpp); no misaligned
//                     half-spectrum rows in the column pass
//   RowsThenColumns   row kernel, then the strided column kernel in place (or, for the
//                     inverse real transform, columns out of place then the real rows)
//   TransposedPasses  the "transpose" method for the Stockham implementations: rows stored
//                     transposed, then the columns as rows of the workspace, stored transposed
//                     back; the transposes ride on the passes' LDS tiles (fft2_transposed.hpp),
//                     two HBM round trips instead of the reference's four (fft2d.cu:138-187)
//   Transposes        the "transpose" method otherwise (naive, arrays with a side of 1, real
//                     rows of 2, and complex arrays with a side beyond 1024): rows, a
//                     transpose, the columns as contiguous rows, a transpose back (remap.hip's
//                     tiled kernel)
//
// The inverse's 1 / (n1 n2) comes from the 1D passes: 1/n2 in the rows, 1/n1 in the columns.

#include "fft_api.hpp"

#include <algorithm>
#include <climits>

// The complex transform's two transposing passes stage T = 8192 / N transforms per workgroup
// beyond 512 points, so at 2048 and 4096 points their transposed side moves runs of only 32 and
// 16 bytes. There the four-kernel route (whole 64 x 64 transpose tiles) measured faster: fft2_c2c
// 2048^2 282.7 -> 180.8 us and 4096^2 471.5 -> 192.9 us over 2^24 points (three alternated
// rounds on MI355X). The real transforms keep the two passes at every size (rfft2 2048^2: 74.4
// against 101.1 us). A larger value here keeps the complex transform's two passes beyond 1024.
#ifndef SPX_TRANSPOSED_PASSES_MAX_C2C
#define SPX_TRANSPOSED_PASSES_MAX_C2C 1024
#endif

namespace spx {
namespace {

enum class Kind { C2c, R2c, C2r };
enum class Route { SinglePass, ColumnFirst, RowsThenColumns, TransposedPasses, Transposes };

struct Plan2d {
    Route route;
    int n1;
    int n2;
    int batch;
    int regions;         // array-sized workspace regions the route passes through (0 .. 2)
    std::size_t region;  // cf32 values per region
    std::size_t real;    // scratch of the generic real rows (implementations that need it)

    std::size_t words() const { return static_cast<std::size_t>(regions) * region + real; }
    cf32* at(cf32* work, int i) const { return work + static_cast<std::size_t>(i) * region; }
    cf32* real_scratch(cf32* work) const
    {
        return real > 0 ? work + static_cast<std::size_t>(regions) * region : nullptr;
    }
};

std::size_t values(int rows, int cols, int batch)
{
    return static_cast<std::size_t>(batch) * static_cast<std::size_t>(rows)
           * static_cast<std::size_t>(cols);
}

// The shape checks and their messages are the reference's API (fft2d.cu:100-128).
void validate(const FftImpl& impl, Columns columns, int n1, int n2, int batch, bool real)
{
    const std::string name = impl.name;
    const int max_n2 = real ? impl.max_real_n : impl.max_n;
    if (!is_pow2(n1) || n1 > impl.max_n) {
        throw InvalidArgument("fft2: " + name + " needs n1 to be a power of two up to "
                              + str(impl.max_n) + ", got " + str(n1));
    }
    if (!is_pow2(n2) || n2 > max_n2 || (real && n2 < 2)) {
        throw InvalidArgument("fft2: " + name + " needs n2 to be a power of two"
                              + (real ? std::string(" from 2") : std::string()) + " up to "
                              + str(max_n2) + ", got " + str(n2));
    }
    if (batch < 1) {
        throw InvalidArgument("fft2: batch must be at least 1, got " + str(batch));
    }
    if (static_cast<long long>(batch) * std::max(n1, n2) > INT_MAX) {
        throw InvalidArgument("fft2: too many transforms");
    }
    if (columns == Columns::Strided && impl.columns == nullptr) {
        throw InvalidArgument("fft2: " + name
                              + " has no strided column kernel; use the transpose method");
    }
}

Plan2d plan_2d(const FftImpl& impl, Columns columns, Kind kind, int n1, int n2, int batch)
{
    validate(impl, columns, n1, n2, batch, kind != Kind::C2c);
    Plan2d p{Route::Transposes, n1, n2, batch, 0, 0, 0};
    const int w = kind == Kind::C2c ? n2 : n2 / 2 + 1;
    const std::size_t real_rows =
        kind != Kind::C2c && impl.real_needs_work ? values(n1, n2 / 2, batch) : 0;
    const Fused2dFns* f = impl.fused;
    if (columns == Columns::Transpose) {
        if (f != nullptr && n1 >= 2 && n2 >= (kind == Kind::C2c ? 2 : 4) &&
            (kind != Kind::C2c || std::max(n1, n2) <= SPX_TRANSPOSED_PASSES_MAX_C2C)) {
            p.route = Route::TransposedPasses;
            p.regions = 1;
            p.region = values(n1, w, batch);
            return p;
        }
        p.regions = 2;
        p.region = values(n1, w, batch);
        p.real = real_rows;
        return p;
    }
    if (kind == Kind::C2c) {
        p.route = f != nullptr && f->c2c_supports(n1, n2) ? Route::SinglePass
                                                          : Route::RowsThenColumns;
        return p;
    }
    if (f != nullptr && f->supports(n1, n2)) {
        p.route = Route::SinglePass;
    } else if (f != nullptr && n2 >= 32) {
        p.route = Route::ColumnFirst;
        p.regions = 1;
        p.region = values(n1, n2 / 2, batch);
    } else {
        p.route = Route::RowsThenColumns;
        p.real = real_rows;
        if (kind == Kind::C2r) {  // columns out of place: the input is the caller's
            p.regions = 1;
            p.region = values(n1, w, batch);
        }
    }
    return p;
}

// batch arrays of rows x cols -> cols x rows
void transpose_arrays(const cf32* x, cf32* y, int rows, int cols, int batch, hipStream_t stream)
{
    const Remap r{cols, rows, cols, static_cast<long long>(rows) * cols, batch,
                  AxisMap::identity(rows), AxisMap::identity(cols)};
    remap(x, y, r, true, stream);
}

}  // namespace

void transpose(const cf32* x, cf32* y, int rows, int cols, int batch, hipStream_t stream)
{
    if (rows < 1 || cols < 1 || batch < 1) {
        throw InvalidArgument("transpose: need rows, cols, batch >= 1");
    }
    transpose_arrays(x, y, rows, cols, batch, stream);
}

std::size_t fft2_c2c_workspace(const FftImpl& impl, Columns columns, int n1, int n2, int batch)
{
    return plan_2d(impl, columns, Kind::C2c, n1, n2, batch).words();
}

std::size_t fft2_r2c_workspace(const FftImpl& impl, Columns columns, int n1, int n2, int batch)
{
    return plan_2d(impl, columns, Kind::R2c, n1, n2, batch).words();
}

std::size_t fft2_c2r_workspace(const FftImpl& impl, Columns columns, int n1, int n2, int batch)
{
    return plan_2d(impl, columns, Kind::C2r, n1, n2, batch).words();
}

void fft2_c2c(const FftImpl& impl, Columns columns, const cf32* x, cf32* y, int n1, int n2,
              int batch, Direction direction, cf32* work, hipStream_t stream)
{
    const Plan2d p = plan_2d(impl, columns, Kind::C2c, n1, n2, batch);
    switch (p.route) {
    case Route::SinglePass:
        impl.fused->c2c(x, y, n1, n2, batch, direction, stream);
        return;
    case Route::RowsThenColumns:
        // The row pass writes y, which the column pass then transforms in place.
        if (impl.fused != nullptr) {
            impl.fused->c2c_rows(x, y, n2, batch * n1, direction, stream);
        } else {
            impl.c2c(x, y, n2, batch * n1, direction, stream);
        }
        impl.columns(y, y, n1, n2, batch, direction, stream);
        return;
    case Route::TransposedPasses:
        impl.fused->c2c_transposed(x, y, p.at(work, 0), n1, n2, batch, direction, stream);
        return;
    default: {
        cf32* a = p.at(work, 0);
        cf32* b = p.at(work, 1);
        impl.c2c(x, a, n2, batch * n1, direction, stream);
        transpose_arrays(a, b, n1, n2, batch, stream);
        impl.c2c(b, a, n1, batch * n2, direction, stream);
        transpose_arrays(a, y, n2, n1, batch, stream);
        return;
    }
    }
}

void fft2_r2c(const FftImpl& impl, Columns columns, const float* x, cf32* y, int n1, int n2,
              int batch, cf32* work, hipStream_t stream)
{
    const Plan2d p = plan_2d(impl, columns, Kind::R2c, n1, n2, batch);
    const int w = n2 / 2 + 1;
    switch (p.route) {
    case Route::SinglePass:
        impl.fused->r2c(x, y, n1, n2, 0, w, batch, stream);
        return;
    case Route::ColumnFirst:
        impl.fused->r2c_columns(reinterpret_cast<const cf32*>(x), p.at(work, 0), n1, n2 / 2,
                                batch, stream);
        impl.fused->r2c_rows(p.at(work, 0), y, n1, n2 / 2, batch, stream);
        return;
    case Route::RowsThenColumns:
        impl.r2c(x, y, n2, batch * n1, p.real_scratch(work), stream);
        impl.columns(y, y, n1, w, batch, Direction::Forward, stream);
        return;
    case Route::TransposedPasses:
        impl.fused->r2c_transposed(x, y, p.at(work, 0), n1, n2, batch, stream);
        return;
    default: {
        cf32* a = p.at(work, 0);
        cf32* b = p.at(work, 1);
        impl.r2c(x, a, n2, batch * n1, p.real_scratch(work), stream);
        transpose_arrays(a, b, n1, w, batch, stream);
        impl.c2c(b, a, n1, batch * w, Direction::Forward, stream);
        transpose_arrays(a, y, w, n1, batch, stream);
        return;
    }
    }
}

void fft2_c2r(const FftImpl& impl, Columns columns, const cf32* x, float* y, int n1, int n2,
              int batch, cf32* work, hipStream_t stream)
{
    const Plan2d p = plan_2d(impl, columns, Kind::C2r, n1, n2, batch);
    const int w = n2 / 2 + 1;
    switch (p.route) {
    case Route::SinglePass:
        impl.fused->c2r(x, y, n1, n2, 0, w, batch, stream);
        return;
    case Route::ColumnFirst:
        impl.fused->c2r_rows(x, p.at(work, 0), n1, n2 / 2, batch, stream);
        impl.columns(p.at(work, 0), reinterpret_cast<cf32*>(y), n1, n2 / 2, batch,
                     Direction::Inverse, stream);
        return;
    case Route::RowsThenColumns:
        impl.columns(x, p.at(work, 0), n1, w, batch, Direction::Inverse, stream);
        impl.c2r(p.at(work, 0), y, n2, batch * n1, p.real_scratch(work), stream);
        return;
    case Route::TransposedPasses:
        impl.fused->c2r_transposed(x, y, p.at(work, 0), n1, n2, batch, stream);
        return;
    default: {
        cf32* a = p.at(work, 0);
        cf32* b = p.at(work, 1);
        transpose_arrays(x, a, n1, w, batch, stream);
        impl.c2c(a, b, n1, batch * w, Direction::Inverse, stream);
        transpose_arrays(b, a, w, n1, batch, stream);
        impl.c2r(a, y, n2, batch * n1, p.real_scratch(work), stream);
        return;
    }
    }
}

}  // namespace spx
