// Two-dimensional FFTs from the 1D kernels (reference fft2d.hpp:3-16, fft2d.cu:15-187): rows
// first, then the columns either in place with the strided column kernel ("strided"), or by
// transposing, running rows, and transposing back ("transpose", every implementation). Real
// transforms keep n2/2 + 1 columns on the complex side. Forward unnormalized; the inverse divides
// by n1 * n2, split between the two passes (1/n2 in the rows, 1/n1 in the columns).
//
// The transpose is an LDS-tiled 64 x 64 copy sized for wave64: each wavefront reads one tile row
// of 64 complex values (512 contiguous bytes) and writes one transposed row, through a tile padded
// to 65 columns so the column-order LDS reads fall in distinct banks.

#include "fft_api.hpp"

#include <algorithm>
#include <climits>

namespace spx {
namespace {

constexpr int kTile = 64;
constexpr int kTileRows = 4;  // 64 x 4 lanes move a 64 x 64 tile in 16 steps

__global__ void __launch_bounds__(kTile * kTileRows)
    transpose_kernel(const cf32* __restrict__ x, cf32* __restrict__ y, int rows, int cols,
                     int batch)
{
    __shared__ cf32 tile[kTile][kTile + 1];
    const std::size_t size = static_cast<std::size_t>(rows) * static_cast<std::size_t>(cols);
    const int tx = threadIdx.x;  // 0 .. 63
    const int ty = threadIdx.y;  // 0 .. 3
    for (int b = blockIdx.z; b < batch; b += gridDim.z) {
        const cf32* xs = x + static_cast<std::size_t>(b) * size;
        cf32* ys = y + static_cast<std::size_t>(b) * size;
        const int c = blockIdx.x * kTile + tx;
#pragma unroll
        for (int k = 0; k < kTile; k += kTileRows) {
            const int r = blockIdx.y * kTile + ty + k;
            if (r < rows && c < cols) {
                tile[ty + k][tx] = xs[static_cast<std::size_t>(r) * cols + c];
            }
        }
        __syncthreads();
        const int r_out = blockIdx.y * kTile + tx;  // a row of y is a column of x
#pragma unroll
        for (int k = 0; k < kTile; k += kTileRows) {
            const int c_out = blockIdx.x * kTile + ty + k;
            if (r_out < rows && c_out < cols) {
                ys[static_cast<std::size_t>(c_out) * rows + r_out] = tile[tx][ty + k];
            }
        }
        __syncthreads();  // the tile is reused for the next array
    }
}

std::size_t count(int n1, int n2, int batch)
{
    return static_cast<std::size_t>(batch) * static_cast<std::size_t>(n1)
           * static_cast<std::size_t>(n2);
}

// Throws unless the shape suits the implementation, the method exists, and every intermediate
// transform count fits an int (reference fft2d.cu:100-128, same messages).
void check(const FftImpl& impl, Columns columns, int n1, int n2, int batch, bool real)
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

std::size_t real_work(const FftImpl& impl, int n1, int n2, int batch)
{
    return impl.real_needs_work ? count(n1, n2 / 2, batch) : 0;
}

// The strided method runs as one single-pass kernel when the implementation has one for the shape.
bool fused(const FftImpl& impl, Columns columns, int n1, int n2)
{
    return columns == Columns::Strided && impl.fused != nullptr && impl.fused->supports(n1, n2);
}

// Otherwise, from n2 = 32, column-first (fft2_pairs.hpp): columns over the real array read as
// n1 x n2/2 complex values, whose rows are whole 128-byte lines, and one row-pair pass on the
// other side; the row-then-column order would run its column pass over half-spectrum rows of
// n2/2 + 1 values, misaligned.
bool column_first(const FftImpl& impl, Columns columns, int n1, int n2)
{
    return columns == Columns::Strided && impl.fused != nullptr && !impl.fused->supports(n1, n2)
           && n2 >= 32;
}

}  // namespace

void transpose(const cf32* x, cf32* y, int rows, int cols, int batch, hipStream_t stream)
{
    if (rows < 1 || cols < 1 || batch < 1) {
        throw InvalidArgument("transpose: need rows, cols, batch >= 1");
    }
    const dim3 block(kTile, kTileRows);
    const dim3 grid(static_cast<unsigned>((cols + kTile - 1) / kTile),
                    static_cast<unsigned>((rows + kTile - 1) / kTile),
                    static_cast<unsigned>(std::min(batch, 65535)));
    hipLaunchKernelGGL(transpose_kernel, grid, block, 0, stream, x, y, rows, cols, batch);
    SPX_LAUNCH_CHECK();
}

std::size_t fft2_c2c_workspace(const FftImpl&, Columns columns, int n1, int n2, int batch)
{
    return columns == Columns::Strided ? 0 : 2 * count(n1, n2, batch);
}

void fft2_c2c(const FftImpl& impl, Columns columns, const cf32* x, cf32* y, int n1, int n2,
              int batch, Direction direction, cf32* work, hipStream_t stream)
{
    check(impl, columns, n1, n2, batch, false);
    if (columns == Columns::Strided && impl.fused != nullptr && impl.fused->c2c_supports(n1, n2)) {
        impl.fused->c2c(x, y, n1, n2, batch, direction, stream);
        return;
    }
    if (columns == Columns::Strided) {
        if (impl.fused != nullptr) {
            impl.fused->c2c_rows(x, y, n2, batch * n1, direction, stream);
        } else {
            impl.c2c(x, y, n2, batch * n1, direction, stream);
        }
        impl.columns(y, y, n1, n2, batch, direction, stream);
        return;
    }
    cf32* a = work;
    cf32* b = work + count(n1, n2, batch);
    impl.c2c(x, a, n2, batch * n1, direction, stream);
    transpose(a, b, n1, n2, batch, stream);
    impl.c2c(b, a, n1, batch * n2, direction, stream);
    transpose(a, y, n2, n1, batch, stream);
}

std::size_t fft2_r2c_workspace(const FftImpl& impl, Columns columns, int n1, int n2, int batch)
{
    if (fused(impl, columns, n1, n2)) {
        return 0;
    }
    if (column_first(impl, columns, n1, n2)) {
        return count(n1, n2 / 2, batch);
    }
    const std::size_t half = columns == Columns::Strided ? 0 : 2 * count(n1, n2 / 2 + 1, batch);
    return half + real_work(impl, n1, n2, batch);
}

void fft2_r2c(const FftImpl& impl, Columns columns, const float* x, cf32* y, int n1, int n2,
              int batch, cf32* work, hipStream_t stream)
{
    check(impl, columns, n1, n2, batch, true);
    const int w = n2 / 2 + 1;
    if (fused(impl, columns, n1, n2)) {
        impl.fused->r2c(x, y, n1, n2, 0, w, batch, stream);
        return;
    }
    if (column_first(impl, columns, n1, n2)) {
        impl.fused->r2c_columns(reinterpret_cast<const cf32*>(x), work, n1, n2 / 2, batch, stream);
        impl.fused->r2c_rows(work, y, n1, n2 / 2, batch, stream);
        return;
    }
    if (columns == Columns::Strided) {
        cf32* rwork = impl.real_needs_work ? work : nullptr;
        impl.r2c(x, y, n2, batch * n1, rwork, stream);
        impl.columns(y, y, n1, w, batch, Direction::Forward, stream);
        return;
    }
    cf32* a = work;
    cf32* b = work + count(n1, w, batch);
    cf32* rwork = impl.real_needs_work ? work + 2 * count(n1, w, batch) : nullptr;
    impl.r2c(x, a, n2, batch * n1, rwork, stream);
    transpose(a, b, n1, w, batch, stream);
    impl.c2c(b, a, n1, batch * w, Direction::Forward, stream);
    transpose(a, y, w, n1, batch, stream);
}

std::size_t fft2_c2r_workspace(const FftImpl& impl, Columns columns, int n1, int n2, int batch)
{
    if (fused(impl, columns, n1, n2)) {
        return 0;
    }
    const std::size_t q = count(n1, n2 / 2 + 1, batch);
    return (columns == Columns::Strided ? q : 2 * q) + real_work(impl, n1, n2, batch);
}

void fft2_c2r(const FftImpl& impl, Columns columns, const cf32* x, float* y, int n1, int n2,
              int batch, cf32* work, hipStream_t stream)
{
    check(impl, columns, n1, n2, batch, true);
    const int w = n2 / 2 + 1;
    if (fused(impl, columns, n1, n2)) {
        impl.fused->c2r(x, y, n1, n2, 0, w, batch, stream);
        return;
    }
    if (column_first(impl, columns, n1, n2)) {
        // The workspace holds n1 x (n2/2 + 1) per array, more than the n1 x n2/2 used here.
        impl.fused->c2r_rows(x, work, n1, n2 / 2, batch, stream);
        impl.columns(work, reinterpret_cast<cf32*>(y), n1, n2 / 2, batch, Direction::Inverse,
                     stream);
        return;
    }
    const std::size_t q = count(n1, w, batch);
    if (columns == Columns::Strided) {
        // Columns first, out of place (the input is the caller's), then the real rows.
        cf32* a = work;
        cf32* rwork = impl.real_needs_work ? work + q : nullptr;
        impl.columns(x, a, n1, w, batch, Direction::Inverse, stream);
        impl.c2r(a, y, n2, batch * n1, rwork, stream);
        return;
    }
    cf32* a = work;
    cf32* b = work + q;
    cf32* rwork = impl.real_needs_work ? work + 2 * q : nullptr;
    transpose(x, a, n1, w, batch, stream);
    impl.c2c(a, b, n1, batch * w, Direction::Inverse, stream);
    transpose(b, a, w, n1, batch, stream);
    impl.c2r(a, y, n2, batch * n1, rwork, stream);
}

}  // namespace spx
