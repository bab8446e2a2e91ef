// Index remaps: one pass that copies batch arrays through a row map and a column map, either in
// the same orientation or transposed. It is the transpose of the 2D "transpose" method, the
// gather of FNO modes out of a full half spectrum, and the scatter back (whose zeros it writes in
// the same pass: every output value is written exactly once).
//
// Design for gfx950 (wave64, LDS of 64 banks of 4 bytes, read by half-waves for 8-byte values):
//
// * Transposed: a workgroup of eight waves moves a 64 x 64 tile of complex values. A wave reads
//   one input row segment per step (64 lanes x 8 bytes, 512 contiguous bytes), holds all 8 of
//   its steps' loads in registers before touching LDS (every load in flight together), then
//   writes them to the tile; after one barrier it reads tile columns and writes output rows,
//   again 512 contiguous bytes per wave step. Against four waves of 16 steps: 2-5 % faster on
//   1024 x 16384 matrices and on 512 x 257 spectra, equal elsewhere; 16-byte accesses
//   (pairs of values per lane) were 7-28 % slower.
//   The tile is unpadded and XOR-swizzled: element (p, q) sits at p * 64 + (q ^ (p mod 32)).
//   A half-wave writing a row (fixed p, 32 consecutive q) and a half-wave reading a column
//   (fixed q, 32 consecutive p) both cover 32 distinct 8-byte bank slots, so neither phase has a
//   bank conflict (SQ_LDS_BANK_CONFLICT reads 0), and the tile needs no padding column (32 KiB;
//   four workgroups of eight waves fill a CU).
//   The grid is those resident workgroups (persistent), each looping over tiles and issuing its
//   next tile's loads as soon as the current tile is in LDS, so they are in flight during the
//   current tile's column reads and stores (bounded to 64 VGPRs, eight waves per SIMD). Against
//   one tile per workgroup, three alternated rounds of the transpose method: 512^2 x 64
//   100.2-100.6 -> 97.7-98.0 us (rfft2) and 95.0-95.4 -> 93.1-93.3 us (irfft2); 128^2 x 1024
//   0.5 % faster. Two or three resident workgroups per CU, each with more tiles, ran the same
//   (within 0.5 us).
// * Not transposed: each output row is walked by a power-of-two group of lanes as wide as the row
//   (up to a wave), so short rows (16 modes) still fill whole waves with several rows each. The
//   row and column maps are evaluated per lane; no flat-index division per value.
// * Transposed, a size of 64k + 1 (a real spectrum's n/2 + 1 values): the last full tile's
//   workgroup also copies the one row or column past it, straight from HBM to HBM, so no
//   workgroup carries a 64 x 1 sliver tile (whose 64 strided loads and near-idle lanes made
//   128 x 65 transposes take 37.7 us against 26.0 us for 128 x 64; now 28.3 us).
// * Output rows that do not start on 128-byte lines (a width not a multiple of 16 values): runs of
//   8 consecutive tiles go to one XCD (xcd_grouped), so the partial lines that neighbouring tiles
//   share meet in one L2: 257 x 512 -> 512 x 257 went 33.0 -> 28.4 us.
// * Transposed, arrays with fewer than 32 rows or columns: one lane per output value, the arrays
//   walked flat (stores coalesced; an array's reads stay within a few cache lines). A 64 x 64 tile
//   per array would leave most of each workgroup idle: at 4 x 3 arrays (2^24-point 4 x 4 real
//   transforms) the tiles took 5.2 ms where the flat walk takes tens of microseconds.

#include "fft_api.hpp"

#include <algorithm>
#include <climits>

namespace spx {
namespace {

constexpr int kThreads = 256;      // the row remap's workgroup
constexpr int kTileThreads = 512;  // the transposed remap's: eight waves
constexpr int kTile = 64;
constexpr int kSteps = kTile / (kTileThreads / 64);  // tile rows per wave: 8
constexpr int kTilesPerCu = 4;                       // resident tile workgroups per CU
constexpr int kTileWavesPerSimd = kTilesPerCu * kTileThreads / 64 / 4;  // 8: at most 64 VGPRs
constexpr long long kMaxBlocks = 1 << 20;        // the loops below cover any remainder

__device__ __forceinline__ cf32 zero() { return cf32{0.0f, 0.0f}; }

// extra_p / extra_q: the output has one column / row past its last full tile (a width of
// 64k + 1, as a real spectrum's n/2 + 1 values): the workgroup of that last tile copies it
// directly, one value per lane, instead of a workgroup per sliver tile of 64 x 1 (which made
// 128 x 65 transposes 45 % slower than 128 x 64 ones).
// Workgroup b runs on XCD b mod 8, each XCD with its own L2. With group > 1, each span of
// 8 group workgroups is renumbered so that every XCD takes `group` consecutive tiles (tiles
// next to each other in the output, which share the partial cache lines of rows that do not
// start on a line); a trailing partial span keeps its order.
__device__ __forceinline__ long long xcd_grouped(long long b, long long grid, int group)
{
    const long long span = 8LL * group;
    if (group <= 1 || b >= grid / span * span) {
        return b;
    }
    const long long base = b / span * span;
    const long long rest = b - base;
    return base + (rest % 8) * group + rest / 8;
}

__global__ void __launch_bounds__(kTileThreads, kTileWavesPerSimd)
    remap_tiles_kernel(const cf32* __restrict__ x, cf32* __restrict__ y, Remap r, int tiles_p,
                       int tiles_q, long long tiles, int extra_p, int extra_q, int group)
{
    __shared__ cf32 tile[kTile * kTile];
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const long long per_array = static_cast<long long>(tiles_p) * tiles_q;
    const long long grid = gridDim.x;

    // Tile t: array b, output columns p0 .. p0 + 63 (input rows), output rows q0 .. q0 + 63
    // (input columns).
    struct Place {
        long long b;
        int tp;
        int tq;
    };
    const auto place = [&](long long t) {
        Place pl;
        pl.b = t / per_array;
        const int rest = static_cast<int>(t - pl.b * per_array);
        pl.tq = rest / tiles_p;
        pl.tp = rest - pl.tq * tiles_p;
        return pl;
    };
    // Input row rows(p) at column cols(q): lane -> q, wave + 8 k -> p.
    const auto fetch = [&](const Place& pl, cf32 (&v)[kSteps]) {
        const int p0 = pl.tp * kTile;
        const int q_in = pl.tq * kTile + lane;
        const cf32* xs = x + pl.b * r.x_array;
        const int xc = q_in < r.y_rows ? r.cols(q_in) : -1;
#pragma unroll
        for (int k = 0; k < kSteps; ++k) {
            const int p = p0 + wave + 8 * k;
            const int xr = p < r.y_cols ? r.rows(p) : -1;
            v[k] = (xr >= 0 && xc >= 0) ? xs[static_cast<long long>(xr) * r.x_pitch + xc] : zero();
        }
    };

    // Workgroup b takes tiles first(b), first(b) + grid, ...: the grid holds as many
    // workgroups as fit on the device, and each issues its next tile's loads right after the
    // current tile has reached LDS, so they are in flight during its LDS reads and stores.
    const long long first = xcd_grouped(blockIdx.x, grid, group);
    cf32 v[kSteps];
    if (first < tiles) {
        fetch(place(first), v);
    }
    for (long long t = first; t < tiles; t += grid) {
        const Place pl = place(t);
        const int p0 = pl.tp * kTile;
        const int q0 = pl.tq * kTile;
#pragma unroll
        for (int k = 0; k < kSteps; ++k) {
            const int pl_row = wave + 8 * k;
            tile[pl_row * kTile + (lane ^ (pl_row & 31))] = v[k];
        }
        __syncthreads();
        if (t + grid < tiles) {
            fetch(place(t + grid), v);
        }
        // Output row q0 + wave + 8 k, column p0 + lane: tile column, read across p.
        const cf32* xs = x + pl.b * r.x_array;
        cf32* ys = y + pl.b * static_cast<long long>(r.y_rows) * r.y_cols;
        const int p_out = p0 + lane;
#pragma unroll
        for (int k = 0; k < kSteps; ++k) {
            const int q = q0 + wave + 8 * k;
            if (q < r.y_rows && p_out < r.y_cols) {
                ys[static_cast<long long>(q) * r.y_cols + p_out] =
                    tile[lane * kTile + ((wave + 8 * k) ^ (lane & 31))];
            }
        }
        // The extra output row (input column y_rows - 1) across this tile's columns: wave 0. The
        // extra output column (input row y_cols - 1) across its rows: wave 1. Their corner: wave 2.
        const bool last_q = extra_q != 0 && pl.tq == tiles_q - 1;
        const bool last_p = extra_p != 0 && pl.tp == tiles_p - 1;
        if (last_q && wave == 0 && p_out < r.y_cols - extra_p) {
            const int q = r.y_rows - 1;
            const int xr = r.rows(p_out);
            const int xc2 = r.cols(q);
            ys[static_cast<long long>(q) * r.y_cols + p_out] =
                (xr >= 0 && xc2 >= 0) ? xs[static_cast<long long>(xr) * r.x_pitch + xc2] : zero();
        }
        if (last_p && wave == 1 && q0 + lane < r.y_rows - extra_q) {
            const int p = r.y_cols - 1;
            const int q = q0 + lane;
            const int xr = r.rows(p);
            const int xc2 = r.cols(q);
            ys[static_cast<long long>(q) * r.y_cols + p] =
                (xr >= 0 && xc2 >= 0) ? xs[static_cast<long long>(xr) * r.x_pitch + xc2] : zero();
        }
        if (last_p && last_q && wave == 2 && lane == 0) {
            const int xr = r.rows(r.y_cols - 1);
            const int xc2 = r.cols(r.y_rows - 1);
            ys[static_cast<long long>(r.y_rows - 1) * r.y_cols + r.y_cols - 1] =
                (xr >= 0 && xc2 >= 0) ? xs[static_cast<long long>(xr) * r.x_pitch + xc2] : zero();
        }
        __syncthreads();  // the next tile overwrites the LDS
    }
}

__global__ void __launch_bounds__(kThreads)
    remap_rows_kernel(const cf32* __restrict__ x, cf32* __restrict__ y, Remap r, int lanes_log2,
                      long long total_rows)
{
    const int lanes = 1 << lanes_log2;
    const int sub = static_cast<int>(threadIdx.x) >> lanes_log2;  // row within the workgroup
    const int lane = static_cast<int>(threadIdx.x) & (lanes - 1);
    const int rows_per_block = kThreads >> lanes_log2;
    for (long long row = static_cast<long long>(blockIdx.x) * rows_per_block + sub;
         row < total_rows; row += static_cast<long long>(gridDim.x) * rows_per_block) {
        const long long b = row / r.y_rows;
        const int xr = r.rows(static_cast<int>(row - b * r.y_rows));
        cf32* ys = y + row * r.y_cols;
        if (xr < 0) {
            for (int p = lane; p < r.y_cols; p += lanes) {
                ys[p] = zero();
            }
            continue;
        }
        const cf32* xs = x + b * r.x_array + static_cast<long long>(xr) * r.x_pitch;
        for (int p = lane; p < r.y_cols; p += lanes) {
            const int xc = r.cols(p);
            ys[p] = xc >= 0 ? xs[xc] : zero();
        }
    }
}

template <bool Transposed, class Index>
__global__ void __launch_bounds__(kThreads)
    remap_flat_kernel(const cf32* __restrict__ x, cf32* __restrict__ y, Remap r, Index total)
{
    const Index area = static_cast<Index>(r.y_rows) * static_cast<Index>(r.y_cols);
    const Index stride = static_cast<Index>(gridDim.x) * kThreads;
    for (Index e = static_cast<Index>(blockIdx.x) * kThreads + threadIdx.x; e < total;
         e += stride) {
        // The offset within an array stays in Index: one array may hold more than 2^31 values
        // (16 x 2^28 fits in HBM). Its row and column each fit an int.
        const Index b = e / area;
        const Index rest = e - b * area;
        const Index q_wide = rest / static_cast<Index>(r.y_cols);
        const int q = static_cast<int>(q_wide);
        const int p = static_cast<int>(rest - q_wide * static_cast<Index>(r.y_cols));
        const int xr = r.rows(Transposed ? p : q);
        const int xc = r.cols(Transposed ? q : p);
        y[e] = (xr >= 0 && xc >= 0)
                   ? x[static_cast<long long>(b) * r.x_array
                       + static_cast<long long>(xr) * r.x_pitch + xc]
                   : zero();
    }
}

unsigned blocks(long long work) { return static_cast<unsigned>(std::min(work, kMaxBlocks)); }

}  // namespace

void remap(const cf32* x, cf32* y, const Remap& r, bool transposed, hipStream_t stream)
{
    if (r.y_rows < 1 || r.y_cols < 1 || r.batch < 1) {
        throw InvalidArgument("remap: need at least one row, one column and one array");
    }
    if (transposed && (r.y_rows < kTile / 2 || r.y_cols < kTile / 2)) {
        const long long total = static_cast<long long>(r.y_rows) * r.y_cols * r.batch;
        const unsigned grid = blocks((total + kThreads - 1) / kThreads);
        if (total <= INT_MAX) {
            hipLaunchKernelGGL((remap_flat_kernel<true, unsigned>), dim3(grid), dim3(kThreads), 0,
                               stream, x, y, r, static_cast<unsigned>(total));
        } else {
            hipLaunchKernelGGL((remap_flat_kernel<true, unsigned long long>), dim3(grid),
                               dim3(kThreads), 0, stream, x, y, r,
                               static_cast<unsigned long long>(total));
        }
    } else if (transposed) {
        // Sizes here are at least 32, so a size of 64k + 1 has k >= 1 full tiles.
        const int extra_p = r.y_cols % kTile == 1 ? 1 : 0;
        const int extra_q = r.y_rows % kTile == 1 ? 1 : 0;
        const int tiles_p = (r.y_cols - extra_p + kTile - 1) / kTile;
        const int tiles_q = (r.y_rows - extra_q + kTile - 1) / kTile;
        const long long tiles = static_cast<long long>(tiles_p) * tiles_q * r.batch;
        // Output rows that do not start on 128-byte lines: runs of 8 consecutive tiles (the
        // tiles of a band, then the next bands and arrays, which share lines at their edges) on
        // one XCD each.
        const int group = r.y_cols % 16 != 0 ? 8 : 1;
        // Persistent: the workgroups that fit on the device at once (four of eight waves per CU,
        // by registers and the 32 KiB tile).
        const long long resident = static_cast<long long>(device_cus()) * kTilesPerCu;
        hipLaunchKernelGGL(remap_tiles_kernel, dim3(blocks(std::min(tiles, resident))),
                           dim3(kTileThreads), 0, stream, x, y, r, tiles_p, tiles_q, tiles,
                           extra_p, extra_q, group);
    } else {
        int lanes_log2 = 0;
        while (lanes_log2 < 6 && (1 << lanes_log2) < r.y_cols) {
            ++lanes_log2;
        }
        const long long rows = static_cast<long long>(r.y_rows) * r.batch;
        const long long per_block = kThreads >> lanes_log2;
        hipLaunchKernelGGL(remap_rows_kernel, dim3(blocks((rows + per_block - 1) / per_block)),
                           dim3(kThreads), 0, stream, x, y, r, lanes_log2, rows);
    }
    SPX_LAUNCH_CHECK();
}

}  // namespace spx
