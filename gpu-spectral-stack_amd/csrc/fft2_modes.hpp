#pragma once

// Single-pass pruned 2D real FFTs for few kept columns: rfft2_modes / irfft2_modes (reference
// pruned.cu:172-209, the FNO layout of pruned.cu:27-39) with w <= n2/8 kept columns, one array
// per workgroup.
//
// The general single-pass kernels keep a whole half spectrum in LDS (at 128 x 128, 70 KB: two
// arrays per CU), although only w columns outlive the row pass. Here the row transforms exchange
// through a scratch of one pass's rows, and only the w kept bins of each row go to a narrow
// column tile (N1 rows by TC >= w values): at 128 x 128 with w <= 16, 40 KB, so four arrays share
// a CU and more of the HBM traffic overlaps the transforms.
//
//   forward  every row pass's loads first, then per pass: row transform (exchanges in the
//            scratch), bins X[k], k < w, into the tile; the w columns in place down the tile;
//            the kept rows (0 .. m1-1, n1-m1 .. n1-1) of those columns stored flat.
//   inverse  the kept modes into the tile (the other rows read as zeros); inverse columns; per
//            pass: each lane forms its row-inverse inputs straight from the tile row (the c2r
//            prepare), inverse row transform, the real rows stored.
//
// Normalization follows numpy: forward none, inverse 1 / (n1 n2).

#include "fft2_fused.hpp"

namespace spx::dev {

template <int N1_, int M_, int R, bool Table>
struct Modes2d {
    static constexpr int N1 = N1_;  // rows (column transform length)
    static constexpr int M = M_;    // complex values per real row (n2 / 2)
    static constexpr bool kTable = Table;
    static constexpr int WMax = M / 4;  // kept columns this kernel takes
    using PR = Plan<M, R, default_e<M, R>()>;
    using PC = Plan<N1, column_radix<N1, R>(), column_values<N1, R>()>;  // as Fused2d's
    static constexpr int NT = 256;
    static constexpr int RPP = NT / PR::L;        // rows per pass
    static constexpr int kPasses = N1 / RPP;
    // LDS layouts (64 banks of 4 bytes, 8-byte accesses served a half-wave at a time). Scratch
    // rows of 64 values sit 72 apart (8 mod 32), other lengths an odd stride. Tile (n1 >= 64,
    // rows of 64 values or more): row f in tile row pad(f), tile rows TC = 4 mod 8 apart. Bank
    // conflicts in the 128 x 128 kernels' row and column passes: 20 % and 14 % of LDS cycles,
    // against 56 % and 50 % with odd strides.
    static constexpr int TR = M == 64 ? 72 : (pad(M) + 1) | 1;  // scratch row stride
    static constexpr bool kPadRows = N1 >= 64 && M >= 64;
    static constexpr int TC = kPadRows ? (WMax + 3) / 8 * 8 + 4 : WMax | 1;  // tile row stride
    static constexpr int kScratch = RPP * TR;
    static constexpr int kTile = (kPadRows ? pad(N1 - 1) + 1 : N1) * TC;
    using ColLay = std::conditional_t<kPadRows, PaddedRows<TC>, Strided<TC>>;
    __host__ __device__ static constexpr int tile_row(int f)
    {
        return (kPadRows ? pad(f) : f) * TC;
    }
    static constexpr int kMaxIo = (N1 * WMax + NT - 1) / NT;  // flat modes per lane, at most

    static_assert(kPasses >= 1 && N1 % RPP == 0, "row passes cover the rows exactly");
    static_assert(kPasses * PR::E <= 32, "every pass's row inputs fit in registers");
    static_assert(PR::L <= 64 && PC::L <= 64, "row and column transforms stay inside a wave");
    static_assert(WMax < PR::L * (WMax / PR::L + 1), "the bin loop covers k < WMax");
    static_assert(static_cast<long long>(N1) * WMax * N1 * WMax < (1LL << 31), "FastDiv range");

    __device__ __forceinline__ static int row_of(int f, int m1)
    {
        return f >= m1 ? f + N1 - 2 * m1 : f;
    }
};

// Forward: z = the real arrays viewed as complex (batch x N1 x M), y = batch arrays of 2 m1 x w
// modes. wdiv divides by w.
template <class F>
__global__ void __launch_bounds__(F::NT)
    rfft2_modes_kernel(const cf32* __restrict__ z, cf32* __restrict__ y, int m1, int w,
                       FastDiv wdiv, const cf32* table)
{
    using PR = typename F::PR;
    using PC = typename F::PC;
    __shared__ cf32 lds[F::kScratch + F::kTile];
    cf32* const tile = lds + F::kScratch;
    const long long array = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid % PR::L;
    const int prow = tid / PR::L;  // row within a pass
    cf32* const s = lds + prow * F::TR;

    // Every pass's loads in pass order, so pass p's transform waits for its own loads only.
    constexpr int R0 = PR::template radix<0>();
    const cf32* const src = z + array * F::N1 * F::M;
    cf32 v[F::kPasses][PR::E];
    static_for<0, F::kPasses>([&](auto pi) {
        constexpr int p = decltype(pi)::value;
        const cf32* const row = src + (p * F::RPP + prow) * F::M;
#pragma unroll
        for (int b = 0; b < PR::E / R0; ++b) {
#pragma unroll
            for (int r = 0; r < R0; ++r) {
                v[p][b * R0 + r] = row[input_index<PR, 0>(lane, b, r)];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    });

    // Rows: transform, then X[k] = E[k] + exp(-pi i k / M) O[k] for k < w into the tile. The
    // lane holds Z[k] for its k = lane + j L; the partner Z[M - k] is element (L - lane) + (E - 1
    // - j) L, held by lane L - lane of the row (lane 0: its own element (E - j) L), and is read
    // across lanes. Against writing the row to the scratch and reading both back (six
    // alternated rounds over 2048 arrays, m = n / 8): 64^2 8.76 -> 8.29 us, 128^2 28.78 ->
    // 28.32 us.
    static_assert(F::WMax <= (PR::E - 1) * PR::L, "partners lie in the row's last E - 1 slots");
    const cf32 base = twiddle_of<2 * F::M, false>(lane);
    const int wave_lane = tid & 63;
    const int mirror = (wave_lane & ~(PR::L - 1)) | ((PR::L - lane) & (PR::L - 1));
    static_for<0, F::kPasses>([&](auto pi) {
        constexpr int p = decltype(pi)::value;
        run_stages<PR, 0, false, F::kTable, RowExchange<PR, F::TR>>(v[p], s, lane, table);
        cf32* const trow = tile + F::tile_row(p * F::RPP + prow);
        static_for<0, (F::WMax + PR::L - 1) / PR::L>([&](auto ji) {
            constexpr int j = decltype(ji)::value;
            const cf32 zk = v[p][out_slot<PR>(j)];
            const cf32 across = lane_value(v[p][out_slot<PR>(PR::E - 1 - j)], mirror);
            const cf32 zm = lane == 0 ? v[p][out_slot<PR>((PR::E - j) % PR::E)] : across;
            const int k = lane + j * PR::L;
            if (k < w) {
                const cf32 ev{0.5f * (zk.re + zm.re), 0.5f * (zk.im - zm.im)};
                const cf32 od{0.5f * (zk.im + zm.im), -0.5f * (zk.re - zm.re)};
                constexpr cf32 c = const_twiddle<false>(j * PR::L, 2 * F::M);
                trow[k] = cadd(ev, cmul(j == 0 ? base : cmul(base, c), od));
            }
        });
    });
    __syncthreads();

    // Columns 0 .. w-1, in place down the tile.
    constexpr int CPP = F::NT / PC::L;
#pragma unroll 1
    for (int c0 = 0; c0 < w; c0 += CPP) {
        const int c = c0 + tid / PC::L;
        const int clane = tid % PC::L;
        if (c < w) {
            cf32* const col = tile + c;
            cf32 u[PC::E];
            stage_read<PC, 0, typename F::ColLay>(col, u, clane);
            run_stages<PC, 0, false, F::kTable, typename F::ColLay>(u, col, clane, table);
            lds_sync<true>();
            final_write<PC, typename F::ColLay>(col, u, clane);
        }
    }
    __syncthreads();

    // The kept rows of those columns, one contiguous run of 2 m1 w values.
    const int total = 2 * m1 * w;
    cf32* const dst = y + array * total;
    for (int e = tid; e < total; e += F::NT) {
        const int f = static_cast<int>(wdiv.div(static_cast<unsigned>(e)));
        st_stream(dst + e, tile[F::tile_row(F::row_of(f, m1)) + (e - f * w)]);
    }
}

// Inverse: x = batch arrays of 2 m1 x w modes (the other frequencies zero), z = the real outputs
// viewed as complex (batch x N1 x M). wdiv divides by w.
// W and M1: compile-time bounds on w and m1 (w <= W <= WMax, m1 <= M1 <= N1 / 2, powers of two),
// so that which of a lane's row slots and column slots can hold a kept mode is known at compile
// time and the others are constant zeros in the first stages. Tile columns w .. W-1, and tile
// rows m1 .. M1-1 and N1-M1 .. N1-m1-1 of the kept columns, are zeroed with the load.
template <class F, int W, int M1>
__global__ void __launch_bounds__(F::NT)
    irfft2_modes_kernel(const cf32* __restrict__ x, cf32* __restrict__ z, int m1, int w,
                        FastDiv wdiv, const cf32* table)
{
    static_assert(W >= 1 && W <= F::WMax && (W & (W - 1)) == 0 && F::NT % W == 0,
                  "W is a power of two within the tile's columns");
    static_assert(M1 >= 1 && 2 * M1 <= F::N1 && (M1 & (M1 - 1)) == 0,
                  "M1 is a power of two, at most half the rows");
    using PR = typename F::PR;
    using PC = typename F::PC;
    __shared__ cf32 lds[F::kScratch + F::kTile];
    cf32* const tile = lds + F::kScratch;
    const long long array = blockIdx.x;
    const int tid = threadIdx.x;

    // The modes into their tile rows, every load in flight before any LDS write.
    const int total = 2 * m1 * w;
    const cf32* const src = x + array * total;
    cf32 val[F::kMaxIo];
#pragma unroll
    for (int k = 0; k < F::kMaxIo; ++k) {
        if (k * F::NT < total) {
            val[k] = src[cmin(tid + k * F::NT, total - 1)];
        }
    }
#pragma unroll
    for (int k = 0; k < F::kMaxIo; ++k) {
        if (k * F::NT < total) {
            const int e = cmin(tid + k * F::NT, total - 1);
            const int f = static_cast<int>(wdiv.div(static_cast<unsigned>(e)));
            tile[F::tile_row(F::row_of(f, m1)) + (e - f * w)] = val[k];
        }
    }
    // Columns w .. W-1 of every row are zeros, read as such by the row prepare below (the column
    // pass touches only columns below w).
    if (w < W) {
        const int c = tid % W;
        if (c >= w) {
            for (int f = tid / W; f < F::N1; f += F::NT / W) {
                tile[F::tile_row(f) + c] = czero();
            }
        }
    }
    if (m1 < M1) {
        // Row q of the 2 (M1 - m1) rows to clear: m1 + q, then N1 - M1 + (q - (M1 - m1)).
        const int gap = M1 - m1;
        for (int e = tid; e < 2 * gap * w; e += F::NT) {
            const int q = static_cast<int>(wdiv.div(static_cast<unsigned>(e)));
            const int f = q < gap ? m1 + q : F::N1 - M1 + (q - gap);
            tile[F::tile_row(f) + (e - q * w)] = czero();
        }
    }
    __syncthreads();

    // Inverse columns 0 .. w-1 in place; rows past the bound M1 are read as zeros (every row of a
    // column is overwritten by its transform).
    constexpr int CPP = F::NT / PC::L;
    constexpr int RC = PC::template radix<0>();
#pragma unroll 1
    for (int c0 = 0; c0 < w; c0 += CPP) {
        const int c = c0 + tid / PC::L;
        const int clane = tid % PC::L;
        if (c < w) {
            cf32* const col = tile + c;
            cf32 u[PC::E];
#pragma unroll
            for (int b = 0; b < PC::E / RC; ++b) {
#pragma unroll
                for (int r = 0; r < RC; ++r) {
                    const int i = input_index<PC, 0>(clane, b, r);
                    u[b * RC + r] =
                        (i < M1 || i >= F::N1 - M1) ? col[F::ColLay::at(i)] : czero();
                }
            }
            run_stages<PC, 0, true, F::kTable, typename F::ColLay>(u, col, clane, table);
            lds_sync<true>();
            final_write<PC, typename F::ColLay>(col, u, clane);
        }
    }
    __syncthreads();

    // Rows. Lane slot k (k = lane + off) takes Z[k] = E + i O, E = (X[k] + conj X[M-k]) / 2,
    // O = exp(pi i k / M) (X[k] - conj X[M-k]) / 2, from the tile row (X[k] = 0 for k >= w; the
    // imaginary part of X[0] dropped; X[M] is never kept, w < M). The scale 1 / (N1 M), which
    // with the halves makes the row inverse numpy's irfft and covers both passes, rides on the
    // halves. A slot whose k lies in [W, M - W] for every lane of the row is zero, known at
    // compile time; the tile's columns w .. W-1 hold zeros, so reads below W need no test of w.
    constexpr float half = 0.5f / static_cast<float>(F::N1 * F::M);
    constexpr int R0 = PR::template radix<0>();
    const int lane = tid % PR::L;
    const int prow = tid / PR::L;
    cf32* const s = lds + prow * F::TR;
    cf32* const out = z + array * F::N1 * F::M;
    const cf32 base = twiddle_of<2 * F::M, true>(lane);
#pragma unroll 1
    for (int p = 0; p < F::kPasses; ++p) {
        const int row = p * F::RPP + prow;
        const cf32* const trow = tile + F::tile_row(row);
        cf32 v[PR::E];
        static_for<0, PR::E>([&](auto ei) {
            constexpr int e = decltype(ei)::value;
            constexpr int off = (e / R0) * PR::L + (e % R0) * (PR::N / R0);
            if constexpr (off >= W && F::M - off - (PR::L - 1) >= W) {
                v[e] = czero();
                return;
            }
            const int k = lane + off;
            cf32 xk = k < W ? trow[k] : czero();
            const cf32 xm = (k > 0 && F::M - k < W) ? trow[F::M - k] : czero();
            if (k == 0) {
                xk.im = 0.0f;
            }
            const cf32 ev{half * (xk.re + xm.re), half * (xk.im - xm.im)};
            const cf32 d{half * (xk.re - xm.re), half * (xk.im + xm.im)};
            constexpr cf32 c = const_twiddle<true>(off, 2 * F::M);
            const cf32 od = cmul(d, off == 0 ? base : cmul(base, c));
            v[e] = cf32{ev.re - od.im, ev.im + od.re};
        });
        run_stages<PR, 0, true, F::kTable, RowExchange<PR, F::TR>>(v, s, lane, table);
        if constexpr (PR::L >= 16) {
            // Rows of 16 lanes or more: every store is a run of at least 128 bytes.
            cf32* const dst = out + row * F::M;
            constexpr int RL = PR::template radix<PR::kStages - 1>();
#pragma unroll
            for (int b = 0; b < PR::E / RL; ++b) {
#pragma unroll
                for (int r = 0; r < RL; ++r) {
                    st_stream(dst + lane + b * PR::L + r * (PR::N / RL), v[b * RL + r]);
                }
            }
            lds_sync<true>();  // the scratch is read before the next pass reuses it
        } else {
            // Short rows: back to the scratch, then each wave stores its 64 / L consecutive rows
            // (consecutive in z too) as one contiguous run.
            lds_sync<true>();
            final_write<PR>(s, v, lane);
            lds_sync<true>();
            constexpr int kWaveRows = 64 / PR::L;
            const int r0 = (tid / 64) * kWaveRows;  // first scratch row of this wave
            cf32* const dst = out + (p * F::RPP + r0) * F::M;
#pragma unroll
            for (int k = 0; k < PR::E; ++k) {
                const int e = tid % 64 + k * 64;
                st_stream(dst + e, lds[(r0 + e / F::M) * F::TR + pad(e % F::M)]);
            }
            lds_sync<true>();
        }
    }
}

}  // namespace spx::dev
