#pragma once

// Single-pass 2D real FFTs for arrays whose half spectrum fits in LDS: rfft2 / irfft2 and the
// pruned FNO transforms (rfft2_modes / irfft2_modes) as ONE kernel and one HBM round trip per
// array, where the row-then-column drivers (reference fft2d.cu:138-187, pruned.cu:172-209) need two
// kernels and write the spectrum to HBM in between.
//
// A workgroup owns AP whole arrays (AP n1 n2 ~ 16384 points) and keeps each array's half spectrum
// in an LDS tile of n1 rows of TS complex values (TS > pad(n2/2), so a row can also hold a padded
// row transform; the layout that keeps the tile's rows and columns on distinct banks is
// Fused2d's):
//
//   forward  rows: each row of n2 reals is read as n2/2 complex values, transformed in registers
//            (Stockham stages, exchanges in the tile row itself) and combined in place into its
//            n2/2 + 1 bins; columns: the first w columns, transformed in place down the tile
//            (element i of column c at tile[row_at(i) + pad(c)]); store: the kept rows (all n1, or
//            rows 0 .. m1-1 and n1-m1 .. n1-1) of those w columns, contiguous and coalesced.
//   inverse  the mirror: load the kept rows and columns (zero elsewhere), inverse columns, then per
//            row the c2r prepare, an inverse n2/2-point transform, and the real row stored.
//
// When all n2/2 + 1 columns are kept, the DC and Nyquist columns (real in every row after the row
// transforms) travel as one complex column and are split after the column pass (forward) or
// joined before it (inverse), so n2/2 column transforms cover n2/2 + 1 columns.
//
// Normalization follows numpy: forward none, inverse 1 / (n1 n2) (the column and row scales are
// folded into the row pass). The butterflies, twiddles and exchanges are the ones of stockham.hpp.

#include "stockham.hpp"

namespace spx::dev {

// floor(x / d) as one 32-bit multiply-high: m = ceil(2^31 / d) (2^31 at d = 1, so it fits), and
// mulhi(2 x, m) = floor(x / d + x e / 2^31) with 0 <= e < 1. The fraction of x / d is at most
// (d - 1) / d, so the quotient is exact whenever x e / 2^31 < 1 / d, i.e. whenever x d < 2^31.
struct FastDiv {
    unsigned d;
    unsigned m;

    static FastDiv of(unsigned d)
    {
        return {d, static_cast<unsigned>(((1ULL << 31) + d - 1) / d)};
    }
    __device__ __forceinline__ unsigned div(unsigned x) const { return __umulhi(x << 1, m); }
};

// Values per lane of the single-pass kernels' column transforms: 16 from 128 rows on.
template <int N1, int R>
constexpr int column_values()
{
    return N1 >= 128 ? cmax(16, default_e<N1, R>()) : default_e<N1, R>();
}

// Their radix. Where a lane holds 16 values, the radix-8 variants run radix-16 stages: 128 rows
// as 16 x 8 (one LDS exchange and one twiddle stage, against 8 x 8 x 2's two of each), 256 as
// 16 x 16. Measured at 128 x 128 x 1024 (four alternated rounds, one box): rfft2 32.35 -> 31.08
// us, irfft2 34.79 -> 31.28 us; and at C4's 2048 arrays of 128 x 128 (m = 16), 29.05 -> 28.84
// and 28.58 -> 28.23 us.
template <int N1, int R>
constexpr int column_radix()
{
    return (kRadix16 && R == 8 && column_values<N1, R>() >= 16) ? 16 : R;
}

// Complex kernels' tile rows hold M values, pad(M - 1) + 1 slots; real ones the M + 1 bins,
// pad(M) + 1. Sized as complex, a 128 x 128 complex tile takes the padded layout below within
// 160 KB (rows 136 values apart, 146,880 B); sized as real it needs rows 168 apart, which does
// not fit, and falls back to odd strides. 0 sizes complex rows as real ones, for A/B builds.
#ifndef SPX_COMPLEX_TILE_ROWS
#define SPX_COMPLEX_TILE_ROWS 1
#endif

template <int N1_, int M_, int R, bool Table, int BudgetKB = 80, int Threads = 512,
          bool Complex = false>
struct Fused2d {
    static constexpr int N1 = N1_;                 // rows (column transform length)
    static constexpr int M = M_;                   // complex values per real row (n2 / 2)
    static constexpr int N2 = 2 * M;
    static constexpr bool kTable = Table;
    using PR = Plan<M, R, default_e<M, R>()>;     // row transforms
    // Column transforms: 16 values per lane from 128 rows, so a 512-lane workgroup covers 64
    // columns per pass (65 columns of a 128 x 128 half spectrum in two passes, not three);
    // measured 5-9 % faster at 128 x 128, neutral at 64 x 64. With 16 values per lane the
    // radix-8 variants take radix-16 stages (column_radix).
    using PC = Plan<N1, column_radix<N1, R>(), column_values<N1, R>()>;
    // Tile layout: row f, column c of array a at tile[a kTile + row_at(f) + pad(c)]. A tile row
    // holds kRowValues values (a padded row transform, or the M + 1 bins). One array per
    // workgroup with rows of 64 complex values or more (128 x 128): row f in tile row pad(f),
    // tile rows TS = 8 mod 32 apart, and the column passes interleave their columns across each
    // wave's lanes (col_slot / col_lane), which keeps each half-wave on distinct banks in all but
    // the first stage's writes (bank conflicts 14 % of column and 20 % of row LDS cycles, against
    // 50-56 % for odd strides with contiguous column groups). Otherwise rows are TS apart, TS odd.
    static constexpr int kRowValues =
        (Complex && SPX_COMPLEX_TILE_ROWS != 0) ? pad(M - 1) + 1 : pad(M) + 1;
    static constexpr int kTsOdd = kRowValues | 1;
    static constexpr int kTsPadded = ((kRowValues + 23) / 32) * 32 + 8;
    static constexpr int kRowsPadded = pad(N1 - 1) + 1;
    static constexpr bool kPadRows = N1 * 2 * M >= 16384 && M >= 64 && N1 >= 16
                                     && kRowsPadded * kTsPadded * 8 <= BudgetKB * 1024;
    static constexpr int TS = kPadRows ? kTsPadded : kTsOdd;  // tile row stride
    static constexpr int kTile = (kPadRows ? kRowsPadded : N1) * TS;  // values per array
    using ColLay = std::conditional_t<kPadRows, PaddedRows<TS>, Strided<TS>>;
    __host__ __device__ static constexpr int row_at(int f) { return (kPadRows ? pad(f) : f) * TS; }
    // Arrays per workgroup: about 16384 points, as many as the 80 KB tile budget allows (a
    // power of two, so the row passes still cover the rows exactly).
    static constexpr int kLdsArrays =
        BudgetKB * 1024 / (kTile * static_cast<int>(sizeof(cf32)));
    static constexpr int AP = cmin(cmax(1, 16384 / (N1 * N2)),
                                   1 << (31 - __builtin_clz(cmax(1, kLdsArrays))));
    static constexpr int NT = Threads;             // lanes per workgroup
    static constexpr int NW = NT / 64;
    static constexpr int kRows = AP * N1;
    static constexpr int RPP = NT / PR::L;         // rows per pass
    static constexpr int CPP = NT / PC::L;         // columns per pass
    static constexpr int kMaxLoads = (AP * N1 * (M + 1) + NT - 1) / NT;  // inverse: loads per lane
    static constexpr int kColsPerWave = 64 / PC::L;

    // Column slot (0 .. CPP-1) and lane of a column pass.
    __device__ __forceinline__ static int col_slot(int tid)
    {
        return kPadRows ? (tid / 64) * kColsPerWave + tid % kColsPerWave : tid / PC::L;
    }
    __device__ __forceinline__ static int col_lane(int tid)
    {
        return kPadRows ? (tid % 64) / kColsPerWave : tid % PC::L;
    }

    static_assert(PR::L <= 64 && PC::L <= 64, "row and column transforms stay inside a wave");
    static_assert(!kPadRows || AP == 1, "padded tile rows: one array per workgroup");
    static_assert(kRows % RPP == 0, "row passes cover the rows exactly");
    static_assert(AP * kTile * sizeof(cf32) <= BudgetKB * 1024, "tile exceeds the LDS budget");
    // Flat indices stay below AP N1 (M + 1) and divisors at most N1 (M + 1): FastDiv is exact.
    static_assert(static_cast<long long>(AP) * N1 * (M + 1) * N1 * (M + 1) < (1LL << 31),
                  "FastDiv range");

    // Tile row holding frequency-row f of the kept rows (all rows when m1 = 0).
    __device__ __forceinline__ static int row_of(int f, int m1)
    {
        return (m1 > 0 && f >= m1) ? f + N1 - 2 * m1 : f;
    }
};

// Combine of the real forward transform for one row held in place at s (Padded): pair k (0 < k
// <= M / 2) reads Z[k] and Z[M-k] and writes X[k] and X[M-k] into the same slots; tw =
// exp(-pi i k / M). k = 0 gives the two real bins X[0] and X[M]: with pack, both go to slot 0 as
// X[0] + i X[M] (the packed DC / Nyquist column), else X[0] alone (X[M] is not kept).
template <int M>
__device__ __forceinline__ void combine_pair(cf32* s, int k, cf32 tw, bool pack)
{
    if (k == 0) {
        const cf32 z0 = s[0];
        s[0] = cf32{z0.re + z0.im, pack ? z0.re - z0.im : 0.0f};
        return;
    }
    const cf32 zk = s[pad(k)];
    const cf32 zm = s[pad(M - k)];
    const cf32 ev{0.5f * (zk.re + zm.re), 0.5f * (zk.im - zm.im)};
    const cf32 od{0.5f * (zk.im + zm.im), -0.5f * (zk.re - zm.re)};
    const cf32 wo = cmul(tw, od);
    s[pad(k)] = cadd(ev, wo);
    if (k < M - k) {
        s[pad(M - k)] = cconj(csub(ev, wo));
    }
}

// The combines of one row's pairs k = lane + j L <= kmax (L lanes per row). A lane evaluates one
// twiddle, exp(-pi i lane / M), and reaches its other pairs' through compile-time constants.
template <int M, int L>
__device__ __forceinline__ void combine_row(cf32* s, int lane, int kmax, bool pack)
{
    const cf32 base = twiddle_of<2 * M, false>(lane);
    static_for<0, M / 2 / L + 1>([&](auto ji) {
        constexpr int j = decltype(ji)::value;
        const int k = lane + j * L;
        if (k <= kmax) {
            if constexpr (j == 0) {
                combine_pair<M>(s, k, base, pack);
            } else {
                constexpr cf32 c = const_twiddle<false>(j * L, 2 * M);
                combine_pair<M>(s, k, cmul(base, c), pack);
            }
        }
    });
}

// Prepare of the real inverse transform for one row, formed in registers. Each lane computes the
// stage-0 inputs of its own slots straight from the row's half spectrum at s (Padded): X[k] for
// k < w, zero beyond; imaginary parts of X[0] and X[M] dropped; with pack, slot 0 holds
// X[0] + i X[M] (both already real). Slot e of lane l holds element
// i = l + (e / R0) L + (e % R0) M / R0, and Z[i] = E + i O with E = (X[i] + conj X[M - i]) / 2
// and O = exp(pi i i / M) (X[i] - conj X[M - i]) / 2, times half = 1/2 of the inverse's scale,
// which the (linear) row transform carries to its outputs. One twiddle per lane: the slots'
// offsets are compile-time constants. Against a pass over the pairs (k, M - k) that wrote Z back
// in place for stage_read (six alternated rounds of irfft2 over 2^24 points on MI355X): 128^2
// 29.18 -> 28.72 us, 64^2 35.22 -> 33.87 us, 32^2 35.39 -> 34.62 us.
template <class P, int M>
__device__ __forceinline__ void prepare_to_registers(const cf32* s, cf32 (&u)[P::E], int lane,
                                                     int w, bool pack, float half)
{
    static_assert(P::N == M, "the row transform has M points");
    constexpr int R0 = P::template radix<0>();
    const cf32 base = twiddle_of<2 * M, true>(lane);
    static_for<0, P::E>([&](auto ei) {
        constexpr int e = decltype(ei)::value;
        constexpr int off = (e / R0) * P::L + (e % R0) * (P::N / R0);
        const int k = lane + off;
        cf32 xk;
        cf32 xm;
        if (off == 0 && k == 0) {
            const cf32 p = s[0];
            xk = cf32{p.re, 0.0f};
            xm = cf32{pack ? p.im : 0.0f, 0.0f};
        } else {
            xk = k < w ? s[pad(k)] : czero();
            xm = M - k < w ? s[pad(M - k)] : czero();
        }
        const cf32 ev{half * (xk.re + xm.re), half * (xk.im - xm.im)};
        const cf32 d{half * (xk.re - xm.re), half * (xk.im + xm.im)};
        constexpr cf32 c = const_twiddle<true>(off, 2 * M);
        const cf32 od = cmul(d, off == 0 ? base : cmul(base, c));
        u[e] = cf32{ev.re - od.im, ev.im + od.re};
    });
}

// Columns 0 and M of a forward tile from the packed column P = C0 + i CM, where C0 and CM are the
// transforms of the real columns X[., 0] and X[., M] and so Hermitian: C0 = (P + conj P[-k]) / 2
// and CM = (P - conj P[-k]) / 2i. Task (array, k1), k1 = 0 .. N1 / 2, owns rows k1 and -k1.
template <class F>
__device__ __forceinline__ void unpack_dc_nyquist(cf32* tile, int tid)
{
    constexpr int H = F::N1 / 2 + 1;
    for (int e = tid; e < F::AP * H; e += F::NT) {
        const int a = e / H;
        const int k1 = e - a * H;
        const int k2 = (F::N1 - k1) & (F::N1 - 1);
        cf32* const t = tile + a * F::kTile;
        const cf32 p = t[F::row_at(k1)];
        const cf32 q = t[F::row_at(k2)];
        const cf32 c0{0.5f * (p.re + q.re), 0.5f * (p.im - q.im)};
        const cf32 cm{0.5f * (p.im + q.im), -0.5f * (p.re - q.re)};
        t[F::row_at(k1)] = c0;
        t[F::row_at(k1) + pad(F::M)] = cm;
        t[F::row_at(k2)] = cconj(c0);
        t[F::row_at(k2) + pad(F::M)] = cconj(cm);
    }
}

// The inverse's mirror: columns 0 and M of the loaded spectrum into one column P = H0 + i HM,
// where H = (c + conj c[-k]) / 2 is the Hermitian part of a column, whose inverse transform is
// the real part of the column's (what the row inverse keeps of the DC and Nyquist bins). With
// m1 > 0 the kept rows are 0 .. m1-1 and N1-m1 .. N1-1, so row -m1 is kept and its mirror m1 is
// not: dropped rows are read as zeros here, P is written to row m1 too, and the packed column's
// load reads rows 0 .. m1 (packed_kept).
template <class F>
__device__ __forceinline__ bool kept_row(int i, int m1)
{
    return m1 == 0 || i < m1 || i >= F::N1 - m1;
}

template <class F>
__device__ __forceinline__ void pack_dc_nyquist(cf32* tile, int m1, int tid)
{
    constexpr int H = F::N1 / 2 + 1;
    for (int e = tid; e < F::AP * H; e += F::NT) {
        const int a = e / H;
        const int k1 = e - a * H;
        const int k2 = (F::N1 - k1) & (F::N1 - 1);
        const bool kept1 = kept_row<F>(k1, m1);
        const bool kept2 = kept_row<F>(k2, m1);
        if (!kept1 && !kept2) {
            continue;
        }
        cf32* const t = tile + a * F::kTile;
        const cf32 a0 = kept1 ? t[F::row_at(k1)] : czero();
        const cf32 b0 = kept2 ? t[F::row_at(k2)] : czero();
        const cf32 am = kept1 ? t[F::row_at(k1) + pad(F::M)] : czero();
        const cf32 bm = kept2 ? t[F::row_at(k2) + pad(F::M)] : czero();
        const cf32 h0{0.5f * (a0.re + b0.re), 0.5f * (a0.im - b0.im)};
        const cf32 hm{0.5f * (am.re + bm.re), 0.5f * (am.im - bm.im)};
        t[F::row_at(k1)] = cf32{h0.re - hm.im, h0.im + hm.re};
        t[F::row_at(k2)] = cf32{h0.re + hm.im, hm.re - h0.im};
    }
}

// Rows of column c read from the tile by the inverse column pass; the others are zeros.
template <class F>
__device__ __forceinline__ bool packed_kept(int i, int m1, bool packed_column)
{
    return kept_row<F>(i, m1) || (packed_column && i == m1);
}

// Whole half spectra (m1 = 0, w = M + 1), HBM -> tile, for rows of M >= 32 complex values: row
// by row, with no index division. Wave v owns rows v RPW .. v RPW + RPW-1 of the workgroup's
// arrays (arrays are contiguous in the tile, kTile apart, and in HBM); lane l holds column
// c = l mod M (plus 64 j, j < CW, when M = 128) of row l / M of each step, so a step's tile and
// HBM addresses are the lane's own plus compile-time offsets. Column M (the Nyquist bins) takes
// one more step, lane l < RPW holding row l's. (The same order for the forward's stores measured
// 15-30 % slower than flat stores: its runs start off the 128-byte lines.)
template <class F>
struct FullRows {
    static constexpr bool kUse = F::M >= 32;
    static constexpr int RPW = F::kRows / F::NW;            // rows per wave
    static constexpr int RW = F::M >= 64 ? 1 : 64 / F::M;   // rows per step
    static constexpr int CW = F::M > 64 ? F::M / 64 : 1;    // steps per row
    static constexpr int kSteps = RPW / RW;
    static constexpr int kPitch = F::M + 1;                 // HBM row length
    static_assert(!kUse || (RPW % RW == 0 && RPW <= 64 && kSteps * CW <= 16),
                  "whole rows per wave, the Nyquist bins in one step");

    // A wave's rows stay inside one 16-row block of the padded tile (rows RPW-aligned, RPW a
    // divisor of 16, one row per step), or the tile is unpadded: either way step i's tile row is
    // the lane's first plus i RW TS, a compile-time offset.
    static constexpr bool kLinearRows = !F::kPadRows || (RW == 1 && 16 % RPW == 0);

    // A lane's values of one load: kSteps x CW row values and a Nyquist bin.
    struct Regs {
        cf32 val[kSteps][CW];
        cf32 ny;
    };

    // src: the workgroup's first array; rows of arrays >= count read the last row instead. With
    // one array per workgroup count is 1 and every row exists, so the addresses are the lane's
    // own plus compile-time offsets (no clamp).
    __device__ __forceinline__ static void fetch(Regs& g, const cf32* src, int count, int tid)
    {
        const int row = (tid / 64) * RPW + (tid % 64) / (F::M >= 64 ? 64 : F::M);
        const int col = F::M >= 64 ? tid % 64 : tid % F::M;
        const int last = count * F::N1 - 1;
        const cf32* const lane_src = src + row * kPitch + col;
        static_for<0, kSteps>([&](auto ii) {
            constexpr int i = decltype(ii)::value;
            static_for<0, CW>([&](auto jj) {
                constexpr int j = decltype(jj)::value;
                if constexpr (F::AP == 1) {
                    g.val[i][j] = lane_src[i * RW * kPitch + 64 * j];
                } else {
                    g.val[i][j] = src[cmin(row + i * RW, last) * kPitch + col + 64 * j];
                }
            });
        });
        const int nrow = cmin((tid / 64) * RPW + tid % 64, F::kRows - 1);
        g.ny = src[cmin(nrow, last) * kPitch + F::M];
    }

    __device__ __forceinline__ static void put(cf32* tile, const Regs& g, int tid)
    {
        const int row = (tid / 64) * RPW + (tid % 64) / (F::M >= 64 ? 64 : F::M);
        const int col = F::M >= 64 ? tid % 64 : tid % F::M;
        cf32* const lane_tile = tile + F::row_at(row) + pad(col);
        static_for<0, kSteps>([&](auto ii) {
            constexpr int i = decltype(ii)::value;
            static_for<0, CW>([&](auto jj) {
                constexpr int j = decltype(jj)::value;
                if constexpr (kLinearRows) {
                    lane_tile[i * RW * F::TS + pad(64 * j)] = g.val[i][j];
                } else {
                    tile[F::row_at(row + i * RW) + pad(col + 64 * j)] = g.val[i][j];
                }
            });
        });
        if (tid % 64 < RPW) {
            const int nrow = cmin((tid / 64) * RPW + tid % 64, F::kRows - 1);
            tile[F::row_at(nrow) + pad(F::M)] = g.ny;
        }
    }

    // Every lane's loads in flight before its first LDS write.
    __device__ __forceinline__ static void load(cf32* tile, const cf32* src, int count, int tid)
    {
        Regs g;
        fetch(g, src, count, tid);
        put(tile, g, tid);
    }
};

// Whole half spectra, tile -> HBM (dst: the workgroup's first array), flat: element e = row W + c
// (W = M + 1, rows counted across the workgroup's arrays) goes to dst[e] from tile[row_at(row) +
// pad(c)], lane t taking e = t + k NT. (row, c) advances by a compile-time step from one k to
// the next, so no element needs a division; stores are full 128-byte lines.
template <class F>
__device__ __forceinline__ void store_full(const cf32* tile, cf32* dst, int count, int tid)
{
    constexpr int W = F::M + 1;
    constexpr int K = (F::AP * F::N1 * W + F::NT - 1) / F::NT;
    constexpr int kChunk = 8;
    const int total = count * F::N1 * W;
    int row = tid / W;
    int c = tid - row * W;
    static_for<0, (K + kChunk - 1) / kChunk>([&](auto gi) {
        constexpr int g = decltype(gi)::value;
        constexpr int n = cmin(kChunk, K - g * kChunk);
        cf32 val[n];
        static_for<0, n>([&](auto ki) {
            constexpr int k = decltype(ki)::value;
            val[k] = tile[F::row_at(cmin(row, F::kRows - 1)) + pad(c)];
            c += F::NT % W;
            row += F::NT / W;
            if (c >= W) {
                c -= W;
                ++row;
            }
        });
        static_for<0, n>([&](auto ki) {
            constexpr int k = decltype(ki)::value;
            const int e = tid + (g * kChunk + k) * F::NT;
            if (e < total) {
                st_stream(dst + e, val[k]);
            }
        });
    });
}

// Forward: z = the real arrays viewed as complex (batch x N1 x M), y = batch arrays of rows_out x w
// values (rows_out = 2 m1 when m1 > 0, else N1). wdiv divides by w, odiv by rows_out w.
template <class F, bool Full = false>
__global__ void __launch_bounds__(F::NT)
    rfft2_fused_kernel(const cf32* __restrict__ z, cf32* __restrict__ y, int m1_arg, int w_arg,
                       FastDiv wdiv, FastDiv odiv, long long batch, const cf32* table)
{
    using PR = typename F::PR;
    using PC = typename F::PC;
    __shared__ cf32 tile[F::AP * F::kTile];
    // Full: the whole half spectrum (m1 = 0, w = M + 1) as compile-time facts, so the combine's
    // bounds and the store's route fold away.
    const int m1 = Full ? 0 : m1_arg;
    const int w = Full ? F::M + 1 : w_arg;

    const long long first = static_cast<long long>(blockIdx.x) * F::AP;
    const int count = static_cast<int>(batch - first < F::AP ? batch - first : F::AP);
    const int tid = threadIdx.x;
    // All M + 1 columns kept: the real DC and Nyquist columns travel as one complex column, so
    // M column transforms (one pass at 128 x 128) cover M + 1 columns.
    const bool pack = w == F::M + 1;
    const int ncols = pack ? F::M : w;

    // Rows: load straight from HBM, transform, combine in place. Every pass's loads are issued
    // before the first pass's transform, so later passes' loads arrive during earlier passes'
    // work. (Staging short rows flat through the tile first, as the complex kernel does,
    // measured 10-20 % slower here.)
    constexpr int kPasses = F::kRows / F::RPP;
    constexpr int R0 = PR::template radix<0>();
    static_assert(kPasses * PR::E <= 32, "all row passes' inputs fit in registers");
    const int lane = tid % PR::L;
    cf32 v[kPasses][PR::E];
    static_for<0, kPasses>([&](auto pi) {
        constexpr int p = decltype(pi)::value;
        // Row of the workgroup's arrays; rows of arrays past the batch read the last array's
        // (their tile rows are never stored), so every load is unconditional.
        const int row = p * F::RPP + tid / PR::L;
        const int a = cmin(row / F::N1, count - 1);
        const cf32* src = z + (first * F::N1 + a * F::N1 + row % F::N1) * F::M;
#pragma unroll
        for (int b = 0; b < PR::E / R0; ++b) {
#pragma unroll
            for (int r = 0; r < R0; ++r) {
                v[p][b * R0 + r] = src[input_index<PR, 0>(lane, b, r)];
            }
        }
        // Keep the passes' loads in pass order, so pass 0's transform waits for its own loads
        // only (the memory counter retires loads in issue order).
        __builtin_amdgcn_sched_barrier(0);
    });
    static_for<0, kPasses>([&](auto pi) {
        constexpr int p = decltype(pi)::value;
        const int row = p * F::RPP + tid / PR::L;
        cf32* const s = tile + (row / F::N1) * F::kTile + F::row_at(row % F::N1);
        run_stages<PR, 0, false, F::kTable, RowExchange<PR, F::TS>>(v[p], s, lane, table);
        lds_sync<true>();
        final_write<PR>(s, v[p], lane);
        lds_sync<true>();
        // Pairs (k, M - k) up to M / 2; with w <= M / 2 kept columns only X[k], k < w, is read.
        combine_row<F::M, PR::L>(s, lane, w > F::M / 2 ? F::M / 2 : w - 1, pack);
    });
    __syncthreads();

    // Columns 0 .. ncols-1 of every array, in place down the tile.
    const int total_cols = F::AP * ncols;
#pragma unroll 1
    for (int c0 = 0; c0 < total_cols; c0 += F::CPP) {
        const int cg = c0 + F::col_slot(tid);
        const int lane = F::col_lane(tid);
        if (cg < total_cols) {
            const int a = pack ? cg / F::M : static_cast<int>(wdiv.div(static_cast<unsigned>(cg)));
            const int c = cg - a * ncols;
            cf32* const s = tile + a * F::kTile + pad(c);
            cf32 v[PC::E];
            stage_read<PC, 0, typename F::ColLay>(s, v, lane);
            run_stages<PC, 0, false, F::kTable, typename F::ColLay>(v, s, lane, table);
            lds_sync<true>();
            final_write<PC, typename F::ColLay>(s, v, lane);
        }
    }
    __syncthreads();
    if (pack) {
        unpack_dc_nyquist<F>(tile, tid);
        __syncthreads();
    }

    if (pack && m1 == 0) {
        store_full<F>(tile, y + first * F::N1 * (F::M + 1), count, tid);
        return;
    }

    // Store the kept rows of the first w columns. The workgroup's output is one contiguous run of
    // count x rows_out x w values: the lanes walk it flat, coalesced whatever w is (rows of a
    // few values, as at 4 x 4, would otherwise leave most of a wave idle), reading kStoreChunk
    // tile values into registers before storing them. The reads are unconditional (lanes past
    // the end read the last value again), so they issue back to back.
    const int per_array = (m1 > 0 ? 2 * m1 : F::N1) * w;
    const int total = count * per_array;
    cf32* const dst = y + first * per_array;
    constexpr int kStoreChunk = 8;
#pragma unroll 1
    for (int e0 = 0; e0 < total; e0 += F::NT * kStoreChunk) {
        cf32 val[kStoreChunk];
#pragma unroll
        for (int k = 0; k < kStoreChunk; ++k) {
            const int e = cmin(e0 + k * F::NT + tid, total - 1);
            const int a = F::AP == 1 ? 0 : static_cast<int>(odiv.div(static_cast<unsigned>(e)));
            const int r = e - a * per_array;
            const int f = static_cast<int>(wdiv.div(static_cast<unsigned>(r)));
            val[k] = tile[a * F::kTile + F::row_at(F::row_of(f, m1)) + pad(r - f * w)];
        }
#pragma unroll
        for (int k = 0; k < kStoreChunk; ++k) {
            const int e = e0 + k * F::NT + tid;
            if (e < total) {
                st_stream(dst + e, val[k]);
            }
        }
    }
}

// Inverse: x = batch arrays of rows_in x w values (rows_in = 2 m1 when m1 > 0, else N1; the other
// frequencies are zero), z = the real outputs viewed as complex (batch x N1 x M). wdiv divides by
// w, adiv by rows_in w.
template <class F, bool Full = false>
__global__ void __launch_bounds__(F::NT)
    irfft2_fused_kernel(const cf32* __restrict__ x, cf32* __restrict__ z, int m1_arg, int w_arg,
                        FastDiv wdiv, FastDiv adiv, long long batch, const cf32* table)
{
    using PR = typename F::PR;
    using PC = typename F::PC;
    __shared__ cf32 tile[F::AP * F::kTile];
    // Full: the whole half spectrum (m1 = 0, w = M + 1) as compile-time facts, so the column
    // reads and the prepare's bounds fold away.
    const int m1 = Full ? 0 : m1_arg;
    const int w = Full ? F::M + 1 : w_arg;

    const long long first = static_cast<long long>(blockIdx.x) * F::AP;
    const int count = static_cast<int>(batch - first < F::AP ? batch - first : F::AP);
    const int tid = threadIdx.x;

    const bool pack = w == F::M + 1;  // DC and Nyquist columns as one (see pack_dc_nyquist)
    const int ncols = pack ? F::M : w;

    // Load the kept rows of the first w columns (contiguous in x: count arrays of rows_in x w),
    // every lane's loads in flight before any LDS write.
    bool loaded = false;
    if constexpr (FullRows<F>::kUse) {
        if (pack && m1 == 0) {
            FullRows<F>::load(tile, x + first * F::N1 * (F::M + 1), count, tid);
            loaded = true;
        }
    }
    if (!loaded) {
        const int rows_in = m1 > 0 ? 2 * m1 : F::N1;
        const int per_array = rows_in * w;
        const int total = count * per_array;
        const cf32* const src = x + first * per_array;
        // Steps past the end are skipped whole (a test uniform over the workgroup); within the
        // last step, lanes past the end load and write the last value again (same value, same
        // slot), so no load or LDS write waits on a per-lane branch.
        cf32 val[F::kMaxLoads];
#pragma unroll
        for (int k = 0; k < F::kMaxLoads; ++k) {
            if (k * F::NT < total) {
                val[k] = src[cmin(tid + k * F::NT, total - 1)];
            }
        }
#pragma unroll
        for (int k = 0; k < F::kMaxLoads; ++k) {
            if (k * F::NT < total) {
                const int e = cmin(tid + k * F::NT, total - 1);
                const int a =
                    F::AP == 1 ? 0 : static_cast<int>(adiv.div(static_cast<unsigned>(e)));
                const int rem = e - a * per_array;
                const int f = static_cast<int>(wdiv.div(static_cast<unsigned>(rem)));
                const int c = rem - f * w;
                tile[a * F::kTile + F::row_at(F::row_of(f, m1)) + pad(c)] = val[k];
            }
        }
    }
    __syncthreads();
    if (pack) {
        pack_dc_nyquist<F>(tile, m1, tid);
        __syncthreads();
    }

    // Inverse columns 0 .. ncols-1, in place. The dropped rows (m1 > 0) are read as zeros, never
    // from the tile: the column's later stages overwrite all its rows anyway.
    const int total_cols = F::AP * ncols;
    constexpr int R0 = PC::template radix<0>();
#pragma unroll 1
    for (int c0 = 0; c0 < total_cols; c0 += F::CPP) {
        const int cg = c0 + F::col_slot(tid);
        const int lane = F::col_lane(tid);
        if (cg < total_cols) {
            const int a = pack ? cg / F::M : static_cast<int>(wdiv.div(static_cast<unsigned>(cg)));
            const int c = cg - a * ncols;
            cf32* const s = tile + a * F::kTile + pad(c);
            cf32 v[PC::E];
            if (m1 == 0) {
                stage_read<PC, 0, typename F::ColLay>(s, v, lane);
            } else {
#pragma unroll
                for (int b = 0; b < PC::E / R0; ++b) {
#pragma unroll
                    for (int r = 0; r < R0; ++r) {
                        const int i = input_index<PC, 0>(lane, b, r);
                        const bool kept = packed_kept<F>(i, m1, pack && c == 0);
                        v[b * R0 + r] = kept ? s[F::ColLay::at(i)] : czero();
                    }
                }
            }
            run_stages<PC, 0, true, F::kTable, typename F::ColLay>(v, s, lane, table);
            lds_sync<true>();
            final_write<PC, typename F::ColLay>(s, v, lane);
        }
    }
    __syncthreads();

    // Rows: prepare in registers, inverse transform, store the real row. The scale 1 / (N1 M)
    // covers both passes (the prepare's halves make 1 / M the row inverse of numpy's irfft) and
    // rides on those halves.
    constexpr float half = 0.5f / static_cast<float>(F::N1 * F::M);
#pragma unroll 1
    for (int p = 0; p < F::kRows / F::RPP; ++p) {
        const int row = p * F::RPP + tid / PR::L;
        const int lane = tid % PR::L;
        const int a = row / F::N1;
        cf32* const s = tile + a * F::kTile + F::row_at(row % F::N1);
        cf32 v[PR::E];
        prepare_to_registers<PR, F::M>(s, v, lane, w, pack, half);
        run_stages<PR, 0, true, F::kTable, RowExchange<PR, F::TS>>(v, s, lane, table);
        if constexpr (PR::L >= 16) {
            // Rows of 16 lanes or more: every store is a run of at least 128 bytes.
            if (a < count) {
                cf32* const dst = z + (first * F::N1 + row) * F::M;
                constexpr int RL = PR::template radix<PR::kStages - 1>();
#pragma unroll
                for (int b = 0; b < PR::E / RL; ++b) {
#pragma unroll
                    for (int r = 0; r < RL; ++r) {
                        st_stream(dst + lane + b * PR::L + r * (PR::N / RL), v[b * RL + r]);
                    }
                }
            }
        } else {
            // Short rows: back to the tile row, then each wave stores its 64 / L consecutive rows
            // (consecutive in z too) as one contiguous run.
            lds_sync<true>();
            final_write<PR>(s, v, lane);
            lds_sync<true>();
            const int row0 = p * F::RPP + (tid / 64) * (64 / PR::L);
#pragma unroll
            for (int k = 0; k < PR::E; ++k) {
                const int e = tid % 64 + k * 64;
                const int rw = row0 + e / F::M;
                const int i = e % F::M;
                const int aw = rw / F::N1;
                if (aw < count) {
                    st_stream(z + (first * F::N1 + rw) * F::M + i,
                              tile[aw * F::kTile + F::row_at(rw % F::N1) + pad(i)]);
                }
            }
        }
    }
}

// Complex 2D (fft2_c2c): x, y = batch arrays of N1 x M complex values (here M is the row length,
// n2). Rows straight from HBM, transformed into the tile, then the columns in place, then a flat
// store; inverse scale 1 / (N1 M) on the way out.
template <class F, bool Inv>
__global__ void __launch_bounds__(F::NT)
    fft2_fused_kernel(const cf32* __restrict__ x, cf32* __restrict__ y, long long batch,
                      float scale, const cf32* table)
{
    using PR = typename F::PR;
    using PC = typename F::PC;
    __shared__ cf32 tile[F::AP * F::kTile];
    constexpr int kPerArray = F::N1 * F::M;

    const long long first = static_cast<long long>(blockIdx.x) * F::AP;
    const int count = static_cast<int>(batch - first < F::AP ? batch - first : F::AP);
    const int tid = threadIdx.x;
    constexpr int R0 = PR::template radix<0>();

    // Rows of fewer than 16 lanes would load a few bytes per row per instruction: those load the
    // workgroup's arrays flat (one contiguous run) into the tile rows first.
    constexpr bool kStaged = PR::L < 16;
    if constexpr (kStaged) {
        constexpr int kLoads = F::AP * kPerArray / F::NT;
        static_assert(F::AP * kPerArray % F::NT == 0, "whole load steps");
        const int total = count * kPerArray;
        const cf32* src = x + first * kPerArray;
        cf32 val[kLoads];
#pragma unroll
        for (int k = 0; k < kLoads; ++k) {
            const int e = tid + k * F::NT;
            val[k] = e < total ? ld_stream(src + e) : czero();
        }
#pragma unroll
        for (int k = 0; k < kLoads; ++k) {
            const int e = tid + k * F::NT;
            const int a = e / kPerArray;
            const int r = e - a * kPerArray;
            const int f = r / F::M;
            tile[a * F::kTile + F::row_at(f) + pad(r - f * F::M)] = val[k];
        }
        __syncthreads();
    }
#pragma unroll 1
    for (int p = 0; p < F::kRows / F::RPP; ++p) {
        const int row = p * F::RPP + tid / PR::L;  // row of the workgroup's arrays
        const int lane = tid % PR::L;
        const int a = row / F::N1;
        cf32* const s = tile + a * F::kTile + F::row_at(row % F::N1);
        cf32 v[PR::E];
        if constexpr (kStaged) {
            stage_read<PR, 0>(s, v, lane);
        } else {
            const cf32* src = x + (first * F::N1 + row) * F::M;
#pragma unroll
            for (int b = 0; b < PR::E / R0; ++b) {
#pragma unroll
                for (int r = 0; r < R0; ++r) {
                    v[b * R0 + r] =
                        a < count ? ld_stream(src + input_index<PR, 0>(lane, b, r)) : czero();
                }
            }
        }
        run_stages<PR, 0, Inv, F::kTable, RowExchange<PR, F::TS>>(v, s, lane, table);
        lds_sync<true>();
        final_write<PR>(s, v, lane);
    }
    __syncthreads();

#pragma unroll 1
    for (int c0 = 0; c0 < F::AP * F::M; c0 += F::CPP) {
        const int cg = c0 + F::col_slot(tid);
        const int lane = F::col_lane(tid);
        if (cg < F::AP * F::M) {
            const int a = cg / F::M;
            const int c = cg - a * F::M;
            cf32* const s = tile + a * F::kTile + pad(c);
            cf32 v[PC::E];
            stage_read<PC, 0, typename F::ColLay>(s, v, lane);
            run_stages<PC, 0, Inv, F::kTable, typename F::ColLay>(v, s, lane, table);
            lds_sync<true>();
            final_write<PC, typename F::ColLay>(s, v, lane);
        }
    }
    __syncthreads();

    const int total = count * kPerArray;
    cf32* const dst = y + first * kPerArray;
    constexpr int kStoreChunk = 8;
#pragma unroll 1
    for (int e0 = 0; e0 < total; e0 += F::NT * kStoreChunk) {
        cf32 val[kStoreChunk];
#pragma unroll
        for (int k = 0; k < kStoreChunk; ++k) {
            const int e = e0 + k * F::NT + tid;
            if (e < total) {
                const int a = e / kPerArray;
                const int r = e - a * kPerArray;
                const int f = r / F::M;
                val[k] = tile[a * F::kTile + F::row_at(f) + pad(r - f * F::M)];
            }
        }
#pragma unroll
        for (int k = 0; k < kStoreChunk; ++k) {
            const int e = e0 + k * F::NT + tid;
            if (e < total) {
                st_stream(dst + e, cscale(val[k], scale));
            }
        }
    }
}

// Persistent inverse for one array per workgroup (irfft2 of arrays of 16384 points: 128 x 128,
// 256 x 64, 64 x 256). The LDS tile of such an array takes half a CU's LDS, so two workgroups
// share a CU, and with one array per workgroup each runs its phases in sequence: the loads, the
// LDS work, the stores. Here workgroup g takes arrays g, g + G, g + 2G, ... (G = gridDim.x, the
// workgroups that fit on the device at once). Once array k's columns are done, it issues array
// k + G's loads into registers; they are in flight during array k's row pass and stores. At the
// top of the next turn the wave waits for all of them, its stores included, before writing the
// new array into the tile.
//
// Measured at 128 x 128 x 1024 on one box, alternated with one array per workgroup: 32.3 against
// 36.5 us. Letting the wait skip the stores (the compiler can count them when the path from the
// loads to their first use is straight) measured slower, 37.1 us. So did the same prefetch in
// the forward transform, which stays one array per workgroup (33.1 against 32.6 us).

template <class F>
__global__ void __launch_bounds__(F::NT)
    irfft2_full_persistent_kernel(const cf32* __restrict__ x, cf32* __restrict__ z,
                                  long long batch, const cf32* table)
{
    static_assert(F::AP == 1 && FullRows<F>::kUse, "one array per workgroup, rows of 32 or more");
    using PR = typename F::PR;
    using PC = typename F::PC;
    using Rows = FullRows<F>;
    __shared__ cf32 tile[F::kTile];
    constexpr int W = F::M + 1;
    constexpr float half = 0.5f / static_cast<float>(F::N1 * F::M);

    typename Rows::Regs g;
    long long a = blockIdx.x;
    Rows::fetch(g, x + a * F::N1 * W, 1, threadIdx.x);
#pragma unroll 1
    for (; a < batch; a += gridDim.x) {
        const int tid = opaque_tid<F::NT>();
        Rows::put(tile, g, tid);
        __syncthreads();
        pack_dc_nyquist<F>(tile, 0, tid);
        __syncthreads();

        // Inverse columns 0 .. M-1 (column 0 the packed DC / Nyquist column), in place.
#pragma unroll 1
        for (int c0 = 0; c0 < F::M; c0 += F::CPP) {
            const int c = c0 + F::col_slot(tid);
            if (c < F::M) {
                cf32* const s = tile + pad(c);
                const int cl = F::col_lane(tid);
                cf32 u[PC::E];
                stage_read<PC, 0, typename F::ColLay>(s, u, cl);
                run_stages<PC, 0, true, F::kTable, typename F::ColLay>(u, s, cl, table);
                lds_sync<true>();
                final_write<PC, typename F::ColLay>(s, u, cl);
            }
        }
        __syncthreads();
        const long long next = a + gridDim.x;
        if (next < batch) {
            Rows::fetch(g, x + next * F::N1 * W, 1, tid);
        }

        // Rows: prepare in registers, inverse transform, store the real row (scale 1 / (N1 M) on
        // the prepare's halves).
        cf32* const dst = z + a * F::N1 * F::M;
#pragma unroll 1
        for (int p = 0; p < F::N1 / F::RPP; ++p) {
            const int row = p * F::RPP + tid / PR::L;
            const int lane = tid % PR::L;
            cf32* const s = tile + F::row_at(row);
            cf32 u[PR::E];
            prepare_to_registers<PR, F::M>(s, u, lane, W, true, half);
            run_stages<PR, 0, true, F::kTable, RowExchange<PR, F::TS>>(u, s, lane, table);
            if constexpr (PR::L >= 16) {
                constexpr int RL = PR::template radix<PR::kStages - 1>();
#pragma unroll
                for (int b = 0; b < PR::E / RL; ++b) {
#pragma unroll
                    for (int r = 0; r < RL; ++r) {
                        st_stream(dst + row * F::M + lane + b * PR::L + r * (PR::N / RL),
                                  u[b * RL + r]);
                    }
                }
            } else {
                // Short rows: back to the tile row, then each wave stores its 64 / L
                // consecutive rows as one contiguous run.
                lds_sync<true>();
                final_write<PR>(s, u, lane);
                lds_sync<true>();
                const int row0 = p * F::RPP + (tid / 64) * (64 / PR::L);
#pragma unroll
                for (int k = 0; k < PR::E; ++k) {
                    const int e = tid % 64 + k * 64;
                    const int rw = row0 + e / F::M;
                    const int i = e % F::M;
                    st_stream(dst + rw * F::M + i, tile[F::row_at(rw) + pad(i)]);
                }
            }
        }
        __syncthreads();  // the next array's values overwrite the tile
    }
}

// Persistent complex 2D for one array per workgroup whose rows load straight from HBM (fft2 /
// ifft2 of 128 x 128: a 140 KB tile, one workgroup per CU, so no other workgroup's traffic
// overlaps its LDS phases). Workgroup g takes arrays g, g + G, ...: every row pass's loads are
// issued before the first pass's transform, and the next array's rows are issued once the
// current array's rows are in the tile, so they are in flight during its column pass and
// stores. The wave waits for them, with its stores, at the top of the next turn.
template <class F, bool Inv>
__global__ void __launch_bounds__(F::NT)
    fft2_full_persistent_kernel(const cf32* __restrict__ x, cf32* __restrict__ y,
                                long long batch, float scale, const cf32* table)
{
    static_assert(F::AP == 1 && F::PR::L >= 16, "one array per workgroup, rows loaded directly");
    using PR = typename F::PR;
    using PC = typename F::PC;
    __shared__ cf32 tile[F::kTile];
    constexpr int kPerArray = F::N1 * F::M;
    constexpr int kPasses = F::N1 / F::RPP;
    constexpr int R0 = PR::template radix<0>();
    static_assert(kPasses * PR::E <= 32, "all row passes' inputs fit in registers");

    cf32 v[kPasses][PR::E];
    const auto fetch = [&](long long a, int tid) __attribute__((always_inline)) {
        const int lane = tid % PR::L;
        static_for<0, kPasses>([&](auto pi) {
            constexpr int p = decltype(pi)::value;
            const cf32* const src = x + (a * F::N1 + p * F::RPP + tid / PR::L) * F::M;
#pragma unroll
            for (int b = 0; b < PR::E / R0; ++b) {
#pragma unroll
                for (int r = 0; r < R0; ++r) {
                    v[p][b * R0 + r] = ld_stream(src + input_index<PR, 0>(lane, b, r));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    long long a = blockIdx.x;
    fetch(a, threadIdx.x);
#pragma unroll 1
    for (; a < batch; a += gridDim.x) {
        const int tid = opaque_tid<F::NT>();
        {
            const int lane = tid % PR::L;
            static_for<0, kPasses>([&](auto pi) {
                constexpr int p = decltype(pi)::value;
                cf32* const s = tile + F::row_at(p * F::RPP + tid / PR::L);
                run_stages<PR, 0, Inv, F::kTable, RowExchange<PR, F::TS>>(v[p], s, lane,
                                                                       table);
                lds_sync<true>();
                final_write<PR>(s, v[p], lane);
            });
        }
        __syncthreads();
        const long long next = a + gridDim.x;
        if (next < batch) {
            fetch(next, tid);
        }

#pragma unroll 1
        for (int c0 = 0; c0 < F::M; c0 += F::CPP) {
            const int c = c0 + F::col_slot(tid);
            if (c < F::M) {
                cf32* const s = tile + pad(c);
                const int cl = F::col_lane(tid);
                cf32 u[PC::E];
                stage_read<PC, 0, typename F::ColLay>(s, u, cl);
                run_stages<PC, 0, Inv, F::kTable, typename F::ColLay>(u, s, cl, table);
                lds_sync<true>();
                final_write<PC, typename F::ColLay>(s, u, cl);
            }
        }
        __syncthreads();

        cf32* const dst = y + a * kPerArray;
        constexpr int kStoreChunk = 8;
        static_assert(kPerArray % (F::NT * kStoreChunk) == 0, "whole store steps");
#pragma unroll 1
        for (int e0 = 0; e0 < kPerArray; e0 += F::NT * kStoreChunk) {
            cf32 val[kStoreChunk];
#pragma unroll
            for (int k = 0; k < kStoreChunk; ++k) {
                const int e = e0 + k * F::NT + tid;
                const int f = e / F::M;
                val[k] = tile[F::row_at(f) + pad(e - f * F::M)];
            }
#pragma unroll
            for (int k = 0; k < kStoreChunk; ++k) {
                st_stream(dst + e0 + k * F::NT + tid, cscale(val[k], scale));
            }
        }
        __syncthreads();  // the next array's rows overwrite the tile
    }
}

}  // namespace spx::dev
