#pragma once

// Host drivers of one Stockham variant (radix R, computed or table twiddles): argument checks,
// dispatch on the transform size, launch. Each stockham_*.hip file instantiates this header for
// one variant so the variants compile in parallel.
//
// The checks and their messages follow the reference's drivers (stockham.cuh:489-620,
// real.cu:160-180, fourstep.cuh:110-131): callers and tests match on them.

#include "fft2_fused.hpp"
#include "fft2_modes.hpp"
#include "fft2_pairs.hpp"
#include "fft2_transposed.hpp"
#include "fft_api.hpp"
#include "rf.hpp"
#include "stockham.hpp"

#include <algorithm>
#include <atomic>
#include <climits>
#include <optional>
#include <type_traits>

namespace spx {

// Validation shared by the variants.
void check_size(int n, const char* who);
void check_keep(int keep, int n, const char* who);
void check_real_arguments(const void* real_side, const void* complex_side, int n, int batch,
                          int complex_row, int max_n, const char* who);
// n = 2 real transforms (m = 1, where the complex transform is the identity): the combine or
// prepare alone, one row per lane (real.hip).
void r2c_n2(const float* x, cf32* y, int batch, int keep, hipStream_t stream);
void c2r_n2(const cf32* x, float* y, int batch, int keep, hipStream_t stream);
// n = 4 inverse (m = 2) in closed form, one row per lane; false (nothing queued) when y is not
// 16-byte aligned.
bool c2r_n4(const cf32* x, float* y, int batch, int keep, hipStream_t stream);
// The table of exp(-2 pi i m / kTableN) on the current device, built on first use.
const cf32* twiddle_table();
// Whether the current device's default memory pool keeps what is freed into it (its release
// threshold raised to the maximum on first use), so the stream-ordered workspaces of the large
// transforms reuse one reservation across calls instead of returning memory to the driver at
// every synchronization and mapping it again (the reference's fourstep.cu:9-37 policy). False on
// a device without memory pools: the caller then allocates synchronously.
bool pool_retained();

namespace dev {

template <class P, bool Inv, bool Table, class Io>
void launch(const Io& io, long long batch, hipStream_t stream)
{
    const long long blocks = (batch + P::T - 1) / P::T;
    const cf32* table = Table ? twiddle_table() : nullptr;
    hipLaunchKernelGGL((fft_kernel<P, Inv, Table, Io>), dim3(static_cast<unsigned>(blocks)),
                       dim3(P::kThreads), 0, stream, io, batch, table);
    SPX_LAUNCH_CHECK();
}

// The radix of the single-pass plan of N points. The radix-8 variants take 4096 points as three
// radix-16 stages (16 values per lane, two LDS exchanges instead of three): C2C 4096 unchanged
// (50.1 us), R2C / C2R 8192 (whose complex half is this plan) 29.4 -> 28.2 / 30.9 -> 29.1 us
// over 2^24 points, four alternated rounds on one box.
template <int N, int R>
constexpr int plan_radix()
{
    return (kRadix16 && R == 8 && N == 4096) ? 16 : R;
}

template <int N, int R>
constexpr int plan_e()
{
    return (kRadix16 && R == 8 && N == 4096) ? 16 : default_e<N, R>();
}

template <int R, bool Inv, bool Table, class Io>
void dispatch(int n, const Io& io, long long batch, hipStream_t stream)
{
    switch (n) {
#define SPX_CASE(N)                                                                          \
    case N:                                                                                  \
        launch<Plan<N, plan_radix<N, R>(), plan_e<N, R>()>, Inv, Table>(io, batch, stream);   \
        break;
        SPX_CASE(2)
        SPX_CASE(4)
        SPX_CASE(8)
        SPX_CASE(16)
        SPX_CASE(32)
        SPX_CASE(64)
        SPX_CASE(128)
        SPX_CASE(256)
        SPX_CASE(512)
        SPX_CASE(1024)
        SPX_CASE(2048)
        SPX_CASE(4096)
#undef SPX_CASE
    default:
        throw InvalidArgument("stockham: unsupported size " + str(n));
    }
}

// Strided columns: the plans of column_e / column_threads.
// The column plans' launch: persistent (tiles_persistent_kernel) for I/O policies whose load
// splits into a register fetch and an LDS park, else fft_kernel. Defined below.
template <class P, bool Inv, bool Table, class Io>
void launch_tiles(const Io& io, long long batch, hipStream_t stream);

template <int R, bool Inv, bool Table, class Io>
void dispatch_columns(int n, const Io& io, long long batch, hipStream_t stream)
{
    switch (n) {
#define SPX_CASE(N)                                                                          \
    case N:                                                                                  \
        launch_tiles<Plan<N, R, column_e<N, R>(), column_threads<N, R>()>, Inv, Table>(       \
            io, batch, stream);                                                              \
        break;
        SPX_CASE(2)
        SPX_CASE(4)
        SPX_CASE(8)
        SPX_CASE(16)
        SPX_CASE(32)
        SPX_CASE(64)
        SPX_CASE(128)
        SPX_CASE(256)
        SPX_CASE(512)
        SPX_CASE(1024)
        SPX_CASE(2048)
        SPX_CASE(4096)
#undef SPX_CASE
    default:
        throw InvalidArgument("stockham: unsupported size " + str(n));
    }
}

// The persistent strided column kernel over as many workgroups as fit on the device at once.
// Workgroups per CU depend only on the kernel and the architecture (gfx950 everywhere this
// library runs), so the first query serves every device; the CU count is per device.
template <class P, bool Inv, bool Table, int C = 0>
void launch_columns_persistent(const StridedIo& io, long long batch, hipStream_t stream)
{
    static const int per_cu = [] {
        int blocks = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &blocks, reinterpret_cast<const void*>(&columns_kernel<P, Inv, Table, C>),
            P::kThreads, 0);
        return e == hipSuccess && blocks > 0 ? blocks : 1;
    }();
    const long long tiles = (batch + P::T - 1) / P::T;
    const long long grid = std::min(tiles, static_cast<long long>(device_cus()) * per_cu);
    const cf32* table = Table ? twiddle_table() : nullptr;
    hipLaunchKernelGGL((columns_kernel<P, Inv, Table, C>), dim3(static_cast<unsigned>(grid)),
                       dim3(P::kThreads), 0, stream, io, batch, table);
    SPX_LAUNCH_CHECK();
}

// A persistent kernel whose workgroup g takes items g, g + G, ... of `items`: G = the workgroups
// that fit on the device at once (at most `items`). The workgroups per CU are queried once per
// kernel (a template argument, so kernels of one signature keep their own count). Kernel
// arguments follow `stream`.
template <auto Kernel, class... Args>
void launch_persistent(int threads, long long items, hipStream_t stream, Args... args)
{
    static const int per_cu = [threads] {
        int blocks = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &blocks, reinterpret_cast<const void*>(Kernel), threads, 0);
        return e == hipSuccess && blocks > 0 ? blocks : 1;
    }();
    const long long grid = std::min(items, static_cast<long long>(device_cus()) * per_cu);
    hipLaunchKernelGGL(Kernel, dim3(static_cast<unsigned>(grid)), dim3(threads), 0, stream,
                       args...);
    SPX_LAUNCH_CHECK();
}

// The single-pass irfft2 and the complex fft2 of one array per workgroup run persistent (the
// next array's loads overlap the current one's later phases); 0 keeps one array per workgroup.
#ifndef SPX_FUSED_PERSISTENT
#define SPX_FUSED_PERSISTENT 1
#endif
inline constexpr bool kFusedPersistent = SPX_FUSED_PERSISTENT != 0;

// The single-pass 16384-point C2C runs persistent (fft_persistent_kernel); 0 keeps one transform
// per workgroup.
#ifndef SPX_LARGE_PERSISTENT
#define SPX_LARGE_PERSISTENT 1
#endif
inline constexpr bool kPersistentLarge = SPX_LARGE_PERSISTENT != 0;

// Strided columns of 256, 512 and 1024 points, and of 64 and 128 points in wide matrices, run
// persistent (columns_kernel); other lengths keep one tile per workgroup. The 1024-point tiles hold
// 8 columns of 16 values per lane, one wave per column (workgroups of 512 lanes), in XCD order:
// 72.0 us for the columns of 2^20-point transforms over 2^24 points on MI355X, against 90.8 us for
// one tile per workgroup of 1024 lanes (8 values per lane, two waves per column) and 85.3 us for
// the same persistent kernel in plain order.
template <int R, bool Inv, bool Table>
void dispatch_strided_columns(int n, const StridedIo& io, long long batch, hipStream_t stream)
{
    switch (n) {
    case 64:
    case 128:
        // Wide matrices (the two-pass split's 64 x 512 and 128 x 512 at 2^15 and 2^16 points)
        // run persistent with workgroups of 512 lanes, 64- or 32-column tiles (512- or 256-byte
        // runs): over 2^24 points 56.8 -> 48.8 us at 64 and 63.8 -> 51.7 us at 128 on MI355X.
        if (io.cols >= 256) {
            if (n == 64) {
                launch_columns_persistent<Plan<64, R, column_e<64, R>(), 512>, Inv, Table>(
                    io, batch, stream);
            } else {
                launch_columns_persistent<Plan<128, R, column_e<128, R>(), 512>, Inv, Table>(
                    io, batch, stream);
            }
        } else {
            dispatch_columns<R, Inv, Table>(n, io, batch, stream);
        }
        break;
    case 256:
        // Wide matrices take workgroups of 1024 lanes, 32-column tiles with the radix-8 plans
        // (256-byte runs): 59.7 -> 55.6 us on 256 x 16384 matrices (2^22 points); at 128
        // columns (a 256^2 real array's) those measured 3 % slower than 16-column tiles.
        if (io.cols >= 1024) {
            launch_columns_persistent<Plan<256, R, column_e<256, R>(), 1024>, Inv, Table>(
                io, batch, stream);
        } else {
            launch_columns_persistent<Plan<256, R, column_e<256, R>(), column_threads<256, R>()>,
                                      Inv, Table>(io, batch, stream);
        }
        break;
    case 512:
        launch_columns_persistent<Plan<512, R, column_e<512, R>(), column_threads<512, R>()>, Inv,
                                  Table>(io, batch, stream);
        break;
    case 1024:
        // Radix 16 in the radix-8 variants (two exchanges instead of three): the 2^20-point
        // C2C over 2^24 points 115.6 -> 112.0 us in interleaved runs.
        launch_columns_persistent<Plan<1024, (R == 8 ? 16 : R), 16, 512>, Inv, Table, 32>(
            io, batch, stream);
        break;
    default:
        dispatch_columns<R, Inv, Table>(n, io, batch, stream);
    }
}

// Single-pass transforms beyond 4096 points: one transform per workgroup of 1024 lanes (N / 1024
// values per lane), the whole transform in LDS between stages (69,640 B at 8192 points, two
// workgroups per CU; 139,272 B at 16384, one). Measured on MI355X at 2^24 points: 8192 ran at
// 62-64 % of the 8 TB/s peak for radix 4 and 8 with 1024 lanes (512 or 256 lanes: 58-61 %);
// 16384 at 50 % (radix 8) and 53 % (radix 16), where the four-step split took 8 % and 13 %.
template <int N, int R>
using LargePlan = Plan<N, (N == 16384 && R == 8) ? 16 : R, N / kMaxBlock, kMaxBlock>;

template <class Io, class = void>
struct HasFetch : std::false_type {};
template <class Io>
struct HasFetch<Io, std::void_t<decltype(Io::kFetch)>> : std::bool_constant<Io::kFetch> {};

// The transposed-side passes of the transpose column method run persistent where their policy
// has fetch / park, at 512 points: 16-transform tiles of 1024 lanes, two per CU. irfft2 512² x 64
// by that method went from 59.7 to 53.6 us (four alternated rounds). At 64-256 points (tiles of
// 256 or 512 lanes, more per CU) and at 1024 (8-transform tiles) the loop measured 3-4 % slower,
// so those keep one tile per workgroup. SPX_TILES_PERSISTENT=0: one tile per workgroup at every
// size, for A/B builds.
#ifndef SPX_TILES_PERSISTENT
#define SPX_TILES_PERSISTENT 1
#endif

template <class P, bool Inv, bool Table, class Io>
void launch_tiles(const Io& io, long long batch, hipStream_t stream)
{
    if constexpr (SPX_TILES_PERSISTENT != 0 && HasFetch<Io>::value && P::N == 512) {
        launch_persistent<tiles_persistent_kernel<P, Inv, Table, Io>>(
            P::kThreads, (batch + P::T - 1) / P::T, stream, io, batch,
            Table ? twiddle_table() : nullptr);
    } else {
        launch<P, Inv, Table>(io, batch, stream);
    }
}

// The single-pass large plans. Where one workgroup fills a CU's LDS (16384 points, 139 KB),
// complex rows run persistent (fft_persistent_kernel): nothing else overlaps that workgroup's
// load phase. Measured over 2^24 points (four alternated rounds): 16384 66.1 -> 64.2 us, but
// 8192 (two workgroups per CU) 60.3 -> 63.4 us, so 8192 and the real transforms' combine and
// prepare keep one transform per workgroup.
template <class P, bool Inv, bool Table, class Io>
void launch_large(const Io& io, long long batch, hipStream_t stream)
{
    if constexpr (kPersistentLarge && P::N >= 16384 && Io::template direct_in<P>() &&
                  Io::template direct_out<P>() && !HasInAll<Io>::value && !HasFinal<Io>::value &&
                  !HasStage0<Io>::value) {
        launch_persistent<fft_persistent_kernel<P, Inv, Table, Io>>(
            P::kThreads, batch, stream, io, batch, Table ? twiddle_table() : nullptr);
    } else {
        launch<P, Inv, Table>(io, batch, stream);
    }
}

template <int R, bool Inv, bool Table, class Io>
void dispatch_large(int n, const Io& io, long long batch, hipStream_t stream)
{
    if (n == 8192) {
        launch_large<LargePlan<8192, R>, Inv, Table>(io, batch, stream);
    } else if (n == 16384) {
        launch_large<LargePlan<16384, R>, Inv, Table>(io, batch, stream);
    } else {
        throw InvalidArgument("stockham: unsupported size " + str(n));
    }
}

template <int R, bool Table, class Io>
void dispatch_dir(int n, bool inverse, const Io& io, long long batch, hipStream_t stream)
{
    if (inverse) {
        dispatch<R, true, Table>(n, io, batch, stream);
    } else {
        dispatch<R, false, Table>(n, io, batch, stream);
    }
}

// Four-step (Bailey) rows: batch * n1 rows of N values; element i of row t is multiplied by
// exp(sign 2 pi i k1 i / (n1 N)), k1 = t mod n1, before the row transform. k1 * i < 2^24 and
// 2 / (n1 N) is a power of two, so the angle is exact in float.
struct TwiddleRowsIo {
    static constexpr bool kGroupIsBlock = false;
    const cf32* x;
    cf32* y;
    float scale;
    float sign;
    int n1;
    float two_over_n;

    template <class P>
    static constexpr bool direct_in() { return P::L >= 16; }
    template <class P>
    static constexpr bool direct_out() { return P::L >= 16; }

    __device__ __forceinline__ cf32 twiddled(long long t, int i, cf32 v) const
    {
        const int k1 = static_cast<int>(t & (n1 - 1));
        cf32 w = expi_pi(static_cast<float>(k1 * i) * two_over_n);
        w.im *= sign;
        return cmul(v, w);
    }

    template <class P>
    __device__ __forceinline__ cf32 in(long long t, int i) const
    {
        return twiddled(t, i, x[t * P::N + i]);
    }

    // A lane's stage-0 elements are i = lane + L m, m = b + r E / R0 < E, so the twiddle factors:
    // w^(k1 i) = w^(k1 lane) w^(k1 L m). When a wave lies inside one transform (L >= 64: k1 is the
    // same on all its lanes) lane j computes w^(k1 L j) and every lane reads factor m from lane m:
    // two sincospi per lane instead of E. Both angles are exact in float (k1 L m < n1 N <= 2^24).
    static constexpr bool kInAll = true;
    template <class P>
    __device__ __forceinline__ void in_all(long long t, int lane, cf32 (&v)[P::E]) const
    {
        constexpr int R0 = P::template radix<0>();
        const cf32* const row = x + t * P::N;
        if constexpr (P::L >= 64 && P::E <= 64) {
            const int k1 = static_cast<int>(t & (n1 - 1));
            const int j = static_cast<int>(threadIdx.x & 63) % P::E;
            const cf32 base = expi_pi(static_cast<float>(k1 * lane) * two_over_n);
            const cf32 step = expi_pi(static_cast<float>(k1 * P::L * j) * two_over_n);
#pragma unroll
            for (int b = 0; b < P::E / R0; ++b) {
#pragma unroll
                for (int r = 0; r < R0; ++r) {
                    constexpr int kPerR = P::E / R0;
                    const int m = b + r * kPerR;
                    const cf32 f{__builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                     __builtin_bit_cast(int, step.re), m)),
                                 __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                     __builtin_bit_cast(int, step.im), m))};
                    cf32 w = cmul(base, f);
                    w.im *= sign;
                    v[b * R0 + r] = cmul(row[lane + P::L * m], w);
                }
            }
        } else {
#pragma unroll
            for (int b = 0; b < P::E / R0; ++b) {
#pragma unroll
                for (int r = 0; r < R0; ++r) {
                    const int i = input_index<P, 0>(lane, b, r);
                    v[b * R0 + r] = twiddled(t, i, row[i]);
                }
            }
        }
    }

    template <class P>
    __device__ __forceinline__ void out(long long t, int i, cf32 v) const
    {
        y[t * P::N + i] = cscale(v, scale);
    }

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        using S = Staged<G, P::N>;
        const cf32* src = x + first * P::N;
        cf32 val[S::kSteps];
        S::each(count, tid, [&](int k, int u, int i, bool valid) {
            val[k] = valid ? src[u * P::N + i] : czero();
        });
        S::each(count, tid, [&](int k, int u, int i, bool valid) {
            if (valid) {
                lds[u * P::kStride + pad(i)] = twiddled(first + u, i, val[k]);
            }
        });
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long first, int count,
                                          int tid) const
    {
        C2cIo<false>{nullptr, y, scale, P::N, P::N}.template store<P, G>(lds, first, count, tid);
    }
};

// Four-step rows that also transpose (the second of two passes): T consecutive rows k1 of one
// n1 x N matrix per workgroup, twiddled on the way in like TwiddleRowsIo, and element k2 of row
// k1 stored at y[slab n + k1 + n1 k2]. Staged through LDS, the store walks k1 fastest, so every
// k2 is one run of T * 8 bytes: the transposed layout comes out of the row kernel itself.
struct TwiddleRowsTransposedIo {
    static constexpr bool kGroupIsBlock = true;
    TwiddleRowsIo rows;  // input side: x, the twiddle and the scale
    long long n;         // n1 * N

    template <class P>
    static constexpr bool direct_in() { return P::L >= 16; }
    template <class P>
    static constexpr bool direct_out() { return false; }

    template <class P>
    __device__ __forceinline__ cf32 in(long long t, int i) const { return rows.in<P>(t, i); }
    static constexpr bool kInAll = true;
    template <class P>
    __device__ __forceinline__ void in_all(long long t, int lane, cf32 (&v)[P::E]) const
    {
        rows.in_all<P>(t, lane, v);
    }
    template <class P>
    __device__ __forceinline__ void out(long long, int, cf32) const {}

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        rows.load<P, G>(lds, first, count, tid);
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long first, int count,
                                          int tid) const
    {
        static_assert(G::kT == P::T, "the rows of a workgroup are stored together");
        constexpr int kTotal = P::T * P::N;
        static_assert(kTotal % G::kThreads == 0, "whole steps");
        const long long slab = first / rows.n1;  // T divides n1: one slab per workgroup
        const int k1 = static_cast<int>(first - slab * rows.n1);
        cf32* const dst = rows.y + slab * n + k1;
#pragma unroll
        for (int k = 0; k < kTotal / G::kThreads; ++k) {
            const int e = tid + k * G::kThreads;
            const int u = e % P::T;
            const int k2 = e / P::T;
            if (G::kFull || u < count) {
                st_stream(dst + u + static_cast<long long>(rows.n1) * k2,
                          cscale(lds[u * P::kStride + pad(k2)], rows.scale));
            }
        }
    }
};

// One of two passes of a long column transform (n = n1c x n2c points down the columns of
// slabs x n x cols arrays), each staging whole column runs like StridedIo. Transform t is column
// c = t mod cols of group g = (t / cols) mod groups of slab t / (cols groups); its element i is
// read at x[slab slab_elems + g step_in + i stride_in + c] and its output k written at
// y[slab slab_elems + g step_out + k stride_out + c], times exp(sign 2 pi i g k two_over_n / 2)
// when twiddled (two_over_n = 2 / n; g k < n, exact in float). With j = j1 n2c + j2 and
// k = k1 + n1c k2:
//   pass A: group g = j2, input rows j1 n2c + j2, output rows k1 n2c + j2, twiddle w_n^(j2 k1);
//   pass B: group g = k1, input rows k1 n2c + j2, output rows k1 + n1c k2 = X[k].
struct ColumnStepIo {
    static constexpr bool kGroupIsBlock = true;
    const cf32* x;
    cf32* y;
    int cols;
    int groups;
    long long slab_elems;
    long long step_in;
    long long stride_in;
    long long step_out;
    long long stride_out;
    float scale;
    bool twiddle;
    float sign;
    float two_over_n;
    bool stream_in;   // nontemporal loads (a caller's input), else plain (the pass-A workspace)
    bool stream_out;  // nontemporal stores (a final output), else plain (a workspace read next)

    template <class P>
    static constexpr bool direct_in() { return false; }
    template <class P>
    static constexpr bool direct_out() { return false; }

    template <class P>
    __device__ __forceinline__ cf32 in(long long, int) const { return czero(); }
    template <class P>
    __device__ __forceinline__ void out(long long, int, cf32) const {}

    // Base offset (without the element term) and group of transform t.
    __device__ __forceinline__ long long origin(long long t, bool input, int& g) const
    {
        const long long q = t / cols;
        const int c = static_cast<int>(t - q * cols);
        const long long slab = q / groups;
        g = static_cast<int>(q - slab * groups);
        return slab * slab_elems + g * (input ? step_in : step_out) + c;
    }

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        static_assert(G::kT == P::T, "column runs stage a whole workgroup");
        constexpr int kRowsPerStep = G::kThreads / P::T;
        constexpr int kSteps = P::N / kRowsPerStep;
        const int j = tid % P::T;
        if (!G::kFull && j >= count) {
            return;
        }
        int g = 0;
        const cf32* const base = x + origin(first + j, true, g);
        cf32 val[kSteps];
#pragma unroll
        for (int k = 0; k < kSteps; ++k) {
            const int i = tid / P::T + k * kRowsPerStep;
            val[k] = stream_in ? ld_stream(base + i * stride_in) : base[i * stride_in];
        }
#pragma unroll
        for (int k = 0; k < kSteps; ++k) {
            lds[j * P::kStride + pad(tid / P::T + k * kRowsPerStep)] = val[k];
        }
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long first, int count,
                                          int tid) const
    {
        constexpr int kRowsPerStep = G::kThreads / P::T;
        constexpr int kSteps = P::N / kRowsPerStep;
        const int j = tid % P::T;
        if (!G::kFull && j >= count) {
            return;
        }
        int g = 0;
        cf32* const base = y + origin(first + j, false, g);
        // The lane's rows are i = tid / T + k S (S = kRowsPerStep): w^(g i) is w^(g tid / T)
        // times k steps of w^(g S), two sincospi per lane instead of one per value (the
        // three-pass C2C at 2^21 points: 145 -> 140 us over 2^24 points; 0.5-1.5 % elsewhere).
        cf32 w{1.0f, 0.0f};
        cf32 step{1.0f, 0.0f};
        if (twiddle) {
            w = expi_pi(static_cast<float>(g * (tid / P::T)) * two_over_n);
            step = expi_pi(static_cast<float>(g * kRowsPerStep) * two_over_n);
            w.im *= sign;
            step.im *= sign;
        }
#pragma unroll
        for (int k = 0; k < kSteps; ++k) {
            const int i = tid / P::T + k * kRowsPerStep;
            cf32 v = cscale(lds[j * P::kStride + pad(i)], scale);
            if (twiddle) {
                v = cmul(v, w);
                w = cmul(w, step);
            }
            if (stream_out) {
                st_stream(base + i * stride_out, v);
            } else {
                base[i * stride_out] = v;
            }
        }
    }
};

// Rows of the two-pass split: 1024 lanes holding 16 rows of 512 points or 8 rows of 1024, so
// the transposed store writes 128- or 64-byte runs. At 1024 points 8 rows (64 KiB of LDS, two
// workgroups per CU) measured 64.3 us over 2^24 points on MI355X against 67.2 us for 16 rows
// (128 KiB, one workgroup per CU).
template <int N>
constexpr int transposed_rows() { return N <= 512 ? 16 : 8; }
template <int N, int R>
using TransposedRowsPlan =
    Plan<N, R, cmax(cmax(R, 4), N * transposed_rows<N>() / kMaxBlock), kMaxBlock>;

}  // namespace dev

// Stream-ordered scratch memory for one large-transform call: allocated on `stream` from the
// device's retained default pool, freed on it after the kernels queued in between, so no
// device-wide synchronization is needed. Without memory pools: hipMalloc / hipFree.
class StreamWorkspace {
public:
    StreamWorkspace(std::size_t count, hipStream_t stream)
        : stream_(stream), pooled_(pool_retained())
    {
        void* raw = nullptr;
        if (pooled_) {
            SPX_HIP_CHECK(hipMallocAsync(&raw, count * sizeof(cf32), stream));
        } else {
            SPX_HIP_CHECK(hipMalloc(&raw, count * sizeof(cf32)));
        }
        ptr_ = static_cast<cf32*>(raw);
    }
    ~StreamWorkspace() { (void)(pooled_ ? hipFreeAsync(ptr_, stream_) : hipFree(ptr_)); }
    StreamWorkspace(const StreamWorkspace&) = delete;
    StreamWorkspace& operator=(const StreamWorkspace&) = delete;
    cf32* get() const { return ptr_; }

private:
    cf32* ptr_ = nullptr;
    hipStream_t stream_;
    bool pooled_;
};

// The scratch of one large-transform call: `given` when the caller brings it (at least
// n x batch values), otherwise a StreamWorkspace of that size.
class CallScratch {
public:
    CallScratch(cf32* given, std::size_t count, hipStream_t stream) : ptr_(given)
    {
        if (ptr_ == nullptr) {
            own_.emplace(count, stream);
            ptr_ = own_->get();
        }
    }
    cf32* get() const { return ptr_; }

private:
    cf32* ptr_;
    std::optional<StreamWorkspace> own_;
};

template <int R, bool Table>
struct Stockham {
    // Complex transforms of n <= 4096 points. keep prunes the frequency side: forward writes the
    // first keep outputs, inverse reads the first keep inputs (the rest zero).
    static void c2c_single(const cf32* x, cf32* y, int n, int batch, Direction direction,
                           hipStream_t stream, int keep)
    {
        check_size(n, "stockham");
        if (batch < 1) {
            throw InvalidArgument("stockham: batch must be at least 1, got " + str(batch));
        }
        if (keep < 1 || keep > n) {
            throw InvalidArgument("stockham: keep must be in [1, " + str(n) + "], got "
                                  + str(keep));
        }
        const bool inverse = direction == Direction::Inverse;
        const int row_in = inverse ? keep : n;
        const int row_out = inverse ? n : keep;
        const auto rows = static_cast<std::size_t>(batch);
        if (x < y + rows * row_out && y < x + rows * row_in) {
            throw InvalidArgument("stockham: x and y must not overlap (out-of-place only)");
        }
        if (n == 1) {
            SPX_HIP_CHECK(hipMemcpyAsync(y, x, rows * sizeof(cf32), hipMemcpyDeviceToDevice,
                                         stream));
            return;
        }
        const float scale = inverse ? 1.0f / static_cast<float>(n) : 1.0f;
        if (keep == n) {
            dev::dispatch_dir<R, Table>(n, inverse, dev::C2cIo<false>{x, y, scale, n, n}, batch,
                                        stream);
        } else {
            dev::dispatch_dir<R, Table>(n, inverse,
                                        dev::C2cIo<true>{x, y, scale, row_in, row_out}, batch,
                                        stream);
        }
    }

    // n = n1 x n2 in two passes, for kSinglePassMaxN < n <= kTwoPassMaxN: n1-point transforms down
    // the n2 columns of each n1 x n2 matrix (x -> work), then the twiddled n2-point rows, stored
    // transposed (work -> y): X[k1 + n1 k2] is row k1's element k2.
    static void two_pass(const cf32* x, cf32* y, int n, int batch, Direction direction,
                         hipStream_t stream, cf32* given)
    {
        const int n2 = n <= (1 << 18) ? 512 : 1024;
        const int n1 = n / n2;
        if (static_cast<long long>(batch) * n1 > INT_MAX
            || static_cast<long long>(batch) * n2 > INT_MAX) {
            throw InvalidArgument("fourstep: too many transforms");
        }
        const bool inverse = direction == Direction::Inverse;
        const std::size_t total = static_cast<std::size_t>(n) * static_cast<std::size_t>(batch);
        const CallScratch work(given, total, stream);
        columns_impl(x, work.get(), n1, n2, batch, direction, stream, 0, 0, false);
        const dev::TwiddleRowsTransposedIo rows{
            dev::TwiddleRowsIo{work.get(), y, inverse ? 1.0f / static_cast<float>(n2) : 1.0f,
                               inverse ? 1.0f : -1.0f, n1, 2.0f / static_cast<float>(n)},
            n};
        const long long transforms = static_cast<long long>(batch) * n1;
        if (n2 == 512) {
            launch_rows<512>(rows, inverse, transforms, stream);
        } else {
            launch_rows<1024>(rows, inverse, transforms, stream);
        }
    }

    template <int N2>
    static void launch_rows(const dev::TwiddleRowsTransposedIo& rows, bool inverse,
                            long long transforms, hipStream_t stream)
    {
        using P = dev::TransposedRowsPlan<N2, R>;
        if (inverse) {
            dev::launch<P, true, Table>(rows, transforms, stream);
        } else {
            dev::launch<P, false, Table>(rows, transforms, stream);
        }
    }

    // Any power of two up to kFourStepMaxN: one kernel up to kSinglePassMaxN, two passes up to
    // kTwoPassMaxN, three beyond.
    // work: nullptr, or the caller's scratch of c2c_scratch_values(n, batch) values.
    static void c2c(const cf32* x, cf32* y, int n, int batch, Direction direction,
                    hipStream_t stream, cf32* work = nullptr)
    {
        if (n <= kStockhamMaxN) {
            c2c_single(x, y, n, batch, direction, stream, n);
            return;
        }
        if (!is_pow2(n) || n > kFourStepMaxN) {
            throw InvalidArgument("fourstep: n must be a power of two up to "
                                  + str(kFourStepMaxN) + ", got " + str(n));
        }
        if (batch < 1) {
            throw InvalidArgument("fourstep: batch must be at least 1, got " + str(batch));
        }
        const std::size_t total = static_cast<std::size_t>(n) * static_cast<std::size_t>(batch);
        if (x < y + total && y < x + total) {
            throw InvalidArgument("fourstep: x and y must not overlap (out-of-place only)");
        }
        if (n <= kSinglePassMaxN) {
            const bool inverse = direction == Direction::Inverse;
            const dev::C2cIo<false> io{x, y, inverse ? 1.0f / static_cast<float>(n) : 1.0f, n, n};
            if (inverse) {
                dev::dispatch_large<R, true, Table>(n, io, batch, stream);
            } else {
                dev::dispatch_large<R, false, Table>(n, io, batch, stream);
            }
            return;
        }
        if (n <= kTwoPassMaxN) {
            two_pass(x, y, n, batch, direction, stream, work);
            return;
        }
        three_pass(x, y, n, batch, direction, stream, work);
    }

    // n = n1 x 512 for kTwoPassMaxN < n <= kFourStepMaxN (n1 = 4096 .. 32768): two_pass with
    // its n1-point columns split again as 64 x n1b (ColumnStepIo, n1b = n1 / 64 = 64 .. 512).
    // Pass A: 64-point transforms over rows j1 n1b + j2 of each n1 x 512 matrix, twiddled by
    // w_n1^(j2 k1) (x -> y); pass B: n1b-point transforms over rows k1 n1b + j2, written to row
    // k1 + 64 k2 (y -> work); then two_pass's twiddled 512-point rows, 16 per workgroup, stored
    // transposed in 128-byte runs (work -> y). Each pass stages whole column runs or transposes
    // through LDS, so there is no separate transpose. Against the four-step it replaces (columns,
    // 16384-point rows, transpose), over 2^24 points on MI355X: 2^22 158 -> 140 us, 2^24
    // 183 -> 143 us; rows of 1024 (8 per workgroup, 64-byte runs) measured 3-7 % slower, and the
    // persistent column kernel 4-12 % slower than one tile per workgroup for both steps.
    static void three_pass(const cf32* x, cf32* y, int n, int batch, Direction direction,
                           hipStream_t stream, cf32* given)
    {
        constexpr int n2 = 512;
        constexpr int n1a = 64;
        const int n1 = n / n2;
        const int n1b = n1 / n1a;
        if (static_cast<long long>(batch) * n1 > INT_MAX) {
            throw InvalidArgument("fourstep: too many transforms");
        }
        const bool inverse = direction == Direction::Inverse;
        const float sign = inverse ? 1.0f : -1.0f;
        const std::size_t total = static_cast<std::size_t>(n) * static_cast<std::size_t>(batch);
        const CallScratch work(given, total, stream);
        const long long wide = static_cast<long long>(n1b) * n2;
        const dev::ColumnStepIo a{x,    y,    n2,   n1b,  n,    n2,    wide, n2,
                                  wide, 1.0f, true, sign, 2.0f / static_cast<float>(n1),
                                  true, false};
        const dev::ColumnStepIo b{y,
                                  work.get(),
                                  n2,
                                  n1a,
                                  n,
                                  wide,
                                  n2,
                                  n2,
                                  static_cast<long long>(n1a) * n2,
                                  inverse ? 1.0f / static_cast<float>(n1) : 1.0f,
                                  false,
                                  1.0f,
                                  0.0f,
                                  false,
                                  false};
        const long long transforms_a = static_cast<long long>(batch) * n1b * n2;
        const long long transforms_b = static_cast<long long>(batch) * n1a * n2;
        if (inverse) {
            dev::dispatch_columns<R, true, Table>(n1a, a, transforms_a, stream);
            dev::dispatch_columns<R, true, Table>(n1b, b, transforms_b, stream);
        } else {
            dev::dispatch_columns<R, false, Table>(n1a, a, transforms_a, stream);
            dev::dispatch_columns<R, false, Table>(n1b, b, transforms_b, stream);
        }
        const dev::TwiddleRowsTransposedIo rows{
            dev::TwiddleRowsIo{work.get(), y, inverse ? 1.0f / static_cast<float>(n2) : 1.0f,
                               sign, n1, 2.0f / static_cast<float>(n)},
            n};
        launch_rows<n2>(rows, inverse, static_cast<long long>(batch) * n1, stream);
    }

    // Columns of n = 2048 or 4096 points as two passes of 64 x (n / 64) (a four-step split of
    // the column axis): a single pass would stage only 4 or 2 columns per workgroup, reading
    // runs of 32 or 16 bytes; each of these passes stages 32 columns of 64 points (256-byte
    // runs). Pass A runs
    // the 64-point transforms over rows j1 (n/64) + j2 and twiddles them (x -> work); pass B runs
    // the (n/64)-point transforms over rows k1 (n/64) + j2 and writes row k1 + 64 k2 (work -> y).
    static void long_columns(const cf32* x, cf32* y, int n, int cols, int slabs,
                             Direction direction, hipStream_t stream, bool stream_out)
    {
        constexpr int n1c = 64;
        const int n2c = n / n1c;
        const bool inverse = direction == Direction::Inverse;
        const long long slab_elems = static_cast<long long>(n) * cols;
        const std::size_t total = static_cast<std::size_t>(slab_elems) * slabs;
        StreamWorkspace work(total, stream);
        const dev::ColumnStepIo a{x,
                                  work.get(),
                                  cols,
                                  n2c,
                                  slab_elems,
                                  cols,
                                  static_cast<long long>(n2c) * cols,
                                  cols,
                                  static_cast<long long>(n2c) * cols,
                                  1.0f,
                                  true,
                                  inverse ? 1.0f : -1.0f,
                                  2.0f / static_cast<float>(n),
                                  true,
                                  false};
        const dev::ColumnStepIo b{work.get(),
                                  y,
                                  cols,
                                  n1c,
                                  slab_elems,
                                  static_cast<long long>(n2c) * cols,
                                  cols,
                                  cols,
                                  static_cast<long long>(n1c) * cols,
                                  inverse ? 1.0f / static_cast<float>(n) : 1.0f,
                                  false,
                                  1.0f,
                                  0.0f,
                                  false,
                                  stream_out};
        const long long transforms_a = static_cast<long long>(slabs) * n2c * cols;
        const long long transforms_b = static_cast<long long>(slabs) * n1c * cols;
        if (inverse) {
            dev::dispatch_columns<R, true, Table>(n1c, a, transforms_a, stream);
            dev::dispatch_columns<R, true, Table>(n2c, b, transforms_b, stream);
        } else {
            dev::dispatch_columns<R, false, Table>(n1c, a, transforms_a, stream);
            dev::dispatch_columns<R, false, Table>(n2c, b, transforms_b, stream);
        }
    }

    // stream_out: y is a final output (nontemporal stores); false for an intermediate that the
    // next pass reads.
    static void columns_impl(const cf32* x, cf32* y, int n, int cols, int slabs,
                             Direction direction, hipStream_t stream, int m1_in, int m1_out,
                             bool stream_out = true)
    {
        check_size(n, "stockham columns");
        if (cols < 1 || slabs < 1 || static_cast<long long>(cols) * slabs > INT_MAX) {
            throw InvalidArgument("stockham columns: need 1 <= cols * slabs <= INT_MAX");
        }
        if (m1_in < 0 || m1_out < 0 || 2 * m1_in > n || 2 * m1_out > n) {
            throw InvalidArgument("stockham columns: need 0 <= 2 m1 <= n = " + str(n));
        }
        if ((m1_in > 0 || m1_out > 0) && x == y) {
            throw InvalidArgument("stockham columns: a pruned transform cannot run in place");
        }
        const long long batch = static_cast<long long>(cols) * slabs;
        if (n >= 2048 && m1_in == 0 && m1_out == 0 && cols >= 32) {
            long_columns(x, y, n, cols, slabs, direction, stream, stream_out);
            return;
        }
        if (n == 1) {
            if (x != y) {
                SPX_HIP_CHECK(hipMemcpyAsync(y, x, static_cast<std::size_t>(batch) * sizeof(cf32),
                                             hipMemcpyDeviceToDevice, stream));
            }
            return;
        }
        const bool inverse = direction == Direction::Inverse;
        const float scale = inverse ? 1.0f / static_cast<float>(n) : 1.0f;
        const dev::StridedIo io{x, y, cols, scale, m1_in, m1_out, stream_out};
        if (inverse) {
            dev::dispatch_strided_columns<R, true, Table>(n, io, batch, stream);
        } else {
            dev::dispatch_strided_columns<R, false, Table>(n, io, batch, stream);
        }
    }

    // Rows of a row-then-column 2D transform: full C2C rows into y, which the column pass reads
    // next in place, with plain stores.
    static void c2c_rows(const cf32* x, cf32* y, int n, int batch, Direction direction,
                         hipStream_t stream)
    {
        const auto rows = static_cast<std::size_t>(batch);
        if (n == 1 || batch < 1 || (x < y + rows * n && y < x + rows * n)) {
            c2c_single(x, y, n, batch, direction, stream, n);  // its checks and n = 1 copy
            return;
        }
        check_size(n, "stockham");
        const bool inverse = direction == Direction::Inverse;
        const float scale = inverse ? 1.0f / static_cast<float>(n) : 1.0f;
        dev::dispatch_dir<R, Table>(n, inverse, dev::C2cIo<false, true>{x, y, scale, n, n}, batch,
                                    stream);
    }

    static void columns(const cf32* x, cf32* y, int n, int cols, int slabs, Direction direction,
                        hipStream_t stream)
    {
        columns_impl(x, y, n, cols, slabs, direction, stream, 0, 0);
    }

    // plain_out: y is a workspace that the next pass reads (plain stores).
    static void r2c_impl(const float* x, cf32* y, int n, int batch, hipStream_t stream, int keep,
                         bool plain_out = false)
    {
        check_keep(keep, n, "stockham r2c");
        check_real_arguments(x, y, n, batch, keep, 2 * kStockhamMaxN, "stockham r2c");
        const int m = n / 2;
        const auto* z = reinterpret_cast<const cf32*>(x);
        if (m == 1) {
            r2c_n2(x, y, batch, keep, stream);
            return;
        }
        if (plain_out) {
            dev::dispatch_dir<R, Table>(m, false, dev::R2cIoT<true>{z, y, keep}, batch, stream);
        } else {
            dev::dispatch_dir<R, Table>(m, false, dev::R2cIo{z, y, keep}, batch, stream);
        }
    }

    static void c2r_impl(const cf32* x, float* y, int n, int batch, hipStream_t stream, int keep)
    {
        check_keep(keep, n, "stockham c2r");
        check_real_arguments(y, x, n, batch, keep, 2 * kStockhamMaxN, "stockham c2r");
        const int m = n / 2;
        auto* z = reinterpret_cast<cf32*>(y);
        if (m == 1) {
            c2r_n2(x, y, batch, keep, stream);
            return;
        }
        if (m == 2 && c2r_n4(x, y, batch, keep, stream)) {
            return;
        }
        const float scale = 1.0f / static_cast<float>(m);
        dev::dispatch_dir<R, Table>(m, true, dev::C2rIo{x, z, scale, keep}, batch, stream);
    }

    static void r2c(const float* x, cf32* y, int n, int batch, cf32*, hipStream_t stream)
    {
        r2c_impl(x, y, n, batch, stream, n / 2 + 1);
    }

    static void c2r(const cf32* x, float* y, int n, int batch, cf32*, hipStream_t stream)
    {
        c2r_impl(x, y, n, batch, stream, n / 2 + 1);
    }

    static void pruned_c2c(const cf32* x, cf32* y, int n, int batch, int keep,
                           Direction direction, hipStream_t stream)
    {
        c2c_single(x, y, n, batch, direction, stream, keep);
    }

    static void pruned_r2c(const float* x, cf32* y, int n, int batch, int keep,
                           hipStream_t stream)
    {
        r2c_impl(x, y, n, batch, stream, keep);
    }

    static void pruned_c2r(const cf32* x, float* y, int n, int batch, int keep,
                           hipStream_t stream)
    {
        c2r_impl(x, y, n, batch, stream, keep);
    }

    static void pruned_columns(const cf32* x, cf32* y, int n, int cols, int slabs, int m1_in,
                               int m1_out, Direction direction, hipStream_t stream)
    {
        columns_impl(x, y, n, cols, slabs, direction, stream, m1_in, m1_out);
    }

    // The same two into a workspace that the next pass reads: plain stores.
    static void pruned_r2c_work(const float* x, cf32* y, int n, int batch, int keep,
                                hipStream_t stream)
    {
        r2c_impl(x, y, n, batch, stream, keep, true);
    }

    static void pruned_columns_work(const cf32* x, cf32* y, int n, int cols, int slabs,
                                    int m1_in, int m1_out, Direction direction,
                                    hipStream_t stream)
    {
        columns_impl(x, y, n, cols, slabs, direction, stream, m1_in, m1_out, false);
    }

    // Not constexpr on purpose: a constant-initialized table of host function addresses would
    // also be emitted for the device, where those functions do not exist.
    static PrunedFns pruned_fns()
    {
        return {&pruned_c2c,     &pruned_r2c,      &pruned_c2r,
                &pruned_columns, &pruned_r2c_work, &pruned_columns_work};
    }
};

// The (n1, n2) shapes with a single-pass 2D kernel: both in 4 .. 16, or both in 32 .. 256 with the
// half spectrum (plus row padding) within the 80 KB LDS tile of fft2_fused.hpp.
#define SPX_FUSED_SHAPES(X)                                                                     \
    X(4, 4) X(8, 4) X(16, 4) X(4, 8) X(8, 8) X(16, 8) X(4, 16) X(8, 16) X(16, 16)                \
    X(32, 32) X(64, 32) X(128, 32) X(256, 32) X(32, 64) X(64, 64) X(128, 64) X(256, 64)         \
    X(32, 128) X(64, 128) X(128, 128) X(32, 256) X(64, 256)

// The (n1, n2) shapes with a single-pass complex 2D kernel: an array of n1 x n2 complex values
// (plus row padding) within the same 80 KB tile, and 128 x 128 alone in a 140 KB one (one
// workgroup per CU).
#define SPX_FUSED_C2C_SHAPES(X)                                                                 \
    X(4, 4) X(8, 8) X(16, 16) X(32, 32) X(32, 64) X(64, 32) X(64, 64) X(64, 128) X(128, 64)      \
    X(128, 128)

// The fused shapes whose pruned transforms with w <= n2/8 kept columns take the narrow-tile
// kernels of fft2_modes.hpp (n2 >= 64, and n1 at least one row pass, at most 128 rows).
#define SPX_MODES_SHAPES(X)                                                                     \
    X(64, 64) X(128, 64) X(32, 128) X(64, 128) X(128, 128) X(32, 256) X(64, 256)

template <int N1, int N2>
constexpr bool modes_shape()
{
#define SPX_X(A, B) || (N1 == (A) && N2 == (B))
    return false SPX_MODES_SHAPES(SPX_X);
#undef SPX_X
}

// Single-pass 2D drivers of one variant (radix 4 and up; radix 2 has none).
template <int R, bool Table>
struct Fused2dDriver {
    static bool supports(int n1, int n2)
    {
        if constexpr (R >= 4) {
#define SPX_X(A, B)                 \
    if (n1 == (A) && n2 == (B)) {   \
        return true;                \
    }
            SPX_FUSED_SHAPES(SPX_X)
#undef SPX_X
        }
        (void)n1;
        (void)n2;
        return false;
    }

    static void check(const void* real_side, const void* complex_side, int n1, int n2, int m1,
                      int w, int batch)
    {
        if (!supports(n1, n2)) {
            throw InvalidArgument("fused 2D: no kernel for " + str(n1) + " x " + str(n2));
        }
        if (batch < 1 || m1 < 0 || 2 * m1 > n1 || w < 1 || w > n2 / 2 + 1) {
            throw InvalidArgument("fused 2D: bad batch, m1 or w");
        }
        const auto* r = static_cast<const char*>(real_side);
        const auto* c = static_cast<const char*>(complex_side);
        const std::size_t real_bytes =
            static_cast<std::size_t>(batch) * static_cast<std::size_t>(n1) * n2 * sizeof(float);
        const std::size_t complex_bytes = static_cast<std::size_t>(batch)
                                          * static_cast<std::size_t>(m1 > 0 ? 2 * m1 : n1) * w
                                          * sizeof(cf32);
        if (r < c + complex_bytes && c < r + real_bytes) {
            throw InvalidArgument("fused 2D: input and output must not overlap");
        }
    }

    template <int N1, int M>
    static void launch_r2c(const float* x, cf32* y, int m1, int w, int batch, hipStream_t stream)
    {
        if constexpr (modes_shape<N1, 2 * M>()) {
            if (m1 > 0 && w <= M / 4) {
                using F = dev::Modes2d<N1, M, R, Table>;
                hipLaunchKernelGGL((dev::rfft2_modes_kernel<F>), dim3(static_cast<unsigned>(batch)),
                                   dim3(F::NT), 0, stream, reinterpret_cast<const cf32*>(x), y, m1,
                                   w, dev::FastDiv::of(static_cast<unsigned>(w)),
                                   Table ? twiddle_table() : nullptr);
                SPX_LAUNCH_CHECK();
                return;
            }
        }
        using F = dev::Fused2d<N1, M, R, Table>;
        const long long blocks = (static_cast<long long>(batch) + F::AP - 1) / F::AP;
        const cf32* table = Table ? twiddle_table() : nullptr;
        const int rows_out = m1 > 0 ? 2 * m1 : N1;
        // The whole half spectrum (rfft2 itself) takes the variant with m1 and w fixed at
        // compile time.
        const auto kernel = (m1 == 0 && w == M + 1) ? dev::rfft2_fused_kernel<F, true>
                                                    : dev::rfft2_fused_kernel<F, false>;
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(F::NT), 0, stream,
                           reinterpret_cast<const cf32*>(x), y, m1, w,
                           dev::FastDiv::of(static_cast<unsigned>(w)),
                           dev::FastDiv::of(static_cast<unsigned>(rows_out * w)),
                           static_cast<long long>(batch), table);
        SPX_LAUNCH_CHECK();
    }

    template <int N1, int M>
    static void launch_c2r(const cf32* x, float* y, int m1, int w, int batch, hipStream_t stream)
    {
        if constexpr (modes_shape<N1, 2 * M>()) {
            if (m1 > 0 && w <= M / 4) {
                using F = dev::Modes2d<N1, M, R, Table>;
                // Compile-time bounds on w (half the tile's columns, or all of them) and on m1
                // (an eighth, a quarter or half of the rows): the smallest that hold them.
                const auto pick = [m1](auto wb) {
                    constexpr int kW = decltype(wb)::value;
                    return m1 <= N1 / 8   ? dev::irfft2_modes_kernel<F, kW, N1 / 8>
                           : m1 <= N1 / 4 ? dev::irfft2_modes_kernel<F, kW, N1 / 4>
                                          : dev::irfft2_modes_kernel<F, kW, N1 / 2>;
                };
                const auto kernel = w <= F::WMax / 2
                                        ? pick(std::integral_constant<int, F::WMax / 2>{})
                                        : pick(std::integral_constant<int, F::WMax>{});
                hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(batch)), dim3(F::NT), 0,
                                   stream, x, reinterpret_cast<cf32*>(y), m1, w,
                                   dev::FastDiv::of(static_cast<unsigned>(w)),
                                   Table ? twiddle_table() : nullptr);
                SPX_LAUNCH_CHECK();
                return;
            }
        }
        using F = dev::Fused2d<N1, M, R, Table>;
        const long long blocks = (static_cast<long long>(batch) + F::AP - 1) / F::AP;
        const cf32* table = Table ? twiddle_table() : nullptr;
        if constexpr (F::AP == 1 && dev::kFusedPersistent && dev::FullRows<F>::kUse) {
            if (m1 == 0 && w == M + 1) {
                dev::launch_persistent<dev::irfft2_full_persistent_kernel<F>>(
                    F::NT, batch, stream, x, reinterpret_cast<cf32*>(y),
                    static_cast<long long>(batch), table);
                return;
            }
        }
        const int rows_in = m1 > 0 ? 2 * m1 : N1;
        const auto kernel = (m1 == 0 && w == M + 1) ? dev::irfft2_fused_kernel<F, true>
                                                    : dev::irfft2_fused_kernel<F, false>;
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(F::NT), 0, stream, x,
                           reinterpret_cast<cf32*>(y), m1, w,
                           dev::FastDiv::of(static_cast<unsigned>(w)),
                           dev::FastDiv::of(static_cast<unsigned>(rows_in * w)),
                           static_cast<long long>(batch), table);
        SPX_LAUNCH_CHECK();
    }

    static void r2c(const float* x, cf32* y, int n1, int n2, int m1, int w, int batch,
                    hipStream_t stream)
    {
        check(x, y, n1, n2, m1, w, batch);
        if constexpr (R >= 4) {
#define SPX_X(A, B)                                                  \
    if (n1 == (A) && n2 == (B)) {                                    \
        launch_r2c<(A), (B) / 2>(x, y, m1, w, batch, stream);        \
        return;                                                      \
    }
            SPX_FUSED_SHAPES(SPX_X)
#undef SPX_X
        }
    }

    // Not constexpr, like Stockham::pruned_fns: host function addresses only.
    static bool c2c_supports(int n1, int n2)
    {
        if constexpr (R >= 4) {
#define SPX_X(A, B)                 \
    if (n1 == (A) && n2 == (B)) {   \
        return true;                \
    }
            SPX_FUSED_C2C_SHAPES(SPX_X)
#undef SPX_X
        }
        (void)n1;
        (void)n2;
        return false;
    }

    template <int N1, int N2>
    static void launch_c2c(const cf32* x, cf32* y, int batch, bool inverse, hipStream_t stream)
    {
        // M = N2: complex rows of n2 values; 128 x 128 takes a 143 KB tile. With 128 rows, one
        // array per workgroup of 1024 lanes: 128 x 128 76.4 -> 71.7 us and 128 x 64 56.4 ->
        // 53.4 us over 2^24 points on MI355X against 512 lanes (64 x 128 unchanged; the real
        // kernels at 128 x 128 measured 39 % slower with 1024, and still 3-6 % slower with one
        // row pass, 8-value columns and 43-55 VGPRs, i.e. 8 waves per SIMD).
        using F = dev::Fused2d<N1, N2, R, Table, (N1 * N2 > 8192 ? 160 : 80),
                               (N1 >= 128 ? 1024 : 512), true>;
        const long long blocks = (static_cast<long long>(batch) + F::AP - 1) / F::AP;
        const cf32* table = Table ? twiddle_table() : nullptr;
        const float scale = inverse ? 1.0f / static_cast<float>(N1 * N2) : 1.0f;
        if constexpr (F::AP == 1 && F::PR::L >= 16 && dev::kFusedPersistent) {
            if (inverse) {
                dev::launch_persistent<dev::fft2_full_persistent_kernel<F, true>>(
                    F::NT, batch, stream, x, y, static_cast<long long>(batch), scale, table);
            } else {
                dev::launch_persistent<dev::fft2_full_persistent_kernel<F, false>>(
                    F::NT, batch, stream, x, y, static_cast<long long>(batch), scale, table);
            }
            return;
        }
        if (inverse) {
            hipLaunchKernelGGL((dev::fft2_fused_kernel<F, true>),
                               dim3(static_cast<unsigned>(blocks)), dim3(F::NT), 0, stream, x, y,
                               static_cast<long long>(batch), scale, table);
        } else {
            hipLaunchKernelGGL((dev::fft2_fused_kernel<F, false>),
                               dim3(static_cast<unsigned>(blocks)), dim3(F::NT), 0, stream, x, y,
                               static_cast<long long>(batch), scale, table);
        }
        SPX_LAUNCH_CHECK();
    }

    static void c2c(const cf32* x, cf32* y, int n1, int n2, int batch, Direction direction,
                    hipStream_t stream)
    {
        if (!c2c_supports(n1, n2) || batch < 1) {
            throw InvalidArgument("fused 2D: no complex kernel for " + str(n1) + " x " + str(n2));
        }
        const std::size_t bytes = static_cast<std::size_t>(batch) * n1 * n2 * sizeof(cf32);
        const auto* a = reinterpret_cast<const char*>(x);
        const auto* b = reinterpret_cast<const char*>(y);
        if (a < b + bytes && b < a + bytes) {
            throw InvalidArgument("fused 2D: input and output must not overlap");
        }
        const bool inverse = direction == Direction::Inverse;
        if constexpr (R >= 4) {
#define SPX_X(A, B)                                             \
    if (n1 == (A) && n2 == (B)) {                               \
        launch_c2c<(A), (B)>(x, y, batch, inverse, stream);     \
        return;                                                 \
    }
            SPX_FUSED_C2C_SHAPES(SPX_X)
#undef SPX_X
        }
        (void)inverse;
    }

    // Row-pair passes (fft2_pairs.hpp).
    template <class Io>
    static void pairs(int m, bool inverse, const Io& io, long long transforms,
                      hipStream_t stream)
    {
        switch (m) {
#define SPX_CASE(M)                                                                   \
    case M:                                                                           \
        if (inverse) {                                                                \
            dev::launch<dev::PairPlan<M, R>, true, Table>(io, transforms, stream);    \
        } else {                                                                      \
            dev::launch<dev::PairPlan<M, R>, false, Table>(io, transforms, stream);   \
        }                                                                             \
        break;
            SPX_CASE(16)
            SPX_CASE(32)
            SPX_CASE(64)
            SPX_CASE(128)
            SPX_CASE(256)
            SPX_CASE(512)
            SPX_CASE(1024)
            SPX_CASE(2048)
            SPX_CASE(4096)
#undef SPX_CASE
        default:
            throw InvalidArgument("fft2 row pairs: unsupported m " + str(m));
        }
    }

    static void c2c_rows(const cf32* x, cf32* y, int n, int batch, Direction direction,
                         hipStream_t stream)
    {
        Stockham<R, Table>::c2c_rows(x, y, n, batch, direction, stream);
    }

    // The forward's column pass, into the workspace that r2c_rows reads next (plain stores).
    static void r2c_columns(const cf32* x, cf32* z, int n1, int m, int batch, hipStream_t stream)
    {
        Stockham<R, Table>::columns_impl(x, z, n1, m, batch, Direction::Forward, stream, 0, 0,
                                         false);
    }

    static void r2c_rows(const cf32* z, cf32* y, int n1, int m, int batch, hipStream_t stream)
    {
        const dev::PairRows rows{n1, n1 / 2 + 1};
        pairs(m, false, dev::PairR2cIo{z, y, rows}, 2LL * batch * rows.pairs, stream);
    }

    static void c2r_rows(const cf32* x, cf32* z, int n1, int m, int batch, hipStream_t stream)
    {
        const dev::PairRows rows{n1, n1 / 2 + 1};
        pairs(m, true, dev::PairC2rIo{x, z, rows, 1.0f / static_cast<float>(m)},
              2LL * batch * rows.pairs, stream);
    }

    // The transpose column method in two passes (fft2_transposed.hpp), on the column plans
    // (T = 16 transforms per workgroup up to N = 512: 128-byte runs on the transposed side).
    // work: batch arrays of n2 x n1 (complex) or (n2/2 + 1) x n1 (real) values.
    template <class Io>
    static void columns_plan(int n, bool inverse, const Io& io, long long transforms,
                             hipStream_t stream)
    {
        if (inverse) {
            dev::dispatch_columns<R, true, Table>(n, io, transforms, stream);
        } else {
            dev::dispatch_columns<R, false, Table>(n, io, transforms, stream);
        }
    }

    // Rows of n2 (x -> work, stored transposed), then the columns as rows of n1 (work -> y,
    // stored transposed back). The inverse's 1/n2 and 1/n1 ride on the two passes' stores.
    static void c2c_transposed(const cf32* x, cf32* y, cf32* work, int n1, int n2, int batch,
                               Direction direction, hipStream_t stream)
    {
        const bool inverse = direction == Direction::Inverse;
        const float s2 = inverse ? 1.0f / static_cast<float>(n2) : 1.0f;
        const float s1 = inverse ? 1.0f / static_cast<float>(n1) : 1.0f;
        columns_plan(n2, inverse, dev::RowsToTransposedIo{x, work, n1, s2, true, false},
                     static_cast<long long>(batch) * n1, stream);
        columns_plan(n1, inverse, dev::RowsToTransposedIo{work, y, n2, s1, false, true},
                     static_cast<long long>(batch) * n2, stream);
    }

    // Real rows of n2 = 2m to half spectra, stored transposed (x -> work); then the m + 1
    // columns as rows of n1 (work -> y, stored transposed back).
    static void r2c_transposed(const float* x, cf32* y, cf32* work, int n1, int n2, int batch,
                               hipStream_t stream)
    {
        const int m = n2 / 2;
        columns_plan(m, false,
                     dev::R2cRowsToTransposedIo{reinterpret_cast<const cf32*>(x), work, n1},
                     static_cast<long long>(batch) * n1, stream);
        columns_plan(n1, false, dev::RowsToTransposedIoT<8>{work, y, m + 1, 1.0f, false, false},
                     static_cast<long long>(batch) * (m + 1), stream);
    }

    // The m + 1 columns of the half spectra read transposed, inverted and written as rows of n1
    // (x -> work); then the real rows read transposed from there (work -> y).
    static void c2r_transposed(const cf32* x, float* y, cf32* work, int n1, int n2, int batch,
                               hipStream_t stream)
    {
        const int m = n2 / 2;
        columns_plan(n1, true,
                     dev::TransposedToRowsIoT<8>{x, work, m + 1, 1.0f / static_cast<float>(n1),
                                                 false, false},
                     static_cast<long long>(batch) * (m + 1), stream);
        columns_plan(m, true,
                     dev::C2rTransposedToRowsIo{work, reinterpret_cast<cf32*>(y), n1,
                                                1.0f / static_cast<float>(m)},
                     static_cast<long long>(batch) * n1, stream);
    }

    static Fused2dFns fns()
    {
        return {&supports,       &r2c,           &c2r,           &r2c_columns, &r2c_rows,
                &c2r_rows,       &c2c_supports,  &c2c,           &c2c_rows,    &c2c_transposed,
                &r2c_transposed, &c2r_transposed};
    }

    static void c2r(const cf32* x, float* y, int n1, int n2, int m1, int w, int batch,
                    hipStream_t stream)
    {
        check(y, x, n1, n2, m1, w, batch);
        if constexpr (R >= 4) {
#define SPX_X(A, B)                                                  \
    if (n1 == (A) && n2 == (B)) {                                    \
        launch_c2r<(A), (B) / 2>(x, y, m1, w, batch, stream);        \
        return;                                                      \
    }
            SPX_FUSED_SHAPES(SPX_X)
#undef SPX_X
        }
    }
};

// The radio callers' kernels of one variant (rf.hpp): the plans of dispatch and dispatch_large.
template <int R, bool Table>
struct RfDriver {
    template <int N>
    using PlanOf =
        std::conditional_t<(N > kStockhamMaxN), dev::LargePlan<N, R>,
                           dev::Plan<N, dev::plan_radix<N, R>(), dev::plan_e<N, R>()>>;

    // The FIR's blocks, a forward and an inverse transform each, are bound by their arithmetic
    // and exchanges rather than by HBM. At 1024 points the radix-8 variants run them as radix 16
    // with 16 values per lane: one wave per transform, so its exchanges need no workgroup
    // barrier. rf.fir with 255 taps (1024-point blocks) over 2^22 samples: 27.2 -> 25.6 us (four
    // alternated rounds); at 256 and 512 points the same change measured 11 % slower, at 2048
    // no different.
    template <int N>
    using FirPlanOf =
        std::conditional_t<(dev::kRadix16 && R == 8 && N == 1024), dev::Plan<N, 16, 16>, PlanOf<N>>;

    static void check(long long n, int nfft, long long rows, const char* who)
    {
        if (!is_pow2(nfft) || nfft < 2 || nfft > kSinglePassMaxN) {
            throw InvalidArgument(std::string(who) + ": nfft must be a power of two from 2 to "
                                  + str(kSinglePassMaxN) + ", got " + str(nfft));
        }
        if (n < 0 || rows < 0) {
            throw InvalidArgument(std::string(who) + ": n and rows must not be negative");
        }
    }

    template <class F>
    static void by_size(int nfft, F&& f)
    {
        switch (nfft) {
#define SPX_CASE(N)                                     \
    case N:                                             \
        f(std::integral_constant<int, N>{});            \
        break;
            SPX_CASE(2)
            SPX_CASE(4)
            SPX_CASE(8)
            SPX_CASE(16)
            SPX_CASE(32)
            SPX_CASE(64)
            SPX_CASE(128)
            SPX_CASE(256)
            SPX_CASE(512)
            SPX_CASE(1024)
            SPX_CASE(2048)
            SPX_CASE(4096)
            SPX_CASE(8192)
            SPX_CASE(16384)
#undef SPX_CASE
        default:
            throw InvalidArgument("rf: unsupported nfft " + str(nfft));
        }
    }

    static void spectrum(const cf32* x, const float* window, cf32* y, long long n, int nfft,
                         long long rows, hipStream_t stream)
    {
        check(n, nfft, rows, "spectrum");
        const long long frames = n > nfft ? (n + nfft - 1) / nfft : 1;
        const long long transforms = rows * frames;
        if (transforms == 0) {
            return;
        }
        const dev::FramesIo io{x, window, y, n, frames};
        by_size(nfft, [&](auto size) {
            dev::launch<PlanOf<decltype(size)::value>, false, Table>(io, transforms, stream);
        });
    }

    static void fir(const cf32* x, const cf32* h, cf32* y, long long n, int taps, int nfft,
                    long long rows, hipStream_t stream)
    {
        check(n, nfft, rows, "fir");
        if (taps < 1 || taps > nfft) {
            throw InvalidArgument("fir: nfft must be a power of two of at least len(taps) = "
                                  + str(taps) + ", got " + str(nfft));
        }
        const int step = nfft - taps + 1;
        const long long blocks = n > step ? (n + step - 1) / step : 1;
        if (rows == 0 || n == 0) {
            return;
        }
        const cf32* table = Table ? twiddle_table() : nullptr;
        by_size(nfft, [&](auto size) {
            dev::launch_fir<FirPlanOf<decltype(size)::value>, Table>(x, h, y, n, taps, step,
                                                                     blocks, rows * blocks,
                                                                     table, stream);
        });
    }

    static void filter(const void* taps, bool complex_taps, cf32* h, int count, int nfft,
                       hipStream_t stream)
    {
        check(0, nfft, 0, "fir");
        if (count < 1 || count > nfft) {
            throw InvalidArgument("fir: nfft must be a power of two of at least len(taps) = "
                                  + str(count) + ", got " + str(nfft));
        }
        const dev::TapsIo io{taps, complex_taps, count, h};
        by_size(nfft, [&](auto size) {
            dev::launch<PlanOf<decltype(size)::value>, false, Table>(io, 1, stream);
        });
    }

    static RfFns fns() { return {&spectrum, &fir, &filter, kSinglePassMaxN}; }
};

}  // namespace spx

// Defines the registry entry points of one variant (declared by SPX_DECLARE_VARIANT).
#define SPX_DEFINE_VARIANT(NAME, R, TABLE)                                                     \
    namespace spx {                                                                             \
    void c2c_##NAME(const cf32* x, cf32* y, int n, int batch, Direction direction,             \
                    hipStream_t stream)                                                         \
    {                                                                                           \
        Stockham<R, TABLE>::c2c(x, y, n, batch, direction, stream);                             \
    }                                                                                           \
    void c2c_work_##NAME(const cf32* x, cf32* y, int n, int batch, Direction direction,        \
                         cf32* work, hipStream_t stream)                                        \
    {                                                                                           \
        Stockham<R, TABLE>::c2c(x, y, n, batch, direction, stream, work);                       \
    }                                                                                           \
    void r2c_##NAME(const float* x, cf32* y, int n, int batch, cf32* work, hipStream_t stream) \
    {                                                                                           \
        Stockham<R, TABLE>::r2c(x, y, n, batch, work, stream);                                  \
    }                                                                                           \
    void c2r_##NAME(const cf32* x, float* y, int n, int batch, cf32* work, hipStream_t stream) \
    {                                                                                           \
        Stockham<R, TABLE>::c2r(x, y, n, batch, work, stream);                                  \
    }                                                                                           \
    void columns_##NAME(const cf32* x, cf32* y, int n, int cols, int slabs,                    \
                        Direction direction, hipStream_t stream)                                \
    {                                                                                           \
        Stockham<R, TABLE>::columns(x, y, n, cols, slabs, direction, stream);                   \
    }                                                                                           \
    const PrunedFns pruned_##NAME = Stockham<R, TABLE>::pruned_fns();                           \
    const Fused2dFns fused_##NAME = Fused2dDriver<R, TABLE>::fns();                             \
    const RfFns rf_##NAME = RfDriver<R, TABLE>::fns();                                          \
    }
