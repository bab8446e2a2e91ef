#pragma once

// Batched power-of-two FFTs for gfx950: the Stockham autosort recurrence, one workgroup pass per
// group of transforms, data in registers between stages and LDS only for the exchanges.
//
// The recurrence (a textbook algorithm, the same one the reference's stockham.cuh:169-209 runs):
// a stage of radix R turns sub-transforms of length ns into sub-transforms of length ns * R.
// Butterfly j (k = j mod ns) takes inputs in[j + r N/R] for r < R, multiplies input r by
// w^(k r) with w = exp(sign 2 pi i / (ns R)), takes an R-point DFT, and writes output r to
// out[(j - k) R + k + r ns]. After the last stage the result is in natural order.
//
// How this file maps it onto CDNA4 (the design is this repository's own):
//
// * Elements per lane E is a separate parameter from the radix. A transform of N points is
//   owned by L = N / E lanes; each lane holds E values in VGPRs and runs E / R butterflies per
//   stage (j = lane + b L). The radix only sets the stage count: radix 8 at N = 1024 is
//   8 x 8 x 8 x 2; with E = 8 a lane runs one radix-8 butterfly per stage, then four radix-2.
// * A workgroup is 256 lanes (four wave64s) and holds T = 256 / L transforms. When L <= 64 every
//   transform lives inside one wavefront, so the LDS exchanges between stages need only a
//   wavefront-scope fence (no s_barrier): the four waves of a workgroup never wait for each other.
//   E is chosen per (N, R) by default_e: small, for occupancy.
// * Contiguous rows (L >= 16) skip LDS on the way in and out: the first stage's inputs
//   in[j + r N/R] are read straight from HBM (for fixed b, r the lanes of a transform read
//   consecutive values, runs of L * 8 >= 128 bytes), and the last stage's outputs
//   out[j + r N/R] are written straight back. Only the stage exchanges touch LDS.
// * Other access patterns (small N, strided columns, the real-FFT combine that pairs k with
//   N - k) stage through LDS: the group loads cooperatively and coalesced, then the first stage
//   reads LDS.
// * LDS rows are padded by one complex value per 16 (index i is stored at i + i / 16), and the
//   per-transform stride is odd, so stride-R stage writes and column-major staging spread over
//   the banks.
// * Twiddles: one evaluation per lane per stage (exact integer reduction to a quadrant, then
//   short Taylor series; or, in the table variants, one lookup in a table built once in double
//   precision), its powers by complex products, and compile-time constants for the lane's other
//   butterflies. LDS addresses are a
//   per-lane base plus compile-time offsets.

#include "spx_common.hpp"

#include <cstdint>
#include <type_traits>

namespace spx::dev {

constexpr int kBlock = 256;      // lanes per workgroup, unless one transform needs more
constexpr int kMaxBlock = 1024;  // the largest workgroup

__host__ __device__ constexpr int clog2(int n)
{
    int r = 0;
    while ((1 << r) < n) {
        ++r;
    }
    return r;
}

__host__ __device__ constexpr int cmin(int a, int b) { return a < b ? a : b; }
__host__ __device__ constexpr int cmax(int a, int b) { return a > b ? a : b; }

// LDS position of element i of a transform: one complex of padding after every 16.
__host__ __device__ constexpr int pad(int i) { return i + (i >> 4); }

// --- complex arithmetic ---------------------------------------------------------------------

__device__ __forceinline__ cf32 cadd(cf32 a, cf32 b) { return {a.re + b.re, a.im + b.im}; }
__device__ __forceinline__ cf32 csub(cf32 a, cf32 b) { return {a.re - b.re, a.im - b.im}; }
__device__ __forceinline__ cf32 cmul(cf32 a, cf32 b)
{
    return {a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re};
}
__device__ __forceinline__ cf32 cscale(cf32 a, float s) { return {a.re * s, a.im * s}; }
__device__ __forceinline__ cf32 cconj(cf32 a) { return {a.re, -a.im}; }
__device__ __forceinline__ cf32 czero() { return {0.0f, 0.0f}; }

// a * (sign i), sign = -1 forward, +1 inverse: a swap and one negation.
template <bool Inv>
__device__ __forceinline__ cf32 mul_si(cf32 a)
{
    if constexpr (Inv) {
        return {-a.im, a.re};
    } else {
        return {a.im, -a.re};
    }
}

// exp(i pi a); sincospif reduces pi * a without rounding pi.
__device__ __forceinline__ cf32 expi_pi(float a)
{
    float s = 0.0f;
    float c = 0.0f;
    sincospif(a, &s, &c);
    return {c, s};
}

// --- streaming global accesses ---------------------------------------------------------------
//
// Every HBM byte of a transform is read once and written once. Stores of final outputs carry the
// nontemporal hint (they stream through the caches instead of displacing other lines), and so do
// the loads of complex-to-complex transforms (+4-6 % of peak with both hints on MI355X). The
// real transforms' loads take the hint where it measured faster (R2cIoT, C2rIo).

using f2v = float __attribute__((ext_vector_type(2)));

__device__ __forceinline__ cf32 ld_stream(const cf32* p)
{
    const f2v v = __builtin_nontemporal_load(reinterpret_cast<const f2v*>(p));
    return {v.x, v.y};
}

__device__ __forceinline__ void st_stream(cf32* p, cf32 a)
{
    __builtin_nontemporal_store(f2v{a.re, a.im}, reinterpret_cast<f2v*>(p));
}

// A load sent straight to LDS (global_load_lds_dwordx4, nontemporal): each lane of the wave reads
// 16 bytes at `src`, and lane k's bytes land at lds_base + 16 k. lds_base must be the same for
// every lane of the wave (the instruction takes it from M0) and 16-byte aligned.
__device__ __forceinline__ void ld_lds16(const cf32* src, cf32* lds_base)
{
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(src),
                                     (__attribute__((address_space(3))) void*)lds_base, 16, 0, 2);
}

// --- R-point DFTs in registers, X[q] = sum_p v[p] exp(sign 2 pi i p q / R) ---------------------

template <int R, bool Inv>
struct Dft;

template <bool Inv>
struct Dft<1, Inv> {
    __device__ __forceinline__ static void run(cf32*) {}
};

template <bool Inv>
struct Dft<2, Inv> {
    __device__ __forceinline__ static void run(cf32* v)
    {
        const cf32 a = v[0];
        v[0] = cadd(a, v[1]);
        v[1] = csub(a, v[1]);
    }
};

template <bool Inv>
struct Dft<4, Inv> {
    __device__ __forceinline__ static void run(cf32* v)
    {
        const cf32 s02 = cadd(v[0], v[2]);
        const cf32 d02 = csub(v[0], v[2]);
        const cf32 s13 = cadd(v[1], v[3]);
        const cf32 d13 = mul_si<Inv>(csub(v[1], v[3]));
        v[0] = cadd(s02, s13);
        v[2] = csub(s02, s13);
        v[1] = cadd(d02, d13);
        v[3] = csub(d02, d13);
    }
};

// 8 = 2 x 4: DFT4 of the even and of the odd inputs, then X[q] = E[q] + w8^q O[q] and
// X[q + 4] = E[q] - w8^q O[q]. w8 = (1 + sign i) / sqrt 2, w8^2 = sign i, w8^3 = sign i w8.
template <bool Inv>
struct Dft<8, Inv> {
    __device__ __forceinline__ static void run(cf32* v)
    {
        cf32 e[4] = {v[0], v[2], v[4], v[6]};
        cf32 o[4] = {v[1], v[3], v[5], v[7]};
        Dft<4, Inv>::run(e);
        Dft<4, Inv>::run(o);
        constexpr float h = 0.707106781186547524f;
        const cf32 o1 = cscale(cadd(o[1], mul_si<Inv>(o[1])), h);   // w8 o1
        const cf32 o2 = mul_si<Inv>(o[2]);                          // w8^2 o2
        const cf32 o3 = cscale(csub(mul_si<Inv>(o[3]), o[3]), h);   // w8^3 o3
        v[0] = cadd(e[0], o[0]);
        v[4] = csub(e[0], o[0]);
        v[1] = cadd(e[1], o1);
        v[5] = csub(e[1], o1);
        v[2] = cadd(e[2], o2);
        v[6] = csub(e[2], o2);
        v[3] = cadd(e[3], o3);
        v[7] = csub(e[3], o3);
    }
};

// 16 = 4 x 4: DFT4 over p for each residue a (inputs v[a + 4 p]), twiddle by w16^(a c), then
// DFT4 over a; X[c + 4 d] = sum_a w4^(a d) w16^(a c) A_a[c].
template <bool Inv>
struct Dft<16, Inv> {
    __device__ __forceinline__ static void run(cf32* v)
    {
        cf32 a[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                a[r][p] = v[r + 4 * p];
            }
            Dft<4, Inv>::run(a[r]);
        }
        constexpr float c1 = 0.923879532511286756f;  // cos(pi/8)
        constexpr float s1 = 0.382683432365089772f;  // sin(pi/8)
        constexpr float h = 0.707106781186547524f;
        constexpr float sg = Inv ? 1.0f : -1.0f;
        // w16^m for m = 1, 2, 3, 4, 6, 9 (a * c with a, c in 1..3).
        const cf32 w1{c1, sg * s1};
        const cf32 w2{h, sg * h};
        const cf32 w3{s1, sg * c1};
        a[1][1] = cmul(a[1][1], w1);
        a[1][2] = cmul(a[1][2], w2);
        a[1][3] = cmul(a[1][3], w3);
        a[2][1] = cmul(a[2][1], w2);
        a[2][2] = mul_si<Inv>(a[2][2]);                  // w16^4 = sign i
        a[2][3] = mul_si<Inv>(cmul(a[2][3], w2));        // w16^6 = sign i w16^2
        a[3][1] = cmul(a[3][1], w3);
        a[3][2] = mul_si<Inv>(cmul(a[3][2], w2));        // w16^6
        a[3][3] = cmul(a[3][3], cf32{-c1, -sg * s1});    // w16^9 = -w16^1
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            cf32 t[4] = {a[0][c], a[1][c], a[2][c], a[3][c]};
            Dft<4, Inv>::run(t);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                v[c + 4 * d] = t[d];
            }
        }
    }
};

// --- compile-time loops ---------------------------------------------------------------------

// f(integral_constant<int, I>) for I = Begin .. End-1, unrolled at compile time, so values that
// depend on I (twiddle constants, LDS offsets) are constant expressions.
template <int Begin, int End, class F>
__device__ __forceinline__ void static_for(F&& f)
{
    if constexpr (Begin < End) {
        f(std::integral_constant<int, Begin>{});
        static_for<Begin + 1, End>(f);
    }
}

// --- twiddles -------------------------------------------------------------------------------
//
// exp(sign 2 pi i k / Span) with exact argument reduction in integers: 4k = q Span + rem with
// |rem| <= Span / 2, so the angle is q quarter turns plus r = (pi / 2) rem / Span, |r| <= pi / 4.
// sin r and cos r come from their Taylor series (through r^9 and r^10; the first omitted terms
// are below 2e-9 on |r| <= pi/4, far under float rounding), and the quarter turns are applied
// exactly by swapping and negating. Multiples of a quarter turn come out exact.

constexpr double kPi = 3.14159265358979323846264338327950288;

// Taylor series of sin and cos in double, for compile-time constants (|x| <= pi / 4).
__host__ __device__ constexpr double taylor_sin(double x)
{
    double term = x;
    double sum = x;
    for (int n = 1; n < 16; ++n) {
        term *= -x * x / static_cast<double>((2 * n) * (2 * n + 1));
        sum += term;
    }
    return sum;
}

__host__ __device__ constexpr double taylor_cos(double x)
{
    double term = 1.0;
    double sum = 1.0;
    for (int n = 1; n < 16; ++n) {
        term *= -x * x / static_cast<double>((2 * n - 1) * (2 * n));
        sum += term;
    }
    return sum;
}

// exp(sign 2 pi i m / span) rounded once to float, at compile time.
template <bool Inv>
__host__ __device__ constexpr cf32 const_twiddle(long long m, long long span)
{
    m %= span;
    const long long m4 = 4 * m;
    const long long q = (m4 + span / 2) / span;  // nearest quarter turn
    const double r = kPi / 2.0 * static_cast<double>(m4 - q * span) / static_cast<double>(span);
    const double c = taylor_cos(r);
    const double s = taylor_sin(r);
    double re = (q & 1) ? -s : c;
    double im = (q & 1) ? c : s;
    if (q & 2) {
        re = -re;
        im = -im;
    }
    return cf32{static_cast<float>(re), static_cast<float>(Inv ? im : -im)};
}

// The same at run time, for integer k >= 0 (k < 2^29) and a compile-time power-of-two Span.
template <int Span, bool Inv>
__device__ __forceinline__ cf32 twiddle_of(int k)
{
    constexpr int kShift = clog2(Span);
    constexpr double c = kPi / (2.0 * Span);  // r = rem * c, c split so r is rounded once
    constexpr float c_hi = static_cast<float>(c);
    constexpr float c_lo = static_cast<float>(c - static_cast<double>(c_hi));
    const int k4 = k << 2;
    const int q = (k4 + Span / 2) >> kShift;
    const float rem = static_cast<float>(k4 - (q << kShift));
    const float r = fmaf(rem, c_hi, rem * c_lo);
    const float r2 = r * r;
    constexpr float s3 = static_cast<float>(-1.0 / 6.0);
    constexpr float s5 = static_cast<float>(1.0 / 120.0);
    constexpr float s7 = static_cast<float>(-1.0 / 5040.0);
    constexpr float s9 = static_cast<float>(1.0 / 362880.0);
    constexpr float c2 = -0.5f;
    constexpr float c4 = static_cast<float>(1.0 / 24.0);
    constexpr float c6 = static_cast<float>(-1.0 / 720.0);
    constexpr float c8 = static_cast<float>(1.0 / 40320.0);
    constexpr float c10 = static_cast<float>(-1.0 / 3628800.0);
    const float sn = fmaf(r * r2, fmaf(r2, fmaf(r2, fmaf(r2, s9, s7), s5), s3), r);
    const float cs = fmaf(r2, fmaf(r2, fmaf(r2, fmaf(r2, fmaf(r2, c10, c8), c6), c4), c2), 1.0f);
    float re = (q & 1) ? -sn : cs;
    float im = (q & 1) ? cs : sn;
    if (q & 2) {
        re = -re;
        im = -im;
    }
    return {re, Inv ? im : -im};
}

// Size of the precomputed table: exp(-2 pi i m / kTableN), m < kTableN, rounded once from double.
// Stages whose span exceeds it (single-pass transforms beyond 4096 points) compute their twiddles.
constexpr int kTableN = 4096;

// --- plans ----------------------------------------------------------------------------------

// N-point transform, stages of radix R (then one stage of the leftover factor), E values per lane,
// Threads lanes per workgroup (0: 256, or L when one transform needs more).
template <int N_, int R_, int E_, int Threads_ = 0>
struct Plan {
    static constexpr int N = N_;
    static constexpr int R = R_ < N_ ? R_ : N_;
    static constexpr int E = E_;
    static constexpr int L = N / E;                         // lanes per transform
    static constexpr int kThreads = Threads_ > 0 ? Threads_ : (L > kBlock ? L : kBlock);
    static constexpr int T = kThreads / L;                    // transforms per workgroup
    static constexpr int kFull = clog2(N) / clog2(R);       // radix-R stages
    static constexpr int kFinal = N >> (kFull * clog2(R));  // leftover radix (1: none)
    static constexpr int kStages = kFull + (kFinal > 1 ? 1 : 0);
    static constexpr int kStride = (pad(N) + 1) | 1;        // odd: LDS distance between transforms
    static constexpr bool kWaveLocal = L <= 64;             // each transform inside one wave

    static_assert(N >= 2 && (N & (N - 1)) == 0, "N must be a power of two");
    static_assert(E <= N && N % E == 0 && L <= kMaxBlock, "bad lane split");
    static_assert(kThreads % L == 0 && kThreads <= kMaxBlock, "bad workgroup size");
    static_assert(R <= E && kFinal <= E, "a lane must hold a whole butterfly");

    template <int S>
    static constexpr int radix() { return S < kFull ? R : kFinal; }
    template <int S>
    static constexpr int span_before() { return 1 << (S * clog2(R)); }
};

// Radix-16 stages where a lane holds 16 values anyway (the 4096-point plan, the single-pass 2D
// columns, the FIR's 1024-point blocks): one LDS exchange and one twiddle stage fewer than radix
// 8 at the same lanes and registers. 0 keeps radix 8 there, for A/B builds.
#ifndef SPX_RADIX16
#define SPX_RADIX16 1
#endif
inline constexpr bool kRadix16 = SPX_RADIX16 != 0;

// Values per lane for an N-point transform with radix-R stages: as few as hold one butterfly (and
// at least 4: radix-2 plans with E = 2 measured 15-20 % slower), but enough that a transform needs
// at most 256 lanes. Fewer values per lane means fewer VGPRs and more resident waves, and on
// MI355X that is what raised the sustained bandwidth: at N = 1024 radix 4, E = 4 / 8 / 16 measured
// 76 / 75 / 72 % of the 8 TB/s peak; larger workgroups (N = 4096 with E = 8 or 4) measured lower.
template <int N, int R>
constexpr int default_e()
{
    return cmin(N, cmax(cmax(R, 4), N / kBlock));
}

// Strided columns (StridedIo) stage T neighbouring columns per workgroup, so every row access is a
// run of T * 8 bytes: T = 16 (128-byte runs) up to N = 512; beyond, T shrinks to keep the column
// tile near 70 KB of LDS (two workgroups per CU). E grows with T so a workgroup stays within 1024
// lanes.
template <int N>
constexpr int column_t()
{
    return N <= 512 ? 16 : 8192 / N;
}

template <int N, int R>
constexpr int column_e()
{
    return cmax(default_e<N, R>(), cmin(N, N * column_t<N>() / kMaxBlock));
}

template <int N, int R>
constexpr int column_threads()
{
    return cmax(kBlock, column_t<N>() * (N / column_e<N, R>()));
}

// --- synchronization ------------------------------------------------------------------------

template <bool WaveLocal>
__device__ __forceinline__ void lds_sync()
{
    if constexpr (WaveLocal) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else {
        __syncthreads();
    }
}

// --- stage pieces ---------------------------------------------------------------------------
//
// A transform's values sit in LDS in one of these layouts: element i at s[Lay::at(i)].
//   Padded         one complex of padding after every 16 (a transform stored as a row)
//   Padded8        one after every 8 (the 64-point rows' exchange, see RowExchange)
//   Strided<ST>    every ST values (a column of a row-major tile whose rows are ST long)
//   PaddedRows<ST> a column of a tile with a spare row after every 16 rows
// LDS addresses are a per-lane base plus a compile-time offset. For Strided that is linearity;
// for Padded, pad(a + c) = pad(a) + pad(c) whenever the low four bits of a and c add without a
// carry, and for every access pattern below that holds for all lanes (power-of-two strides,
// lane < L). read_splits / write_splits check it exhaustively at compile time for each
// instantiated plan, stage and layout, so a plan where it failed would not build.

struct Padded {
    __host__ __device__ static constexpr int at(int i) { return pad(i); }
};

struct Padded8 {
    __host__ __device__ static constexpr int at(int i) { return i + (i >> 3); }
};

// The layout of a row transform's stage exchanges when four rows of a half-wave sit RowStride
// values apart. The 64-point plan (8 lanes of 8, two radix-8 stages) with rows 8 mod 32 apart
// exchanges free of bank conflicts in Padded8 (64 banks of 4 bytes, 8-byte accesses served a
// half-wave at a time): the first stage's writes, lane l at 8 l + r, fill all 32 eight-byte
// slots of the four rows, where Padded leaves them 2-way conflicted at every row stride. It
// needs 71 slots per row (Padded: 67). SPX_ROW_EXCHANGE_PAD8=0 keeps Padded, for A/B builds.
#ifndef SPX_ROW_EXCHANGE_PAD8
#define SPX_ROW_EXCHANGE_PAD8 1
#endif
template <class P, int RowStride>
using RowExchange =
    std::conditional_t<(SPX_ROW_EXCHANGE_PAD8 != 0 && P::N == 64 && P::L == 8 &&
                        RowStride % 32 == 8 && RowStride >= 71),
                       Padded8, Padded>;

template <int Stride>
struct Strided {
    __host__ __device__ static constexpr int at(int i) { return i * Stride; }
};

// A column of a tile whose element i sits in tile row pad(i) (one spare row after every 16),
// tile rows Stride apart.
template <int Stride>
struct PaddedRows {
    __host__ __device__ static constexpr int at(int i) { return pad(i) * Stride; }
};

template <class P, class Lay>
constexpr bool read_splits(int R)
{
    for (int lane = 0; lane < P::L; ++lane) {
        for (int b = 0; b < P::E / R; ++b) {
            for (int r = 0; r < R; ++r) {
                const int off = b * P::L + r * (P::N / R);
                if (Lay::at(lane + off) != Lay::at(lane) + Lay::at(off)) {
                    return false;
                }
            }
        }
    }
    return true;
}

template <class P, class Lay>
constexpr bool write_splits(int R, int NS)
{
    for (int lane = 0; lane < P::L; ++lane) {
        const int k0 = lane & (NS - 1);
        const int base = (lane - k0) * R + k0;
        for (int b = 0; b < P::E / R; ++b) {
            const int kb = (b * P::L) % NS;
            for (int r = 0; r < R; ++r) {
                const int off = (b * P::L - kb) * R + kb + r * NS;
                const int j = lane + b * P::L;  // the definition: k = j mod NS
                const int k = j & (NS - 1);
                if ((j - k) * R + k + r * NS != base + off
                    || Lay::at(base + off) != Lay::at(base) + Lay::at(off)) {
                    return false;
                }
            }
        }
    }
    return true;
}

// Stage S: twiddles, then E / R DFTs of radix R. Input r of butterfly b (j = lane + b L,
// k = j mod NS) is multiplied by w^(k r), w = exp(sign 2 pi i / (NS R)). k = (lane mod NS) +
// ((b L) mod NS), the second term a compile-time multiple of L, so a lane evaluates (or looks up)
// one twiddle per stage, w^(lane mod NS), takes its powers, and reaches the other butterflies'
// twiddles through compile-time constants.
template <class P, int S, bool Inv, bool Table>
__device__ __forceinline__ void stage_compute(cf32 (&v)[P::E], int lane, const cf32* table)
{
    constexpr int R = P::template radix<S>();
    constexpr int NS = P::template span_before<S>();
    constexpr int SP = NS * R;
    constexpr int B = P::E / R;
    if constexpr (NS > 1) {
        const int k0 = lane & (NS - 1);
        cf32 p[R];  // p[r] = w^(k0 r)
        if constexpr (Table && kTableN % SP == 0) {
            const cf32 w = table[k0 * (kTableN / SP)];  // k0 < SP: no wrap
            p[1] = Inv ? cconj(w) : w;
        } else {
            p[1] = twiddle_of<SP, Inv>(k0);
        }
#pragma unroll
        for (int r = 2; r < R; ++r) {
            p[r] = (r % 2 == 0) ? cmul(p[r / 2], p[r / 2]) : cmul(p[r - 1], p[1]);
        }
        static_for<0, B>([&](auto bi) {
            constexpr int b = decltype(bi)::value;
            constexpr int kb = (b * P::L) % NS;
            static_for<1, R>([&](auto ri) {
                constexpr int r = decltype(ri)::value;
                if constexpr (kb == 0) {
                    v[b * R + r] = cmul(v[b * R + r], p[r]);
                } else {
                    constexpr cf32 c = const_twiddle<Inv>(static_cast<long long>(kb) * r, SP);
                    v[b * R + r] = cmul(cmul(v[b * R + r], c), p[r]);
                }
            });
        });
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {
        Dft<R, Inv>::run(&v[b * R]);
    }
}

// Stage S's outputs to their Stockham positions in LDS: output r of butterfly j goes to
// (j - k) R + k + r NS.
template <class P, int S, class Lay = Padded>
__device__ __forceinline__ void stage_write(cf32* s, const cf32 (&v)[P::E], int lane)
{
    constexpr int R = P::template radix<S>();
    constexpr int NS = P::template span_before<S>();
    static_assert(write_splits<P, Lay>(R, NS), "LDS offsets do not split for this plan");
    const int k0 = lane & (NS - 1);
    cf32* const base = s + Lay::at((lane - k0) * R + k0);
    static_for<0, P::E / R>([&](auto bi) {
        constexpr int b = decltype(bi)::value;
        constexpr int kb = (b * P::L) % NS;
        static_for<0, R>([&](auto ri) {
            constexpr int r = decltype(ri)::value;
            base[Lay::at((b * P::L - kb) * R + kb + r * NS)] = v[b * R + r];
        });
    });
}

// Stage S's inputs from LDS: v[b R + r] = s[j + r N / R], j = lane + b L.
template <class P, int S, class Lay = Padded>
__device__ __forceinline__ void stage_read(const cf32* s, cf32 (&v)[P::E], int lane)
{
    constexpr int R = P::template radix<S>();
    static_assert(read_splits<P, Lay>(R), "LDS offsets do not split for this plan");
    const cf32* const base = s + Lay::at(lane);
    static_for<0, P::E / R>([&](auto bi) {
        constexpr int b = decltype(bi)::value;
        static_for<0, R>([&](auto ri) {
            constexpr int r = decltype(ri)::value;
            v[b * R + r] = base[Lay::at(b * P::L + r * (P::N / R))];
        });
    });
}

// Index of the value held in v[b R + r] as input of stage S (natural order of the transform).
template <class P, int S>
__device__ __forceinline__ constexpr int input_index(int lane, int b, int r)
{
    return lane + b * P::L + r * (P::N / P::template radix<S>());
}

// --- the exchange between two stages in registers ------------------------------------------
//
// A 64-point transform held by 8 lanes of 8 values in two radix-8 stages exchanges through an
// 8 x 8 transpose: after stage 0, lane l holds elements 8 l .. 8 l + 7, and stage 1 needs
// elements l, l + 8, .., l + 56. Three rounds of swaps between partner lanes l ^ 1, l ^ 2, l ^ 4
// (each swapping the off-diagonal halves of 2 x 2 blocks of the lane x register matrix) do it
// without LDS: DPP quad_perm moves a dword to the partner lane within a quad (^ 1, ^ 2), and
// ds_swizzle in bit mode (and 0x1F, xor 4) across a quad pair (^ 4). Per lane that is 24 moves,
// 24 DPP / swizzle ops and their selects, against 8 LDS writes and 8 LDS reads of 8 bytes.
// It applies to transforms whose 8 lanes are 8 consecutive lanes of a wave in order
// (lane = thread index mod 8, the row layout Padded), every lane of the group running it.
//
// Off by default: measured on MI355X against the LDS exchange (three alternated rounds at
// 2^24 points, and SQ counters), it kept the same LDS instruction count (ds_write2 / ds_read2
// move two values per instruction, and ds_swizzle is an LDS instruction too), raised VALU
// instructions per wave by 18-40 % (C2C n = 64: 226 -> 316) and ran 2-9 % slower (R2C n = 128
// 24.2 -> 26.7 us), irfft2 128^2 unchanged. Build with -DSPX_EXCHANGE_IN_REGISTERS=1 to
// measure it (build.py --define SPX_EXCHANGE_IN_REGISTERS=1 --lib-dir DIR).
#ifndef SPX_EXCHANGE_IN_REGISTERS
#define SPX_EXCHANGE_IN_REGISTERS 0
#endif
constexpr bool kExchangeInRegisters = SPX_EXCHANGE_IN_REGISTERS != 0;

template <class P, int S, class Lay>
constexpr bool exchange_in_registers()
{
    return kExchangeInRegisters && std::is_same_v<Lay, Padded> && P::N == 64 && P::E == 8
           && P::L == 8 && S == 0 && P::kStages == 2 && P::template radix<0>() == 8
           && P::template radix<1>() == 8;
}

// One dword from the partner lane (lane ^ D) of the lane's group of 8.
template <int D>
__device__ __forceinline__ float from_partner(float x)
{
    const int i = __builtin_bit_cast(int, x);
    if constexpr (D == 1) {
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(i, 0xB1, 0xF, 0xF, false));
    } else if constexpr (D == 2) {
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(i, 0x4E, 0xF, 0xF, false));
    } else {
        static_assert(D == 4, "partners within groups of 8 lanes");
        return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(i, 0x101F));
    }
}

// Round D: lanes with bit D clear swap their registers r | D for the partner's registers r.
template <int D>
__device__ __forceinline__ void swap_with_partner(cf32 (&v)[8], int lane)
{
    const bool hi = (lane & D) != 0;
    static_for<0, 8>([&](auto ri) {
        constexpr int r0 = decltype(ri)::value;
        if constexpr ((r0 & D) == 0) {
            constexpr int r1 = r0 | D;
            const cf32 send = hi ? v[r0] : v[r1];
            const cf32 recv{from_partner<D>(send.re), from_partner<D>(send.im)};
            v[r0] = hi ? recv : v[r0];
            v[r1] = hi ? v[r1] : recv;
        }
    });
}

template <class P>
__device__ __forceinline__ void transpose_lanes(cf32 (&v)[P::E], int lane)
{
    static_assert(P::E == 8 && P::L == 8, "an 8 x 8 transpose");
    swap_with_partner<1>(v, lane);
    swap_with_partner<2>(v, lane);
    swap_with_partner<4>(v, lane);
}

// Runs stages S .. kStages-1. On entry v holds stage S's inputs; on exit the last stage's
// outputs, output r of butterfly b being element lane + b L + r N / R_last.
template <class P, int S, bool Inv, bool Table, class Lay = Padded>
__device__ __forceinline__ void run_stages(cf32 (&v)[P::E], cf32* s, int lane, const cf32* table)
{
    stage_compute<P, S, Inv, Table>(v, lane, table);
    if constexpr (S + 1 < P::kStages) {
        if constexpr (exchange_in_registers<P, S, Lay>()) {
            transpose_lanes<P>(v, lane);
        } else {
            lds_sync<P::kWaveLocal>();  // every lane has read the previous contents of s
            stage_write<P, S, Lay>(s, v, lane);
            lds_sync<P::kWaveLocal>();
            stage_read<P, S + 1, Lay>(s, v, lane);
        }
        run_stages<P, S + 1, Inv, Table, Lay>(v, s, lane, table);
    }
}

// Slot of the first stage's inputs that holds the element the last stage leaves in slot e_out.
// Both hold the same elements of a lane, lane + q L for q < E (b L + r N / R covers every q
// once at any radix), in different register orders: a transform's output can feed another
// transform's first stage (an inverse after a forward, on the same lanes) by renaming registers.
template <class P>
constexpr int forward_slot_of(int e_out)
{
    constexpr int RL = P::template radix<P::kStages - 1>();
    constexpr int R0 = P::template radix<0>();
    const int idx = (e_out / RL) * P::L + (e_out % RL) * (P::N / RL);  // lane 0's element
    for (int e = 0; e < P::E; ++e) {
        if ((e / R0) * P::L + (e % R0) * (P::N / R0) == idx) {
            return e;
        }
    }
    return -1;
}

template <class P>
constexpr bool slots_match()
{
    for (int e = 0; e < P::E; ++e) {
        if (forward_slot_of<P>(e) < 0) {
            return false;
        }
    }
    return true;
}

// After a plan's last stage, lane l holds element l + q L of its transform (q < E) in register
// slot out_slot<P>(q).
template <class P>
constexpr int out_slot(int q)
{
    constexpr int RL = P::template radix<P::kStages - 1>();
    for (int e = 0; e < P::E; ++e) {
        if ((e / RL) * P::L + (e % RL) * (P::N / RL) == q * P::L) {
            return e;
        }
    }
    return -1;
}

// v as held by wave lane `from` (ds_bpermute: a cross-lane read through the LDS crossbar that
// touches no LDS memory). Every lane of the wave must execute it.
__device__ __forceinline__ cf32 lane_value(cf32 v, int from)
{
    const int addr = from << 2;
    return {__builtin_bit_cast(float,
                               __builtin_amdgcn_ds_bpermute(addr, __builtin_bit_cast(int, v.re))),
            __builtin_bit_cast(float,
                               __builtin_amdgcn_ds_bpermute(addr, __builtin_bit_cast(int, v.im)))};
}

// Writes the last stage's outputs to LDS in natural order (for a staged store).
template <class P, class Lay = Padded>
__device__ __forceinline__ void final_write(cf32* s, const cf32 (&v)[P::E], int lane)
{
    constexpr int R = P::template radix<P::kStages - 1>();
    static_assert(read_splits<P, Lay>(R), "LDS offsets do not split for this plan");
    cf32* const base = s + Lay::at(lane);
    static_for<0, P::E / R>([&](auto bi) {
        constexpr int b = decltype(bi)::value;
        static_for<0, R>([&](auto ri) {
            constexpr int r = decltype(ri)::value;
            base[Lay::at(b * P::L + r * (P::N / R))] = v[b * R + r];
        });
    });
}

// --- groups and staged access ---------------------------------------------------------------
//
// A group is the set of lanes that stage their transforms through LDS together: one wavefront
// when a transform fits in one (and the I/O policy allows it), otherwise the whole workgroup.
// Full: all kT transforms of the group exist; otherwise the group holds the batch's tail and
// only its first `count` transforms touch global memory.
template <int T_, int Threads_, bool Full_>
struct Group {
    static constexpr int kT = T_;
    static constexpr int kThreads = Threads_;
    static constexpr bool kFull = Full_;
    static constexpr bool kWave = Threads_ <= 64;
};

// The staged loop over a group's transforms of Row elements each, row-major: element
// e = u * Row + i goes to lane e mod kThreads at step e / kThreads, so the lanes of a wavefront
// take consecutive elements and global accesses coalesce whatever Row is. The step count is a
// compile-time constant: the loops unroll, and a caller that first gathers every step's loads
// into registers and only then writes LDS keeps all of a lane's loads in flight together.
template <class G, int Row>
struct Staged {
    static constexpr int kTotal = G::kT * Row;
    static constexpr int kSteps = (kTotal + G::kThreads - 1) / G::kThreads;

    // f(step, u, i, valid); valid: element exists (inside the group and the batch).
    template <class F>
    __device__ __forceinline__ static void each(int count, int tid, F&& f)
    {
#pragma unroll
        for (int k = 0; k < kSteps; ++k) {
            const int e = tid + k * G::kThreads;
            const int u = e / Row;
            const int i = e - u * Row;
            const bool valid =
                (kTotal % G::kThreads == 0 || e < kTotal) && (G::kFull || u < count);
            f(k, u, i, valid);
        }
    }
};

// The group's rows of Row values written out as one run: row u of LDS (lds + u * Stride, value
// i at pad(i)) to dst[u * Row + i] for u < count. Consecutive lanes take consecutive values of
// the run, walked from the 128-byte boundary at or before dst, so every wave store covers whole
// lines whatever the row length: rows of odd length (a half spectrum's m + 1 values) start at
// 8-byte offsets, and a store straddling lines leaves partial lines that nontemporal writes
// send to memory separately. put(address, value) does the store.
template <class G, int Row, int Stride, class Put>
__device__ __forceinline__ void store_run_aligned(const cf32* lds, cf32* dst, int count, int tid,
                                                  Put&& put)
{
    constexpr int kTotal = G::kT * Row;
    constexpr int kSteps = (kTotal + 15 + G::kThreads - 1) / G::kThreads;
    const int shift = static_cast<int>((reinterpret_cast<std::uintptr_t>(dst) / sizeof(cf32)) & 15);
    const int total = (G::kFull ? G::kT : count) * Row;
#pragma unroll
    for (int k = 0; k < kSteps; ++k) {
        const int e = tid + k * G::kThreads - shift;
        if (e >= 0 && e < total) {
            const int u = e / Row;
            const int i = e - u * Row;
            put(dst + e, lds[u * Stride + pad(i)]);
        }
    }
}

// The same for rows that are not adjacent in memory: row u of LDS to dst(u)[0 .. Row), or
// nowhere when dst(u) is null. Each row is walked over a span of whole 128-byte lines from the
// boundary at or before its start (Span slots, enough for any start), consecutive lanes on
// consecutive slots.
template <class G, int Row, int Stride, class Dst, class Put>
__device__ __forceinline__ void store_rows_aligned(const cf32* lds, int count, int tid, Dst&& dst,
                                                   Put&& put)
{
    constexpr int kSpan = (Row + 15 + 15) / 16 * 16;
    constexpr int kSteps = (G::kT * kSpan + G::kThreads - 1) / G::kThreads;
    const int rows = G::kFull ? G::kT : count;
#pragma unroll
    for (int k = 0; k < kSteps; ++k) {
        const int e = tid + k * G::kThreads;
        const int u = e / kSpan;
        cf32* const d = u < rows ? dst(u) : nullptr;
        if (d != nullptr) {
            const int shift = static_cast<int>((reinterpret_cast<std::uintptr_t>(d) / sizeof(cf32))
                                               & 15);
            const int i = e - u * kSpan - shift;
            if (i >= 0 && i < Row) {
                put(d + i, lds[u * Stride + pad(i)]);
            }
        }
    }
}

// --- the kernel -----------------------------------------------------------------------------
//
// An I/O policy `Io` supplies, for transform t of the batch:
//   direct_in<P>() / direct_out<P>()   whether the stage-0 inputs are read from global memory by
//                                the lanes that use them, and the outputs written by the lanes
//                                that hold them
//   in<P>(t, i), out<P>(t, i, value)   those direct accesses (element i of transform t)
//   load<P, G>(lds, first, count, tid)   otherwise: fill lds[u * kStride + pad(i)] for the
//   store<P, G>(lds, first, count, tid)  group's transforms u < count, or write them out from
//                                there; tid is the lane's index within the group
//   kGroupIsBlock                the staged accesses need the whole workgroup (strided columns)
//
// Transforms past the end of the batch still run the stages (on whatever is in registers) but
// touch no global memory, so every lane reaches every barrier.
// An I/O policy with `static constexpr bool kStage0 = true` forms the stage-0 inputs itself from
// what its staged load left in LDS (stage0<P>(s, v, lane)), instead of stage_read.
template <class Io, class = void>
struct HasStage0 : std::false_type {};
template <class Io>
struct HasStage0<Io, std::void_t<decltype(Io::kStage0)>> : std::bool_constant<Io::kStage0> {};

// An I/O policy with `static constexpr bool kFinal = true` takes the last stage's outputs from
// registers itself (final<P, WaveLocal>(s, v, lane, t, batch), t the lane's transform) instead of
// final_write: it leaves in LDS what its staged store reads, or stores them itself.
template <class Io, class = void>
struct HasFinal : std::false_type {};
template <class Io>
struct HasFinal<Io, std::void_t<decltype(Io::kFinal)>> : std::bool_constant<Io::kFinal> {};

// A direct-input policy with `static constexpr bool kInAll = true` reads a lane's E stage-0 inputs
// itself (in_all<P>(t, lane, v), v[b R0 + r] = element input_index<P, 0>(lane, b, r) of transform
// t), for work shared between them (a twiddle factored over the lane's elements).
template <class Io, class = void>
struct HasInAll : std::false_type {};
template <class Io>
struct HasInAll<Io, std::void_t<decltype(Io::kInAll)>> : std::bool_constant<Io::kInAll> {};

// A policy with `template <class P> static constexpr bool lds_dma_in()` true for plan P sends the
// workgroup's stage-0 inputs straight to LDS (lds_dma<P>(lds, first, batch, tid): transform u of
// the workgroup's T at lds + u N, densely), and each lane reads its stage-0 values from there.
template <class Io, class P, class = void>
struct HasLdsDmaIn : std::false_type {};
template <class Io, class P>
struct HasLdsDmaIn<Io, P, std::void_t<decltype(Io::template lds_dma_in<P>())>>
    : std::bool_constant<Io::template lds_dma_in<P>()> {};

// Workgroup order across the XCDs. The dispatcher hands workgroup b to XCD b mod 8, and each XCD
// has its own L2, so in plain order the neighbouring tiles of a strided pass (whose rows share
// cache lines and DRAM pages) run on different XCDs. An I/O policy with
// `static constexpr int kXcdChunk = C` renumbers each span of 8 C workgroups so that every XCD
// takes C consecutive tiles of the span; a trailing partial span keeps its order. Spans stay
// short: the XCDs then work on neighbouring regions, where XCDs working on regions far apart
// (C = grid / 8) measured slower than plain order.
template <class Io, class = void>
struct XcdChunk : std::integral_constant<int, 0> {};
template <class Io>
struct XcdChunk<Io, std::void_t<decltype(Io::kXcdChunk)>>
    : std::integral_constant<int, Io::kXcdChunk> {};

template <int C>
__device__ __forceinline__ long long xcd_order(long long b, long long grid)
{
    if constexpr (C == 0) {
        return b;
    } else {
        constexpr long long kSpan = 8LL * C;
        if (b >= grid / kSpan * kSpan) {
            return b;
        }
        const long long base = b / kSpan * kSpan;
        const long long r = b - base;
        return base + (r % 8) * C + r / 8;
    }
}

template <class P, bool Inv, bool Table, class Io>
__global__ void __launch_bounds__(P::kThreads) fft_kernel(Io io, long long batch, const cf32* table)
{
    __shared__ cf32 lds[P::T * P::kStride];

    constexpr bool kWaveGroups = P::kWaveLocal && !Io::kGroupIsBlock;
    constexpr int kGroupThreads = kWaveGroups ? 64 : P::kThreads;
    constexpr int kGroupT = kGroupThreads / P::L;  // transforms per group
    using Full = Group<kGroupT, kGroupThreads, true>;
    using Tail = Group<kGroupT, kGroupThreads, false>;

    const int tid = threadIdx.x;
    const int u = tid / P::L;  // transform within the workgroup
    const int lane = tid % P::L;
    const long long block = xcd_order<XcdChunk<Io>::value>(blockIdx.x, gridDim.x);
    const long long t = block * P::T + u;
    const int group = tid / kGroupThreads;
    const int gtid = tid % kGroupThreads;
    const long long group_first = block * P::T + group * kGroupT;
    const long long left = batch - group_first;
    const int group_count = left >= kGroupT ? kGroupT : (left > 0 ? static_cast<int>(left) : 0);
    cf32* const group_lds = lds + group * kGroupT * P::kStride;
    cf32* const s = lds + u * P::kStride;

    cf32 v[P::E];
    if constexpr (HasLdsDmaIn<Io, P>::value) {
        static_assert(!P::kWaveLocal, "the first exchange's workgroup barrier orders these reads");
        io.template lds_dma<P>(lds, block * P::T, batch, tid);
        __builtin_amdgcn_s_waitcnt(0);  // this wave's loads have landed in LDS
        __syncthreads();                // and every other wave's
        const cf32* const d = lds + u * P::N;
#pragma unroll
        for (int b = 0; b < P::E / P::template radix<0>(); ++b) {
#pragma unroll
            for (int r = 0; r < P::template radix<0>(); ++r) {
                v[b * P::template radix<0>() + r] = d[input_index<P, 0>(lane, b, r)];
            }
        }
    } else if constexpr (Io::template direct_in<P>()) {
        if (t < batch) {
            if constexpr (HasInAll<Io>::value) {
                io.template in_all<P>(t, lane, v);
            } else {
#pragma unroll
                for (int b = 0; b < P::E / P::template radix<0>(); ++b) {
#pragma unroll
                    for (int r = 0; r < P::template radix<0>(); ++r) {
                        v[b * P::template radix<0>() + r] =
                            io.template in<P>(t, input_index<P, 0>(lane, b, r));
                    }
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < P::E; ++e) {
                v[e] = czero();
            }
        }
    } else {
        if (group_count == kGroupT) {
            io.template load<P, Full>(group_lds, group_first, kGroupT, gtid);
        } else {
            io.template load<P, Tail>(group_lds, group_first, group_count, gtid);
        }
        lds_sync<kWaveGroups>();
        if constexpr (HasStage0<Io>::value) {
            io.template stage0<P>(s, v, lane);
        } else {
            stage_read<P, 0>(s, v, lane);
        }
    }

    run_stages<P, 0, Inv, Table>(v, s, lane, table);

    if constexpr (Io::template direct_out<P>()) {
        if (t < batch) {
            constexpr int RL = P::template radix<P::kStages - 1>();
#pragma unroll
            for (int b = 0; b < P::E / RL; ++b) {
#pragma unroll
                for (int r = 0; r < RL; ++r) {
                    io.template out<P>(t, lane + b * P::L + r * (P::N / RL), v[b * RL + r]);
                }
            }
        }
    } else {
        if constexpr (HasFinal<Io>::value) {
            io.template final<P, kWaveGroups>(s, v, lane, t, batch);
        } else {
            lds_sync<kWaveGroups>();
            final_write<P>(s, v, lane);
            lds_sync<kWaveGroups>();
        }
        if (group_count == kGroupT) {
            io.template store<P, Full>(group_lds, group_first, kGroupT, gtid);
        } else {
            io.template store<P, Tail>(group_lds, group_first, group_count, gtid);
        }
    }
}

// The lane's index within the workgroup, as a value the compiler cannot see through. Taken once
// per turn of a persistent loop, it keeps the lane's loop-invariant values (twiddle bases,
// addresses) from being hoisted out of the loop and held in registers across all of it: the
// loop body then needs about the registers of one item's work (the single-pass irfft2 at
// 128 x 128: 110 VGPRs against 152 without), so as many workgroups fit on a CU as without the
// loop. The bound 0 <= tid < NT is restated for the compiler.
template <int NT>
__device__ __forceinline__ int opaque_tid()
{
    int tid = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(tid));
    __builtin_assume(tid >= 0 && tid < NT);
    return tid;
}

// Persistent fft_kernel for plans of one transform per workgroup whose I/O policy reads and
// writes HBM directly (the 16384-point C2C: 1024 lanes, 139 KB of LDS, one per CU). Workgroup
// g takes transforms g, g + G, ... (G = gridDim.x, the workgroups resident at once). Before a
// transform's stages it issues the next transform's loads into a second register set, so they
// are in flight during the stages' exchanges and the stores. Each exchange of run_stages starts
// with a barrier, so one transform's stages do not write the LDS before the previous
// transform's last reads.
template <class P, bool Inv, bool Table, class Io>
__global__ void __launch_bounds__(P::kThreads)
    fft_persistent_kernel(Io io, long long batch, const cf32* table)
{
    static_assert(P::T == 1 && Io::template direct_in<P>() && Io::template direct_out<P>() &&
                      !HasInAll<Io>::value,
                  "one transform per workgroup, loaded and stored directly");
    __shared__ cf32 lds[P::kStride];
    constexpr int R0 = P::template radix<0>();
    constexpr int RL = P::template radix<P::kStages - 1>();

    cf32 v[P::E];
    const auto fetch = [&](long long t, int lane) __attribute__((always_inline)) {
#pragma unroll
        for (int b = 0; b < P::E / R0; ++b) {
#pragma unroll
            for (int r = 0; r < R0; ++r) {
                v[b * R0 + r] = io.template in<P>(t, input_index<P, 0>(lane, b, r));
            }
        }
    };

    long long t = blockIdx.x;
    fetch(t, threadIdx.x);
#pragma unroll 1
    for (; t < batch; t += gridDim.x) {
        const int lane = opaque_tid<P::kThreads>();
        cf32 u[P::E];
#pragma unroll
        for (int e = 0; e < P::E; ++e) {
            u[e] = v[e];
        }
        const long long next = t + gridDim.x;
        if (next < batch) {
            fetch(next, lane);
        }
        run_stages<P, 0, Inv, Table>(u, lds, lane, table);
#pragma unroll
        for (int b = 0; b < P::E / RL; ++b) {
#pragma unroll
            for (int r = 0; r < RL; ++r) {
                io.template out<P>(t, lane + b * P::L + r * (P::N / RL), u[b * RL + r]);
            }
        }
    }
}

// --- I/O policies ---------------------------------------------------------------------------

// 1 sends the stage-0 loads of the C2C plans of more than one wave straight to LDS, for A/B
// builds. Off: over 2^24 points those plans ran 0.8-2.9 % slower that way than with register
// loads, and a copy of C1's rows streamed 6.12 against 6.29 TB/s.
#ifndef SPX_C2C_LDS_DMA
#define SPX_C2C_LDS_DMA 0
#endif

// Contiguous complex rows. Pruned: rows of x hold keep_in values (the rest of each transform is
// zero), rows of y keep_out values. PlainOut: plain stores, for an intermediate that the next
// pass reads (nontemporal otherwise).
template <bool Pruned, bool PlainOut = false>
struct C2cIo {
    static constexpr bool kGroupIsBlock = false;
    const cf32* x;
    cf32* y;
    float scale;  // applied on the way out: 1/N for the inverse, else 1
    int keep_in;
    int keep_out;

    template <class P>
    static constexpr bool direct_in() { return P::L >= 16 && !lds_dma_in<P>(); }
    template <class P>
    static constexpr bool direct_out() { return P::L >= 16; }

    // Whole transforms of more than one wave: their stage-0 inputs may go straight to LDS
    // (SPX_C2C_LDS_DMA), in 16-byte pieces that never straddle two transforms.
    template <class P>
    static constexpr bool lds_dma_in()
    {
        return SPX_C2C_LDS_DMA != 0 && !Pruned && !P::kWaveLocal && P::N <= 4096 &&
               (P::T * P::N) % (2 * P::kThreads) == 0 && P::N % 128 == 0;
    }

    // The workgroup's transforms first .. first + T - 1 (those below batch) to lds densely: each
    // wave instruction moves 1 KB, 128 values of one transform.
    template <class P>
    __device__ __forceinline__ void lds_dma(cf32* lds, long long first, long long batch,
                                            int tid) const
    {
        constexpr int kChunk = 2 * P::kThreads;  // values per workgroup instruction
        const int wave = tid / 64;
        const cf32* const src = x + first * P::N;
#pragma unroll
        for (int j = 0; j < P::T * P::N / kChunk; ++j) {
            const int e = j * kChunk + wave * 128;  // the wave's first value
            if (first + e / P::N < batch) {
                ld_lds16(src + e + 2 * (tid % 64), lds + e);
            }
        }
    }

    template <class P>
    __device__ __forceinline__ cf32 in(long long t, int i) const
    {
        if constexpr (Pruned) {
            return i < keep_in ? ld_stream(x + t * keep_in + i) : czero();
        } else {
            return ld_stream(x + t * P::N + i);
        }
    }

    template <class P>
    __device__ __forceinline__ void out(long long t, int i, cf32 v) const
    {
        if constexpr (Pruned) {
            if (i < keep_out) {
                put(y + t * keep_out + i, cscale(v, scale));
            }
        } else {
            put(y + t * P::N + i, cscale(v, scale));
        }
    }

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        using S = Staged<G, P::N>;
        const int row = Pruned ? keep_in : P::N;
        const cf32* src = x + first * row;
        cf32 val[S::kSteps];
        S::each(count, tid, [&](int k, int u, int i, bool valid) {
            val[k] = (valid && (!Pruned || i < keep_in)) ? ld_stream(src + u * row + i) : czero();
        });
        S::each(count, tid, [&](int k, int u, int i, bool valid) {
            if (valid) {
                lds[u * P::kStride + pad(i)] = val[k];
            }
        });
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long first, int count,
                                          int tid) const
    {
        using S = Staged<G, P::N>;
        const int row = Pruned ? keep_out : P::N;
        cf32* dst = y + first * row;
        S::each(count, tid, [&](int, int u, int i, bool valid) {
            if (valid && (!Pruned || i < keep_out)) {
                put(dst + u * row + i, cscale(lds[u * P::kStride + pad(i)], scale));
            }
        });
    }

    __device__ __forceinline__ static void put(cf32* p, cf32 v)
    {
        if constexpr (PlainOut) {
            *p = v;
        } else {
            st_stream(p, v);
        }
    }
};

// The real transforms' pair passes over a group's rows in LDS (row u at lds + u * kStride, value
// k at pad(k)), one pair (k, m - k) per step, both slots read and written by the same lane, so no
// lane touches another lane's slots (k = 0 pairs slot 0 with slot m).
//
// combine_pairs (forward): the m-point transform Z of the row read as complex becomes the half
// spectrum X[0 .. m]: E = (Z[k] + conj Z[m-k]) / 2, O = (Z[k] - conj Z[m-k]) / 2i (indices mod m),
// X[k] = E + exp(-pi i k / m) O, X[m-k] = conj(E - exp(-pi i k / m) O); X[m] lands in slot m.
template <class P, class G>
__device__ __forceinline__ void combine_pairs(cf32* lds, int count, int tid)
{
    constexpr int m = P::N;
    using S = Staged<G, m / 2 + 1>;
    S::each(count, tid, [&](int, int u, int k, bool valid) {
        if (!valid) {
            return;
        }
        cf32* s = lds + u * P::kStride;
        const cf32 zk = s[pad(k & (m - 1))];
        const cf32 zm = s[pad((m - k) & (m - 1))];
        const cf32 ev{0.5f * (zk.re + zm.re), 0.5f * (zk.im - zm.im)};
        const cf32 od{0.5f * (zk.im + zm.im), -0.5f * (zk.re - zm.re)};
        const cf32 wo = cmul(twiddle_of<2 * m, false>(k), od);  // exp(-pi i k / m) O
        s[pad(k)] = cadd(ev, wo);
        if (k < m - k) {
            s[pad(m - k)] = cconj(csub(ev, wo));
        }
    });
}

// prepare_pairs (inverse): the half spectrum X[0 .. m] becomes the m-point inverse's input Z:
// E = (X[k] + conj X[m-k]) / 2, O = exp(pi i k / m) (X[k] - conj X[m-k]) / 2, Z[k] = E + i O,
// Z[m-k] = conj(E - i O), the imaginary parts of X[0] and X[m] dropped; `scale` rides on the
// halves.
template <class P, class G>
__device__ __forceinline__ void prepare_pairs(cf32* lds, int count, int tid, float scale)
{
    constexpr int m = P::N;
    const float half = 0.5f * scale;
    using S = Staged<G, m / 2 + 1>;
    S::each(count, tid, [&](int, int u, int k, bool valid) {
        if (!valid) {
            return;
        }
        cf32* s = lds + u * P::kStride;
        cf32 xk = s[pad(k)];
        cf32 xm = s[pad(m - k)];
        if (k == 0) {
            xk.im = 0.0f;
            xm.im = 0.0f;
        }
        const cf32 ev{half * (xk.re + xm.re), half * (xk.im - xm.im)};
        const cf32 d{half * (xk.re - xm.re), half * (xk.im + xm.im)};
        const cf32 od = cmul(d, twiddle_of<2 * m, true>(k));  // d exp(pi i k / m)
        const cf32 iod{-od.im, od.re};
        if (k < m) {
            s[pad(k)] = cadd(ev, iod);
        }
        if (k > 0 && k < m - k) {
            s[pad(m - k)] = cconj(csub(ev, iod));
        }
    });
}

// Real input (forward). A row of n = 2m reals is read as m complex values z[j] = x[2j] + i x[2j+1]
// (the same bytes), an m-point forward transform gives Z, and the store combines pairs:
//   E = (Z[k] + conj Z[m-k]) / 2,  O = (Z[k] - conj Z[m-k]) / 2i,  w = exp(-pi i k / m),
//   X[k] = E + w O,  X[m-k] = conj(E - w O),
// so one twiddle serves bins k and m-k (k = 0 pairs with m, whose Z index wraps to 0). This is the
// split formula of the reference's real.cuh:7-42, evaluated per pair instead of per bin.
// keep: values per row of y, m + 1 for the whole half spectrum, fewer when pruned.
template <bool PlainOut, bool Aligned = true>
struct R2cIoT {
    static constexpr bool kGroupIsBlock = false;
    static constexpr bool kFinal = true;
    const cf32* z;  // x viewed as complex
    cf32* y;
    int keep;

    // The group's rows leave LDS as one run in whole 128-byte lines (store_run_aligned): rows of
    // m + 1 values start at 8-byte offsets, and stores that straddle lines wrote 5-9 % more bytes
    // than the output holds (WRITE_SIZE, n = 128 .. 8192); in whole lines, 0.2-1.8 %. Rows of
    // fewer than 64 lanes are staged through LDS anyway. Rows of exactly 64 lanes take it when
    // their plan has radix 8 or more and at most 8 values per lane (radix 8, n = 1024: 24.54
    // against 26.25 us for the direct store, four alternated rounds with cache-clean inputs);
    // the other plans store their bins X[k] straight from registers, runs of L values, where
    // the extra LDS pass cost more than it saved: n = 2048 (128 lanes) 29.20 -> 27.35 us in the
    // same rounds, n = 4096 (256 lanes) equal, n = 8192 at 16 values per lane 67.8 -> 64.6 % and
    // radix 4 at n = 1024 73.5 -> 67.0 % of 8 TB/s in earlier interleaved rounds. Aligned = false
    // keeps the direct store for every row of 64 lanes or more and the row-by-row staged store
    // for the others.
    template <class P>
    static constexpr bool aligned_store()
    {
        return Aligned && (P::L < 64 || (P::L == 64 && P::R >= 8 && P::E <= 8));
    }
    template <class P>
    static constexpr bool direct_store() { return !aligned_store<P>() && P::L >= 64; }
    // The combine done by the transform's own lanes from their registers (final) for m = 8 ..
    // 64 and for rows of 16 lanes or more (X then goes back to LDS for the staged store, or out
    // directly), a separate pass over the pairs otherwise.
    template <class P>
    static constexpr bool direct_combine()
    {
        return (P::N >= 8 && P::N <= 64) || P::L >= 16;
    }

    template <class P>
    static constexpr bool direct_in() { return P::L >= 16; }
    template <class P>
    static constexpr bool direct_out() { return false; }

    // Nontemporal loads: with the inputs in rotation beyond the Infinity Cache (twice its size),
    // three alternated A/B rounds at 2^24 points on MI355X ran n = 16 .. 1024 1-2.4 % faster than
    // plain loads (n = 1024: 24.97 -> 24.37 us) and no size slower. (Plain loads had looked
    // faster when the inputs of a three-set rotation could stay in that cache.)
    template <class P>
    __device__ __forceinline__ cf32 in(long long t, int i) const
    {
        return ld_stream(z + t * P::N + i);
    }
    template <class P>
    __device__ __forceinline__ void out(long long, int, cf32) const {}

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        using S = Staged<G, P::N>;
        const cf32* src = z + first * P::N;
        cf32 val[S::kSteps];
        S::each(count, tid, [&](int k, int u, int i, bool valid) {
            val[k] = valid ? ld_stream(src + u * P::N + i) : czero();
        });
        S::each(count, tid, [&](int k, int u, int i, bool valid) {
            if (valid) {
                lds[u * P::kStride + pad(i)] = val[k];
            }
        });
    }

    // Output slot e of the last stage holds Z[k], k = lane + off. With the row's Z in LDS, the
    // lane reads Z[m-k] and forms X[k] = E + exp(-pi i k / m) O, E = (Z[k] + conj Z[m-k]) / 2,
    // O = (Z[k] - conj Z[m-k]) / 2i (indices mod m), and X[m] = E[0] - O[0] at k = 0; then X
    // replaces Z in LDS. A lane's k are lane plus compile-time offsets: one twiddle per lane.
    template <class P, bool WaveLocal>
    __device__ __forceinline__ void final(cf32* s, cf32 (&v)[P::E], int lane, long long t,
                                          long long batch) const
    {
        lds_sync<WaveLocal>();
        final_write<P>(s, v, lane);
        lds_sync<WaveLocal>();
        if constexpr (direct_combine<P>()) {
            constexpr int m = P::N;
            constexpr int RL = P::template radix<P::kStages - 1>();
            const cf32 base = twiddle_of<2 * m, false>(lane);
            cf32 xm{0.0f, 0.0f};
            static_for<0, P::E>([&](auto ei) {
                constexpr int e = decltype(ei)::value;
                constexpr int off = (e / RL) * P::L + (e % RL) * (P::N / RL);
                const int k = lane + off;
                const cf32 zk = v[e];
                const cf32 zm = s[pad((m - k) & (m - 1))];
                const cf32 ev{0.5f * (zk.re + zm.re), 0.5f * (zk.im - zm.im)};
                const cf32 od{0.5f * (zk.im + zm.im), -0.5f * (zk.re - zm.re)};
                constexpr cf32 c = const_twiddle<false>(off, 2 * m);
                v[e] = cadd(ev, cmul(off == 0 ? base : cmul(base, c), od));
                if constexpr (off == 0) {
                    xm = csub(ev, od);  // X[m], kept by the lane with k = 0
                }
            });
            if constexpr (direct_store<P>()) {
                if (t < batch) {
                    cf32* const dst = y + t * keep;
                    static_for<0, P::E>([&](auto ei) {
                        constexpr int e = decltype(ei)::value;
                        constexpr int off = (e / RL) * P::L + (e % RL) * (P::N / RL);
                        if (lane + off < keep) {
                            put(dst + lane + off, v[e]);
                        }
                    });
                    if (lane == 0 && m < keep) {
                        put(dst + m, xm);
                    }
                }
            } else {
                lds_sync<WaveLocal>();  // every partner read is done before X replaces Z
                final_write<P>(s, v, lane);
                if (lane == 0) {
                    s[pad(m)] = xm;
                }
                lds_sync<WaveLocal>();
            }
        }
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long first, int count, int tid) const
    {
        constexpr int m = P::N;
        if constexpr (direct_store<P>()) {
            return;  // stored by final
        }
        if constexpr (!direct_combine<P>()) {
            combine_pairs<P, G>(lds, count, tid);
            lds_sync<G::kWave>();
        }
        // 2. The first `keep` values of each row, stored contiguously.
        cf32* dst = y + first * keep;
        if constexpr (aligned_store<P>()) {
            if (keep == m + 1) {
                store_run_aligned<G, m + 1, P::kStride>(lds, dst, count, tid,
                                                        [](cf32* p, cf32 v) { put(p, v); });
                return;
            }
        }
        using H = Staged<G, m + 1>;
        H::each(count, tid, [&](int, int u, int i, bool valid) {
            if (valid && i < keep) {
                put(dst + u * keep + i, lds[u * P::kStride + pad(i)]);
            }
        });
    }

    // PlainOut: plain stores, for a workspace that the next pass reads (nontemporal otherwise).
    __device__ __forceinline__ static void put(cf32* p, cf32 v)
    {
        if constexpr (PlainOut) {
            *p = v;
        } else {
            st_stream(p, v);
        }
    }
};
using R2cIo = R2cIoT<false>;

// Real output (inverse). Rows of x hold X[0 .. keep-1] of the m + 1 half-spectrum values (the
// rest zero). The load prepares pairs (reference real.cuh:44-61, per pair):
//   E = (X[k] + conj X[m-k]) / 2,  O = (X[k] - conj X[m-k]) / 2 * exp(pi i k / m),
//   Z[k] = E + i O,  Z[m-k] = conj(E - i O),
// with the imaginary parts of X[0] and X[m] dropped; then an m-point inverse transform, scaled
// by 1/m, is the 2m real outputs read as complex.
struct C2rIo {
    static constexpr bool kGroupIsBlock = false;
    static constexpr bool kStage0 = true;
    const cf32* x;
    cf32* z;      // y viewed as complex
    float scale;  // 1/m
    int keep;

    // Stage-0 inputs formed from the raw half spectrum by each lane (stage0) for m = 16 .. 64:
    // measured 7-12 % of peak faster there than a separate prepare pass over the pairs, and
    // 2-4 % slower at m = 4, 128 and 512, which keep the pass. At m = 8 (one lane per
    // transform, each reading its 16 halves from LDS) the pass is faster: 34.4 -> 27.9 us over
    // 2^24 points with cache-clean inputs, three alternated rounds.
    template <class P>
    static constexpr bool direct_prepare() { return P::N >= 16 && P::N <= 64; }

    template <class P>
    static constexpr bool direct_in() { return false; }
    template <class P>
    static constexpr bool direct_out() { return P::L >= 16; }

    template <class P>
    __device__ __forceinline__ cf32 in(long long, int) const { return czero(); }
    // The scale rides on the prepare's halves, so the outputs are stored as they are.
    template <class P>
    __device__ __forceinline__ void out(long long t, int i, cf32 v) const
    {
        st_stream(z + t * P::N + i, v);
    }

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        constexpr int m = P::N;
        static_assert(pad(m) < P::kStride, "a row of m + 1 values fits its LDS stride");
        // The half spectrum X[0 .. m] into LDS (zero beyond keep).
        using H = Staged<G, m + 1>;
        // Nontemporal loads for m <= 32, plain beyond: with cache-clean inputs (three alternated
        // A/B rounds at 2^24 points) nontemporal loads ran n = 8 .. 64 0.2-5 % faster and
        // n = 1024 and 4096 about 2 % slower.
        const cf32* src = x + first * keep;
        cf32 val[H::kSteps];
        H::each(count, tid, [&](int j, int u, int k, bool valid) {
            val[j] = (valid && k < keep)
                         ? (m <= 32 ? ld_stream(src + u * keep + k) : src[u * keep + k])
                         : czero();
        });
        H::each(count, tid, [&](int j, int u, int k, bool valid) {
            if (valid) {
                lds[u * P::kStride + pad(k)] = val[j];
            }
        });
        if constexpr (!direct_prepare<P>()) {
            lds_sync<G::kWave>();
            prepare_pairs<P, G>(lds, count, tid, scale);
        }
    }

    // Stage-0 input slot e holds Z[k], k = lane + off: Z[k] = E + i O with E = (X[k] + conj
    // X[m-k]) / 2 and O = exp(pi i k / m) (X[k] - conj X[m-k]) / 2 (imaginary parts of X[0] and
    // X[m] dropped), read from the row's raw half spectrum in LDS. A lane's k are lane plus
    // compile-time offsets, so it evaluates one twiddle. Either way the scale 1/m rides on the
    // halves.
    template <class P>
    __device__ __forceinline__ void stage0(const cf32* s, cf32 (&v)[P::E], int lane) const
    {
        if constexpr (!direct_prepare<P>()) {
            stage_read<P, 0>(s, v, lane);
        } else {
            constexpr int m = P::N;
            constexpr int R0 = P::template radix<0>();
            const float half = 0.5f * scale;
            const cf32 base = twiddle_of<2 * m, true>(lane);
            static_for<0, P::E>([&](auto ei) {
                constexpr int e = decltype(ei)::value;
                constexpr int off = (e / R0) * P::L + (e % R0) * (P::N / R0);
                const int k = lane + off;
                cf32 xk = s[pad(k)];
                cf32 xm = s[pad(m - k)];
                if (k == 0) {
                    xk.im = 0.0f;
                    xm.im = 0.0f;
                }
                const cf32 ev{half * (xk.re + xm.re), half * (xk.im - xm.im)};
                const cf32 d{half * (xk.re - xm.re), half * (xk.im + xm.im)};
                constexpr cf32 c = const_twiddle<true>(off, 2 * m);
                const cf32 od = cmul(d, off == 0 ? base : cmul(base, c));
                v[e] = cf32{ev.re - od.im, ev.im + od.re};
            });
        }
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long first, int count,
                                          int tid) const
    {
        C2cIo<false>{nullptr, z, 1.0f, P::N, P::N}.template store<P, G>(lds, first, count, tid);
    }
};

// Columns of row-major arrays: slabs arrays of N rows by `cols` columns, back to back; transform
// c is column c % cols of slab c / cols. The whole workgroup stages its T neighbouring columns
// together, so each row read or written is a run of T * 8 contiguous bytes, and a lane keeps the
// same column for its whole staging loop (T divides 256), so the slab/column split is computed
// once.
//
// Pruned (an FNO keeps the lowest frequencies of each column): m1_in > 0 means the arrays of x hold
// only 2 m1_in rows, frequencies 0 .. m1_in-1 then N-m1_in .. N-1 (the rest zero); m1_out > 0
// that y keeps only those 2 m1_out rows. Frequency i sits in row i (i < m1) or i - (N - 2 m1).
// x == y is allowed only unpruned: a workgroup reads all its columns before writing any.
struct StridedIo {
    static constexpr bool kGroupIsBlock = true;
    const cf32* x;
    cf32* y;
    int cols;
    float scale;
    int m1_in;
    int m1_out;
    // Nontemporal stores, for a final output. An intermediate that the next pass reads keeps
    // plain stores: on MI355X nontemporal stores measured 1-3 points faster for the former (the
    // inverse 2D column pass) and 1.4-2.2 slower for the latter (the forward one).
    bool stream_out;

    template <class P>
    static constexpr bool direct_in() { return false; }
    template <class P>
    static constexpr bool direct_out() { return false; }

    template <class P>
    __device__ __forceinline__ cf32 in(long long, int) const { return czero(); }
    template <class P>
    __device__ __forceinline__ void out(long long, int, cf32) const {}

    // Values a lane stages per tile of T columns: the workgroup covers kThreads / T rows of the
    // tile per step.
    template <class P>
    static constexpr int steps() { return P::N / (P::kThreads / P::T); }

    // The global half of the load: lane tid takes column j = tid mod T of the tile starting at
    // transform `first`, rows tid / T + k kThreads / T, into registers (zero for the rows a pruned
    // input does not hold). Lanes of columns past `count` take nothing. nt: nontemporal loads.
    template <class P, bool Full>
    __device__ __forceinline__ void fetch(cf32 (&val)[steps<P>()], long long first, int count,
                                          int tid, bool nt = false) const
    {
        constexpr int kRowsPerStep = P::kThreads / P::T;
        const int j = tid % P::T;
        if (!Full && j >= count) {
            return;
        }
        const long long c = first + j;
        const long long slab = c / cols;
        const int col = static_cast<int>(c - slab * cols);
        const int rows = m1_in > 0 ? 2 * m1_in : P::N;
        const cf32* base = x + slab * rows * cols + col;
#pragma unroll
        for (int k = 0; k < steps<P>(); ++k) {
            const int i = tid / P::T + k * kRowsPerStep;
            int row = i;
            if (m1_in > 0) {
                row = i < m1_in ? i : (i >= P::N - m1_in ? i - (P::N - rows) : -1);
            }
            const cf32* const src = base + static_cast<long long>(row) * cols;
            val[k] = row < 0 ? czero() : (nt ? ld_stream(src) : *src);
        }
    }

    // The LDS half: the fetched values to their tile slots.
    template <class P, bool Full>
    __device__ __forceinline__ void park(cf32* lds, const cf32 (&val)[steps<P>()], int count,
                                         int tid) const
    {
        constexpr int kRowsPerStep = P::kThreads / P::T;
        const int j = tid % P::T;
        if (!Full && j >= count) {
            return;
        }
#pragma unroll
        for (int k = 0; k < steps<P>(); ++k) {
            lds[j * P::kStride + pad(tid / P::T + k * kRowsPerStep)] = val[k];
        }
    }

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        static_assert(G::kT == P::T && G::kThreads == P::kThreads,
                      "strided columns stage a whole workgroup");
        cf32 val[steps<P>()];
        fetch<P, G::kFull>(val, first, count, tid);
        park<P, G::kFull>(lds, val, count, tid);
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
        const long long c = first + j;
        const long long slab = c / cols;
        const int col = static_cast<int>(c - slab * cols);
        const int rows = m1_out > 0 ? 2 * m1_out : P::N;
        cf32* base = y + slab * rows * cols + col;
#pragma unroll
        for (int k = 0; k < kSteps; ++k) {
            const int row = tid / P::T + k * kRowsPerStep;
            if (row < rows) {
                const int i = (m1_out > 0 && row >= m1_out) ? row + (P::N - rows) : row;
                cf32* const dst = base + static_cast<long long>(row) * cols;
                const cf32 v = cscale(lds[j * P::kStride + pad(i)], scale);
                if (stream_out) {
                    st_stream(dst, v);
                } else {
                    *dst = v;
                }
            }
        }
    }
};

// Strided columns, persistent: in round r workgroup b transforms the tile of T columns
// r gridDim.x + xcd_order<C>(b), and issues each next tile's loads into registers before the
// current tile's stages, so they are in flight during its stages and stores. Launched with as
// many workgroups as fit on the device at once. With one tile per workgroup in flight
// (fft_kernel) the loads of the whole device come in bursts between compute phases: at 256- and
// 512-point columns this measured 10-13 points of the 8 TB/s peak faster on MI355X.
// C > 0 (tiles narrower than a cache line, T = 8 at 1024 points) keeps the two tiles that share
// each 128-byte line on one XCD: 90.8 -> 72.0 us for the 1024-point columns of 2^20-point
// transforms (2^24 points), where 128-byte tiles gained nothing at 512 points.
template <class P, bool Inv, bool Table, int C = 0>
__global__ void __launch_bounds__(P::kThreads)
    columns_kernel(StridedIo io, long long batch, const cf32* table)
{
    __shared__ cf32 lds[P::T * P::kStride];
    using Full = Group<P::T, P::kThreads, true>;
    using Tail = Group<P::T, P::kThreads, false>;
    const int tid = threadIdx.x;
    const int lane = tid % P::L;
    cf32* const s = lds + (tid / P::L) * P::kStride;
    const long long tiles = (batch + P::T - 1) / P::T;
    const auto count_of = [batch](long long tile) {
        const long long left = batch - tile * P::T;
        return left >= P::T ? P::T : static_cast<int>(left);
    };
    // The last pass of a transform (final output) also loads nontemporally: 1 point of the peak
    // faster for the inverse 2D and fft2_c2c column passes at 256 and 512 points, where the
    // forward's first pass measured 1-2 points slower with it. Not for tiles narrower than a
    // cache line (C > 0): their neighbour tile, on the same XCD, reads the other half of each line
    // from L2, which nontemporal loads do not leave there. Plain loads there: irfft2 1024^2
    // 64.4 -> 57.0 us and fft2_c2c 1024^2 125.8 -> 103.2 us on MI355X (interleaved rounds).
    const bool nt = io.stream_out && C == 0;
    cf32 val[StridedIo::steps<P>()];
    const long long offset = xcd_order<C>(blockIdx.x, gridDim.x);
    if (offset < tiles) {
        io.template fetch<P, false>(val, offset * P::T, count_of(offset), tid, nt);
    }
    for (long long tile = offset; tile < tiles; tile += gridDim.x) {
        const int count = count_of(tile);
        io.template park<P, false>(lds, val, count, tid);
        lds_sync<false>();
        const long long next = tile + gridDim.x;
        if (next < tiles) {
            io.template fetch<P, false>(val, next * P::T, count_of(next), tid, nt);
        }
        // Columns past the batch run the stages on what the tile holds but store nothing.
        cf32 v[P::E];
        stage_read<P, 0>(s, v, lane);
        run_stages<P, 0, Inv, Table>(v, s, lane, table);
        lds_sync<P::kWaveLocal>();  // a transform's lanes have read s (one wave when L <= 64)
        final_write<P>(s, v, lane);
        lds_sync<false>();
        if (count == P::T) {
            io.template store<P, Full>(lds, tile * P::T, P::T, tid);
        } else {
            io.template store<P, Tail>(lds, tile * P::T, count, tid);
        }
        lds_sync<false>();  // every store has read the tile before the next one lands
    }
}

}  // namespace spx::dev
