#pragma once

// Column-first 2D real transforms, for the shapes too large for a single-pass kernel. A real
// n1 x n2 array read as n1 x M complex values (M = n2 / 2, value c = (x[2c], x[2c+1])) has rows
// of M * 8 bytes, a whole number of 128-byte lines from M = 16; its half spectrum has rows of
// (M + 1) * 8 bytes, which are not. The row-then-column drivers run their column pass over the
// half spectrum, where every 128-byte run of a column tile straddles two lines (a strided copy
// at that pitch measured 36-41 % of peak on MI355X, against 56-63 % at an aligned pitch). So:
//
//   forward  1. n1-point FFTs down the M packed columns, Z = A + i B (A, B the column spectra of
//               the even and odd real columns), x -> work at the aligned pitch;
//            2. per pair of rows (k1, -k1 mod n1) of one array: M-point FFTs of both rows, then
//               X[k1, k] = FA + W^k FB from FA = (F[k1, k] + conj(F[-k1, -k])) / 2 and
//               FB = (F[k1, k] - conj(F[-k1, -k])) / 2i (A and B are Hermitian in k1, since
//               the columns are real), k = 0 .. M, W = exp(-2 pi i / n2); both rows of X are
//               written contiguously (PairR2cIo).
//   inverse  the mirror: per pair of rows, the prepare Z = FA + i FB from X (PairC2rIo), inverse
//            M-point row FFTs (work), then inverse columns into the real output (x read as
//            complex). Columns 0 and M are first made Hermitian across the pair, which is what
//            numpy's irfft2 does with them (it drops the imaginary parts of DC and Nyquist of
//            each row after the column inverse); other columns need nothing.
//
// Transforms come in pairs t = 2 p + slot, pair p = array * pairs + k1 (pairs = n1 / 2 + 1, k1 =
// 0 .. n1 / 2): slot 0 is row k1, slot 1 row -k1 mod n1. Rows 0 and n1 / 2 are their own
// partners; their slot 1 computes the same row again and writes nothing. Each workgroup holds
// an even number of transforms, so a pair never straddles two.

#include "stockham.hpp"

namespace spx::dev {

struct PairRows {
    int n1;
    int pairs;  // n1 / 2 + 1

    // Row of transform t within its array, and the array; dup: slot 1 of a self-paired row.
    __device__ __forceinline__ int row(long long t, long long& array, bool& dup) const
    {
        const long long p = t >> 1;
        array = p / pairs;
        const int k1 = static_cast<int>(p - array * pairs);
        const bool slot = (t & 1) != 0;
        dup = slot && (k1 == 0 || 2 * k1 == n1);
        return slot ? (n1 - k1) & (n1 - 1) : k1;
    }

    // The same for t = first + du, 0 <= du, given first's pair split once as (array0, k10) with
    // `first` even: no division per transform.
    __device__ __forceinline__ int row_after(long long array0, int k10, int du, long long& array,
                                             bool& dup) const
    {
        int k1 = k10 + (du >> 1);
        array = array0;
        while (k1 >= pairs) {
            k1 -= pairs;
            ++array;
        }
        const bool slot = (du & 1) != 0;
        dup = slot && (k1 == 0 || 2 * k1 == n1);
        return slot ? (n1 - k1) & (n1 - 1) : k1;
    }
};

// Forward pass 2: z (arrays x n1 x M, column-transformed packed rows) -> y (arrays x n1 x (M+1)).
struct PairR2cIo {
    static constexpr bool kGroupIsBlock = true;
    static constexpr bool kFinal = true;
    const cf32* z;
    cf32* y;
    PairRows rows;

    // Rows of 16 lanes or more combine their bins in registers (final); shorter rows combine in
    // the staged store.
    template <class P>
    static constexpr bool direct_combine() { return P::L >= 16; }

    template <class P>
    static constexpr bool direct_in() { return P::L >= 16; }
    template <class P>
    static constexpr bool direct_out() { return false; }

    template <class P>
    __device__ __forceinline__ cf32 in(long long t, int i) const
    {
        long long array;
        bool dup;
        const int r = rows.row(t, array, dup);
        return z[(array * rows.n1 + r) * P::N + i];
    }
    template <class P>
    __device__ __forceinline__ void out(long long, int, cf32) const {}

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        using S = Staged<G, P::N>;
        // The group's first transform is even (groups hold an even number): split its pair once.
        const long long array0 = (first >> 1) / rows.pairs;
        const int k10 = static_cast<int>((first >> 1) - array0 * rows.pairs);
        cf32 val[S::kSteps];
        S::each(count, tid, [&](int k, int u, int i, bool valid) {
            cf32 v = czero();
            if (valid) {
                long long array;
                bool dup;
                const int r = rows.row_after(array0, k10, u, array, dup);
                v = z[(array * rows.n1 + r) * P::N + i];
            }
            val[k] = v;
        });
        S::each(count, tid, [&](int k, int u, int i, bool valid) {
            if (valid) {
                lds[u * P::kStride + pad(i)] = val[k];
            }
        });
    }

    // The last stage leaves Z[k] of this row in slot e (k = lane + off); with both rows of the
    // pair in LDS, the lane reads the partner's Z[-k] and forms X[k1, k] = FA + W^k FB (W =
    // exp(-pi i / N); FA, FB as in the staged store below) for its own k, one twiddle per lane,
    // then puts X[0 .. N] in its row's slots for the staged store. X[k1, N] = FA - FB at k = 0.
    template <class P, bool WaveLocal>
    __device__ __forceinline__ void final(cf32* s, cf32 (&v)[P::E], int lane, long long t,
                                          long long) const
    {
        lds_sync<WaveLocal>();
        final_write<P>(s, v, lane);
        lds_sync<WaveLocal>();
        if constexpr (direct_combine<P>()) {
            constexpr int N = P::N;
            constexpr int RL = P::template radix<P::kStages - 1>();
            // Pairs are transforms (2 p, 2 p + 1) of one workgroup (an even number per group).
            const cf32* const partner = (t & 1) != 0 ? s - P::kStride : s + P::kStride;
            const cf32 base = twiddle_of<2 * N, false>(lane);
            cf32 xn{0.0f, 0.0f};
            static_for<0, P::E>([&](auto ei) {
                constexpr int e = decltype(ei)::value;
                constexpr int off = (e / RL) * P::L + (e % RL) * (P::N / RL);
                const int k = lane + off;
                const cf32 fa = v[e];
                const cf32 fb = partner[pad((N - k) & (N - 1))];
                const cf32 ev{0.5f * (fa.re + fb.re), 0.5f * (fa.im - fb.im)};
                const cf32 od{0.5f * (fa.im + fb.im), -0.5f * (fa.re - fb.re)};
                constexpr cf32 c = const_twiddle<false>(off, 2 * N);
                v[e] = cadd(ev, cmul(off == 0 ? base : cmul(base, c), od));
                if constexpr (off == 0) {
                    xn = csub(ev, od);
                }
            });
            lds_sync<WaveLocal>();  // every partner read is done before X replaces Z
            final_write<P>(s, v, lane);
            if (lane == 0) {
                s[pad(N)] = xn;
            }
            lds_sync<WaveLocal>();
        }
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long first, int count,
                                          int tid) const
    {
        if constexpr (direct_combine<P>()) {
            // X[0 .. N] of each row, combined by final: consecutive lanes take consecutive
            // values of a row, each row walked in whole 128-byte lines from the boundary before
            // its start (its N + 1 values start at an 8-byte offset; stores straddling lines
            // wrote 7 % more bytes than the output holds at 512^2). (Storing straight from
            // final's registers, runs of L values, measured 5.0 points of the peak slower at
            // 256^2 and 1.8 at 512^2 than the row-walk store before this one.)
            constexpr int N = P::N;
            const long long array0 = (first >> 1) / rows.pairs;
            const int k10 = static_cast<int>((first >> 1) - array0 * rows.pairs);
            cf32* const out = y;
            const PairRows pr = rows;
            store_rows_aligned<G, N + 1, P::kStride>(
                lds, count, tid,
                [&](int u) -> cf32* {
                    long long array;
                    bool dup;
                    const int r = pr.row_after(array0, k10, u, array, dup);
                    return dup ? nullptr : out + (array * pr.n1 + r) * (N + 1);
                },
                [](cf32* p, cf32 v) { st_stream(p, v); });
            return;
        }
        constexpr int N = P::N;
        using S = Staged<G, N + 1>;
        const long long array0 = (first >> 1) / rows.pairs;
        const int k10 = static_cast<int>((first >> 1) - array0 * rows.pairs);
        S::each(count, tid, [&](int, int u, int k, bool valid) {
            long long array;
            bool dup;
            const int r = rows.row_after(array0, k10, u, array, dup);
            if (!valid || dup) {
                return;
            }
            const cf32 fa = lds[u * P::kStride + pad(k & (N - 1))];
            const cf32 fb = lds[(u ^ 1) * P::kStride + pad((N - k) & (N - 1))];
            const cf32 ev{0.5f * (fa.re + fb.re), 0.5f * (fa.im - fb.im)};
            const cf32 od{0.5f * (fa.im + fb.im), -0.5f * (fa.re - fb.re)};
            st_stream(y + (array * rows.n1 + r) * (N + 1) + k,
                      cadd(ev, cmul(twiddle_of<2 * N, false>(k), od)));
        });
    }
};

// Inverse pass 1: x (arrays x n1 x (M+1)) -> z (arrays x n1 x M, prepared and row-inverted),
// scaled by `scale` (1 / M: with the prepare's halves, the row inverse of numpy's irfft). z is
// the workspace the column pass reads next, so it takes plain stores: nontemporal ones measured
// 1.2-2.4 points of the peak slower end to end at 256^2 .. 2048^2 on MI355X.
struct PairC2rIo {
    static constexpr bool kGroupIsBlock = true;
    const cf32* x;
    cf32* z;
    PairRows rows;
    float scale;

    template <class P>
    static constexpr bool direct_in() { return false; }
    template <class P>
    static constexpr bool direct_out() { return P::L >= 16; }

    template <class P>
    __device__ __forceinline__ cf32 in(long long, int) const { return czero(); }

    template <class P>
    __device__ __forceinline__ void out(long long t, int i, cf32 v) const
    {
        long long array;
        bool dup;
        const int r = rows.row(t, array, dup);
        if (!dup) {
            z[(array * rows.n1 + r) * P::N + i] = cscale(v, scale);
        }
    }

    // Raw rows (M + 1 values each) into LDS, then the prepare in place: task (pair, k) reads
    // slots (a, k) and (b, M - k) and writes the same two, so no two tasks touch one slot.
    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        constexpr int N = P::N;
        static_assert(pad(N) < P::kStride, "a row of N + 1 values fits its LDS stride");
        using S = Staged<G, N + 1>;
        // The group's first transform is even (groups hold an even number): split its pair once.
        const long long array0 = (first >> 1) / rows.pairs;
        const int k10 = static_cast<int>((first >> 1) - array0 * rows.pairs);
        cf32 val[S::kSteps];
        S::each(count, tid, [&](int k, int u, int i, bool valid) {
            cf32 v = czero();
            if (valid) {
                long long array;
                bool dup;
                const int r = rows.row_after(array0, k10, u, array, dup);
                v = x[(array * rows.n1 + r) * (N + 1) + i];
            }
            val[k] = v;
        });
        S::each(count, tid, [&](int k, int u, int i, bool valid) {
            if (valid) {
                lds[u * P::kStride + pad(i)] = val[k];
            }
        });
        lds_sync<false>();
        const int tasks = (count / 2) * N;
        for (int e = tid; e < tasks; e += G::kThreads) {
            const int q = e / N;
            const int k = e - q * N;
            cf32* const a = lds + (2 * q) * P::kStride;
            cf32* const b = a + P::kStride;
            if (k == 0) {
                // Columns 0 and M made Hermitian across the pair, then both rows' Z[0].
                const cf32 a0 = a[0];
                const cf32 b0 = b[0];
                const cf32 an = a[pad(N)];
                const cf32 bn = b[pad(N)];
                const cf32 dc{0.5f * (a0.re + b0.re), 0.5f * (a0.im - b0.im)};
                const cf32 ny{0.5f * (an.re + bn.re), 0.5f * (an.im - bn.im)};
                const cf32 ev{0.5f * (dc.re + ny.re), 0.5f * (dc.im + ny.im)};
                const cf32 d{0.5f * (dc.re - ny.re), 0.5f * (dc.im - ny.im)};
                a[0] = cf32{ev.re - d.im, ev.im + d.re};   // ev + i d
                b[0] = cf32{ev.re + d.im, -ev.im + d.re};  // conj(ev) + i conj(d)
            } else {
                const cf32 xk = a[pad(k)];
                const cf32 xm = b[pad(N - k)];
                const cf32 ev{0.5f * (xk.re + xm.re), 0.5f * (xk.im - xm.im)};
                const cf32 d{0.5f * (xk.re - xm.re), 0.5f * (xk.im + xm.im)};
                const cf32 od = cmul(d, twiddle_of<2 * N, true>(k));
                const cf32 iod{-od.im, od.re};
                a[pad(k)] = cadd(ev, iod);
                b[pad(N - k)] = cconj(csub(ev, iod));
            }
        }
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long first, int count,
                                          int tid) const
    {
        using S = Staged<G, P::N>;
        const long long array0 = (first >> 1) / rows.pairs;
        const int k10 = static_cast<int>((first >> 1) - array0 * rows.pairs);
        S::each(count, tid, [&](int, int u, int i, bool valid) {
            long long array;
            bool dup;
            const int r = rows.row_after(array0, k10, u, array, dup);
            if (valid && !dup) {
                z[(array * rows.n1 + r) * P::N + i] = cscale(lds[u * P::kStride + pad(i)], scale);
            }
        });
    }
};

// Row-pair plans: an even number of transforms per workgroup (at least two).
template <int M, int R>
using PairPlan = Plan<M, R, default_e<M, R>(),
                      cmax(kBlock, 2 * (M / default_e<M, R>()))>;

}  // namespace spx::dev
