#pragma once

// The "transpose" column method of the 2D transforms in two HBM round trips. The reference runs
// it as four kernels (fft2d.cu:138-187): rows, a transpose, the columns as contiguous rows, a
// transpose back. Here the transposes happen inside the 1D passes, on the LDS tile each
// workgroup already stages: a pass reads whole rows and writes them transposed, or reads a
// transposed layout and writes whole rows.
//
// Layouts: `rows` transforms per array; a transform's `len` values on the transposed side sit
// `rows` apart. Transform t is row r = t mod rows of array b = t / rows:
//   rows side        element i of t at  base + t * N + i              (contiguous)
//   transposed side  element k of t at  base + b * rows * len + k * rows + r
// A workgroup stages its T consecutive transforms together (the whole workgroup is the group),
// so every access of the transposed side is a run of T values (T * 8 bytes: 128 bytes for the
// column plans up to N = 512, 256 at N = 64), and a lane keeps one transform for its whole loop:
// lane tid serves transform first + tid mod T at elements tid / T + s L (L lanes per transform).
//
//   RowsToTransposedIo     complex rows in, transposed out            (fft2 both passes; the
//                                                                       forward real 2D's second)
//   R2cRowsToTransposedIo  real rows in (read as m complex values), the half spectrum
//                          X[0 .. m] out transposed (len = m + 1)      (rfft2's first pass)
//   TransposedToRowsIo     transposed complex in, rows out             (irfft2's first pass)
//   C2rTransposedToRowsIo  the half spectrum in transposed (len = m + 1), real rows out
//                                                                      (irfft2's second pass)

#include "stockham.hpp"

namespace spx::dev {

// Where transform first + (tid mod T) keeps its transposed side: base + b rows len + r.
template <class P>
__device__ __forceinline__ long long transposed_origin(long long first, int tid, int rows,
                                                       int len)
{
    const long long t = first + tid % P::T;
    const long long b = t / rows;
    return b * rows * static_cast<long long>(len) + (t - b * rows);
}

// Element k of each staged transform (k < len, from LDS) written transposed. Every lane of the
// workgroup belongs to one of the T transforms (kThreads = T L).
template <class P, class G, class Put>
__device__ __forceinline__ void store_transposed(const cf32* lds, cf32* y, long long first,
                                                 int count, int tid, int rows, int len, Put&& put)
{
    static_assert(G::kT == P::T && G::kThreads == P::kThreads, "the whole workgroup stores");
    const int j = tid % P::T;
    if (!G::kFull && j >= count) {
        return;
    }
    cf32* const base = y + transposed_origin<P>(first, tid, rows, len);
    constexpr int kSteps = (P::N + 1 + P::L - 1) / P::L;  // len is N or N + 1
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        const int k = tid / P::T + s * P::L;
        if ((s + 1) * P::L <= P::N || k < len) {
            put(base + static_cast<long long>(k) * rows, lds[j * P::kStride + pad(k)]);
        }
    }
}

// A lane's values of one transposed load: element tid / T + s L of its transform, s < steps,
// for transforms of len = N + Plus values (Plus 0 or 1).
template <class P, int Plus>
constexpr int transposed_steps()
{
    return (P::N + Plus + P::L - 1) / P::L;
}

// The transposed side's element k < len of each of the count staged transforms into registers
// (lanes of transforms past count load nothing).
template <class P, int Plus>
__device__ __forceinline__ void fetch_transposed(
    cf32 (&val)[(transposed_steps<P, Plus>())], const cf32* x, long long first, int count,
    int tid, int rows, bool stream_in)
{
    constexpr int len = P::N + Plus;
    if (tid % P::T >= count) {
        return;
    }
    const cf32* const base = x + transposed_origin<P>(first, tid, rows, len);
#pragma unroll
    for (int s = 0; s < transposed_steps<P, Plus>(); ++s) {
        const int k = tid / P::T + s * P::L;
        const bool in = (s + 1) * P::L <= P::N || k < len;
        const cf32* const src = base + static_cast<long long>(in ? k : 0) * rows;
        val[s] = in ? (stream_in ? ld_stream(src) : *src) : czero();
    }
}

// The fetched values into their transforms' LDS rows.
template <class P, int Plus>
__device__ __forceinline__ void park_transposed(
    cf32* lds, const cf32 (&val)[(transposed_steps<P, Plus>())], int count, int tid)
{
    constexpr int len = P::N + Plus;
    const int j = tid % P::T;
    if (j >= count) {
        return;
    }
#pragma unroll
    for (int s = 0; s < transposed_steps<P, Plus>(); ++s) {
        const int k = tid / P::T + s * P::L;
        if ((s + 1) * P::L <= P::N || k < len) {
            lds[j * P::kStride + pad(k)] = val[s];
        }
    }
}

// Element k < len of each staged transform read from the transposed side into LDS (every load
// issued before the first LDS write).
template <class P, class G, int Plus>
__device__ __forceinline__ void load_transposed(cf32* lds, const cf32* x, long long first,
                                                int count, int tid, int rows, bool stream_in)
{
    static_assert(G::kT == P::T && G::kThreads == P::kThreads, "the whole workgroup loads");
    cf32 val[transposed_steps<P, Plus>()];
    fetch_transposed<P, Plus>(val, x, first, G::kFull ? P::T : count, tid, rows, stream_in);
    park_transposed<P, Plus>(lds, val, G::kFull ? P::T : count, tid);
}

// Contiguous rows of N complex values into LDS, as the group's staged load.
template <class P, class G>
__device__ __forceinline__ void load_rows(cf32* lds, const cf32* x, long long first, int count,
                                          int tid, bool stream_in)
{
    using S = Staged<G, P::N>;
    const cf32* const src = x + first * P::N;
    cf32 val[S::kSteps];
    S::each(count, tid, [&](int k, int u, int i, bool valid) {
        val[k] = valid ? (stream_in ? ld_stream(src + u * P::N + i) : src[u * P::N + i])
                       : czero();
    });
    S::each(count, tid, [&](int k, int u, int i, bool valid) {
        if (valid) {
            lds[u * P::kStride + pad(i)] = val[k];
        }
    });
}

__device__ __forceinline__ void put_value(cf32* p, cf32 v, bool stream_out)
{
    if (stream_out) {
        st_stream(p, v);
    } else {
        *p = v;
    }
}

// Chunk > 0: runs of Chunk consecutive workgroups on one XCD (xcd_order), for transposed rows that
// do not start on 128-byte lines (a half spectrum's m + 1 values): the partial lines that
// neighbouring tiles share are then written through one L2.
template <int Chunk = 0>
struct RowsToTransposedIoT {
    static constexpr bool kGroupIsBlock = true;
    static constexpr int kXcdChunk = Chunk;
    const cf32* x;
    cf32* y;
    int rows;         // transforms per array
    float scale;      // on the way out
    bool stream_in;   // nontemporal loads: a caller's input (plain: a workspace)
    bool stream_out;  // nontemporal stores: a final output (plain: a workspace read next)

    template <class P>
    static constexpr bool direct_in() { return P::L >= 16; }
    template <class P>
    static constexpr bool direct_out() { return false; }

    template <class P>
    __device__ __forceinline__ cf32 in(long long t, int i) const
    {
        const cf32* const p = x + t * P::N + i;
        return stream_in ? ld_stream(p) : *p;
    }
    template <class P>
    __device__ __forceinline__ void out(long long, int, cf32) const {}

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        load_rows<P, G>(lds, x, first, count, tid, stream_in);
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long first, int count, int tid) const
    {
        const float s = scale;
        const bool nt = stream_out;
        store_transposed<P, G>(lds, y, first, count, tid, rows, P::N,
                               [s, nt](cf32* p, cf32 v) { put_value(p, cscale(v, s), nt); });
    }
};

using RowsToTransposedIo = RowsToTransposedIoT<0>;

struct R2cRowsToTransposedIo {
    static constexpr bool kGroupIsBlock = true;
    const cf32* z;  // the real rows read as complex: m = N values per row
    cf32* y;        // half spectra of m + 1 values, transposed
    int rows;

    // Where the real forward's own final step applies (the combine from each lane's registers,
    // X then written back to LDS rather than stored), it leaves X[0 .. m] in LDS; otherwise
    // the stages' outputs go to LDS as they are and store() combines them pair by pair there.
    using Rows = R2cIoT<true>;
    template <class P>
    static constexpr bool combine_in_registers()
    {
        return Rows::direct_combine<P>() && !Rows::direct_store<P>();
    }
    static constexpr bool kFinal = true;
    template <class P, bool WaveLocal>
    __device__ __forceinline__ void final(cf32* s, cf32 (&v)[P::E], int lane, long long t,
                                          long long batch) const
    {
        if constexpr (combine_in_registers<P>()) {
            Rows{z, y, P::N + 1}.template final<P, WaveLocal>(s, v, lane, t, batch);
        } else {
            lds_sync<WaveLocal>();
            final_write<P>(s, v, lane);
            lds_sync<WaveLocal>();
        }
    }

    template <class P>
    static constexpr bool direct_in() { return P::L >= 16; }
    template <class P>
    static constexpr bool direct_out() { return false; }

    template <class P>
    __device__ __forceinline__ cf32 in(long long t, int i) const { return z[t * P::N + i]; }
    template <class P>
    __device__ __forceinline__ void out(long long, int, cf32) const {}

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        load_rows<P, G>(lds, z, first, count, tid, false);
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long first, int count, int tid) const
    {
        static_assert(pad(P::N) < P::kStride, "X[m] fits the row's LDS stride");
        if constexpr (!combine_in_registers<P>()) {
            combine_pairs<P, G>(lds, count, tid);
            lds_sync<false>();
        }
        store_transposed<P, G>(lds, y, first, count, tid, rows, P::N + 1,
                               [](cf32* p, cf32 v) { *p = v; });
    }
};

template <int Chunk = 0>
struct TransposedToRowsIoT {
    static constexpr bool kGroupIsBlock = true;
    static constexpr int kXcdChunk = Chunk;
    const cf32* x;
    cf32* y;
    int rows;
    float scale;
    bool stream_in;
    bool stream_out;

    template <class P>
    static constexpr bool direct_in() { return false; }
    template <class P>
    static constexpr bool direct_out() { return P::L >= 16; }

    template <class P>
    __device__ __forceinline__ cf32 in(long long, int) const { return czero(); }
    template <class P>
    __device__ __forceinline__ void out(long long t, int i, cf32 v) const
    {
        put_value(y + t * P::N + i, cscale(v, scale), stream_out);
    }

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        load_transposed<P, G, 0>(lds, x, first, count, tid, rows, stream_in);
    }

    // The load in two halves, for the persistent tile loop (tiles_persistent_kernel).
    static constexpr bool kFetch = true;
    template <class P>
    static constexpr int fetch_steps() { return transposed_steps<P, 0>(); }
    template <class P>
    __device__ __forceinline__ void fetch(cf32 (&val)[(transposed_steps<P, 0>())],
                                          long long first, int count, int tid) const
    {
        fetch_transposed<P, 0>(val, x, first, count, tid, rows, stream_in);
    }
    template <class P>
    __device__ __forceinline__ void park(cf32* lds,
                                         const cf32 (&val)[(transposed_steps<P, 0>())],
                                         int count, int tid) const
    {
        park_transposed<P, 0>(lds, val, count, tid);
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long first, int count, int tid) const
    {
        using S = Staged<G, P::N>;
        cf32* const dst = y + first * P::N;
        S::each(count, tid, [&](int, int u, int i, bool valid) {
            if (valid) {
                put_value(dst + u * P::N + i, cscale(lds[u * P::kStride + pad(i)], scale),
                          stream_out);
            }
        });
    }
};

using TransposedToRowsIo = TransposedToRowsIoT<0>;

// Persistent form of fft_kernel for the transposed-side loads: workgroup g takes tiles of T
// transforms g', g' + G, ... (g' = g in the policy's XCD order, G = gridDim.x) and issues the
// next tile's loads into registers once the current tile is in LDS, so they are in flight during
// its stages and stores (the pattern of columns_kernel).
template <class P, bool Inv, bool Table, class Io>
__global__ void __launch_bounds__(P::kThreads) __attribute__((amdgpu_waves_per_eu(8)))
    tiles_persistent_kernel(Io io, long long batch, const cf32* table)
{
    static_assert(Io::kGroupIsBlock && Io::kFetch && !Io::template direct_in<P>(),
                  "loads staged by the whole workgroup, in two halves");
    __shared__ cf32 lds[P::T * P::kStride];
    using Full = Group<P::T, P::kThreads, true>;
    using Tail = Group<P::T, P::kThreads, false>;
    const long long tiles = (batch + P::T - 1) / P::T;
    const auto count_of = [batch](long long tile) {
        const long long left = batch - tile * P::T;
        return left >= P::T ? P::T : static_cast<int>(left);
    };
    cf32 val[Io::template fetch_steps<P>()];
    const long long offset = xcd_order<XcdChunk<Io>::value>(blockIdx.x, gridDim.x);
    if (offset < tiles) {
        io.template fetch<P>(val, offset * P::T, count_of(offset), threadIdx.x);
    }
#pragma unroll 1
    for (long long tile = offset; tile < tiles; tile += gridDim.x) {
        const int tid = opaque_tid<P::kThreads>();
        const int lane = tid % P::L;
        const int u = tid / P::L;
        cf32* const s = lds + u * P::kStride;
        const int count = count_of(tile);
        io.template park<P>(lds, val, count, tid);
        lds_sync<false>();
        const long long next = tile + gridDim.x;
        if (next < tiles) {
            io.template fetch<P>(val, next * P::T, count_of(next), tid);
        }
        // Transforms past the batch run the stages on what the tile holds but store nothing.
        cf32 v[P::E];
        stage_read<P, 0>(s, v, lane);
        run_stages<P, 0, Inv, Table>(v, s, lane, table);
        if constexpr (Io::template direct_out<P>()) {
            if (u < count) {
                constexpr int RL = P::template radix<P::kStages - 1>();
                const long long t = tile * P::T + u;
#pragma unroll
                for (int b = 0; b < P::E / RL; ++b) {
#pragma unroll
                    for (int r = 0; r < RL; ++r) {
                        io.template out<P>(t, lane + b * P::L + r * (P::N / RL), v[b * RL + r]);
                    }
                }
            }
        } else {
            lds_sync<P::kWaveLocal>();
            final_write<P>(s, v, lane);
            lds_sync<false>();
            if (count == P::T) {
                io.template store<P, Full>(lds, tile * P::T, P::T, tid);
            } else {
                io.template store<P, Tail>(lds, tile * P::T, count, tid);
            }
        }
        lds_sync<false>();  // the tile is read before the next one lands
    }
}

struct C2rTransposedToRowsIo {
    static constexpr bool kGroupIsBlock = true;
    const cf32* x;  // half spectra of m + 1 values, transposed
    cf32* z;        // the real rows written as complex: m = N values per row
    int rows;
    float scale;    // 1 / m, on the prepare's halves

    template <class P>
    static constexpr bool direct_in() { return false; }
    template <class P>
    static constexpr bool direct_out() { return P::L >= 16; }

    template <class P>
    __device__ __forceinline__ cf32 in(long long, int) const { return czero(); }
    template <class P>
    __device__ __forceinline__ void out(long long t, int i, cf32 v) const
    {
        st_stream(z + t * P::N + i, v);
    }

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        static_assert(pad(P::N) < P::kStride, "X[m] fits the row's LDS stride");
        load_transposed<P, G, 1>(lds, x, first, count, tid, rows, false);
        lds_sync<false>();
        prepare_pairs<P, G>(lds, count, tid, scale);
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long first, int count, int tid) const
    {
        using S = Staged<G, P::N>;
        cf32* const dst = z + first * P::N;
        S::each(count, tid, [&](int, int u, int i, bool valid) {
            if (valid) {
                st_stream(dst + u * P::N + i, lds[u * P::kStride + pad(i)]);
            }
        });
    }
};

}  // namespace spx::dev
