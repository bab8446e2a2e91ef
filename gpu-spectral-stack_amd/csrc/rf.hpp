#pragma once

// The radio callers' transforms as single kernels: the windowed spectrum of back-to-back frames
// and the overlap-save FIR filter. The reference composes both in PyTorch around its FFT
// (python/spectral/rf.py:86-153): pad, unfold, window or spectrum product, FFT, inverse FFT,
// slice, each a pass through HBM. Here every signal sample is read once and every output written
// once:
//
//   spectrum  frame f of row r is x[r, f nfft .. f nfft + nfft) (zero past the end of the row)
//             times the window, transformed; FramesIo is an I/O policy of fft_kernel, so the
//             frames take the same plans, loads and stores as a batch of C2C transforms.
//   fir       block b of row r is the segment x[r, b step - (M-1) .. + nfft) with zeros outside
//             the row (step = nfft - M + 1, M taps). One kernel runs the forward stages, multiplies
//             by the filter's spectrum H / nfft in registers, runs the inverse stages, and writes
//             the block's last step outputs: y[r, b step + i - (M-1)] for i >= M-1. Circular
//             convolution wraps only into the first M-1 outputs, which are dropped.
//
// The forward transform leaves a lane holding elements lane + q L (q < E) in the last stage's
// slot order, and the inverse transform's first stage takes exactly those elements in its own
// slot order, so the product is handed from one to the other by renaming registers.

#include "fft_api.hpp"
#include "stockham.hpp"

namespace spx::dev {

// Element i of frame t (t = row * frames + f) of rows of n samples, times window[i].
struct FramesIo {
    static constexpr bool kGroupIsBlock = false;
    const cf32* x;
    const float* window;  // nullptr: rectangular
    cf32* y;
    long long n;
    long long frames;

    template <class P>
    static constexpr bool direct_in() { return P::L >= 16; }
    template <class P>
    static constexpr bool direct_out() { return P::L >= 16; }

    template <class P>
    __device__ __forceinline__ cf32 sample(long long t, int i) const
    {
        const long long row = t / frames;
        const long long j = (t - row * frames) * P::N + i;
        if (j >= n) {
            return czero();
        }
        const cf32 v = x[row * n + j];
        return window == nullptr ? v : cscale(v, window[i]);
    }

    template <class P>
    __device__ __forceinline__ cf32 in(long long t, int i) const { return sample<P>(t, i); }

    template <class P>
    __device__ __forceinline__ void out(long long t, int i, cf32 v) const
    {
        st_stream(y + t * P::N + i, v);
    }

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count, int tid) const
    {
        using S = Staged<G, P::N>;
        cf32 val[S::kSteps];
        S::each(count, tid, [&](int k, int u, int i, bool valid) {
            val[k] = valid ? sample<P>(first + u, i) : czero();
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
        cf32* dst = y + first * P::N;
        S::each(count, tid, [&](int, int u, int i, bool valid) {
            if (valid) {
                st_stream(dst + u * P::N + i, lds[u * P::kStride + pad(i)]);
            }
        });
    }
};

// The FIR's filter spectrum h: one transform of N points whose input i is tap i (real float32 or
// complex64), zero from i = taps on. The reference builds it with torch ops around its FFT
// (python/spectral/rf.py:145-147: zeros, a copy of the converted taps, fft); this is one launch.
struct TapsIo {
    static constexpr bool kGroupIsBlock = false;
    const void* taps;
    bool complex_taps;
    int count;
    cf32* h;

    template <class P>
    static constexpr bool direct_in() { return P::L >= 16; }
    template <class P>
    static constexpr bool direct_out() { return P::L >= 16; }

    template <class P>
    __device__ __forceinline__ cf32 in(long long, int i) const
    {
        if (i >= count) {
            return czero();
        }
        return complex_taps ? static_cast<const cf32*>(taps)[i]
                            : cf32{static_cast<const float*>(taps)[i], 0.0f};
    }

    template <class P>
    __device__ __forceinline__ void out(long long, int i, cf32 v) const
    {
        h[i] = v;
    }

    template <class P, class G>
    __device__ __forceinline__ void load(cf32* lds, long long first, int count_, int tid) const
    {
        using S = Staged<G, P::N>;
        S::each(count_, tid, [&](int, int u, int i, bool valid) {
            if (valid) {
                lds[u * P::kStride + pad(i)] = in<P>(first + u, i);
            }
        });
    }

    template <class P, class G>
    __device__ __forceinline__ void store(cf32* lds, long long, int count_, int tid) const
    {
        using S = Staged<G, P::N>;
        S::each(count_, tid, [&](int, int u, int i, bool valid) {
            if (valid) {
                h[i] = lds[u * P::kStride + pad(i)];
            }
        });
    }
};

// Overlap-save blocks: transform t = row * blocks + b.
template <class P, bool Table>
__global__ void __launch_bounds__(P::kThreads)
    fir_kernel(const cf32* __restrict__ x, const cf32* __restrict__ h, cf32* __restrict__ y,
               long long n, int taps, int step, long long blocks, long long transforms,
               const cf32* table)
{
    static_assert(slots_match<P>(), "the forward outputs must be the inverse inputs");
    __shared__ cf32 lds[P::T * P::kStride];
    const int tid = threadIdx.x;
    const int u = tid / P::L;
    const int lane = tid % P::L;
    const long long t = static_cast<long long>(blockIdx.x) * P::T + u;
    const bool valid = t < transforms;
    const long long row = valid ? t / blocks : 0;
    const long long b = valid ? t - row * blocks : 0;
    const long long start = b * step - (taps - 1);  // signal index of segment element 0
    const cf32* const xr = x + row * n;
    cf32* const s = lds + u * P::kStride;

    constexpr int R0 = P::template radix<0>();
    cf32 v[P::E];
#pragma unroll
    for (int bb = 0; bb < P::E / R0; ++bb) {
#pragma unroll
        for (int r = 0; r < R0; ++r) {
            const long long j = start + input_index<P, 0>(lane, bb, r);
            v[bb * R0 + r] = (valid && j >= 0 && j < n) ? ld_stream(xr + j) : czero();
        }
    }
    run_stages<P, 0, false, Table>(v, s, lane, table);

    // Spectrum product, scaled by 1 / nfft, into the inverse's input slots.
    constexpr int RL = P::template radix<P::kStages - 1>();
    constexpr float kInv = 1.0f / static_cast<float>(P::N);
    cf32 w[P::E];
    static_for<0, P::E>([&](auto ei) {
        constexpr int e = decltype(ei)::value;
        const int k = lane + (e / RL) * P::L + (e % RL) * (P::N / RL);
        w[forward_slot_of<P>(e)] = cscale(cmul(v[e], h[k]), kInv);
    });
    run_stages<P, 0, true, Table>(w, s, lane, table);

    if (valid) {
#pragma unroll
        for (int bb = 0; bb < P::E / RL; ++bb) {
#pragma unroll
            for (int r = 0; r < RL; ++r) {
                const int i = lane + bb * P::L + r * (P::N / RL);
                const long long j = start + i;  // output index: b step + i - (taps - 1)
                if (i >= taps - 1 && j < n) {
                    st_stream(y + row * n + j, w[bb * RL + r]);
                }
            }
        }
    }
}

template <class P, bool Table>
void launch_fir(const cf32* x, const cf32* h, cf32* y, long long n, int taps, int step,
                long long blocks, long long transforms, const cf32* table, hipStream_t stream)
{
    const long long grid = (transforms + P::T - 1) / P::T;
    hipLaunchKernelGGL((fir_kernel<P, Table>), dim3(static_cast<unsigned>(grid)),
                       dim3(P::kThreads), 0, stream, x, h, y, n, taps, step, blocks, transforms,
                       table);
    SPX_LAUNCH_CHECK();
}

}  // namespace spx::dev
