// One pseudo-spectral Navier-Stokes stage per field in one kernel: the whole nonlinear term of the
// vorticity equation and the IMEX update, for the pruned (FNO) layout, with every intermediate in
// LDS and registers. This is the MI355X form of the reference's GpuSolver.tendency / step
// (python/spectral/flow/gpu.py:115-129), which runs one batched inverse transform of four fields,
// a product, a forward transform and about fifteen elementwise kernels through HBM per tendency.
// ns_steps_kernel runs the same stage body for many steps per launch (a field's steps depend only
// on that field), in place of the reference's one Python-driven step per call
// (python/spectral/flow/gpu.py:125-142).
//
// State: omega_hat on the 2/3-rule modes in the layout of rfft2_truncated with m = n/3 + 1 (rows
// ky = 0 .. m-1 then -m .. -1, columns kx = 0 .. m-1), (2m) x m complex values per field.
//
// Per field (one workgroup; one lane group per grid row, and per column in the column phases):
//   nonlinear term N = u wx + v wy with u = i ky psi_hat, v = -i kx psi_hat, wx = i kx omega_hat,
//   wy = i ky omega_hat (psi_hat = omega_hat / |k|^2), two real fields per complex transform:
//     for each pair (A, B) = (u, wx), then (v, wy):
//       columns: the inverse column transforms of A's and B's m kept columns into the tile T
//                (2m of the n column slots, one pass)
//       rows:    per grid row ONE n-point complex inverse of Z = A + i B: for real A and B the
//                row spectrum of Z is A~ + i B~ at kx >= 0 and conj(A~) + i conj(B~) at -kx, and
//                A B = Re z Im z in registers
//   forward: per row the n-point complex transform of N (imaginary part zero), its first m bins
//   into T; then the m forward column transforms, and the epilogue on the kept modes:
//           F = f_hat - mask N_hat, and the IMEX update
//             stage 0: out_f = F, out_w = w* = (e w + dt F) i
//             stage 1: out_w = w' = (e w + dt/2 (f0 + F)) i
//           with e = 1 + dt/2 L, i = 1 / (1 - dt/2 L), L = -nu |k|^2 - alpha.
// The state is read from global memory (L2 after the first column pass), so the LDS holds only
// the tile, and each row group uses its own tile row as exchange scratch.
// Normalization: inverse 1 / n^2 over the column and row passes, forward none, as numpy.
//
// Measured on MI355X (n = 128, 256 fields, one stage): 31.2 us for the field-at-a-time form
// (four inverse column and four real row phases), 26.2 us with the fields paired, 18.8 us with
// the tile below free of bank conflicts (62 % of LDS cycles were conflicts). The stage is bound
// by the latency of its chain of dependent phases: one workgroup per CU (146 KB of LDS; the
// batch equals the CU count) with a barrier between phases. Not by VALU issue: a timing-only
// build without the stage twiddle work, a large share of the VALU instructions, ran 1.2 %
// faster.

#include "stockham.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace spx {
namespace dev {
namespace {

__device__ __forceinline__ cf32 mul_ik(float k, cf32 z) { return {-k * z.im, k * z.re}; }

// Kept-mode row of full-spectrum row i (0 .. N-1), or -1 when that row is not kept.
template <class NP>
__device__ __forceinline__ int mode_row(int i)
{
    if (i < NP::m) {
        return i;
    }
    if (i >= NP::N - NP::m) {
        return i - NP::N + 2 * NP::m;
    }
    return -1;
}

template <class NP>
__device__ __forceinline__ float ky_of_mode_row(int r)
{
    return static_cast<float>(r < NP::m ? r : r - 2 * NP::m);
}

// Tile layout, free of LDS bank conflicts (64 banks of 4 bytes, 8-byte accesses served a
// half-wave at a time): grid row y sits in tile row pad(y) (one spare row after every 16), tile
// rows are RS = 8 mod 32 values apart, and a column's lanes are spread over the wave (lane j of
// the column group takes the wave's lanes j kPerWave + 0 .. kPerWave - 1, one per column). A
// half-wave then touches 64 distinct banks in every row and column phase, where odd strides and
// contiguous column groups measured 62 % of LDS cycles in conflicts.
template <int N_, int R, int E>
struct NsPairPlan {
    static constexpr int N = N_;
    static constexpr int m = N / 3 + 1;              // kept modes per axis
    static constexpr int rows = 2 * m;                // kept rows
    using PX = Plan<N, R, E>;                         // rows and columns: N-point complex
    static constexpr int NT = N * PX::L;              // one lane group per grid row
    static constexpr int kTileRows = pad(N - 1) + 1;  // grid row y in tile row pad(y)
    static constexpr int RS = ((kTileRows + 23) / 32) * 32 + 8;  // >= a padded row, 8 mod 32
    static constexpr int kLds = kTileRows * RS;
    static constexpr int kW = rows * m;
    static constexpr int kPerWave = 64 / PX::L;       // column groups per wave

    static_assert(PX::L <= 64 && 64 % PX::L == 0, "a row's or a column's lanes in one wave");
    static_assert(RS >= pad(N - 1) + 1 && RS % 32 == 8, "tile row stride");
    static_assert(NT <= 1024, "one workgroup");
    static_assert(NT / PX::L >= 2 * m && RS >= 2 * m, "both fields' columns in one pass");
    static_assert(slots_match<PX>(), "inverse outputs must be forward inputs");
    static_assert(kLds * sizeof(cf32) <= 160 * 1024, "LDS budget");
};

// Column slot and lane of a column phase: the wave's lanes interleave its kPerWave columns.
template <class NP>
__device__ __forceinline__ int column_slot(int tid)
{
    return (tid / 64) * NP::kPerWave + tid % NP::kPerWave;
}
template <class NP>
__device__ __forceinline__ int column_lane(int tid)
{
    return (tid % 64) / NP::kPerWave;
}

// Inverse column transforms of the pair's two derived fields into tile columns 0 .. m-1 (first)
// and m .. 2m-1 (second).
template <class NP>
__device__ __forceinline__ void pair_columns(const cf32* __restrict__ w, cf32* T, int pair,
                                             int tid)
{
    using PX = typename NP::PX;
    using Lay = PaddedRows<NP::RS>;
    constexpr int R0 = PX::template radix<0>();
    const int slot = column_slot<NP>(tid);
    const int lane = column_lane<NP>(tid);
    if (slot < 2 * NP::m) {
        // Derived field d = i f w with a real multiplier f per mode: u = i (ky / k^2) w,
        // wx = i kx w (pair 0); v = i (-kx / k^2) w, wy = i ky w (pair 1).
        const bool second = slot >= NP::m;
        const int c = second ? slot - NP::m : slot;
        const float kx = static_cast<float>(c);
        const bool on_ky = (pair == 0) != second;  // u and wy take ky, wx and v take kx
        const bool by_k2 = !second;                // u and v divide by |k|^2
        const float sign = (pair == 1 && !second) ? -1.0f : 1.0f;
        cf32 v[PX::E];
#pragma unroll
        for (int b = 0; b < PX::E / R0; ++b) {
#pragma unroll
            for (int r = 0; r < R0; ++r) {
                const int mr = mode_row<NP>(input_index<PX, 0>(lane, b, r));
                cf32 d = czero();
                if (mr >= 0) {
                    const cf32 wv = w[mr * NP::m + c];
                    const float ky = ky_of_mode_row<NP>(mr);
                    const float k2 = kx * kx + ky * ky;
                    float f = sign * (on_ky ? ky : kx);
                    if (by_k2) {
                        f = k2 > 0.0f ? f * __builtin_amdgcn_rcpf(k2) : 0.0f;
                    }
                    d = mul_ik(f, wv);
                }
                v[b * R0 + r] = d;
            }
        }
        cf32* const s = T + slot;
        run_stages<PX, 0, true, false, Lay>(v, s, lane, nullptr);
        lds_sync<true>();
        final_write<PX, Lay>(s, v, lane);
    }
}

// Grid row y's inverse of Z = A + i B from its tile row (A~ in columns 0 .. m-1, B~ in
// m .. 2m-1), scaled by `scale`: on return v holds z at the last stage's slots. The DC bins'
// imaginary parts are dropped (numpy's irfft does the same). The tile row is the exchange
// scratch: run_stages waits for the row group's reads before its first write.
template <class NP>
__device__ __forceinline__ void pair_row_inverse(cf32* row, cf32 (&v)[NP::PX::E], int lane,
                                                 float scale)
{
    using PX = typename NP::PX;
    constexpr int R0 = PX::template radix<0>();
    static_for<0, PX::E>([&](auto ei) {
        constexpr int e = decltype(ei)::value;
        constexpr int off = (e / R0) * PX::L + (e % R0) * (PX::N / R0);
        const int k = lane + off;
        cf32 z = czero();
        if (k < NP::m) {
            cf32 a = row[k];
            cf32 b = row[NP::m + k];
            if (k == 0) {
                a.im = 0.0f;
                b.im = 0.0f;
            }
            z = cf32{a.re - b.im, a.im + b.re};
        } else if (k > NP::N - NP::m) {
            const cf32 a = row[NP::N - k];
            const cf32 b = row[NP::m + NP::N - k];
            z = cf32{a.re + b.im, b.re - a.im};
        }
        v[e] = cscale(z, scale);
    });
    run_stages<PX, 0, true, false>(v, row, lane, nullptr);
}

// One stage of one field (the workgroup's), on the tile T. The arrays hold every field's modes;
// `field` picks this workgroup's. out_f and out_w may overwrite state, w0 or f0 (the C ABI allows
// it): every read of the state happens before the barrier that ends the transforms, and the
// epilogue loads all the values a lane updates before it stores any, so those pointers are not
// restrict. Every lane of the workgroup calls this; it starts by writing T. InLoop: the caller
// runs stages in a loop (below).
template <class NP, bool InLoop>
__device__ __forceinline__ void ns_stage_body(cf32* T, long long field, const cf32* state,
                                              const cf32* w0, const cf32* f0, cf32* out_f,
                                              cf32* out_w, const cf32* __restrict__ forcing_hat,
                                              float nu_f, float drag, float dt, int stage)
{
    using PX = typename NP::PX;
    // In a loop, the lane index is made opaque to the optimizer, so that each stage recomputes
    // the lane's indices and twiddles instead of keeping them live across the loop (which spilled
    // 137 registers at n = 128).
    int tid = threadIdx.x;
    if constexpr (InLoop) {
        asm volatile("" : "+v"(tid));
    }
    const long long base = field * NP::kW;
    const cf32* const w = state + base;
    const int lane = tid % PX::L;
    cf32* const row = T + pad(tid / PX::L) * NP::RS;  // this lane group's grid row
    constexpr float kScale = 1.0f / (static_cast<float>(NP::N) * static_cast<float>(NP::N));

    // u wx + v wy: per pair, both fields' columns into T, then each row's packed inverse.
    // Both pairs unrolled (the pair then known at compile time): 121 VGPRs and no spills at
    // n = 128, where the loop kept at run time spilled 32 bytes per lane.
    float nl[PX::E];
#pragma unroll
    for (int pair = 0; pair < 2; ++pair) {
        pair_columns<NP>(w, T, pair, tid);
        __syncthreads();
        cf32 v[PX::E];
        pair_row_inverse<NP>(row, v, lane, kScale);
#pragma unroll
        for (int e = 0; e < PX::E; ++e) {
            const float p = v[e].re * v[e].im;
            nl[e] = pair == 0 ? p : nl[e] + p;
        }
        __syncthreads();  // every row group is done with its tile row before the next columns
    }

    // Forward row transforms of the product, the first m bins into the tile row.
    {
        cf32 v[PX::E];
        static_for<0, PX::E>([&](auto ei) {
            constexpr int e = decltype(ei)::value;
            v[forward_slot_of<PX>(e)] = cf32{nl[e], 0.0f};
        });
        run_stages<PX, 0, false, false>(v, row, lane, nullptr);
        lds_sync<true>();  // the row group's last exchange reads are done
        constexpr int RL = PX::template radix<PX::kStages - 1>();
        static_for<0, PX::E>([&](auto ei) {
            constexpr int e = decltype(ei)::value;
            const int k = lane + (e / RL) * PX::L + (e % RL) * (PX::N / RL);
            if (k < NP::m) {
                row[k] = v[e];
            }
        });
    }
    __syncthreads();

    // Forward columns of the product's row spectra, in place in T.
    {
        using Lay = PaddedRows<NP::RS>;
        const int c = column_slot<NP>(tid);
        const int clane = column_lane<NP>(tid);
        if (c < NP::m) {
            cf32* const col = T + c;
            cf32 v[PX::E];
            stage_read<PX, 0, Lay>(col, v, clane);
            run_stages<PX, 0, false, false, Lay>(v, col, clane, nullptr);
            lds_sync<true>();
            final_write<PX, Lay>(col, v, clane);
        }
    }
    __syncthreads();

    // Epilogue on the kept modes: every global value a lane reads is loaded before its stores.
    constexpr int kIters = (NP::kW + NP::NT - 1) / NP::NT;
    const float kmax = static_cast<float>(NP::N) / 3.0f;
    cf32 fh[kIters];
    cf32 wv[kIters];
    cf32 fv[kIters];
#pragma unroll
    for (int q = 0; q < kIters; ++q) {
        const int e = tid + q * NP::NT;
        if (e < NP::kW) {
            fh[q] = forcing_hat[e];
            wv[q] = stage == 0 ? w[e] : w0[base + e];
            fv[q] = stage == 0 ? czero() : f0[base + e];
        }
    }
#pragma unroll
    for (int q = 0; q < kIters; ++q) {
        const int e = tid + q * NP::NT;
        if (e < NP::kW) {
            const int r = e / NP::m;
            const int c = e - r * NP::m;
            const float ky = ky_of_mode_row<NP>(r);
            const float kx = static_cast<float>(c);
            const int i = r < NP::m ? r : r - 2 * NP::m + NP::N;
            const bool kept = fabsf(kx) <= kmax && fabsf(ky) <= kmax;
            const cf32 nlh = kept ? T[pad(i) * NP::RS + c] : czero();
            const cf32 F = csub(fh[q], nlh);
            const float linear = -nu_f * (kx * kx + ky * ky) - drag;
            const float ex = 1.0f + 0.5f * dt * linear;
            const float im = 1.0f / (1.0f - 0.5f * dt * linear);
            if (stage == 0) {
                out_f[base + e] = F;
                out_w[base + e] = cscale(cadd(cscale(wv[q], ex), cscale(F, dt)), im);
            } else {
                const cf32 sum = cadd(fv[q], F);
                out_w[base + e] = cscale(cadd(cscale(wv[q], ex), cscale(sum, 0.5f * dt)), im);
            }
        }
    }
}

template <class NP>
__global__ void __launch_bounds__(NP::NT)
    ns_stage_kernel(const cf32* state, const cf32* w0, const cf32* f0, cf32* out_f, cf32* out_w,
                    const cf32* __restrict__ forcing_hat, const float* __restrict__ nu,
                    int nu_stride, float drag, float dt, int stage)
{
    __shared__ cf32 T[NP::kLds];
    const long long field = blockIdx.x;
    ns_stage_body<NP, false>(T, field, state, w0, f0, out_f, out_w, forcing_hat,
                             nu[field * nu_stride], drag, dt, stage);
}

// `steps` whole steps (predictor, then corrector) per field in one launch: the first step reads
// w_in and writes w_out, the later ones advance w_out in place (w_in may be w_out), and each
// step's tendency and predictor go to the field's two slots of `work`. A
// workgroup only ever reads what it wrote itself, so a barrier between the stages orders the
// global accesses (the waves share the CU's L1), and the field's three arrays stay in its
// XCD's L2 from one stage to the next, where separate launches write them back to HBM at the end
// of each stage and read them again at the start of the next.
template <class NP>
__global__ void __launch_bounds__(NP::NT)
    ns_steps_kernel(const cf32* w_in, cf32* w_out, cf32* work,
                    const cf32* __restrict__ forcing_hat, const float* __restrict__ nu,
                    int nu_stride, float drag, float dt, int steps)
{
    __shared__ cf32 T[NP::kLds];
    const long long field = blockIdx.x;
    cf32* const tendency = work;
    cf32* const predicted = work + static_cast<long long>(gridDim.x) * NP::kW;
    const float nu_f = nu[field * nu_stride];
    for (int s = 0; s < steps; ++s) {
        const cf32* const state = s == 0 ? w_in : w_out;
        ns_stage_body<NP, true>(T, field, state, nullptr, nullptr, tendency, predicted,
                                forcing_hat, nu_f, drag, dt, 0);
        __syncthreads();  // the predictor and tendency are written; T is free
        ns_stage_body<NP, true>(T, field, predicted, state, tendency, nullptr, w_out,
                                forcing_hat, nu_f, drag, dt, 1);
        __syncthreads();  // the new state is written; T is free
    }
}

template <int N>
void launch(const cf32* state, const cf32* w0, const cf32* f0, cf32* out_f, cf32* out_w,
            const cf32* forcing_hat, const float* nu, int nu_stride, float drag, float dt,
            int batch, int stage, hipStream_t stream)
{
    // n = 128: radix 16 then 8, 16 values per lane (1024 lanes); n = 64: radix 8 twice, 8 values
    // per lane (512 lanes). Both are two-stage transforms, one LDS exchange each.
    using NP = std::conditional_t<N == 64, NsPairPlan<64, 8, 8>, NsPairPlan<N, 16, 16>>;
    hipLaunchKernelGGL(ns_stage_kernel<NP>, dim3(static_cast<unsigned>(batch)), dim3(NP::NT), 0,
                       stream, state, w0, f0, out_f, out_w, forcing_hat, nu, nu_stride, drag, dt,
                       stage);
    SPX_LAUNCH_CHECK();
}

template <int N>
void launch_steps(const cf32* w_in, cf32* w_out, cf32* work, const cf32* forcing_hat,
                  const float* nu, int nu_stride, float drag, float dt, int batch, int steps,
                  hipStream_t stream)
{
    using NP = std::conditional_t<N == 64, NsPairPlan<64, 8, 8>, NsPairPlan<N, 16, 16>>;
    hipLaunchKernelGGL(ns_steps_kernel<NP>, dim3(static_cast<unsigned>(batch)), dim3(NP::NT), 0,
                       stream, w_in, w_out, work, forcing_hat, nu, nu_stride, drag, dt, steps);
    SPX_LAUNCH_CHECK();
}

}  // namespace
}  // namespace dev

bool ns_supports(int n) { return n == 64 || n == 128; }

void ns_stage(const cf32* state, const cf32* w0, const cf32* f0, cf32* out_f, cf32* out_w,
              const cf32* forcing_hat, const float* nu, int nu_stride, float drag, float dt,
              int n, int batch, int stage, hipStream_t stream)
{
    if (!ns_supports(n)) {
        throw InvalidArgument("ns_stage: the fused Navier-Stokes stage supports n = 64 and 128, "
                              "got " + str(n));
    }
    if (batch < 1 || (stage != 0 && stage != 1) || (nu_stride != 0 && nu_stride != 1)) {
        throw InvalidArgument("ns_stage: need batch >= 1, stage 0 or 1, nu_stride 0 or 1");
    }
    if (stage == 0 && (out_f == nullptr || out_w == nullptr)) {
        throw InvalidArgument("ns_stage: stage 0 writes both the tendency and the predictor");
    }
    if (stage == 1 && (w0 == nullptr || f0 == nullptr || out_w == nullptr)) {
        throw InvalidArgument("ns_stage: stage 1 reads w and f0 and writes the corrected state");
    }
    if (n == 64) {
        dev::launch<64>(state, w0, f0, out_f, out_w, forcing_hat, nu, nu_stride, drag, dt, batch,
                        stage, stream);
    } else {
        dev::launch<128>(state, w0, f0, out_f, out_w, forcing_hat, nu, nu_stride, drag, dt,
                         batch, stage, stream);
    }
}

void ns_steps(const cf32* w_in, cf32* w_out, cf32* work, const cf32* forcing_hat,
              const float* nu, int nu_stride, float drag, float dt, int n, int batch, int steps,
              hipStream_t stream)
{
    if (!ns_supports(n)) {
        throw InvalidArgument("ns_steps: the fused Navier-Stokes stage supports n = 64 and 128, "
                              "got " + str(n));
    }
    if (batch < 1 || steps < 0 || (nu_stride != 0 && nu_stride != 1)) {
        throw InvalidArgument("ns_steps: need batch >= 1, steps >= 0, nu_stride 0 or 1");
    }
    if (w_in == nullptr || w_out == nullptr || work == nullptr || forcing_hat == nullptr ||
        nu == nullptr) {
        throw InvalidArgument("ns_steps: w_in, w_out, work, forcing_hat and nu must not be null");
    }
    const auto m = static_cast<std::uintptr_t>(n / 3 + 1);
    const std::uintptr_t bytes = static_cast<std::uintptr_t>(batch) * 2 * m * m * sizeof(cf32);
    const auto in = reinterpret_cast<std::uintptr_t>(w_in);
    const auto out = reinterpret_cast<std::uintptr_t>(w_out);
    const auto wk = reinterpret_cast<std::uintptr_t>(work);
    const auto overlap = [](std::uintptr_t a, std::uintptr_t a_bytes, std::uintptr_t b,
                            std::uintptr_t b_bytes) { return a < b + b_bytes && b < a + a_bytes; };
    if (overlap(wk, 2 * bytes, in, bytes) || overlap(wk, 2 * bytes, out, bytes)) {
        throw InvalidArgument("ns_steps: work must not overlap w_in or w_out");
    }
    if (in != out && overlap(in, bytes, out, bytes)) {
        throw InvalidArgument("ns_steps: w_in and w_out must be the same array or not overlap");
    }
    if (steps == 0) {
        if (in != out) {
            SPX_HIP_CHECK(hipMemcpyAsync(w_out, w_in, bytes, hipMemcpyDeviceToDevice, stream));
        }
        return;
    }
    if (n == 64) {
        dev::launch_steps<64>(w_in, w_out, work, forcing_hat, nu, nu_stride, drag, dt, batch,
                              steps, stream);
    } else {
        dev::launch_steps<128>(w_in, w_out, work, forcing_hat, nu, nu_stride, drag, dt, batch,
                               steps, stream);
    }
}

}  // namespace spx
