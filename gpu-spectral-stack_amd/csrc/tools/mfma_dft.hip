// spectral_mfma_dft: the column pass of BASELINE C4's pruned forward transform (2048 arrays of
// 128 rows x 16 kept columns in, rows of frequency 0 .. 15 and -16 .. -1 out) computed two ways on
// one MI355X from the same input, to decide whether the fp32 matrix cores pay for the pruned
// transform:
//
//   fft    the library's pruned strided column kernel (spx_pruned_columns, stockham_r8):
//          128-point FFTs down each column, only the kept rows stored
//   mfma   the DFT as a matrix product on the matrix cores in fp32 (no narrowing): per array
//          Z (32 x 16 complex) = H (32 x 128 complex, the DFT rows of the kept frequencies)
//          times Y (128 x 16 complex), as the real product
//          [Zr | Zi] = Hr [Yr | Yi] + Hi [-Yi | Yr], one 32 x 32 tile per wavefront, K = 2 x 128,
//          128 v_mfma_f32_32x32x2_f32 per array; H from a 128-entry twiddle table in LDS
//
// The two must agree to the transforms' tolerance; each is timed as the median of 5 rounds of 20
// launches rotating over 3 buffer sets (the rows say µs per launch and GB/s of the 40 MiB each
// moves). A third row times the mfma kernel on one L2-resident array for every wavefront: its
// arithmetic alone.
//
//   spectral_mfma_dft [--arrays N]

#include "spectral_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#define CHECK(expr)                                                                        \
    do {                                                                                   \
        const hipError_t e_ = (expr);                                                      \
        if (e_ != hipSuccess) {                                                            \
            std::fprintf(stderr, "%s failed: %s\n", #expr, hipGetErrorString(e_));         \
            std::exit(1);                                                                  \
        }                                                                                  \
    } while (0)

namespace {

constexpr int kN = 128;      // column length
constexpr int kCols = 16;    // kept columns
constexpr int kKept = 32;    // kept rows: frequencies 0 .. 15 and -16 .. -1
constexpr int kWaves = 4;    // arrays (wavefronts) per workgroup

struct cf {
    float re;
    float im;
};

using f32x16 = float __attribute__((ext_vector_type(16)));

// One wavefront per array. Lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32] of each
// 32 x 2 by 2 x 32 step and receives D[8 (v / 4) + 4 (l / 32) + v % 4][l % 32] in accumulator v.
// array_stride 0 makes every wavefront read array 0 (the arithmetic alone, from L2).
__global__ void __launch_bounds__(64 * kWaves)
    mfma_columns(const cf* __restrict__ y, cf* __restrict__ z, int arrays, int array_stride)
{
    __shared__ cf tw[kN];  // exp(-2 pi i t / 128)
    if (threadIdx.x < kN) {
        float s = 0.0f;
        float c = 0.0f;
        sincospif(-2.0f * static_cast<float>(threadIdx.x) / kN, &s, &c);
        tw[threadIdx.x] = cf{c, s};
    }
    __syncthreads();
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int array = static_cast<int>(blockIdx.x) * kWaves + (static_cast<int>(threadIdx.x) >> 6);
    if (array >= arrays) {
        return;  // no barrier follows
    }
    const cf* ya = y + static_cast<long long>(array) * array_stride * kN * kCols;
    const int r = lane & 31;             // row of H this lane supplies, column of B
    const int kk = lane >> 5;            // k within a step of 2
    const int f = r < 16 ? r : r - 32;   // frequency of kept row r
    const int col = lane & 15;           // Y column behind B column r
    const bool real_half = r < 16;
    f32x16 acc = {};
#pragma unroll 8
    for (int y0 = 0; y0 < kN; y0 += 2) {
        const int yy = y0 + kk;
        const cf h = tw[(f * yy) & (kN - 1)];
        const cf v = ya[yy * kCols + col];
        const float b1 = real_half ? v.re : v.im;
        const float b2 = real_half ? -v.im : v.re;
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(h.re, b1, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(h.im, b2, acc, 0, 0, 0);
    }
    // D columns 0 .. 15: real parts of Z's columns; 16 .. 31: imaginary parts.
    float* za = reinterpret_cast<float*>(z + static_cast<long long>(array) * kKept * kCols);
    const int j = lane & 31;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int i = 8 * (v / 4) + 4 * (lane >> 5) + (v & 3);
        za[(i * kCols + (j & 15)) * 2 + (j >> 4)] = acc[v];
    }
}

float median(std::vector<float> v)
{
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

template <class Launch>
float time_us(Launch&& launch, hipStream_t stream)
{
    hipEvent_t a;
    hipEvent_t b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    for (int i = 0; i < 3; ++i) {
        launch(i % 3);
    }
    std::vector<float> rounds;
    for (int round = 0; round < 5; ++round) {
        CHECK(hipEventRecord(a, stream));
        for (int i = 0; i < 20; ++i) {
            launch(i % 3);
        }
        CHECK(hipEventRecord(b, stream));
        CHECK(hipEventSynchronize(b));
        float ms = 0.0f;
        CHECK(hipEventElapsedTime(&ms, a, b));
        rounds.push_back(ms * 1000.0f / 20.0f);
    }
    CHECK(hipEventDestroy(a));
    CHECK(hipEventDestroy(b));
    return median(rounds);
}

}  // namespace

int main(int argc, char** argv)
{
    int arrays = 2048;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--arrays" && i + 1 < argc) {
            arrays = std::atoi(argv[++i]);
        } else {
            std::fprintf(stderr, "usage: spectral_mfma_dft [--arrays N]\n");
            return 2;
        }
    }
    if (arrays < 1 || arrays > (1 << 20)) {
        std::fprintf(stderr, "spectral_mfma_dft: --arrays must be in [1, 2^20]\n");
        return 2;
    }
    const int impl = spx_impl_find("stockham_r8");
    const std::size_t in_values = static_cast<std::size_t>(arrays) * kN * kCols;
    const std::size_t out_values = static_cast<std::size_t>(arrays) * kKept * kCols;

    std::vector<cf> host(in_values);
    unsigned state = 12345u;
    for (cf& v : host) {
        state = state * 1664525u + 1013904223u;
        v.re = static_cast<float>(state >> 8) / 16777216.0f - 0.5f;
        state = state * 1664525u + 1013904223u;
        v.im = static_cast<float>(state >> 8) / 16777216.0f - 0.5f;
    }
    cf* in[3];
    cf* out_fft[3];
    cf* out_mfma[3];
    for (int s = 0; s < 3; ++s) {
        CHECK(hipMalloc(&in[s], in_values * sizeof(cf)));
        CHECK(hipMalloc(&out_fft[s], out_values * sizeof(cf)));
        CHECK(hipMalloc(&out_mfma[s], out_values * sizeof(cf)));
        CHECK(hipMemcpy(in[s], host.data(), in_values * sizeof(cf), hipMemcpyHostToDevice));
    }
    hipStream_t stream;
    CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    const unsigned blocks = static_cast<unsigned>((arrays + kWaves - 1) / kWaves);

    auto fft = [&](int s) {
        if (spx_pruned_columns(impl, in[s], out_fft[s], kN, kCols, arrays, 0, kKept / 2, 0,
                               stream) != SPX_OK) {
            std::fprintf(stderr, "spx_pruned_columns: %s\n", spx_last_error());
            std::exit(1);
        }
    };
    auto mfma = [&](int s) {
        hipLaunchKernelGGL(mfma_columns, dim3(blocks), dim3(64 * kWaves), 0, stream, in[s],
                           out_mfma[s], arrays, 1);
    };
    auto mfma_resident = [&](int s) {
        hipLaunchKernelGGL(mfma_columns, dim3(blocks), dim3(64 * kWaves), 0, stream, in[s],
                           out_mfma[s], arrays, 0);
    };

    // Agreement, array by array, on set 0.
    fft(0);
    mfma(0);
    CHECK(hipStreamSynchronize(stream));
    std::vector<cf> a(out_values);
    std::vector<cf> b(out_values);
    CHECK(hipMemcpy(a.data(), out_fft[0], out_values * sizeof(cf), hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(b.data(), out_mfma[0], out_values * sizeof(cf), hipMemcpyDeviceToHost));
    double worst = 0.0;
    for (int t = 0; t < arrays; ++t) {
        double num = 0.0;
        double den = 0.0;
        for (int e = 0; e < kKept * kCols; ++e) {
            const cf& p = a[static_cast<std::size_t>(t) * kKept * kCols + e];
            const cf& q = b[static_cast<std::size_t>(t) * kKept * kCols + e];
            num += (p.re - q.re) * (p.re - q.re) + (p.im - q.im) * (p.im - q.im);
            den += static_cast<double>(p.re) * p.re + static_cast<double>(p.im) * p.im;
        }
        worst = std::max(worst, std::sqrt(num / std::max(den, 1e-300)));
    }
    // Two float32 results of a 128-point transform: each within 8 eps log2 N of the exact one.
    const double tol = 2.0 * 8.0 * std::ldexp(1.0, -23) * 7.0;
    std::printf("# agreement: worst relative L2 difference per array %.3g (bound %.3g): %s\n",
                worst, tol, worst <= tol ? "ok" : "MISMATCH");

    const double bytes = static_cast<double>(in_values + out_values) * sizeof(cf);
    const double mfma_flops = static_cast<double>(arrays) * kKept * 32.0 * 2.0 * kN * 2.0;
    const float t_fft = time_us(fft, stream);
    const float t_mfma = time_us(mfma, stream);
    const float t_res = time_us(mfma_resident, stream);
    std::printf("variant,arrays,us,gbps,tflops\n");
    std::printf("fft_pruned_columns,%d,%.2f,%.1f,\n", arrays, t_fft, bytes / (t_fft * 1e3));
    std::printf("mfma_dft_f32,%d,%.2f,%.1f,%.1f\n", arrays, t_mfma, bytes / (t_mfma * 1e3),
                mfma_flops / (t_mfma * 1e6));
    std::printf("mfma_dft_f32_l2_resident,%d,%.2f,,%.1f\n", arrays, t_res,
                mfma_flops / (t_res * 1e6));
    CHECK(hipDeviceSynchronize());
    return worst <= tol ? 0 : 1;
}
