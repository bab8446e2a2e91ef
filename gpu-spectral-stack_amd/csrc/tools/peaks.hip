// spectral_peaks: the two ceilings of the roofline on this MI355X, measured, as JSON.
//
//   copy_gbps    a streaming copy (dwordx4 loads and stores, bytes read + bytes written) over
//                buffers far larger than the 256 MB Infinity Cache, with the source rotated over
//                several buffer pairs so no launch reads what the previous one left in the cache.
//   fp32_gflops  independent FMA chains, no memory traffic (non-packed VALU FMA: packed FP32 is
//                switched off in every build of this repository).
//
// --patterns times plain copies (no arithmetic) of the HBM access pattern of each pass of the hot
// path, at that pass's size: contiguous rows in 16 KB workgroup chunks (the 1D kernels, the 2D
// row-pair passes), and column tiles of T columns x N rows (the strided column passes). A pass
// cannot stream faster than the copy of its own pattern, so each FFT pass is put against that.
//
// Same role as the reference's csrc/tools/peaks.cu:4-11 (achievable, not datasheet, peaks). The
// copy kernel also serves as the calibration kernel of known size for the rocprof FETCH_SIZE /
// WRITE_SIZE counters: `--copy-only --bytes B --iters K` runs exactly K copies of B bytes.
//
//   spectral_peaks [--copy-only] [--bytes B] [--iters K] [--out FILE]
//   spectral_peaks --patterns

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

#define CHECK(expr)                                                                       \
    do {                                                                                  \
        const hipError_t e_ = (expr);                                                     \
        if (e_ != hipSuccess) {                                                           \
            std::fprintf(stderr, "%s failed: %s (%s:%d)\n", #expr, hipGetErrorString(e_), \
                         __FILE__, __LINE__);                                             \
            std::exit(1);                                                                 \
        }                                                                                 \
    } while (0)

constexpr int kThreads = 256;
constexpr int kVec = 4;  // float4 per lane per step, 64 bytes in flight per lane

// Each lane copies kVec float4 per step, lanes of a wave adjacent (1 KiB runs per load).
__global__ void __launch_bounds__(kThreads)
    copy_kernel(const float4* __restrict__ in, float4* __restrict__ out, std::size_t n)
{
    const std::size_t per_step = static_cast<std::size_t>(gridDim.x) * kThreads * kVec;
    for (std::size_t base = static_cast<std::size_t>(blockIdx.x) * kThreads * kVec + threadIdx.x;
         base < n; base += per_step) {
        float4 v[kVec];
#pragma unroll
        for (int k = 0; k < kVec; ++k) {
            const std::size_t i = base + static_cast<std::size_t>(k) * kThreads;
            if (i < n) {
                v[k] = in[i];
            }
        }
#pragma unroll
        for (int k = 0; k < kVec; ++k) {
            const std::size_t i = base + static_cast<std::size_t>(k) * kThreads;
            if (i < n) {
                out[i] = v[k];
            }
        }
    }
}

typedef float f2v __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ f2v load8(const f2v* p)
{
    if constexpr (NT) {
        return __builtin_nontemporal_load(p);
    } else {
        return *p;
    }
}

template <bool NT>
__device__ __forceinline__ void store8(f2v* p, f2v v)
{
    if constexpr (NT) {
        __builtin_nontemporal_store(v, p);
    } else {
        *p = v;
    }
}

// Contiguous rows: workgroup b copies the Th * V 8-byte values from b Th V, lane t taking values
// t + k Th (runs of 512 bytes per wave access). The grid covers the buffer exactly. NT: both
// accesses nontemporal; StoreNT (default NT): the stores' hint on its own.
template <int Th, int V, bool NT, bool StoreNT = NT>
__global__ void __launch_bounds__(Th) rows_copy_kernel(const f2v* __restrict__ in, f2v* __restrict__ out)
{
    const std::size_t base = static_cast<std::size_t>(blockIdx.x) * Th * V + threadIdx.x;
    f2v v[V];
#pragma unroll
    for (int k = 0; k < V; ++k) {
        v[k] = load8<NT>(in + base + static_cast<std::size_t>(k) * Th);
    }
#pragma unroll
    for (int k = 0; k < V; ++k) {
        store8<StoreNT>(out + base + static_cast<std::size_t>(k) * Th, v[k]);
    }
}

// The same rows with the loads sent straight to LDS (global_load_lds_dwordx4, nontemporal): lane
// k of a wave instruction reads 16 bytes, which land at the wave's LDS base + 16 k. Each wave then
// reads back only what it loaded and stores it as rows_copy_kernel<Th, 8, true> does, 8 bytes per
// lane. Workgroup b moves values b Th 8 .. (b + 1) Th 8 - 1.
template <int Th>
__global__ void __launch_bounds__(Th) rows_lds_dma_kernel(const f2v* __restrict__ in,
                                                        f2v* __restrict__ out)
{
    constexpr int kSteps = 4;           // 16-byte loads per lane
    constexpr int kStep = Th * 2;       // values per workgroup step
    __shared__ f2v lds[kSteps * kStep];  // 16 KB at Th = 256
    const std::size_t base = static_cast<std::size_t>(blockIdx.x) * kSteps * kStep;
    const int wave = threadIdx.x / 64;
    const int l = threadIdx.x % 64;
#pragma unroll
    for (int k = 0; k < kSteps; ++k) {
        const int e = k * kStep + wave * 128;  // the wave's 128 values of this step
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(in + base + e + 2 * l),
                                         (__attribute__((address_space(3))) void*)(lds + e), 16,
                                         0, 2);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < kSteps; ++k) {
        const int e = k * kStep + wave * 128;
        store8<true>(out + base + e + l, lds[e + l]);
        store8<true>(out + base + e + 64 + l, lds[e + 64 + l]);
    }
}

// Uneven mixes: workgroup b reads Th * V contiguous values as rows_copy_kernel does and writes
// Th of them (each lane the sum of its V), or the mirror (Expand: reads Th, writes each V times).
// V = 16 is the byte mix of a pruned 2D transform keeping a sixteenth of its input (C4), V = 2
// that of the real transforms at n = 2 (C2), V = 1 an even copy with plain loads and nontemporal
// stores, as the real transforms access memory.
template <int Th, int V, bool Expand>
__global__ void __launch_bounds__(Th) mix_rows_kernel(const f2v* __restrict__ in, f2v* __restrict__ out)
{
    const std::size_t wide = static_cast<std::size_t>(blockIdx.x) * Th * V + threadIdx.x;
    const std::size_t narrow = static_cast<std::size_t>(blockIdx.x) * Th + threadIdx.x;
    if constexpr (Expand) {
        const f2v v = in[narrow];
#pragma unroll
        for (int k = 0; k < V; ++k) {
            store8<true>(out + wide + static_cast<std::size_t>(k) * Th, v);
        }
    } else {
        f2v v[V];
#pragma unroll
        for (int k = 0; k < V; ++k) {
            v[k] = load8<false>(in + wide + static_cast<std::size_t>(k) * Th);
        }
        f2v sum = v[0];
#pragma unroll
        for (int k = 1; k < V; ++k) {
            sum += v[k];
        }
        store8<true>(out + narrow, sum);
    }
}

// The same 2:1 and 1:2 mixes with one 16-byte access per lane, the way the n = 2 real
// transforms move their rows (a row of two complex values is 16 bytes): Expand reads 8 bytes and
// writes 16, else reads 16 and writes 8. Plain loads, nontemporal stores.
template <int Th, bool Expand>
__global__ void __launch_bounds__(Th) mix16_kernel(const f2v* __restrict__ in, f2v* __restrict__ out)
{
    const std::size_t i = static_cast<std::size_t>(blockIdx.x) * Th + threadIdx.x;
    if constexpr (Expand) {
        const f2v v = in[i];
        __builtin_nontemporal_store(f4v{v.x, v.y, v.y, v.x}, reinterpret_cast<f4v*>(out) + i);
    } else {
        const f4v v = reinterpret_cast<const f4v*>(in)[i];
        store8<true>(out + i, f2v{v.x + v.z, v.y + v.w});
    }
}

// Column tiles: arrays of Rows x Cols 8-byte values; workgroup b copies the tile of T neighbouring
// columns x Rows rows (tile b mod Cols / T of array b / (Cols / T)), lane t taking column t mod T
// and rows t / T + k Th / T: runs of T * 8 bytes, one per row, Cols * 8 bytes apart.
// Side picks the layout of each end: 0 both row-major (the strided column pass in place), 1 the
// output tile-major, 2 the input tile-major. Tile-major stores each tile's Rows x T values as one
// contiguous block (array, tile, row, column in tile), so that end of the copy is contiguous.
template <int Rows, int Cols, int T, int Th, bool NT, int Side = 0>
__global__ void __launch_bounds__(Th) tiles_copy_kernel(const f2v* __restrict__ in, f2v* __restrict__ out)
{
    constexpr int kTiles = Cols / T;
    constexpr int kStep = Th / T;
    constexpr int kK = Rows / kStep;
    static_assert(Cols % T == 0 && Th % T == 0 && Rows % kStep == 0, "tile shape");
    const std::size_t array = blockIdx.x / kTiles;
    const int tile = static_cast<int>(blockIdx.x % kTiles);
    const int col = tile * T + static_cast<int>(threadIdx.x) % T;
    const int row = static_cast<int>(threadIdx.x) / T;
    const std::size_t base = array * Rows * Cols + col + static_cast<std::size_t>(row) * Cols;
    const std::size_t tiled = array * Rows * Cols + static_cast<std::size_t>(tile) * Rows * T
                              + threadIdx.x;
    const std::size_t in_base = Side == 2 ? tiled : base;
    const std::size_t out_base = Side == 1 ? tiled : base;
    constexpr std::size_t kInStep = Side == 2 ? std::size_t(kStep) * T : std::size_t(kStep) * Cols;
    constexpr std::size_t kOutStep = Side == 1 ? std::size_t(kStep) * T : std::size_t(kStep) * Cols;
    f2v v[kK];
#pragma unroll
    for (int k = 0; k < kK; ++k) {
        v[k] = load8<NT>(in + in_base + static_cast<std::size_t>(k) * kInStep);
    }
#pragma unroll
    for (int k = 0; k < kK; ++k) {
        store8<NT>(out + out_base + static_cast<std::size_t>(k) * kOutStep, v[k]);
    }
}

// Whole rows against a tile-major array (tiles of T columns, as above): workgroup b copies G
// consecutive rows of one array, a contiguous run of G * Cols values on the row-major side and,
// on the tile-major side, one run of G * T values in each of the Cols / T tiles. ToTiles: the
// row-major side is the input. Lanes walk the tile-major side in order, the other side in the
// same order (a permuted copy: the floor of the two access patterns, not a layout change).
template <int Rows, int Cols, int T, int G, int Th, bool ToTiles>
__global__ void __launch_bounds__(Th) rows_tiles_copy_kernel(const f2v* __restrict__ in,
                                                             f2v* __restrict__ out)
{
    constexpr int kTotal = G * Cols;
    constexpr int kK = kTotal / Th;
    static_assert(Cols % T == 0 && Rows % G == 0 && kTotal % Th == 0, "row group shape");
    const std::size_t array = blockIdx.x / (Rows / G);
    const int r0 = static_cast<int>(blockIdx.x % (Rows / G)) * G;
    const std::size_t rows_base = array * Rows * Cols + static_cast<std::size_t>(r0) * Cols;
    f2v v[kK];
#pragma unroll
    for (int k = 0; k < kK; ++k) {
        const int e = static_cast<int>(threadIdx.x) + k * Th;
        const int j = e % T;
        const int g = (e / T) % G;
        const int tile = e / (T * G);
        const std::size_t tiled = array * Rows * Cols + static_cast<std::size_t>(tile) * Rows * T
                                  + static_cast<std::size_t>(r0 + g) * T + j;
        v[k] = ToTiles ? in[rows_base + e] : in[tiled];
        if (ToTiles) {
            out[tiled] = v[k];
        } else {
            out[rows_base + e] = v[k];
        }
    }
}

constexpr int kChains = 8;
constexpr int kUnroll = 16;

// a <- a * b + c in kChains independent chains; 0 < b < 1 keeps the values finite. The store is
// behind a test the compiler cannot fold, so the arithmetic stays.
__global__ void __launch_bounds__(kThreads) fma_kernel(float* out, int iters, float b, float c)
{
    float a[kChains];
#pragma unroll
    for (int k = 0; k < kChains; ++k) {
        a[k] = static_cast<float>(threadIdx.x + k);
    }
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) {
#pragma unroll
            for (int k = 0; k < kChains; ++k) {
                a[k] = fmaf(a[k], b, c);
            }
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kChains; ++k) {
        s += a[k];
    }
    if (s == -1.0f) {
        out[blockIdx.x * kThreads + threadIdx.x] = s;
    }
}

float median(std::vector<float> v)
{
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

// --patterns: each pattern copies `values` 8-byte values (in + out = 16 bytes per value) from
// one buffer of a rotating set of eight into another (2 GiB in all, beyond the 256 MB cache);
// the patterns run interleaved over 7 rounds of 20 launches and each reports its median round.
struct Pattern {
    const char* name;
    const char* serves;
    std::size_t values;
    void (*launch)(const f2v*, f2v*, hipStream_t);
    std::vector<float> us;
};

template <int Th, int V, bool NT, bool StoreNT = NT>
void launch_rows(std::size_t values, const f2v* in, f2v* out, hipStream_t s)
{
    hipLaunchKernelGGL((rows_copy_kernel<Th, V, NT, StoreNT>),
                       dim3(static_cast<unsigned>(values / (Th * V))), dim3(Th), 0, s, in, out);
}

template <int Rows, int Cols, int T, int Th, bool NT>
void launch_tiles(std::size_t values, const f2v* in, f2v* out, hipStream_t s)
{
    hipLaunchKernelGGL((tiles_copy_kernel<Rows, Cols, T, Th, NT>),
                       dim3(static_cast<unsigned>(values / (static_cast<std::size_t>(Rows) * T))),
                       dim3(Th), 0, s, in, out);
}

template <int Rows, int Cols, int T, int Th, bool NT, int Side>
void launch_tiles_side(std::size_t values, const f2v* in, f2v* out, hipStream_t s)
{
    hipLaunchKernelGGL((tiles_copy_kernel<Rows, Cols, T, Th, NT, Side>),
                       dim3(static_cast<unsigned>(values / (static_cast<std::size_t>(Rows) * T))),
                       dim3(Th), 0, s, in, out);
}

template <int Rows, int Cols, int T, int G, int Th, bool ToTiles>
void launch_rows_tiles(std::size_t values, const f2v* in, f2v* out, hipStream_t s)
{
    hipLaunchKernelGGL((rows_tiles_copy_kernel<Rows, Cols, T, G, Th, ToTiles>),
                       dim3(static_cast<unsigned>(values / (static_cast<std::size_t>(G) * Cols))),
                       dim3(Th), 0, s, in, out);
}

template <int Th>
void launch_rows_lds_dma(std::size_t values, const f2v* in, f2v* out, hipStream_t s)
{
    hipLaunchKernelGGL((rows_lds_dma_kernel<Th>), dim3(static_cast<unsigned>(values / (Th * 8))),
                       dim3(Th), 0, s, in, out);
}

template <int Th, int V, bool Expand>
void launch_mix(std::size_t wide_values, const f2v* in, f2v* out, hipStream_t s)
{
    hipLaunchKernelGGL((mix_rows_kernel<Th, V, Expand>),
                       dim3(static_cast<unsigned>(wide_values / (Th * V))), dim3(Th), 0, s, in, out);
}

template <int Th, bool Expand>
void launch_mix16(std::size_t rows, const f2v* in, f2v* out, hipStream_t s)
{
    hipLaunchKernelGGL((mix16_kernel<Th, Expand>), dim3(static_cast<unsigned>(rows / Th)), dim3(Th),
                       0, s, in, out);
}

constexpr std::size_t k2e24 = std::size_t(1) << 24;
constexpr std::size_t k2e23 = std::size_t(1) << 23;

int run_patterns()
{
    std::vector<Pattern> ps = {
        {"rows 16 KB chunks, nontemporal", "C1 C2C n = 1024 (2^24 points)", k2e24,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_rows<256, 8, true>(k2e24, i, o, s); }, {}},
        {"rows 16 KB chunks, loads straight to LDS, nontemporal", "C1's size, global_load_lds_dwordx4", k2e24,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_rows_lds_dma<256>(k2e24, i, o, s); }, {}},
        {"rows 16 KB chunks, plain", "2^24 points, plain accesses", k2e24,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_rows<256, 8, false>(k2e24, i, o, s); }, {}},
        {"rows 16 KB chunks, nontemporal", "one pass of C3 512^2 x 64 (2^23 values)", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_rows<256, 8, true>(k2e23, i, o, s); }, {}},
        {"rows 16 KB chunks, plain", "C3 512^2 row-pair pass (2^23 values)", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_rows<256, 8, false>(k2e23, i, o, s); }, {}},
        {"rows 16 KB chunks, plain loads, nontemporal stores", "C2 R2C / C2R n = 8 .. 4096 (64 + 64 MiB)", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_rows<256, 8, false, true>(k2e23, i, o, s); }, {}},
        {"rows 2 KB chunks, plain loads, nontemporal stores", "the same, one value per lane", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_mix<256, 1, false>(k2e23, i, o, s); }, {}},
        {"rows, 2 B read per 1 B written", "C2 C2R n = 2: 128 MiB in, 64 MiB out", (k2e24 + k2e24 / 2) / 2,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_mix<256, 2, false>(k2e24, i, o, s); }, {}},
        {"rows, 1 B read per 2 B written", "C2 R2C n = 2: 64 MiB in, 128 MiB out", (k2e24 + k2e24 / 2) / 2,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_mix<256, 2, true>(k2e24, i, o, s); }, {}},
        {"rows, 16-byte loads, 8-byte stores (2:1)", "C2 C2R n = 2, as its kernel moves rows", (k2e24 + k2e24 / 2) / 2,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_mix16<256, false>(k2e23, i, o, s); }, {}},
        {"rows, 8-byte loads, 16-byte stores (1:2)", "C2 R2C n = 2, as its kernel moves rows", (k2e24 + k2e24 / 2) / 2,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_mix16<256, true>(k2e23, i, o, s); }, {}},
        {"rows, 16 B read per 1 B written", "C4 rfft2_modes: 128 MiB in, 8 MiB out", (k2e24 + k2e24 / 16) / 2,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_mix<256, 16, false>(k2e24, i, o, s); }, {}},
        {"rows, 1 B read per 16 B written", "C4 irfft2_modes: 8 MiB in, 128 MiB out", (k2e24 + k2e24 / 16) / 2,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_mix<256, 16, true>(k2e24, i, o, s); }, {}},
        {"tiles 16 x 512 of 512 x 256, plain", "C3 512^2 column pass (128-byte runs)", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_tiles<512, 256, 16, 1024, false>(k2e23, i, o, s); }, {}},
        {"tiles 16 x 512 of 512 x 256, nontemporal", "C3 512^2 column pass, nontemporal", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_tiles<512, 256, 16, 1024, true>(k2e23, i, o, s); }, {}},
        {"tiles 32 x 512 of 512 x 256, plain", "256-byte runs", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_tiles<512, 256, 32, 1024, false>(k2e23, i, o, s); }, {}},
        {"tiles 64 x 512 of 512 x 256, plain", "512-byte runs", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_tiles<512, 256, 64, 1024, false>(k2e23, i, o, s); }, {}},
        {"tiles 16 x 512 of 512 x 256 in, tile-major out, plain", "column pass into a tile-major workspace", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_tiles_side<512, 256, 16, 1024, false, 1>(k2e23, i, o, s); }, {}},
        {"tile-major in, tiles 16 x 512 of 512 x 256 out, nontemporal", "column pass from a tile-major workspace", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_tiles_side<512, 256, 16, 1024, true, 2>(k2e23, i, o, s); }, {}},
        {"tile-major in (4-row runs, 512 B), rows out", "row-pair pass from a tile-major workspace", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_rows_tiles<512, 256, 16, 4, 256, false>(k2e23, i, o, s); }, {}},
        {"tile-major in (16-row runs, 2 KB), rows out", "row-pair pass, 1024-lane workgroups", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_rows_tiles<512, 256, 16, 16, 1024, false>(k2e23, i, o, s); }, {}},
        {"rows in, tile-major out (4-row runs, 512 B)", "row-pair pass into a tile-major workspace", k2e23,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_rows_tiles<512, 256, 16, 4, 256, true>(k2e23, i, o, s); }, {}},
        {"tiles 8 x 1024 of 1024 x 1024, plain", "2^20-point C2C column pass (64-byte runs)", k2e24,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_tiles<1024, 1024, 8, 512, false>(k2e24, i, o, s); }, {}},
        {"tiles 16 x 1024 of 1024 x 1024, plain", "128-byte runs", k2e24,
         [](const f2v* i, f2v* o, hipStream_t s) { launch_tiles<1024, 1024, 16, 1024, false>(k2e24, i, o, s); }, {}},
    };
    // Eight sets: the smallest inputs here (2^23 values, 64 MiB) then total 512 MiB in rotation,
    // twice the Infinity Cache, so no launch reads what an earlier one left there.
    constexpr int kSets = 8;
    const std::size_t bytes = k2e24 * sizeof(f2v);
    f2v* in[kSets];
    f2v* out[kSets];
    for (int s = 0; s < kSets; ++s) {
        CHECK(hipMalloc(&in[s], bytes));
        CHECK(hipMalloc(&out[s], bytes));
        CHECK(hipMemset(in[s], 0x3c, bytes));
        CHECK(hipMemset(out[s], 0, bytes));
    }
    hipStream_t stream;
    CHECK(hipStreamCreate(&stream));
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    constexpr int kIters = 20;
    for (auto& p : ps) {
        for (int i = 0; i < 3; ++i) {
            p.launch(in[i % kSets], out[i % kSets], stream);
        }
    }
    CHECK(hipGetLastError());
    CHECK(hipStreamSynchronize(stream));
    for (int r = 0; r < 7; ++r) {
        for (auto& p : ps) {
            CHECK(hipEventRecord(e0, stream));
            for (int i = 0; i < kIters; ++i) {
                p.launch(in[i % kSets], out[i % kSets], stream);
            }
            CHECK(hipEventRecord(e1, stream));
            CHECK(hipEventSynchronize(e1));
            float ms = 0.0f;
            CHECK(hipEventElapsedTime(&ms, e0, e1));
            p.us.push_back(1000.0f * ms / kIters);
        }
    }
    CHECK(hipGetLastError());
    std::printf("| pattern | size | serves | us | GB/s |\n|---|---:|---|---:|---:|\n");
    for (auto& p : ps) {
        const double us = median(p.us);
        std::printf("| %s | %.0f MiB in + out | %s | %.2f | %.1f |\n", p.name,
                    p.values * 16.0 / (1 << 20), p.serves, us, p.values * 16.0 / (us * 1e3));
    }
    for (int s = 0; s < kSets; ++s) {
        CHECK(hipFree(in[s]));
        CHECK(hipFree(out[s]));
    }
    return 0;
}

}  // namespace

int main(int argc, char** argv)
{
    bool copy_only = false;
    std::size_t bytes = std::size_t(1) << 30;  // per buffer
    int iters = 20;
    const char* out_path = nullptr;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--patterns") {
            return run_patterns();
        } else if (a == "--copy-only") {
            copy_only = true;
        } else if (a == "--bytes" && i + 1 < argc) {
            bytes = std::strtoull(argv[++i], nullptr, 10);
        } else if (a == "--iters" && i + 1 < argc) {
            iters = std::atoi(argv[++i]);
        } else if (a == "--out" && i + 1 < argc) {
            out_path = argv[++i];
        } else {
            std::fprintf(stderr, "usage: spectral_peaks [--copy-only] [--bytes B] [--iters K] "
                                 "[--out FILE] | --patterns\n");
            return 2;
        }
    }
    if (bytes < 16 || bytes % 16 != 0 || iters < 1) {
        std::fprintf(stderr, "spectral_peaks: --bytes must be a positive multiple of 16 and "
                             "--iters at least 1\n");
        return 2;
    }

    hipDeviceProp_t prop;
    CHECK(hipGetDeviceProperties(&prop, 0));
    const int cus = prop.multiProcessorCount;

    // Rotate the copy over pairs so the sources total at least 1 GiB beyond the cache.
    const int pairs = static_cast<int>(std::max<std::size_t>(1, (std::size_t(3) << 30) / bytes));
    const int npairs = std::min(pairs, 4);
    std::vector<float4*> src(npairs), dst(npairs);
    const std::size_t n = bytes / sizeof(float4);
    for (int p = 0; p < npairs; ++p) {
        CHECK(hipMalloc(&src[p], bytes));
        CHECK(hipMalloc(&dst[p], bytes));
        CHECK(hipMemset(src[p], 0x3c, bytes));
    }
    const unsigned copy_blocks = static_cast<unsigned>(
        std::min<std::size_t>((n + kThreads * kVec - 1) / (kThreads * kVec),
                              static_cast<std::size_t>(cus) * 32));
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));

    if (copy_only) {
        for (int i = 0; i < iters; ++i) {
            hipLaunchKernelGGL(copy_kernel, dim3(copy_blocks), dim3(kThreads), 0, 0,
                               src[i % npairs], dst[i % npairs], n);
        }
        CHECK(hipGetLastError());
        CHECK(hipDeviceSynchronize());
        std::printf("{\"copy_kernel_launches\": %d, \"bytes_read_per_launch\": %zu, "
                    "\"bytes_written_per_launch\": %zu}\n", iters, bytes, bytes);
        return 0;
    }

    // Copy: 3 warm-ups, then 5 rounds of `iters` launches, median per launch.
    for (int i = 0; i < 3; ++i) {
        hipLaunchKernelGGL(copy_kernel, dim3(copy_blocks), dim3(kThreads), 0, 0, src[i % npairs],
                           dst[i % npairs], n);
    }
    std::vector<float> copy_ms;
    for (int r = 0; r < 5; ++r) {
        CHECK(hipEventRecord(e0, 0));
        for (int i = 0; i < iters; ++i) {
            hipLaunchKernelGGL(copy_kernel, dim3(copy_blocks), dim3(kThreads), 0, 0,
                               src[i % npairs], dst[i % npairs], n);
        }
        CHECK(hipEventRecord(e1, 0));
        CHECK(hipEventSynchronize(e1));
        float ms = 0.0f;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        copy_ms.push_back(ms / iters);
    }
    CHECK(hipGetLastError());
    const double copy_gbps = 2.0 * static_cast<double>(bytes) / (median(copy_ms) * 1e6);

    // FMA: enough workgroups for 8 waves per SIMD.
    float* sink = nullptr;
    const unsigned fma_blocks = static_cast<unsigned>(cus) * 8;
    CHECK(hipMalloc(&sink, static_cast<std::size_t>(fma_blocks) * kThreads * sizeof(float)));
    const int fma_iters = 4096;
    hipLaunchKernelGGL(fma_kernel, dim3(fma_blocks), dim3(kThreads), 0, 0, sink, fma_iters, 0.5f,
                       1.0f);
    std::vector<float> fma_ms;
    for (int r = 0; r < 5; ++r) {
        CHECK(hipEventRecord(e0, 0));
        hipLaunchKernelGGL(fma_kernel, dim3(fma_blocks), dim3(kThreads), 0, 0, sink, fma_iters,
                           0.5f, 1.0f);
        CHECK(hipEventRecord(e1, 0));
        CHECK(hipEventSynchronize(e1));
        float ms = 0.0f;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        fma_ms.push_back(ms);
    }
    CHECK(hipGetLastError());
    const double flops = 2.0 * kChains * kUnroll * static_cast<double>(fma_iters) * fma_blocks
                         * kThreads;
    const double fp32_gflops = flops / (median(fma_ms) * 1e6);

    char json[1024];
    std::snprintf(json, sizeof json,
                  "{\"device\": \"%s\", \"arch\": \"%s\", \"cus\": %d, \"copy_bytes_per_buffer\": "
                  "%zu, \"copy_gbps\": %.1f, \"copy_ms\": %.5f, \"fp32_gflops\": %.1f, "
                  "\"datasheet_hbm_gbps\": 8000.0, \"datasheet_fp32_gflops\": 157300.0}\n",
                  prop.name, prop.gcnArchName, cus, bytes, copy_gbps, median(copy_ms),
                  fp32_gflops);
    std::fputs(json, stdout);
    if (out_path != nullptr) {
        FILE* f = std::fopen(out_path, "w");
        if (f == nullptr) {
            std::fprintf(stderr, "spectral_peaks: cannot write %s\n", out_path);
            return 1;
        }
        std::fputs(json, f);
        std::fclose(f);
    }
    for (int p = 0; p < npairs; ++p) {
        CHECK(hipFree(src[p]));
        CHECK(hipFree(dst[p]));
    }
    CHECK(hipFree(sink));
    return 0;
}
