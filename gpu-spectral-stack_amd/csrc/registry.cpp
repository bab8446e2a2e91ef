// Every FFT implementation, by name, in the reference's order (registry.hpp:28-40). The C ABI,
// the PyTorch operators and the benchmark all resolve `impl` through this one table, so a new
// implementation is added here and reaches every test and benchmark.

#include "fft_api.hpp"

namespace spx {
namespace {

const FftImpl kImpls[] = {
    {"naive", &c2c_naive, &r2c_naive, &c2r_naive, nullptr, nullptr, 1 << 30, 1 << 30, 1 << 30,
     true, nullptr, nullptr, nullptr, false},
    {"stockham_r2", &c2c_stockham_r2, &r2c_stockham_r2, &c2r_stockham_r2, &columns_stockham_r2,
     &pruned_stockham_r2, kStockhamMaxN, kFourStepMaxN, 2 * kStockhamMaxN, false, &fused_stockham_r2,
     &rf_stockham_r2, &c2c_work_stockham_r2, false},
    {"stockham_r4", &c2c_stockham_r4, &r2c_stockham_r4, &c2r_stockham_r4, &columns_stockham_r4,
     &pruned_stockham_r4, kStockhamMaxN, kFourStepMaxN, 2 * kStockhamMaxN, false, &fused_stockham_r4,
     &rf_stockham_r4, &c2c_work_stockham_r4, false},
    {"stockham_r8", &c2c_stockham_r8, &r2c_stockham_r8, &c2r_stockham_r8, &columns_stockham_r8,
     &pruned_stockham_r8, kStockhamMaxN, kFourStepMaxN, 2 * kStockhamMaxN, false, &fused_stockham_r8,
     &rf_stockham_r8, &c2c_work_stockham_r8, false},
    {"stockham_r8_table", &c2c_stockham_r8_table, &r2c_stockham_r8_table,
     &c2r_stockham_r8_table, &columns_stockham_r8_table, &pruned_stockham_r8_table,
     kStockhamMaxN, kFourStepMaxN, 2 * kStockhamMaxN, false, &fused_stockham_r8_table,
     &rf_stockham_r8_table, &c2c_work_stockham_r8_table, true},
};

}  // namespace

const FftImpl* impls() { return kImpls; }

int impl_count() { return static_cast<int>(sizeof(kImpls) / sizeof(kImpls[0])); }

std::size_t c2c_scratch_values(const FftImpl& impl, int n, int batch)
{
    if (impl.c2c_work == nullptr || n <= kSinglePassMaxN || batch < 1) {
        return 0;
    }
    return static_cast<std::size_t>(n) * static_cast<std::size_t>(batch);
}

}  // namespace spx
