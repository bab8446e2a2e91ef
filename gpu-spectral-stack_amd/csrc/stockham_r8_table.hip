// Stockham variant stockham_r8_table: radix-8 stages, twiddles from the precomputed table.
#include "variant.hpp"

SPX_DEFINE_VARIANT(stockham_r8_table, 8, true)
