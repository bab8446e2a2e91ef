// Stockham variant stockham_r2: radix-2 stages, twiddles computed with sincospif and powering.
#include "variant.hpp"

SPX_DEFINE_VARIANT(stockham_r2, 2, false)
