// Stockham variant stockham_r4: radix-4 stages, twiddles computed with sincospif and powering.
#include "variant.hpp"

SPX_DEFINE_VARIANT(stockham_r4, 4, false)
