// Stockham variant stockham_r8: radix-8 stages, twiddles computed with sincospif and powering.
#include "variant.hpp"

SPX_DEFINE_VARIANT(stockham_r8, 8, false)
