// Rotation of one (x1, x2) pair with the bf16 rounding sequence of the reference
// (kernels/rope_new.cu:268-269): every product and sum is rounded to bf16.
#pragma once

#include "skv_common.h"

namespace skv {

__device__ __forceinline__ void rope_half_split(uint16_t x1, uint16_t x2, uint16_t c, uint16_t s, uint16_t& y1,
                                                uint16_t& y2) {
  y1 = badd(bmul(x1, c), bmul(bneg(x2), s));
  y2 = badd(bmul(x2, c), bmul(x1, s));
}

}  // namespace skv
