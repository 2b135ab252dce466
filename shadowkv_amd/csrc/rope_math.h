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

// The same rotation on two packed pairs at once: x1, x2, c, s each hold two bf16 (element 0 in
// the low half); returns y1 and y2 packed the same way. Every product and sum is rounded to bf16
// (products of two bf16 are exact in fp32, so one rounding each, as the scalar form).
__device__ __forceinline__ void rope_half_split2(uint32_t x1, uint32_t x2, uint32_t c, uint32_t s, uint32_t& y1,
                                                 uint32_t& y2) {
  const float x1a = bf_lo(x1), x1b = bf_hi(x1), x2a = bf_lo(x2), x2b = bf_hi(x2);
  const float ca = bf_lo(c), cb = bf_hi(c), sa = bf_lo(s), sb = bf_hi(s);
  const uint32_t p = f2bf2(x1a * ca, x1b * cb);
  const uint32_t q = f2bf2(-(x2a * sa), -(x2b * sb));
  const uint32_t r = f2bf2(x2a * ca, x2b * cb);
  const uint32_t t = f2bf2(x1a * sa, x1b * sb);
  y1 = f2bf2(bf_lo(p) + bf_lo(q), bf_hi(p) + bf_hi(q));
  y2 = f2bf2(bf_lo(r) + bf_lo(t), bf_hi(r) + bf_hi(t));
}

}  // namespace skv
