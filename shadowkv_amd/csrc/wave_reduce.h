// Reduce-scatter of M per-lane partial sums over an aligned group of 16 lanes.
//
// Each of the 16 lanes holds v[0..M) (partial dot products over its slice of the head
// dimension). After log2(M) halving exchanges (xor 8, 4, ...) every lane holds the group
// total of one index i = li >> (4 - log2 M), and the remaining xor steps complete it.
// This costs M-1 shuffles per lane instead of the 4*M of M independent butterflies.
#pragma once

#include "skv_common.h"

namespace skv {

template <int COUNT, int O>
struct ReduceScatter16 {
  __device__ __forceinline__ static float run(float* v, int li) {
    if constexpr (O == 0) {
      return v[0];
    } else if constexpr (COUNT > 1) {
      constexpr int HALF = COUNT / 2;
      const bool up = (li & O) != 0;
#pragma unroll
      for (int t = 0; t < HALF; ++t) {
        const float send = up ? v[t] : v[t + HALF];
        const float keep = up ? v[t + HALF] : v[t];
        v[t] = keep + __shfl_xor(send, O, kWave);
      }
      return ReduceScatter16<HALF, O / 2>::run(v, li);
    } else {
      v[0] += __shfl_xor(v[0], O, kWave);
      return ReduceScatter16<1, O / 2>::run(v, li);
    }
  }
};

template <int M>
struct Log2 {
  static constexpr int value = (M <= 1) ? 0 : 1 + Log2<M / 2>::value;
};
template <>
struct Log2<1> {
  static constexpr int value = 0;
};

// Index owned by lane `li` (0..15) after reduce_scatter16<M>.
template <int M>
__device__ __forceinline__ int rs16_owner(int li) {
  return li >> (4 - Log2<M>::value);
}
// True for exactly one lane per owned index (the lowest lane of its replica set).
template <int M>
__device__ __forceinline__ bool rs16_writer(int li) {
  return (li & ((16 / M) - 1)) == 0;
}

template <int M>
__device__ __forceinline__ float reduce_scatter16(float* v, int li) {
  static_assert(M >= 1 && M <= 16 && (M & (M - 1)) == 0, "M must be a power of two <= 16");
  return ReduceScatter16<M, 8>::run(v, li);
}

}  // namespace skv
