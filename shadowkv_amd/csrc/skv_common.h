// Shared device helpers for the ShadowKV sparse-decode kernels (gfx950 / CDNA4).
//
// bf16 values are carried as raw uint16_t bit patterns. Every bf16 arithmetic step
// is done in fp32 and rounded to nearest-even, which is exactly what torch's CPU
// bf16 operators do (they widen to fp32, compute, and narrow with RNE); products and
// sums of two bf16 values are exact or correctly rounded in fp32, so one fp32 op
// followed by RNE equals the single-rounded bf16 op of the reference kernels
// (kernels/rope_new.cu:262-269 uses __hmul/__hadd).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/shadowkv_amd.h"

namespace skv {

constexpr int kWave = 64;

__device__ __forceinline__ float bf2f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// fp32 -> bf16, round to nearest even (gfx950 v_cvt_pk_bf16_f32); NaN -> the canonical quiet NaN
// 0x7fc0, as c10::BFloat16 does.
__device__ __forceinline__ uint16_t f2bf(float f) {
  const uint16_t r = __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  return f != f ? static_cast<uint16_t>(0x7fc0) : r;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> two bf16 in one instruction (a in the low half), round to nearest even. A NaN
// input gives a quiet NaN whose payload is not canonicalised.
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
// The two bf16 of a packed word as fp32 (exact).
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint16_t bmul(uint16_t a, uint16_t b) { return f2bf(bf2f(a) * bf2f(b)); }
// x rounded to bf16 and widened back (exact).
__device__ __forceinline__ float bround(float x) { return bf2f(f2bf(x)); }
// silu(g) * u with vLLM silu_and_mul's roundings (the reference's activation, models/llama.py:212,
// models/glm.py:193): silu(g) = g / (1 + exp(-g)) in fp32 (hardware exp and reciprocal, a few ulp
// of fp32) rounded to bf16, then the bf16 x bf16 product, exact in fp32; the caller rounds the
// result to bf16 once more. Shared by the SiLU-and-mul kernel and the down projection that forms
// the product while reading the gate/up rows, so both agree bit for bit.
__device__ __forceinline__ float silu_mul(float g, float u) { return bround(__fdividef(g, 1.f + __expf(-g))) * u; }
__device__ __forceinline__ uint16_t badd(uint16_t a, uint16_t b) { return f2bf(bf2f(a) + bf2f(b)); }
__device__ __forceinline__ uint16_t bneg(uint16_t a) { return a ^ 0x8000u; }

// Order-preserving map of a bf16 bit pattern to an unsigned key: larger float -> larger key.
__device__ __forceinline__ uint32_t bf16_order_key(uint16_t h) {
  return (h & 0x8000u) ? (static_cast<uint32_t>(~h) & 0xffffu) : (static_cast<uint32_t>(h) | 0x8000u);
}

// Wave-wide reductions over all 64 lanes (result valid in every lane).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
// Wave reductions without LDS round trips: DPP rotations within each 16-lane row (row_ror),
// then the four row results read back as wave-uniform values. Same result on every lane; the
// summation order differs from the butterfly forms above.
template <int N>
__device__ __forceinline__ float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xf, 0xf, false));
}
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, row_ror<8>(v));
  v = fmaxf(v, row_ror<4>(v));
  v = fmaxf(v, row_ror<2>(v));
  v = fmaxf(v, row_ror<1>(v));
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  v += row_ror<1>(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// Softmax normalisers of the m query rows of batch entry z from their per-tile partials (norm:
// tile maximum, sum: tile sum of exp(x - tile maximum); [z][i][tile] arrays of `tiles` entries):
//   gmax[i] = max_t norm[t],   ginv[i] = 1 / sum_t sum[t] * exp(norm[t] - gmax[i]).
// Wave w of the kWaves-wave workgroup takes rows w, w + kWaves, ..., lane l the tiles l, l + 64,
// ... in increasing order, the lanes' sums added by wave_sum_dpp: that assignment alone fixes
// the arithmetic, so every kernel calling this gets bit-identical normalisers. With at most 512
// tiles every row's partials are requested before the first is used (one memory latency for
// the whole merge instead of two per row). gmax/ginv are LDS arrays; the caller synchronises.
template <int kWaves>
__device__ __forceinline__ void merge_softmax_partials(const float* __restrict__ norm, const float* __restrict__ sum,
                                                       int z, int m, int tiles, float* gmax, float* ginv) {
  constexpr int kPL = 8;                 // tiles per lane held in registers
  constexpr int kR = 16 / kWaves;        // rows per wave (m <= 16)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (tiles <= 64 * kPL) {
    float nv[kR][kPL], sv[kR][kPL];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const int i = wave + r * kWaves;
      const int64_t base = (static_cast<int64_t>(z) * m + min(i, m - 1)) * tiles;
#pragma unroll
      for (int u = 0; u < kPL; ++u) {
        const int t = lane + 64 * u;
        const bool ok = i < m && t < tiles;
        nv[r][u] = ok ? norm[base + t] : -INFINITY;
        sv[r][u] = ok ? sum[base + t] : 0.f;
      }
    }
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const int i = wave + r * kWaves;
      if (i >= m) continue;  // wave-uniform (continue, not break: the loop unrolls fully)
      float mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < kPL; ++u) mx = fmaxf(mx, nv[r][u]);
      mx = wave_max_dpp(mx);
      float s = 0.f;
#pragma unroll
      for (int u = 0; u < kPL; ++u)
        if (lane + 64 * u < tiles) s += sv[r][u] * expf(nv[r][u] - mx);
      s = wave_sum_dpp(s);
      if (lane == 0) {
        gmax[i] = mx;
        ginv[i] = 1.f / s;
      }
    }
    return;
  }
  for (int i = wave; i < m; i += kWaves) {
    const float* nr = norm + (static_cast<int64_t>(z) * m + i) * tiles;
    const float* sr = sum + (static_cast<int64_t>(z) * m + i) * tiles;
    float mx = -INFINITY;
    for (int t = lane; t < tiles; t += 64) mx = fmaxf(mx, nr[t]);
    mx = wave_max_dpp(mx);
    float s = 0.f;
    for (int t = lane; t < tiles; t += 64) s += sr[t] * expf(nr[t] - mx);
    s = wave_sum_dpp(s);
    if (lane == 0) {
      gmax[i] = mx;
      ginv[i] = 1.f / s;
    }
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Sum within aligned groups of 16 lanes (result valid in every lane of the group).
__device__ __forceinline__ float group16_sum(float v) {
  v += __shfl_xor(v, 8, kWave);
  v += __shfl_xor(v, 4, kWave);
  v += __shfl_xor(v, 2, kWave);
  v += __shfl_xor(v, 1, kWave);
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wave.
// Inclusive prefix sum over the wave on DPP: shifts within each 16-lane row (lanes shifted in
// from outside the row read 0), then row 0's total into row 1 and row 2's into row 3
// (row_bcast:15), then the total of rows 0-1 into rows 2-3 (row_bcast:31).
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31 into rows 2, 3
  return v;
}

// Exclusive prefix sum over the whole workgroup. `scratch` needs blockDim.x/64 + 1 ints of LDS.
// Returns the exclusive prefix for this thread; *total receives the workgroup sum.
__device__ __forceinline__ int block_exclusive_scan(int v, int* scratch, int* total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nwaves = (blockDim.x + kWave - 1) / kWave;
  int inc = wave_inclusive_scan(v);
  if (lane == kWave - 1) scratch[wave] = inc;
  __syncthreads();
  if (threadIdx.x < kWave) {  // wave 0 scans the per-wave totals (nwaves <= 16)
    const int t = lane < nwaves ? scratch[lane] : 0;
    const int incl = wave_inclusive_scan(t);
    if (lane < nwaves) scratch[lane] = incl - t;
    if (lane == nwaves - 1) scratch[nwaves] = incl;
  }
  __syncthreads();
  int excl = scratch[wave] + inc - v;
  *total = scratch[nwaves];
  __syncthreads();
  return excl;
}

// Wait for every outstanding memory operation of this wave (vector loads included),
// then barrier. Used where a later store by another wave must not overtake a load.
__device__ __forceinline__ void drain_and_barrier() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// 16-byte vector type for chunk copies: a native vector (not a struct), so arrays of it stay in
// registers (a struct is copied with memcpy, which keeps such arrays in private memory).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte load of *p when ok, else zero. p must be readable either way (the caller clamps an
// out-of-range index to a valid one), so the load is issued unconditionally: no branch splits a
// batch of loads, which would make the compiler wait for each before issuing the next.
__device__ __forceinline__ u32x4 load16_or_zero(const void* p, bool ok) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(p);
  return ok ? v : u32x4{0u, 0u, 0u, 0u};
}

// 16-byte load with the non-temporal (streaming) hint: global_load_dwordx4 ... nt. Used for reads
// of pinned host memory over the host link, which are read once (it keeps those long-latency
// requests from holding cache resources that concurrent kernels' HBM traffic needs), and for HBM
// streams read whole lines per wave load (attention's V rows), which it speeds up. Reads that
// split each 128-byte line over two loads (the MFMA operand order) stream slower with it.
__device__ __forceinline__ u32x4 load_nt(const u32x4* p) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
  return u32x4{v.x, v.y, v.z, v.w};
}

// 16-byte store with the non-temporal hint: global_store_dwordx4 ... nt. For large outputs that no
// later instruction of the same kernel reads: they are not kept dirty in the L2, so the write-back
// of dirty L2 lines at the kernel boundary (which the next kernel on the stream waits for) stays
// short (rebuild at batch 8, 33 MB written: 3.2 -> 1.3 us between back-to-back launches).
__device__ __forceinline__ void store_nt(void* p, u32x4 v) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(v4u{v.x, v.y, v.z, v.w}, reinterpret_cast<v4u*>(p));
}

}  // namespace skv

// Host-side error reporting shared by every entry point (defined in skv_api.cpp).
void skv_set_error(const char* fmt, ...);
int skv_check_launch(const char* what);
