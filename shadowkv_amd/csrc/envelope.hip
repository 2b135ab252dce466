// Measurement probes (no counterpart in the reference): the HBM read rate a launch of a given
// size reaches on this GPU, by access order, the ceiling the streaming kernels (landmark scoring,
// attention, rebuild) are read against; and the bf16 MFMA rate of back-to-back matrix
// instructions on register operands, the ceiling of the rebuild's MFMA utilisation.
//
// HBM read probe:
// Each workgroup of 256 threads (4 waves) reads `tiles_per_wg` consecutive tiles of 64 KB
// (4096 16-byte vectors), tile after tile, with all 16 of a thread's loads of a tile issued before
// any is used, and XORs what it read into one vector per thread, written to sink (so no load is
// dead). Two orders within a tile (pattern bit 0), each with plain or non-temporal loads (pattern
// bit 1):
//   kContiguous: load i (0..15) of wave w covers bytes [4096*i + 1024*w, +1024): every wave
//     instruction reads 1 KB of consecutive bytes;
//   kOperand: the tile as 256 rows of 256 bytes, the order in which the scoring and attention
//     kernels fetch MFMA operands: wave w owns rows [64w, 64w + 64); load (kg, ks), kg, ks < 4,
//     gives lane (li = lane % 16, grp = lane / 16) the 16 bytes at byte 64*ks + 16*grp of row
//     64w + 16*kg + li, so one instruction reads 64 bytes from each of 16 rows.
#include "skv_common.h"

namespace {

using skv::u32x4;

constexpr int kThreads = 256;
constexpr int kTileVecs = 4096;  // 64 KB
enum Pattern { kContiguous = 0, kOperand = 1, kNonTemporal = 2 };

template <int kPattern, bool kNt>
__global__ void __launch_bounds__(kThreads) read_probe_kernel(const u32x4* __restrict__ src, int64_t tiles,
                                                              int tiles_per_wg, u32x4* __restrict__ sink) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, li = lane & 15, grp = lane >> 4;
  u32x4 acc = {0u, 0u, 0u, 0u};
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * tiles_per_wg;
  for (int t = 0; t < tiles_per_wg; ++t) {
    if (t0 + t >= tiles) break;  // workgroup-uniform
    const u32x4* tile = src + (t0 + t) * kTileVecs;
    u32x4 r[16];
#pragma unroll
    for (int kg = 0; kg < 4; ++kg)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int v = kPattern == kContiguous ? (kg * 4 + ks) * kThreads + tid
                                              : (wave * 64 + 16 * kg + li) * 16 + 4 * ks + grp;
        r[kg * 4 + ks] = kNt ? skv::load_nt(tile + v) : tile[v];
      }
#pragma unroll
    for (int k = 0; k < 16; ++k) acc ^= r[k];
  }
  sink[static_cast<int64_t>(blockIdx.x) * kThreads + tid] = acc;
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
constexpr int kMfmaChains = 4;  // independent accumulators per wave (cover the instruction's latency)
constexpr int64_t kMfmaFlops = 32 * 32 * 16 * 2;  // one v_mfma_f32_32x32x16_bf16

// Every wave issues iters x kMfmaChains v_mfma_f32_32x32x16_bf16 on operands built from its lane
// id and `seed` (no memory traffic), then writes one float per thread so that no product is dead.
// (The 32x32 form: four named 16-float accumulators stay in place across the loop, where eight
// 16x16x32 chains are shuffled between register tuples by the compiler; measured 2.05 vs 1.95
// PFLOP/s on MI355X.)
__global__ void __launch_bounds__(kThreads) mfma_probe_kernel(int iters, uint32_t seed, float* __restrict__ sink) {
  const uint32_t t = threadIdx.x;
  const uint32_t wa = 0x3f803f80u ^ ((t * 2654435761u + seed) & 0x007f007fu);  // bf16 pairs near 1
  const uint32_t wb = 0x3f803f80u ^ ((t * 2246822519u + seed) & 0x007f007fu);
  const bf16x8_t a = __builtin_bit_cast(bf16x8_t, u32x4{wa, wa ^ 1u, wa ^ 2u, wa ^ 3u});
  const bf16x8_t b = __builtin_bit_cast(bf16x8_t, u32x4{wb, wb ^ 4u, wb ^ 8u, wb ^ 12u});
  f32x16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int i = 0; i < iters; ++i) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
  }
  const f32x16_t q = (c0 + c1) + (c2 + c3);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) s += q[e];
  sink[static_cast<int64_t>(blockIdx.x) * kThreads + t] = s;
}

}  // namespace

extern "C" int skv_mfma_peak_probe(int workgroups, int iters, float* sink, int64_t sink_bytes, void* stream) {
  const char* what = "mfma_peak_probe";
  if (!sink || (reinterpret_cast<uintptr_t>(sink) & 3u)) {
    skv_set_error("%s: null or misaligned sink", what);
    return SKV_EINVAL;
  }
  // The product bounds one launch's work: 2^24 workgroup-iterations of 4 waves x 4 MFMA chains is
  // about 8.8 TFLOP, ~4 ms at the measured rate, far from the GPU's watchdog (the bench runs 2048 x 1024).
  if (workgroups < 1 || workgroups > (1 << 20) || iters < 1 || iters > (1 << 20) ||
      static_cast<int64_t>(workgroups) * iters > (int64_t{1} << 24)) {
    skv_set_error("%s: workgroups=%d (1..2^20) iters=%d (1..2^20), product at most 2^24", what, workgroups, iters);
    return SKV_EINVAL;
  }
  if (sink_bytes < static_cast<int64_t>(workgroups) * kThreads * 4) {
    skv_set_error("%s: sink of %lld bytes, %lld needed", what, (long long)sink_bytes,
                  (long long)workgroups * kThreads * 4);
    return SKV_EINVAL;
  }
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(workgroups), dim3(kThreads), 0, static_cast<hipStream_t>(stream), iters,
                     static_cast<uint32_t>(iters * 31 + workgroups), sink);
  return skv_check_launch(what);
}

extern "C" int64_t skv_mfma_peak_probe_flops(int workgroups, int iters) {
  if (workgroups < 1 || iters < 1) return 0;
  return static_cast<int64_t>(workgroups) * (kThreads / 64) * iters * kMfmaChains * kMfmaFlops;
}

extern "C" int skv_hbm_read_probe(const void* src, int64_t tiles, int tiles_per_workgroup, int pattern, void* sink,
                                  int64_t sink_bytes, void* stream) {
  const char* what = "hbm_read_probe";
  if (!src || !sink) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(sink)) & 15u) {
    skv_set_error("%s: src and sink must be 16-byte aligned", what);
    return SKV_EINVAL;
  }
  if (tiles < 1 || tiles_per_workgroup < 1 || tiles_per_workgroup > 64 || pattern < 0 || pattern > 3) {
    skv_set_error("%s: tiles=%lld tiles_per_workgroup=%d (1..64) pattern=%d (0 contiguous, 1 operand order, +2 "
                  "non-temporal)", what,
                  (long long)tiles, tiles_per_workgroup, pattern);
    return SKV_EINVAL;
  }
  const int64_t grid = (tiles + tiles_per_workgroup - 1) / tiles_per_workgroup;
  if (grid > 0x7fffffff) {
    skv_set_error("%s: %lld workgroups", what, (long long)grid);
    return SKV_EUNSUPPORTED;
  }
  if (sink_bytes < grid * kThreads * 16) {
    skv_set_error("%s: sink of %lld bytes, %lld needed", what, (long long)sink_bytes, (long long)(grid * kThreads * 16));
    return SKV_EINVAL;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const u32x4* in = static_cast<const u32x4*>(src);
  u32x4* out = static_cast<u32x4*>(sink);
  const dim3 g(static_cast<unsigned>(grid)), b(kThreads);
  switch (pattern) {
    case kContiguous: hipLaunchKernelGGL((read_probe_kernel<kContiguous, false>), g, b, 0, s, in, tiles, tiles_per_workgroup, out); break;
    case kOperand: hipLaunchKernelGGL((read_probe_kernel<kOperand, false>), g, b, 0, s, in, tiles, tiles_per_workgroup, out); break;
    case kContiguous | kNonTemporal:
      hipLaunchKernelGGL((read_probe_kernel<kContiguous, true>), g, b, 0, s, in, tiles, tiles_per_workgroup, out);
      break;
    default: hipLaunchKernelGGL((read_probe_kernel<kOperand, true>), g, b, 0, s, in, tiles, tiles_per_workgroup, out); break;
  }
  return skv_check_launch(what);
}
