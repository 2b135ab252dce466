// HBM read envelope probe: the read rate a launch of a given size reaches on this GPU, by access
// order. No counterpart in the reference; it measures the ceiling the streaming kernels
// (landmark scoring, attention, rebuild) are read against.
//
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

}  // namespace

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
