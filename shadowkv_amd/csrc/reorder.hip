// a3: cache-hit reorder of the selected chunk ids against the previous step's slots.
//
// One workgroup (4 wave64) per (batch, kv-head) row. Instead of the reference's LDS hash
// table + warp32 ballots (kernels/map.cuh:475-516), the row is solved by sorting
// (select_core.h, reorder_row): old (id, slot) pairs and new ids are bitonic-sorted in LDS,
// each new id binary-searches the old ids, hits are marked at their old slot so a prefix scan
// over slots emits them in ascending old-slot order, and misses come out of a prefix scan
// over the sorted new ids in ascending id order. The result is the one map.cuh produces after
// its block_sort2 (map.cuh:229-259,503-506); no atomics, no hashing, deterministic.
#include "select_core.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxMap = 2048;

__global__ void __launch_bounds__(kThreads) reorder_kernel(int64_t* __restrict__ cached,
                                                            const int64_t* __restrict__ cur,
                                                            int32_t* __restrict__ offsets,
                                                            int32_t* __restrict__ cnts, int S, int P) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* old_sorted = reinterpret_cast<uint64_t*>(smem);          // P
  uint32_t* new_sorted = reinterpret_cast<uint32_t*>(old_sorted + P);  // P
  int32_t* hit_at_slot = reinterpret_cast<int32_t*>(new_sorted + P);   // S
  int32_t* scan = hit_at_slot + S;                                     // kThreads/64 + 1
  const int64_t base = static_cast<int64_t>(blockIdx.x) * S;
  const int64_t* cur_row = cur + base;
  skv::reorder_row(cached + base, [&](int i) { return cur_row[i]; }, offsets + base, cnts + blockIdx.x, S, P,
                   old_sorted, new_sorted, hit_at_slot, scan);
}

}  // namespace

extern "C" int skv_reorder_keys_and_compute_offsets(int64_t* cached_pos_ids, const int64_t* cur_pos_ids,
                                                    int32_t* offsets, int32_t* cnts, int batch_size,
                                                    int heads, int map_size, void* stream) {
  if (!cached_pos_ids || !cur_pos_ids || !offsets || !cnts) {
    skv_set_error("reorder_keys_and_compute_offsets: null pointer");
    return SKV_EINVAL;
  }
  if (batch_size <= 0 || heads <= 0) {
    skv_set_error("reorder_keys_and_compute_offsets: batch_size=%d heads=%d", batch_size, heads);
    return SKV_EINVAL;
  }
  if (map_size < 1 || map_size > kMaxMap) {
    skv_set_error("reorder_keys_and_compute_offsets: map_size=%d outside [1, %d]", map_size, kMaxMap);
    return SKV_EUNSUPPORTED;
  }
  int P = 64;
  while (P < map_size) P <<= 1;
  const size_t lds = static_cast<size_t>(P) * (8 + 4) + static_cast<size_t>(map_size) * 4 + (kThreads / 64 + 1) * 4;
  hipLaunchKernelGGL(reorder_kernel, dim3(batch_size * heads), dim3(kThreads), lds, static_cast<hipStream_t>(stream),
                     cached_pos_ids, cur_pos_ids, offsets, cnts, map_size, P);
  return skv_check_launch("reorder_keys_and_compute_offsets");
}
