// a3: cache-hit reorder of the selected chunk ids against the previous step's slots.
//
// One workgroup (4 wave64) per (batch, kv-head) row. Instead of the reference's LDS hash
// table + warp32 ballots (kernels/map.cuh:475-516), the row is solved by sorting:
//   1. old (id, slot) pairs and new ids are bitonic-sorted in LDS;
//   2. each new id binary-searches the sorted old ids -> hit slot or miss;
//   3. hits are marked at their old slot, so a prefix scan over slots emits them in
//      ascending old-slot order; misses are emitted by a prefix scan over the sorted
//      new ids, i.e. in ascending id order.
// The output is the one map.cuh produces after its block_sort2 (map.cuh:229-259,503-506):
//   ids     = [hit ids by ascending old slot] ++ [miss ids ascending]
//   offsets = [hit old slots ascending]       ++ [miss ids ascending]
// Everything is deterministic: no atomics, no hashing.
#include "skv_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxMap = 2048;

__device__ __forceinline__ void bitonic_sort_u64(uint64_t* a, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        int ixj = i ^ j;
        if (ixj > i) {
          uint64_t x = a[i], y = a[ixj];
          bool asc = (i & k) == 0;
          if ((x > y) == asc) {
            a[i] = y;
            a[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ void bitonic_sort_u32(uint32_t* a, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        int ixj = i ^ j;
        if (ixj > i) {
          uint32_t x = a[i], y = a[ixj];
          bool asc = (i & k) == 0;
          if ((x > y) == asc) {
            a[i] = y;
            a[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Ids are stored as (id + 1) so that the empty marker -1 sorts first and never matches
// a valid (>= 0) new id.
__global__ void __launch_bounds__(kThreads) reorder_kernel(int64_t* __restrict__ cached,
                                                            const int64_t* __restrict__ cur,
                                                            int32_t* __restrict__ offsets,
                                                            int32_t* __restrict__ cnts, int S, int P) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* old_sorted = reinterpret_cast<uint64_t*>(smem);          // P
  uint32_t* new_sorted = reinterpret_cast<uint32_t*>(old_sorted + P);  // P
  int32_t* hit_at_slot = reinterpret_cast<int32_t*>(new_sorted + P);   // S
  int32_t* scan_tmp = hit_at_slot + S;                                 // kThreads/64 + 1

  const int row = blockIdx.x;
  const int64_t base = static_cast<int64_t>(row) * S;

  for (int i = threadIdx.x; i < P; i += blockDim.x) {
    if (i < S) {
      uint32_t ok = static_cast<uint32_t>(static_cast<int32_t>(cached[base + i]) + 1);
      old_sorted[i] = (static_cast<uint64_t>(ok) << 32) | static_cast<uint32_t>(i);
      new_sorted[i] = static_cast<uint32_t>(static_cast<int32_t>(cur[base + i]) + 1);
      hit_at_slot[i] = -1;
    } else {
      old_sorted[i] = ~0ull;
      new_sorted[i] = 0xffffffffu;
    }
  }
  __syncthreads();
  bitonic_sort_u64(old_sorted, P);
  bitonic_sort_u32(new_sorted, P);

  // Classify the sorted new ids. Thread t owns the contiguous run [t*E, t*E+E).
  const int E = (S + blockDim.x - 1) / blockDim.x;
  const int lo = threadIdx.x * E;
  const int hi = min(lo + E, S);
  uint32_t miss_mask = 0;  // E <= kMaxMap/kThreads = 8 bits
  int my_misses = 0;
  for (int i = lo; i < hi; ++i) {
    uint32_t key = new_sorted[i];
    uint64_t probe = static_cast<uint64_t>(key) << 32;
    int a = 0, b = P;  // lower_bound over old_sorted
    while (a < b) {
      int m = (a + b) >> 1;
      if (old_sorted[m] < probe) a = m + 1; else b = m;
    }
    bool hit = key != 0u && a < P && static_cast<uint32_t>(old_sorted[a] >> 32) == key;
    if (hit) {
      hit_at_slot[static_cast<uint32_t>(old_sorted[a])] = static_cast<int32_t>(key) - 1;
    } else {
      miss_mask |= 1u << (i - lo);
      ++my_misses;
    }
  }
  __syncthreads();

  // Hits in ascending old-slot order.
  int my_hits = 0;
  for (int j = lo; j < hi; ++j) my_hits += hit_at_slot[j] >= 0;
  int total_hits = 0;
  int hrank = skv::block_exclusive_scan(my_hits, scan_tmp, &total_hits);
  int total_misses = 0;
  int mrank = skv::block_exclusive_scan(my_misses, scan_tmp, &total_misses);

  // All reads of `cached` happened before the first barrier; it is safe to overwrite now.
  for (int j = lo; j < hi; ++j) {
    int id = hit_at_slot[j];
    if (id >= 0) {
      cached[base + hrank] = id;
      offsets[base + hrank] = j;
      ++hrank;
    }
  }
  for (int i = lo; i < hi; ++i) {
    if (miss_mask & (1u << (i - lo))) {
      int id = static_cast<int32_t>(new_sorted[i]) - 1;
      cached[base + total_hits + mrank] = id;
      offsets[base + total_hits + mrank] = id;
      ++mrank;
    }
  }
  if (threadIdx.x == 0) cnts[row] = total_hits;
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
  size_t lds = static_cast<size_t>(P) * (8 + 4) + static_cast<size_t>(map_size) * 4 + (kThreads / 64 + 1) * 4;
  hipLaunchKernelGGL(reorder_kernel, dim3(batch_size * heads), dim3(kThreads), lds,
                     static_cast<hipStream_t>(stream), cached_pos_ids, cur_pos_ids, offsets, cnts, map_size, P);
  return skv_check_launch("reorder_keys_and_compute_offsets");
}
