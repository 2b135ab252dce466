// Workgroup-level building blocks of chunk selection, shared by the standalone top-k and
// reorder kernels and the fused selection kernel. All functions are called by every thread
// of the workgroup (they contain barriers).
#pragma once

#include "skv_common.h"

namespace skv {

// Bitonic sort of n (power of two) keys in LDS, ascending.
template <typename T>
__device__ __forceinline__ void block_bitonic_sort(T* a, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const T x = a[i], y = a[ixj];
          if ((x > y) == ((i & k) == 0)) {
            a[i] = y;
            a[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Wave 0 finds bin b with above(b) < want <= above(b) + hist[b], where above(b) counts the
// entries in bins > b; out[0] = b, out[1] = above(b).
__device__ __forceinline__ void select_bin(const uint32_t* hist, int want, int* out) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    uint32_t h[4];
    int local = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      h[u] = hist[255 - 4 * lane - u];
      local += static_cast<int>(h[u]);
    }
    const int incl = wave_inclusive_scan(local);
    int above = incl - local;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (above < want && want <= above + static_cast<int>(h[u])) {
        out[0] = 255 - 4 * lane - u;
        out[1] = above;
      }
      above += static_cast<int>(h[u]);
    }
  }
  __syncthreads();
}

struct TopkShared {
  uint32_t hist[256];
  int found[2];
  int scan[17];
};

// Radix top-k over n 16-bit order keys key(j) (larger key = better). Fills sel[0..k) with
// ((0xffff - key) << 32 | j) for the k winners under (key desc, j asc), sorted ascending,
// i.e. best first; sel must hold P >= k entries (P a power of two), the tail is padded.
// `hist_done` tells that sh.hist already holds the high-byte histogram of all keys.
template <typename KeyFn>
__device__ void radix_topk(KeyFn key, int n, int k, int P, uint64_t* sel, TopkShared& sh, bool hist_done) {
  if (!hist_done) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) sh.hist[i] = 0;
    __syncthreads();
    for (int j = threadIdx.x; j < n; j += blockDim.x) atomicAdd(&sh.hist[key(j) >> 8], 1u);
    __syncthreads();
  }
  select_bin(sh.hist, k, sh.found);
  const uint32_t b1 = static_cast<uint32_t>(sh.found[0]);
  const int above1 = sh.found[1];
  __syncthreads();
  for (int i = threadIdx.x; i < 256; i += blockDim.x) sh.hist[i] = 0;
  __syncthreads();
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    const uint32_t kj = key(j);
    if ((kj >> 8) == b1) atomicAdd(&sh.hist[kj & 255u], 1u);
  }
  __syncthreads();
  select_bin(sh.hist, k - above1, sh.found);
  const uint32_t T = (b1 << 8) | static_cast<uint32_t>(sh.found[0]);
  const int c_gt = above1 + sh.found[1];
  const int need_eq = k - c_gt;

  // Order-preserving compaction, one block of blockDim elements at a time.
  int gt_base = 0, eq_base = 0;
  for (int blk = 0; blk * static_cast<int>(blockDim.x) < n; ++blk) {
    const int j = blk * blockDim.x + threadIdx.x;
    uint32_t kj = 0;
    bool gt = false, eq = false;
    if (j < n) {
      kj = key(j);
      gt = kj > T;
      eq = kj == T;
    }
    int total = 0;
    const int excl = block_exclusive_scan(static_cast<int>(gt) | (static_cast<int>(eq) << 16), sh.scan, &total);
    const uint64_t composite = (static_cast<uint64_t>(0xffffu - kj) << 32) | static_cast<uint32_t>(j);
    if (gt) sel[gt_base + (excl & 0xffff)] = composite;
    if (eq) {
      const int r = eq_base + (excl >> 16);
      if (r < need_eq) sel[c_gt + r] = composite;
    }
    gt_base += total & 0xffff;
    eq_base += total >> 16;
    if (gt_base >= c_gt && eq_base >= need_eq) break;  // workgroup-uniform
  }
  for (int i = k + threadIdx.x; i < P; i += blockDim.x) sel[i] = ~0ull;
  __syncthreads();
  block_bitonic_sort(sel, P);
}

// Reorder of one row: old[0..S) holds the previous slot ids (-1 = empty), new_ids[0..S) the
// newly selected ids (unique, >= 0). Produces, in place of old:
//   old     <- [hit ids by ascending old slot] ++ [miss ids ascending]
//   offsets <- [old slots of the hits, ascending] ++ [miss ids ascending],  *cnt <- #hits.
// LDS: old_sorted[P] (u64), new_sorted[P] (u32), hit_at_slot[S] (int), scan[blockDim/64+1].
// new_ids may alias nothing written here; old is read completely before it is written.
template <typename NewIdFn>
__device__ void reorder_row(int64_t* old, NewIdFn new_id, int32_t* offsets, int32_t* cnt, int S, int P,
                            uint64_t* old_sorted, uint32_t* new_sorted, int32_t* hit_at_slot, int* scan) {
  for (int i = threadIdx.x; i < P; i += blockDim.x) {
    if (i < S) {
      const uint32_t ok = static_cast<uint32_t>(static_cast<int32_t>(old[i]) + 1);
      old_sorted[i] = (static_cast<uint64_t>(ok) << 32) | static_cast<uint32_t>(i);
      new_sorted[i] = static_cast<uint32_t>(static_cast<int32_t>(new_id(i)) + 1);
      hit_at_slot[i] = -1;
    } else {
      old_sorted[i] = ~0ull;
      new_sorted[i] = 0xffffffffu;
    }
  }
  __syncthreads();
  block_bitonic_sort(old_sorted, P);
  block_bitonic_sort(new_sorted, P);

  const int E = (S + blockDim.x - 1) / blockDim.x;  // <= 8 for S <= 2048 and 256 threads
  const int lo = threadIdx.x * E;
  const int hi = min(lo + E, S);
  uint32_t miss_mask = 0;
  int my_misses = 0;
  for (int i = lo; i < hi; ++i) {
    const uint32_t key = new_sorted[i];
    const uint64_t probe = static_cast<uint64_t>(key) << 32;
    int a = 0, b = P;
    while (a < b) {
      const int m = (a + b) >> 1;
      if (old_sorted[m] < probe) a = m + 1; else b = m;
    }
    const bool hit = key != 0u && a < P && static_cast<uint32_t>(old_sorted[a] >> 32) == key;
    if (hit) {
      hit_at_slot[static_cast<uint32_t>(old_sorted[a])] = static_cast<int32_t>(key) - 1;
    } else {
      miss_mask |= 1u << (i - lo);
      ++my_misses;
    }
  }
  __syncthreads();
  int my_hits = 0;
  for (int j = lo; j < hi; ++j) my_hits += hit_at_slot[j] >= 0;
  int total_hits = 0, total_misses = 0;
  int hrank = block_exclusive_scan(my_hits, scan, &total_hits);
  int mrank = block_exclusive_scan(my_misses, scan, &total_misses);
  for (int j = lo; j < hi; ++j) {
    const int id = hit_at_slot[j];
    if (id >= 0) {
      old[hrank] = id;
      offsets[hrank] = j;
      ++hrank;
    }
  }
  for (int i = lo; i < hi; ++i) {
    if (miss_mask & (1u << (i - lo))) {
      const int id = static_cast<int32_t>(new_sorted[i]) - 1;
      old[total_hits + mrank] = id;
      offsets[total_hits + mrank] = id;
      ++mrank;
    }
  }
  if (threadIdx.x == 0) *cnt = total_hits;
}

}  // namespace skv
