// f3: a device chunk cache larger than the selection (a pool of P >= S chunk slots per (b, h) and
// layer), in place of the slot reuse of the reference's reorder (kernels/map.cuh:475-516) when the
// cache is built with one.
//
// pool_assign_kernel: one workgroup per (b, h) row. The step's selected chunk ids are looked up in
// the row's chunk -> slot table; a selected chunk already in the pool is a hit and keeps its slot.
// The misses take the least recently used slots that hold no selected chunk (empty slots first,
// then ascending last-use step, ties to the lowest slot); the k-th miss in selection order takes
// the k-th of those slots in ascending slot order. The tables are updated in place, and the misses
// are listed at the tail [cnts[r], S) of miss_ids / miss_slot, the form the chunk-gather and
// rebuild kernels take (entries i >= cnts[r] are fetched / rebuilt into slot miss_slot[i]).
#include "skv_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxPool = 16384;  // slots per row (LDS bitmap of 2 KB)
constexpr int kMaxSel = 2048;
constexpr int kSelPerThread = kMaxSel / kThreads;

__global__ void __launch_bounds__(kThreads) pool_assign_kernel(const int64_t* __restrict__ selected, int S,
                                                               int chunks, int P, int32_t* __restrict__ slot_of,
                                                               int32_t* __restrict__ slot_chunk,
                                                               int32_t* __restrict__ slot_used,
                                                               int32_t* __restrict__ clock,
                                                               int32_t* __restrict__ slot_list,
                                                               int32_t* __restrict__ miss_ids,
                                                               int32_t* __restrict__ miss_slot,
                                                               int32_t* __restrict__ cnts) {
  __shared__ uint32_t hit_bits[kMaxPool / 32];
  __shared__ int victim[kMaxSel];
  __shared__ int hist[256];
  __shared__ int scan[kThreads / 64 + 1];
  __shared__ int bin_sh, need_sh;
  const int row = blockIdx.x;
  const int64_t* sel = selected + static_cast<int64_t>(row) * S;
  int32_t* so = slot_of + static_cast<int64_t>(row) * chunks;
  int32_t* sc = slot_chunk + static_cast<int64_t>(row) * P;
  int32_t* su = slot_used + static_cast<int64_t>(row) * P;
  int32_t* sl = slot_list + static_cast<int64_t>(row) * S;
  const int32_t t = clock[row] + 1;

  for (int w = threadIdx.x; w < (P + 31) / 32; w += kThreads) hit_bits[w] = 0u;
  __syncthreads();
  // Hits keep their slot. Each thread owns a contiguous range of the selection (order kept) and
  // remembers which of its entries missed.
  const int sper = (S + kThreads - 1) / kThreads;  // <= kSelPerThread
  const int j0 = min(S, static_cast<int>(threadIdx.x) * sper), j1 = min(S, j0 + sper);
  uint32_t miss_mask = 0;
  int misses = 0;
  for (int j = j0; j < j1; ++j) {
    const int64_t c = sel[j];
    const int s = (c >= 0 && c < chunks) ? so[c] : -1;
    if (s >= 0 && s < P) {
      sl[j] = s;
      su[s] = t;
      atomicOr(&hit_bits[s >> 5], 1u << (s & 31));
    } else {
      miss_mask |= 1u << (j - j0);
      ++misses;
    }
  }
  int m;
  int miss_rank = skv::block_exclusive_scan(misses, scan, &m);  // its barriers publish hit_bits

  // Victims: the m smallest keys over the slots, key = last use + 1 (empty slots: 0; hit slots
  // excluded), by a 4-pass 8-bit radix select; ties to the lowest slot.
  const int pper = (P + kThreads - 1) / kThreads;
  const int v0 = min(P, static_cast<int>(threadIdx.x) * pper), v1 = min(P, v0 + pper);
  auto key_of = [&](int v) -> uint32_t {
    if ((hit_bits[v >> 5] >> (v & 31)) & 1u) return 0xffffffffu;
    return static_cast<uint32_t>(su[v] + 1);  // last use >= -1
  };
  uint32_t prefix = 0, mask = 0;
  int need = m;
  if (m > 0) {  // workgroup-uniform
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      for (int i = threadIdx.x; i < 256; i += kThreads) hist[i] = 0;
      __syncthreads();
      for (int v = v0; v < v1; ++v) {
        const uint32_t kk = key_of(v);
        if ((kk & mask) == prefix) atomicAdd(&hist[(kk >> shift) & 255], 1);
      }
      __syncthreads();
      if (threadIdx.x < 64) {
        int c4[4], tot = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          c4[u] = hist[threadIdx.x * 4 + u];
          tot += c4[u];
        }
        int before = skv::wave_inclusive_scan(tot) - tot;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (before < need && need <= before + c4[u]) {
            bin_sh = threadIdx.x * 4 + u;
            need_sh = need - before;
          }
          before += c4[u];
        }
      }
      __syncthreads();
      prefix |= static_cast<uint32_t>(bin_sh) << shift;
      mask |= 0xffu << shift;
      need = need_sh;
      __syncthreads();
    }
  }
  // Victims in ascending slot order: keys below the threshold, and the first `need` keys equal to
  // it (lowest slots); each thread's first victim rank from two block scans over the slot ranges.
  int lt = 0, eq = 0;
  if (m > 0) {
    for (int v = v0; v < v1; ++v) {
      const uint32_t kk = key_of(v);
      lt += kk < prefix;
      eq += kk == prefix;
    }
  }
  int eq_total, taken_total;
  const int eq_before = skv::block_exclusive_scan(eq, scan, &eq_total);
  const int my_ties = max(0, min(eq_before + eq, need) - eq_before);
  int rank = skv::block_exclusive_scan(lt + my_ties, scan, &taken_total);
  if (m > 0) {
    int e = eq_before;
    for (int v = v0; v < v1; ++v) {
      const uint32_t kk = key_of(v);
      bool take = kk < prefix;
      if (kk == prefix) take = e++ < need;
      if (take) victim[rank++] = v;
    }
  }
  __syncthreads();
  // The k-th miss takes victim k; tables and the miss lists are updated. A victim slot holds no
  // selected chunk, so the entries cleared (the victim's old chunk) and set (the miss) are all
  // distinct.
  const int base = S - m;
  for (int j = j0; j < j1; ++j) {
    if (!((miss_mask >> (j - j0)) & 1u)) continue;
    const int64_t c = sel[j];
    const int v = victim[miss_rank];
    const int32_t old = sc[v];
    if (old >= 0 && old < chunks) so[old] = -1;
    if (c >= 0 && c < chunks) so[c] = v;
    sc[v] = static_cast<int32_t>(c);
    su[v] = t;
    sl[j] = v;
    miss_ids[static_cast<int64_t>(row) * S + base + miss_rank] = static_cast<int32_t>(c);
    miss_slot[static_cast<int64_t>(row) * S + base + miss_rank] = v;
    ++miss_rank;
  }
  if (threadIdx.x == 0) {
    cnts[row] = base;
    clock[row] = t;
  }
}

}  // namespace

extern "C" int skv_pool_assign(const int64_t* selected, int rows, int select_sets, int num_chunks, int pool_slots,
                               int32_t* slot_of, int32_t* slot_chunk, int32_t* slot_used, int32_t* clock,
                               int32_t* slot_list, int32_t* miss_ids, int32_t* miss_slot, int32_t* cnts,
                               void* stream) {
  const char* what = "pool_assign";
  if (!selected || !slot_of || !slot_chunk || !slot_used || !clock || !slot_list || !miss_ids || !miss_slot ||
      !cnts) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (rows < 1 || select_sets < 1 || select_sets > kMaxSel || pool_slots < select_sets || pool_slots > kMaxPool ||
      num_chunks < 1) {
    skv_set_error("%s: rows=%d select_sets=%d pool_slots=%d num_chunks=%d (1 <= select_sets <= %d, select_sets "
                  "<= pool_slots <= %d)", what, rows, select_sets, pool_slots, num_chunks, kMaxSel, kMaxPool);
    return SKV_EUNSUPPORTED;
  }
  hipLaunchKernelGGL(pool_assign_kernel, dim3(rows), dim3(kThreads), 0, static_cast<hipStream_t>(stream), selected,
                     select_sets, num_chunks, pool_slots, slot_of, slot_chunk, slot_used, clock, slot_list, miss_ids,
                     miss_slot, cnts);
  return skv_check_launch(what);
}
