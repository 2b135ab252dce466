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

constexpr int kThreads = 1024;
constexpr int kMaxPool = 16384;  // slots per row (LDS bitmap of 2 KB)
constexpr int kMaxSel = 2048;
constexpr int kSelPer = kMaxSel / kThreads;    // selection entries per thread
constexpr int kSlotPer = kMaxPool / kThreads;  // slots per thread

// One histogram count per lane where `count` holds. Last-use keys cluster on a few recent steps,
// so a wave's bins are often all equal: then one atomic adds the wave's count (instead of up to 64
// atomics on one LDS address); otherwise every counting lane adds its own. Called by whole waves.
__device__ __forceinline__ void hist_add(int* hist, uint32_t bin, bool count) {
  const uint64_t act = __ballot(count);
  if (act == 0) return;
  const int leader = __ffsll(static_cast<unsigned long long>(act)) - 1;
  const uint32_t lb = __builtin_amdgcn_readlane(bin, leader);
  if (__ballot(count && bin != lb) == 0) {
    if ((threadIdx.x & 63) == static_cast<unsigned>(leader)) atomicAdd(&hist[lb], __popcll(act));
  } else if (count) {
    atomicAdd(&hist[bin], 1);
  }
}

// Every thread owns a contiguous range of the selection (<= kSelPer entries) and of the slots
// (<= kSlotPer), so block scans over the threads rank entries and slots in index order. All
// global reads are issued up front (the selection and every slot's last use together, then the
// selected chunks' table entries), so a row costs two dependent round trips; the victims' radix
// select runs on the keys held in registers.
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
  __shared__ uint32_t kmin_sh, kmax_sh;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t* sel = selected + static_cast<int64_t>(row) * S;
  int32_t* so = slot_of + static_cast<int64_t>(row) * chunks;
  int32_t* sc = slot_chunk + static_cast<int64_t>(row) * P;
  int32_t* su = slot_used + static_cast<int64_t>(row) * P;
  int32_t* sl = slot_list + static_cast<int64_t>(row) * S;
  const int32_t t = clock[row] + 1;

  const int sper = (S + kThreads - 1) / kThreads;  // <= kSelPer
  const int j0 = min(S, tid * sper), j1 = min(S, j0 + sper);
  const int pper = (P + kThreads - 1) / kThreads;  // <= kSlotPer
  const int v0 = min(P, tid * pper), v1 = min(P, v0 + pper);
  int64_t c[kSelPer];
#pragma unroll
  for (int u = 0; u < kSelPer; ++u) c[u] = (j0 + u < j1) ? sel[j0 + u] : -1;
  // Victim keys: last use + 1 (empty slots: 0); a hit slot's key is replaced below, so a hit's
  // last-use update racing with this read does not matter.
  uint32_t key[kSlotPer];
#pragma unroll
  for (int u = 0; u < kSlotPer; ++u) key[u] = (v0 + u < v1) ? static_cast<uint32_t>(su[v0 + u] + 1) : 0xffffffffu;
  for (int w = tid; w < (P + 31) / 32; w += kThreads) hit_bits[w] = 0u;
  if (tid == 0) {
    kmin_sh = 0xffffffffu;
    kmax_sh = 0u;
  }
  __syncthreads();
  // Hits keep their slot; the thread remembers which of its entries missed.
  int s[kSelPer];
#pragma unroll
  for (int u = 0; u < kSelPer; ++u) s[u] = (c[u] >= 0 && c[u] < chunks) ? so[c[u]] : -1;
  uint32_t miss_mask = 0;
  int misses = 0;
#pragma unroll
  for (int u = 0; u < kSelPer; ++u) {
    if (j0 + u >= j1) continue;
    if (s[u] >= 0 && s[u] < P) {
      sl[j0 + u] = s[u];
      su[s[u]] = t;
      atomicOr(&hit_bits[s[u] >> 5], 1u << (s[u] & 31));
    } else {
      miss_mask |= 1u << u;
      ++misses;
    }
  }
  int m;
  int miss_rank = skv::block_exclusive_scan(misses, scan, &m);  // its barriers publish hit_bits
#pragma unroll
  for (int u = 0; u < kSlotPer; ++u) {
    const int v = v0 + u;
    if (v < v1 && ((hit_bits[v >> 5] >> (v & 31)) & 1u)) key[u] = 0xffffffffu;
  }

  // Victims: the m smallest keys over the slots (hit slots excluded by their key), by an 8-bit
  // radix select; ties to the lowest slot. Keys are step numbers, so the other slots' keys span
  // few values: they are taken relative to their minimum, and the select runs only over the bytes
  // that span needs (one or two passes instead of four for decodes of up to 65536 steps).
  uint32_t prefix = 0, mask = 0;
  int need = m;
  if (m > 0) {  // workgroup-uniform
    uint32_t lmin = 0xffffffffu, lmax = 0u;
#pragma unroll
    for (int u = 0; u < kSlotPer; ++u) {
      if (v0 + u < v1 && key[u] != 0xffffffffu) {
        lmin = min(lmin, key[u]);
        lmax = max(lmax, key[u]);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      lmin = min(lmin, static_cast<uint32_t>(__shfl_xor(static_cast<int>(lmin), off)));
      lmax = max(lmax, static_cast<uint32_t>(__shfl_xor(static_cast<int>(lmax), off)));
    }
    if ((tid & 63) == 0) {
      atomicMin(&kmin_sh, lmin);
      atomicMax(&kmax_sh, lmax);
    }
    __syncthreads();
    const uint32_t lo = kmin_sh, span = kmax_sh - kmin_sh;  // (m > 0: some slot is not a hit)
    const int passes = span < (1u << 8) ? 1 : span < (1u << 16) ? 2 : span < (1u << 24) ? 3 : 4;
#pragma unroll
    for (int u = 0; u < kSlotPer; ++u)
      if (key[u] != 0xffffffffu) key[u] -= lo;
    // the bytes above the passes are zero for every other slot (and not for a hit slot's key)
    mask = passes == 4 ? 0u : ~((1u << (8 * passes)) - 1u);
    for (int pass = 0; pass < passes; ++pass) {
      const int shift = 8 * (passes - 1 - pass);
      for (int i = tid; i < 256; i += kThreads) hist[i] = 0;
      __syncthreads();
#pragma unroll
      for (int u = 0; u < kSlotPer; ++u)
        hist_add(hist, (key[u] >> shift) & 255u, v0 + u < v1 && (key[u] & mask) == prefix);
      __syncthreads();
      if (tid < 64) {
        int c4[4], tot = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          c4[u] = hist[tid * 4 + u];
          tot += c4[u];
        }
        int before = skv::wave_inclusive_scan(tot) - tot;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (before < need && need <= before + c4[u]) {
            bin_sh = tid * 4 + u;
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
#pragma unroll
    for (int u = 0; u < kSlotPer; ++u) {
      if (v0 + u >= v1) continue;
      lt += key[u] < prefix;
      eq += key[u] == prefix;
    }
  }
  int eq_total, taken_total;
  const int eq_before = skv::block_exclusive_scan(eq, scan, &eq_total);
  const int my_ties = max(0, min(eq_before + eq, need) - eq_before);
  int rank = skv::block_exclusive_scan(lt + my_ties, scan, &taken_total);
  if (m > 0) {
    int e = eq_before;
#pragma unroll
    for (int u = 0; u < kSlotPer; ++u) {
      if (v0 + u >= v1) continue;
      bool take = key[u] < prefix;
      if (key[u] == prefix) take = e++ < need;
      if (take) victim[rank++] = v0 + u;
    }
  }
  __syncthreads();
  // The k-th miss takes victim k; tables and the miss lists are updated. A victim slot holds no
  // selected chunk, so the entries cleared (the victim's old chunk) and set (the miss) are all
  // distinct.
  const int base = S - m;
#pragma unroll
  for (int u = 0; u < kSelPer; ++u) {
    if (!((miss_mask >> u) & 1u)) continue;
    const int64_t cu = c[u];
    const int v = victim[miss_rank];
    const int32_t old = sc[v];
    if (old >= 0 && old < chunks) so[old] = -1;
    if (cu >= 0 && cu < chunks) so[cu] = v;
    sc[v] = static_cast<int32_t>(cu);
    su[v] = t;
    sl[j0 + u] = v;
    miss_ids[static_cast<int64_t>(row) * S + base + miss_rank] = static_cast<int32_t>(cu);
    miss_slot[static_cast<int64_t>(row) * S + base + miss_rank] = v;
    ++miss_rank;
  }
  if (tid == 0) {
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
