// a4/a5: chunk copies into the GPU-resident sparse K/V region.
//
// The reference moves 2 KB chunks with one 128-thread block per (b,h) and a pair of blocks
// coupled by a spin flag (kernels/copy.cuh:438-498). Here the work is split into two
// stream-ordered kernels, so no workgroup ever waits on another:
//   compact_hits_kernel  — one workgroup per row performs the in-place forward compaction
//                          slot[i] <- slot[offsets[i]] for i < cnt (offsets ascending, offsets[i] >= i);
//   gather_chunks_kernel — a bounded grid of workgroups fetches the miss chunks i >= cnt straight
//                          from the pinned host store (zero-copy 16-byte non-temporal loads over
//                          the host link), each workgroup keeping 8 loads per lane in flight.
// The copy unit is a chunk of chunk_elems bf16 values, moved as 16-byte vectors.
#include <algorithm>
#include <cstdlib>

#include "fetch_role.h"
#include "skv_common.h"

namespace {

using skv::u32x4;

constexpr int kThreads = 256;
constexpr int kUnroll = 8;  // 16-byte vectors in flight per lane (hit compaction)
using skv::fetch_workgroups;
using skv::kChunksPerFetchWG;

// In-place forward compaction of the hit chunks of one row. Offsets are strictly ascending
// with offsets[i] >= i, so the hits whose offset equals their index form a prefix that is
// already in place; the rest are moved in batches. Within a batch every load is drained
// before any store (a source slot of one chunk can be the destination of another chunk of
// the same batch); a later batch only reads slots beyond every destination of earlier ones.
// One workgroup per row: the row's offsets are read once into LDS (map_size <= kCompactLdsMap;
// beyond that they are read from global memory), so a batch costs one round trip for its loads
// and one for its stores. Long maps (>= kCompactWideMap slots) take 1024 threads (batches of 64
// chunks of 2 KB); short ones 256, which keeps the many small rows of a batched decode step from
// crowding the concurrent host-link fetch (Llama-3.1-8B batch 8, 256 slots: 1024 threads cost
// 1.7 of 383 tokens/s; Llama-3-8B-1M, 2048 slots: the value-hit move takes 7 µs against 29 µs
// with 256 threads re-reading the offsets per batch).
constexpr int kCompactLdsMap = 8192;
constexpr int kCompactWideMap = 1024;

template <bool kLdsOffsets, int kCompactThreads>
__global__ void __launch_bounds__(kCompactThreads) compact_hits_kernel(u32x4* __restrict__ buf,
                                                                        const int32_t* __restrict__ offsets,
                                                                        const int32_t* __restrict__ cnts,
                                                                        int64_t row_stride_vec, int64_t row_offset_vec,
                                                                        int S, int chunk_vec) {
  __shared__ int offs_lds[kLdsOffsets ? kCompactLdsMap : 1];
  __shared__ int first_moved;
  const int row = blockIdx.x;
  const int cnt = min(cnts[row], S);
  if (cnt <= 0) return;
  const int32_t* offs = offsets + static_cast<int64_t>(row) * S;
  if (threadIdx.x == 0) first_moved = cnt;
  __syncthreads();
  for (int j = threadIdx.x; j < cnt; j += blockDim.x) {
    const int o = offs[j];
    if (kLdsOffsets) offs_lds[j] = o;
    if (o != j) atomicMin(&first_moved, j);
  }
  __syncthreads();
  const int32_t* src_of = kLdsOffsets ? offs_lds : offs;
  const int p = first_moved;
  u32x4* base = buf + static_cast<int64_t>(row) * row_stride_vec + row_offset_vec;
  const int total = (cnt - p) * chunk_vec;  // < 2^31: map_size * chunk_vec is bounded on the host
  for (int v0 = 0; v0 < total; v0 += static_cast<int>(blockDim.x) * kUnroll) {
    u32x4 r[kUnroll];
    int dst[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int v = v0 + u * static_cast<int>(blockDim.x) + static_cast<int>(threadIdx.x);
      dst[u] = -1;
      if (v < total) {
        const int j = p + v / chunk_vec;
        const int e = v - (j - p) * chunk_vec;
        const int src = src_of[j];
        if (src >= 0 && src < S) {
          r[u] = base[static_cast<int64_t>(src) * chunk_vec + e];
          dst[u] = j * chunk_vec + e;
        }
      }
    }
    skv::drain_and_barrier();
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (dst[u] >= 0) base[dst[u]] = r[u];
  }
}

void launch_compact_hits(u32x4* buf, const int32_t* offsets, const int32_t* cnts, int rows, int64_t row_stride_vec,
                         int64_t row_offset_vec, int S, int chunk_vec, hipStream_t s) {
  if (S < kCompactWideMap)
    hipLaunchKernelGGL((compact_hits_kernel<true, 256>), dim3(rows), dim3(256), 0, s, buf, offsets, cnts,
                       row_stride_vec, row_offset_vec, S, chunk_vec);
  else if (S <= kCompactLdsMap)
    hipLaunchKernelGGL((compact_hits_kernel<true, 1024>), dim3(rows), dim3(1024), 0, s, buf, offsets, cnts,
                       row_stride_vec, row_offset_vec, S, chunk_vec);
  else
    hipLaunchKernelGGL((compact_hits_kernel<false, 1024>), dim3(rows), dim3(1024), 0, s, buf, offsets, cnts,
                       row_stride_vec, row_offset_vec, S, chunk_vec);
}

// The miss gather over a grid of fetch workgroups (skv::fetch_role).
template <typename IdxT>
__global__ void __launch_bounds__(kThreads) gather_chunks_kernel(skv::FetchArgs<IdxT> f) {
  skv::fetch_role(f, blockIdx.x, gridDim.x);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_common(const char* what, const void* a, const void* b, int batch_size, int heads, int map_size,
                 int chunk_elems) {
  if ((a != nullptr && !aligned16(a)) || (b != nullptr && !aligned16(b))) {
    skv_set_error("%s: buffers must be 16-byte aligned", what);
    return SKV_EINVAL;
  }
  if (batch_size <= 0 || heads <= 0 || map_size <= 0) {
    skv_set_error("%s: batch_size=%d heads=%d map_size=%d", what, batch_size, heads, map_size);
    return SKV_EINVAL;
  }
  if (chunk_elems <= 0 || chunk_elems % 8 != 0) {
    skv_set_error("%s: chunk_elems=%d must be a positive multiple of 8 (16-byte units)", what, chunk_elems);
    return SKV_EUNSUPPORTED;
  }
  if (static_cast<int64_t>(map_size) * chunk_elems > (int64_t{1} << 31)) {
    skv_set_error("%s: map_size=%d chunks of %d elements exceed 2^31 elements per row", what, map_size, chunk_elems);
    return SKV_EUNSUPPORTED;
  }
  return SKV_OK;
}

}  // namespace

extern "C" int skv_gather_copy_d2d_with_offsets(void* keys, const int32_t* offsets, const int32_t* cnts,
                                                int batch_size, int heads, int64_t gpu_k_length,
                                                int64_t gpu_k_offset, int64_t gpu_k_stride, int map_size,
                                                int chunk_elems, void* stream) {
  const char* what = "gather_copy_d2d_with_offsets";
  if (!keys || !offsets || !cnts) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  int rc = check_common(what, keys, nullptr, batch_size, heads, map_size, chunk_elems);
  if (rc) return rc;
  if (gpu_k_offset % 8 || gpu_k_stride % 8 || gpu_k_length != static_cast<int64_t>(map_size) * chunk_elems) {
    skv_set_error("%s: offset=%lld stride=%lld must be multiples of 8, length=%lld must be map_size*chunk_elems", what,
                  (long long)gpu_k_offset, (long long)gpu_k_stride, (long long)gpu_k_length);
    return SKV_EINVAL;
  }
  launch_compact_hits(static_cast<u32x4*>(keys), offsets, cnts, batch_size * heads, gpu_k_stride / 8, gpu_k_offset / 8,
                      map_size, chunk_elems / 8, static_cast<hipStream_t>(stream));
  return skv_check_launch(what);
}

namespace {

// The fetch role's arguments for rows of map_size slots (int32 chunk ids at `offsets`).
void fetch_args(const void* values, void* v_cache_buffer, const int32_t* offsets, const int32_t* cnts, int rows,
               int64_t cpu_v_length, int64_t gpu_v_offset, int64_t gpu_v_stride, int map_size, int chunk_elems,
               const int32_t* dst_slot, int pool_slots, skv::FetchArgs<int32_t>* f) {
  f->src = static_cast<const u32x4*>(values);
  f->src_row_vec = cpu_v_length / 8;
  f->dst = static_cast<u32x4*>(v_cache_buffer);
  f->dst_row_vec = gpu_v_stride / 8;
  f->dst_offset_vec = gpu_v_offset / 8;
  f->ids = offsets;
  f->cnts = cnts;
  f->dst_slot = dst_slot;
  f->pool_slots = pool_slots;
  f->S = map_size;
  f->chunk_vec = chunk_elems / 8;
  f->src_chunks = cpu_v_length / chunk_elems;
  f->rows = rows;
  f->tiles = (map_size + kChunksPerFetchWG - 1) / kChunksPerFetchWG;
  f->workgroups = skv::fetch_workgroups_for(values, rows * f->tiles);
}

// Shared by the two value-fetch entry points: argument checks, then (compact) the in-buffer hit
// move and the host-link gather of the misses, in that order on one stream.
int value_fetch(const char* what, bool compact, const void* values, void* v_cache_buffer, const int32_t* offsets,
                const int32_t* cnts, int batch_size, int heads, int64_t cpu_v_length, int64_t gpu_v_length,
                int64_t gpu_v_offset, int64_t gpu_v_stride, int map_size, int chunk_elems, void* stream,
                const int32_t* dst_slot = nullptr, int pool_slots = 0) {
  if (!values || !v_cache_buffer || !offsets || !cnts) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  int rc = check_common(what, values, v_cache_buffer, batch_size, heads, map_size, chunk_elems);
  if (rc) return rc;
  if (cpu_v_length % 8 || gpu_v_offset % 8 || gpu_v_stride % 8 ||
      gpu_v_length != static_cast<int64_t>(map_size) * chunk_elems) {
    skv_set_error("%s: cpu_v_length=%lld offset=%lld stride=%lld must be multiples of 8, gpu_v_length=%lld must be "
                  "map_size*chunk_elems", what, (long long)cpu_v_length, (long long)gpu_v_offset,
                  (long long)gpu_v_stride, (long long)gpu_v_length);
    return SKV_EINVAL;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rows = batch_size * heads;
  if (compact) {
    launch_compact_hits(static_cast<u32x4*>(v_cache_buffer), offsets, cnts, rows, gpu_v_stride / 8, gpu_v_offset / 8,
                        map_size, chunk_elems / 8, s);
    rc = skv_check_launch(what);
    if (rc) return rc;
  }
  skv::FetchArgs<int32_t> f{};
  fetch_args(values, v_cache_buffer, offsets, cnts, rows, cpu_v_length, gpu_v_offset, gpu_v_stride, map_size,
             chunk_elems, dst_slot, pool_slots, &f);
  hipLaunchKernelGGL(gather_chunks_kernel<int32_t>, dim3(f.workgroups), dim3(kThreads), 0, s, f);
  return skv_check_launch(what);
}

}  // namespace

extern "C" int skv_gather_copy_with_offsets(const void* values, void* v_cache_buffer, const int32_t* offsets,
                                            const int32_t* cnts, int batch_size, int heads, int64_t cpu_v_length,
                                            int64_t gpu_v_length, int64_t gpu_v_offset, int64_t gpu_v_stride,
                                            int map_size, int chunk_elems, void* stream) {
  return value_fetch("gather_copy_with_offsets", true, values, v_cache_buffer, offsets, cnts, batch_size, heads,
                     cpu_v_length, gpu_v_length, gpu_v_offset, gpu_v_stride, map_size, chunk_elems, stream);
}

extern "C" int skv_gather_copy_misses_to_slots(const void* values, void* v_cache_buffer, const int32_t* miss_ids,
                                               const int32_t* cnts, const int32_t* miss_slot, int batch_size,
                                               int heads, int64_t cpu_v_length, int64_t pool_offset,
                                               int64_t gpu_v_stride, int map_size, int pool_slots, int chunk_elems,
                                               void* stream) {
  if (!miss_slot || pool_slots < map_size) {
    skv_set_error("gather_copy_misses_to_slots: miss_slot=%p pool_slots=%d map_size=%d",
                  static_cast<const void*>(miss_slot), pool_slots, map_size);
    return SKV_EINVAL;
  }
  return value_fetch("gather_copy_misses_to_slots", false, values, v_cache_buffer, miss_ids, cnts, batch_size, heads,
                     cpu_v_length, static_cast<int64_t>(map_size) * chunk_elems, pool_offset, gpu_v_stride, map_size,
                     chunk_elems, stream, miss_slot, pool_slots);
}

extern "C" int skv_gather_copy_misses_with_offsets(const void* values, void* v_cache_buffer, const int32_t* offsets,
                                                   const int32_t* cnts, int batch_size, int heads,
                                                   int64_t cpu_v_length, int64_t gpu_v_length, int64_t gpu_v_offset,
                                                   int64_t gpu_v_stride, int map_size, int chunk_elems, void* stream) {
  return value_fetch("gather_copy_misses_with_offsets", false, values, v_cache_buffer, offsets, cnts, batch_size,
                     heads, cpu_v_length, gpu_v_length, gpu_v_offset, gpu_v_stride, map_size, chunk_elems, stream);
}

extern "C" int skv_gather_copy(const void* values, void* v_cache_buffer, const int64_t* position_ids, int batch_size,
                               int heads, int64_t cpu_v_length, int64_t gpu_v_length, int map_size, int chunk_elems,
                               void* stream) {
  const char* what = "gather_copy";
  if (!values || !v_cache_buffer || !position_ids) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  int rc = check_common(what, values, v_cache_buffer, batch_size, heads, map_size, chunk_elems);
  if (rc) return rc;
  if (cpu_v_length % 8 || gpu_v_length % 8 || gpu_v_length < static_cast<int64_t>(map_size) * chunk_elems) {
    skv_set_error("%s: cpu_v_length=%lld gpu_v_length=%lld invalid", what, (long long)cpu_v_length,
                  (long long)gpu_v_length);
    return SKV_EINVAL;
  }
  const int rows = batch_size * heads;
  skv::FetchArgs<int64_t> f{};
  f.src = static_cast<const u32x4*>(values);
  f.src_row_vec = cpu_v_length / 8;
  f.dst = static_cast<u32x4*>(v_cache_buffer);
  f.dst_row_vec = gpu_v_length / 8;
  f.dst_offset_vec = 0;
  f.ids = position_ids;
  f.S = map_size;
  f.chunk_vec = chunk_elems / 8;
  f.src_chunks = cpu_v_length / chunk_elems;
  f.rows = rows;
  f.tiles = (map_size + kChunksPerFetchWG - 1) / kChunksPerFetchWG;
  f.workgroups = skv::fetch_workgroups_for(values, rows * f.tiles);
  hipLaunchKernelGGL(gather_chunks_kernel<int64_t>, dim3(f.workgroups), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), f);
  return skv_check_launch(what);
}
