// The value-fetch role: miss chunks gathered from the pinned host store (zero-copy 16-byte
// non-temporal loads over the host link) into the GPU value buffer. Shared by gather_chunks_kernel
// (gather_copy.hip) and by the one-launch value fetch + key rebuild (rebuild.hip), where the first
// workgroups of the grid take this role.
#pragma once

#include <cstdlib>

#include "skv_common.h"

namespace skv {

constexpr int kFetchUnroll = 8;        // 16-byte vectors in flight per lane
constexpr int kChunksPerFetchWG = 16;  // miss chunks per fetch tile
// Upper bound on fetch workgroups (environment SKV_FETCH_WGS overrides it, read once). The
// fetch is host-link bound, and every host read in flight also slows the HBM traffic of kernels
// running concurrently (measured: a 4096x28672 GEMM 1.9x slower beside 32 workgroups, 2.7x
// beside 256; landmark scoring 1.1x vs 3.1x). 48 workgroups of 256 threads (1.5 MiB of
// non-temporal loads in flight) give the fastest pipelined Llama-3-8B decode step on MI355X
// (tokens/s at 32/40/44/48/52/56/64/96 workgroups: 354/368/375/381/376/365/344/305), and the
// fastest GLM-4-9B one (418.5 vs 414.0 / 415.3 / 407.4 at 32 / 96 / 160).
constexpr int kDefaultFetchWGs = 48;

inline int fetch_workgroups() {
  static const int wgs = [] {
    const char* e = getenv("SKV_FETCH_WGS");
    const int v = e ? atoi(e) : 0;
    return (v >= 1 && v <= 65536) ? v : kDefaultFetchWGs;
  }();
  return wgs;
}

// Fetch workgroups (of 4 waves' worth) of a launch that also rebuilds keys (fetch_rebuild_kernel,
// one-lane decoders, where nothing else runs beside the fetch); environment SKV_FUSED_FETCH_WGS
// overrides it, read once. Measured on MI355X, GLM-4-9B batch 4 (128 tiles of 16 chunks, 2-wave
// workgroups): 443 tokens/s with 128 workgroups (one tile each), 441 with 64, 428 with 96 and 414
// with 112 (a second round of tiles for some of them); Llama-3-8B-1M (1024 tiles): 38.0-38.5 from
// 32 to 64 four-wave workgroups, 35.3 with 24.
constexpr int kDefaultFusedFetchWGs = 64;

inline int fused_fetch_workgroups_target() {
  static const int wgs = [] {
    const char* e = getenv("SKV_FUSED_FETCH_WGS");
    const int v = e ? atoi(e) : 0;
    return (v >= 1 && v <= 65536) ? v : kDefaultFusedFetchWGs;
  }();
  return wgs;
}

// Whether the value store at p is device memory (a store kept in HBM, e.g. value_store="device"
// of the cache) rather than pinned host memory read over the host link; false when the runtime
// cannot tell. A gather from HBM has none of the host reads' cost to concurrent kernels and wants
// the whole GPU: the fetch launches then take kDeviceFetchWGs workgroups (MI355X, Llama-3.1-8B
// batch 8 ctx 122880 with the store in HBM, one-launch fetch + rebuild, tokens/s at 64 / 128 /
// 256 / 512 fetch workgroups: 741.7 / 887.0 / 989.8 / 997.8).
constexpr int kDeviceFetchWGs = 512;

inline bool is_device_memory(const void* p) {
  hipPointerAttribute_t a{};
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();  // (an unregistered host pointer: not device memory; clear the error it left)
    return false;
  }
  return a.type == hipMemoryTypeDevice;
}

// Fetch workgroups for a launch over `tiles` fetch tiles reading `src`: every tile its own
// workgroup up to kDeviceFetchWGs for a store in device memory, fetch_workgroups() for one in
// pinned host memory.
inline int fetch_workgroups_for(const void* src, int tiles) {
  const int cap = is_device_memory(src) ? kDeviceFetchWGs : fetch_workgroups();
  return tiles < cap ? tiles : cap;
}

// dst slot i of row <- src chunk ids[row*S + i] of row, for i in [start, S) where start =
// cnts[row] (or 0 without cnts). With dst_slot, entry i goes to destination slot
// dst_slot[row*S + i] (skipped outside [0, pool_slots)). Ids outside [0, src_chunks) are
// skipped, so a bad id can never read past the source row.
template <typename IdxT>
struct FetchArgs {
  const u32x4* src;
  int64_t src_row_vec;
  u32x4* dst;
  int64_t dst_row_vec, dst_offset_vec;
  const IdxT* ids;
  const int32_t* cnts;
  const int32_t* dst_slot;
  int pool_slots;
  int S, chunk_vec;
  int64_t src_chunks;
  int rows, tiles;  // tiles of kChunksPerFetchWG slots per row
  int workgroups;   // workgroups taking this role
};

// Copies slots [i0, i1) of one row, 16-byte vectors, kFetchUnroll loads in flight per lane.
template <typename IdxT>
__device__ __forceinline__ void fetch_tile(const FetchArgs<IdxT>& f, int row, int i0, int i1) {
  const int64_t total = static_cast<int64_t>(i1 - i0) * f.chunk_vec;
  const u32x4* s = f.src + static_cast<int64_t>(row) * f.src_row_vec;
  u32x4* d = f.dst + static_cast<int64_t>(row) * f.dst_row_vec + f.dst_offset_vec;
  const IdxT* id = f.ids + static_cast<int64_t>(row) * f.S;
  const int32_t* ds = f.dst_slot ? f.dst_slot + static_cast<int64_t>(row) * f.S : nullptr;
  for (int64_t v0 = 0; v0 < total; v0 += static_cast<int64_t>(blockDim.x) * kFetchUnroll) {
    u32x4 r[kFetchUnroll];
#pragma unroll
    for (int u = 0; u < kFetchUnroll; ++u) {
      int64_t v = v0 + static_cast<int64_t>(u) * blockDim.x + threadIdx.x;
      if (v < total) {
        int i = i0 + static_cast<int>(v / f.chunk_vec);
        int e = static_cast<int>(v % f.chunk_vec);
        int64_t c = static_cast<int64_t>(id[i]);
        if (c >= 0 && c < f.src_chunks) r[u] = load_nt(s + c * f.chunk_vec + e);
      }
    }
#pragma unroll
    for (int u = 0; u < kFetchUnroll; ++u) {
      int64_t v = v0 + static_cast<int64_t>(u) * blockDim.x + threadIdx.x;
      if (v < total) {
        int i = i0 + static_cast<int>(v / f.chunk_vec);
        int e = static_cast<int>(v % f.chunk_vec);
        int64_t c = static_cast<int64_t>(id[i]);
        const int slot = ds ? ds[i] : i;
        if (c >= 0 && c < f.src_chunks && (!ds || (slot >= 0 && slot < f.pool_slots)))
          d[static_cast<int64_t>(slot) * f.chunk_vec + e] = r[u];
      }
    }
  }
}

// Workgroup wg of nwg: tile t of a row covers kChunksPerFetchWG consecutive slots starting at
// start + t*kChunksPerFetchWG. The rows * tiles tiles are numbered row by row and walked with a
// stride of nwg; within row r they are rotated by r * tiles / nwg, so that the rows one workgroup
// visits (nwg / tiles apart) give it every tile position in turn. With cache hits only a row's
// first tiles hold misses: unrotated, a stride that is a multiple of the tiles per row would give
// workgroup wg tile wg mod tiles of every row it visits, and most workgroups would find no misses.
// MI355X, Llama-3.1-8B batch 8 ctx 122880, tokens/s (rotated / unrotated / tiles dealt
// tile-major): 2% hits, two lanes 408.6 / 408.9 / 407.0; a pool of 4096 slots (33% hits, two
// lanes) 492.7 / 463.3 / 488.9; 12288 slots (75% hits, one lane) 611.6 / 527.4 / 609.0.
template <typename IdxT>
__device__ void fetch_role(const FetchArgs<IdxT>& f, int wg, int nwg) {
  const int total_tiles = f.rows * f.tiles;
  for (int tile = wg; tile < total_tiles; tile += nwg) {
    const int row = tile / f.tiles;
    const int t = (tile - row * f.tiles + static_cast<int>(static_cast<int64_t>(row) * f.tiles / nwg)) % f.tiles;
    const int start = f.cnts ? max(0, f.cnts[row]) : 0;
    const int i0 = start + t * kChunksPerFetchWG;
    if (i0 >= f.S) continue;
    fetch_tile(f, row, i0, min(i0 + kChunksPerFetchWG, f.S));
  }
}

}  // namespace skv
