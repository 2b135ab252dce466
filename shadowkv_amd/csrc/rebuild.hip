// a6 (+a7): low-rank pre-RoPE key rebuild K = U[gathered rows] . SV^T on MFMA, with the RoPE
// push fused into the epilogue.
//
// Per (batch, kv-head) `bh` and cache row r of the sparse region (r < num_chunks*chunk):
//   pos(r) = ids[bh, r/chunk]*chunk + r%chunk,  k(r) = bf16(sum_k U[b(,h), pos(r), k] * SV[b,h,:,k])
// and only miss rows r >= cnt[bh]*chunk are produced (the reference recomputes whole 128-row
// tiles, kernels/gemm_universal_batch_gather_indices.h:678-680). In RoPE mode the bf16 k(r) is
// rotated with cos_sin row pos(r) and written to cache row sparse_start + r; in plain mode the
// bf16 k(r) itself is written (reference batch_gather_gemm output).
//
// Work decomposition (gfx950, wave64):
//   * workgroup = kNW waves, owns up to kTileRows = kNW x kIters x 32 consecutive rows of one head
//     (256 = 4 waves x 2 iterations when the grid has enough workgroups to fill the GPU, 256 = 8 x
//     1 where that gives one workgroup per CU, else 128 = 4 x 1 or 64 = 2 x 1, so that few rows
//     still spread over the CUs); the grid has the
//     tiles of a head with no hits, and a head's miss rows are dealt evenly over its tiles, so
//     hits shorten every workgroup instead of idling some. At entry it stages
//     SV of that head (128 x rank bf16, 40 KB at rank 160) and the U row of each of its rows
//     (chunk id * chunk + r % chunk) into LDS;
//   * a wave computes 32 rows x 128 columns per iteration, two iterations, with
//     v_mfma_f32_16x16x32_bf16 where A = SV (16 output dims x 32 k, from LDS, shared by both
//     16-row halves) and B = the gathered U rows (16-byte loads straight from HBM). The next
//     iteration's U rows are in flight while the current one computes;
//   * the fp32 result of a 16-row half is rounded to bf16 and staged in a per-wave LDS tile
//     (a lane holds 4 consecutive dims of one row: one 8-byte write per column tile); the
//     epilogue then works in row-contiguous 16-byte units: a lane takes dims [8j, 8j+8) (and,
//     for the half-split rotation, [64+8j, 72+8j)) of one row, with its cos/sin loaded as
//     16-byte vectors before the MFMAs, and stores the rotated row with 16-byte non-temporal
//     stores (skv::store_nt: the output is not re-read by this kernel);
//   * blockIdx -> (head, tile) is XCD-aware: all tiles of a head land on the same XCD
//     (workgroups are dealt round-robin over the 8 XCDs), so SV is fetched from HBM once per
//     head and re-read from that XCD's L2.
#include <algorithm>

#include "fetch_role.h"
#include "rope_math.h"

namespace {

using skv::u32x4;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMaxWaves = 8;
constexpr int kMaxTileRows = 256;  // rows per workgroup: at most 4 waves x 2 iterations x 32 rows
constexpr int kHeadDim = 128;
constexpr int kMaxRank = 192;
constexpr int kXcds = 8;
constexpr int kStLd = kHeadDim + 8;  // staging row (elements), padded against bank conflicts

enum Mode { kPlain = 0, kRopeHalf = 1, kRopeGlm = 2 };

struct RebuildArgs {
  const uint16_t* u;
  int64_t u_sb, u_sh, u_sr, u_rows;
  const uint16_t* sv;
  int64_t sv_sb, sv_sh, sv_sn;
  const void* ids;
  int64_t id_sb, id_sh;
  const int32_t* cnts;
  const uint16_t* cs;
  int64_t cs_stride, cs_rows;
  uint16_t* out;
  int64_t o_sb, o_sh, o_ss;
  int o_start;
  int B, H, S, chunk, rank, tiles;
  int spread;  // deal a head's miss rows evenly over its tiles (else whole tiles, hit tiles idle)
  int grid_tiles;  // tile workgroups of the unfused grid (heads padded to 8 x tiles)
  int rebuild_wgs;  // fused launch: cap on the rebuild workgroups, which then loop over the tiles (0: one per tile)
  // Optional destination slots (chunk pool): row r of entry i goes to cache row
  // o_start + dst_slot[i] * chunk + r % chunk; entries outside [0, pool_slots) are skipped.
  const int32_t* dst_slot;
  int64_t ds_sb, ds_sh;
  int pool_slots;
};

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ uint16_t lo16(uint32_t w) { return static_cast<uint16_t>(w & 0xffffu); }
__device__ __forceinline__ uint16_t hi16(uint32_t w) { return static_cast<uint16_t>(w >> 16); }
__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}
// 8 bf16 of a 16-byte vector as an array (element 2i in the low half of word i).
__device__ __forceinline__ void unpack8(const u32x4& v, uint16_t* e) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    e[2 * i] = lo16(w[i]);
    e[2 * i + 1] = hi16(w[i]);
  }
}
__device__ __forceinline__ u32x4 pack8(const uint16_t* e) {
  return u32x4{pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]), pack2(e[6], e[7])};
}

// Rows handled by one epilogue lane-unit of a 16-row tile: a half-split unit covers dims
// [8j, 8j+8) and [64+8j, 72+8j) (8 units per row); GLM and plain units cover [8j, 8j+8)
// (16 units per row).
template <int kMode>
struct Units {
  static constexpr int kPerRow = kMode == kRopeHalf ? 8 : 16;
  static constexpr int kPerLane = 16 * kPerRow / 64;
};

// The rebuild of tile workgroup `bid` (blockIdx.x of rebuild_kernel; offset by the fetch
// workgroups in fetch_rebuild_kernel).
template <int kMode, int KS, typename IdxT, int kNW, int kIters>
__device__ __forceinline__ void rebuild_role(const RebuildArgs& a, int bid) {
  using U = Units<kMode>;
  constexpr int kThreads = kNW * 64;
  constexpr int kTileRows = kNW * kIters * 32;
  static_assert(kTileRows <= kThreads, "the position staging gives each thread at most one row");
  extern __shared__ __align__(16) unsigned char smem[];
  const int ldr = a.rank + 8;  // padded SV row (elements)
  uint16_t* sv_lds = reinterpret_cast<uint16_t*>(smem);                         // [128][ldr]
  int32_t* pos_lds = reinterpret_cast<int32_t*>(sv_lds + kHeadDim * ldr);      // [kTileRows]
  int32_t* orow_lds = pos_lds + kTileRows;                                      // [kTileRows]
  uint16_t* kst = reinterpret_cast<uint16_t*>(orow_lds + kTileRows);           // [kNW][16][kStLd]

  const int xcd = bid % kXcds;
  const int local = bid / kXcds;
  const int head = xcd + kXcds * (local / a.tiles);
  const int tile = local % a.tiles;
  const int BH = a.B * a.H;
  if (head >= BH) return;
  const int b = head / a.H;
  const int h = head - b * a.H;

  // spread: the head's miss rows [miss_begin, total_rows) are dealt evenly over its a.tiles
  // workgroups in 32-row blocks (span <= kTileRows, as a.tiles covers total_rows), so cache hits
  // shorten every workgroup of the head instead of idling whole tiles. Otherwise tile t owns rows
  // [t, t + 1) x kTileRows and tiles of hits only return at once.
  const int total_rows = a.S * a.chunk;
  const int miss_begin = min(max(a.cnts[head], 0), a.S) * a.chunk;  // (a count outside [0, S] is clamped)
  const int miss_rows = total_rows - miss_begin;
  const int span = a.spread ? ((miss_rows + a.tiles - 1) / a.tiles + 31) / 32 * 32 : kTileRows;
  const int row_begin = a.spread ? miss_begin + tile * span : tile * kTileRows;
  const int row_end = min(row_begin + span, total_rows);
  if (row_end <= miss_begin || row_begin >= row_end) return;

  // Issue order (vector loads retire in order): this thread's chunk id, the SV tile, then, after
  // the positions are shared, every U and cos/sin row the wave needs for both iterations; SV is
  // written to LDS last, so its wait leaves the row loads in flight. Every load is unconditional
  // (clamped index, value zeroed), so no branch splits the batches.
  const IdxT* ids = static_cast<const IdxT*>(a.ids) + b * a.id_sb + h * a.id_sh;
  int64_t my_id = 0;
  {
    const int row = row_begin + min(static_cast<int>(threadIdx.x), kTileRows - 1);  // at most one row per thread
    my_id = ids[min(row, total_rows - 1) / a.chunk];
  }
  const int k8 = a.rank / 8;
  const uint16_t* svp = a.sv + b * a.sv_sb + h * a.sv_sh;
  constexpr int kVecs = (kHeadDim * (KS * 32) / 8 + kThreads - 1) / kThreads;  // >= 128*rank/8/256
  u32x4 svv[kVecs];
#pragma unroll
  for (int i = 0; i < kVecs; ++i) {
    const int idx = static_cast<int>(threadIdx.x) + i * kThreads;
    const int ic = min(idx, kHeadDim * k8 - 1);
    const int n = ic / k8, kk = (ic - n * k8) * 8;
    svv[i] = *reinterpret_cast<const u32x4*>(&svp[n * a.sv_sn + kk]);
  }
  if (static_cast<int>(threadIdx.x) < kTileRows) {
    const int row = row_begin + static_cast<int>(threadIdx.x);
    int32_t p = -1, orow = row;
    if (row < row_end) {
      const int64_t q = my_id * a.chunk + row % a.chunk;
      if (q >= 0 && q <= 0x7fffffff) p = static_cast<int32_t>(q);
    }
    if (a.dst_slot) {  // uniform
      const int32_t sl = a.dst_slot[b * a.ds_sb + h * a.ds_sh + min(row, total_rows - 1) / a.chunk];
      orow = (sl >= 0 && sl < a.pool_slots) ? sl * a.chunk + row % a.chunk : -1;
    }
    pos_lds[threadIdx.x] = p;
    orow_lds[threadIdx.x] = orow;
  }
  __syncthreads();

  const uint16_t* ubase = a.u + b * a.u_sb + h * a.u_sh;
  uint16_t* obase = a.out + b * a.o_sb + h * a.o_sh;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;  // B column (row within a 16-row half) / D column
  const int lk = lane >> 4;  // k-slab of A and B; D row quad
  uint16_t* st = kst + wave * 16 * kStLd;
  const u32x4 zero4 = {0u, 0u, 0u, 0u};

  // 32-row block of iteration it: blocks go to the waves first (block it * kNW + wave), so a span
  // shorter than the tile keeps every wave busy on its first iteration.
  auto lr_of = [&](int it) { return (it * kNW + wave) * 32; };
  bool active[kIters];
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int rb = row_begin + lr_of(it);
    active[it] = rb < row_end && rb + 32 > miss_begin;  // wave-uniform
  }
  // U fragments (B operand) of both 32-row blocks.
  bf16x8_t uf[kIters][2][KS];
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int r = lr_of(it) + m * 16 + li;
      const int grow = row_begin + r;
      const int32_t pos = pos_lds[r];
      const bool valid = active[it] && grow >= miss_begin && grow < row_end && pos >= 0 && pos < a.u_rows;
      const uint16_t* up = ubase + static_cast<int64_t>(valid ? pos : 0) * a.u_sr;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int kk = ks * 32 + lk * 8;
        uf[it][m][ks] = as_bf16x8(skv::load16_or_zero(up + min(kk, a.rank - 8), valid && kk < a.rank));
      }
    }
  }
  // cos/sin of both blocks' epilogue units.
  u32x4 cs_c[kIters][2][U::kPerLane], cs_s[kIters][2][U::kPerLane];
#pragma unroll
  for (int it = 0; it < kIters; ++it)
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int q = 0; q < U::kPerLane; ++q) {
        cs_c[it][m][q] = zero4;
        cs_s[it][m][q] = zero4;
        if (kMode == kPlain) continue;
        const int unit = lane + 64 * q;
        const int r = unit / U::kPerRow, j = unit % U::kPerRow;
        const int32_t pos = pos_lds[lr_of(it) + m * 16 + r];
        const bool ok = active[it] && pos >= 0 && pos < a.cs_rows;
        const uint16_t* c = a.cs + static_cast<int64_t>(ok ? pos : 0) * a.cs_stride;
        if (kMode == kRopeHalf) {
          cs_c[it][m][q] = skv::load16_or_zero(c + 8 * j, ok);
          cs_s[it][m][q] = skv::load16_or_zero(c + 64 + 8 * j, ok);
        } else {  // GLM: 4 pairs per unit, cos at [4j], sin at [32 + 4j]; units j >= 8 pass through
          const int jc = min(j, 7);
          const u32x2 cc = *reinterpret_cast<const u32x2*>(c + 4 * jc);
          const u32x2 ss = *reinterpret_cast<const u32x2*>(c + 32 + 4 * jc);
          const bool use = ok && j < 8;
          cs_c[it][m][q] = use ? u32x4{cc.x, cc.y, 0u, 0u} : zero4;
          cs_s[it][m][q] = use ? u32x4{ss.x, ss.y, 0u, 0u} : zero4;
        }
      }
#pragma unroll
  for (int i = 0; i < kVecs; ++i) {
    const int idx = static_cast<int>(threadIdx.x) + i * kThreads;
    const int n = idx / k8, kk = (idx - n * k8) * 8;
    if (idx < kHeadDim * k8) *reinterpret_cast<u32x4*>(&sv_lds[n * ldr + kk]) = svv[i];
  }
  __syncthreads();

#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    if (!active[it]) continue;
    const int lr = lr_of(it);

    f32x4_t acc[2][8];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[m][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int kk = ks * 32 + lk * 8;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const u32x4 sv = *reinterpret_cast<const u32x4*>(&sv_lds[(t * 16 + li) * ldr + min(kk, a.rank - 8)]);
        const bf16x8_t svf = as_bf16x8(kk < a.rank ? sv : zero4);
        acc[0][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(svf, uf[it][0][ks], acc[0][t], 0, 0, 0);
        acc[1][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(svf, uf[it][1][ks], acc[1][t], 0, 0, 0);
      }
    }

#pragma unroll
    for (int m = 0; m < 2; ++m) {
      // D[dim][row]: this lane holds dims t*16 + 4*lk + v (v = 0..3) of row li.
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const u32x2 w = {skv::f2bf2(acc[m][t][0], acc[m][t][1]), skv::f2bf2(acc[m][t][2], acc[m][t][3])};
        *reinterpret_cast<u32x2*>(&st[li * kStLd + t * 16 + 4 * lk]) = w;
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the tile is in LDS before any lane reads it
#pragma unroll
      for (int q = 0; q < U::kPerLane; ++q) {
        const int unit = lane + 64 * q;
        const int r = unit / U::kPerRow, j = unit % U::kPerRow;
        const int grow = row_begin + lr + m * 16 + r;
        const int32_t pos = pos_lds[lr + m * 16 + r];
        const int32_t prow = orow_lds[lr + m * 16 + r];
        bool valid = grow >= miss_begin && grow < row_end && prow >= 0;
        if (kMode != kPlain) valid = valid && pos >= 0 && pos < a.cs_rows;
        if (!valid) continue;
        uint16_t* orow = obase + static_cast<int64_t>(a.o_start + prow) * a.o_ss;
        const u32x4 x1v = *reinterpret_cast<const u32x4*>(&st[r * kStLd + 8 * j]);
        if (kMode == kPlain) {
          skv::store_nt(orow + 8 * j, x1v);
        } else if (kMode == kRopeHalf) {
          const u32x4 x2v = *reinterpret_cast<const u32x4*>(&st[r * kStLd + 64 + 8 * j]);
          const u32x4 cv = cs_c[it][m][q], sv = cs_s[it][m][q];
          uint32_t y1[4], y2[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) skv::rope_half_split2(x1v[e], x2v[e], cv[e], sv[e], y1[e], y2[e]);
          skv::store_nt(orow + 8 * j, u32x4{y1[0], y1[1], y1[2], y1[3]});
          skv::store_nt(orow + 64 + 8 * j, u32x4{y2[0], y2[1], y2[2], y2[3]});
        } else {  // GLM: interleaved pairs on dims 0..63, dims 64..127 unchanged
          if (j < 8) {
            uint16_t x[8], c[8], sn[8], y[8];
            unpack8(x1v, x);
            unpack8(cs_c[it][m][q], c);
            unpack8(cs_s[it][m][q], sn);
#pragma unroll
            for (int p = 0; p < 4; ++p) skv::rope_half_split(x[2 * p], x[2 * p + 1], c[p], sn[p], y[2 * p], y[2 * p + 1]);
            skv::store_nt(orow + 8 * j, pack8(y));
          } else {
            skv::store_nt(orow + 8 * j, x1v);
          }
        }
      }
    }
  }
}

template <int kMode, int KS, typename IdxT, int kNW, int kIters>
__global__ void __launch_bounds__(kNW * 64, kNW > 4 ? 1 : 2) rebuild_kernel(RebuildArgs a) {
  rebuild_role<kMode, KS, IdxT, kNW, kIters>(a, blockIdx.x);
}

// Fused instances whose rebuild workgroups can loop over several tiles without spilling (half-split
// RoPE, ranks up to 160, 128-row tiles of 4 waves: the tiles of a decode lane); the others keep
// one workgroup per tile.
template <int kMode, int KS, int kNW, int kIters>
constexpr bool kFusedLoops = kIters == 1 && KS <= 5 && kNW == 4 && kMode == kRopeHalf;

// The value fetch of the misses and the key rebuild in one launch: workgroups [0, f.workgroups)
// gather the miss chunks from the pinned host store (skv::fetch_role, host-link bound), the rest
// rebuild the key rows (HBM bound), side by side. Both need only the selection's offsets and
// counts, with the hits already moved in both buffers; one launch on one stream then replaces a
// fetch on a second stream and the two cross-stream waits around it (~5 us each on MI355X).
// f.workgroups is a multiple of 8, so rebuild tile `bid` keeps the XCD of blockIdx bid.
template <int kMode, int KS, typename IdxT, int kNW, int kIters>
__global__ void __launch_bounds__(kNW * 64, 2) fetch_rebuild_kernel(RebuildArgs a, skv::FetchArgs<int32_t> f) {
  const int wg = blockIdx.x;
  if (wg < f.workgroups) {
    skv::fetch_role(f, wg, f.workgroups);
    return;
  }
  // The rebuild workgroups (a multiple of 8) walk the tiles with their count as the stride, so a
  // tile keeps the XCD of its unfused workgroup; each pass ends at a barrier before the next
  // tile's LDS writes.
  if constexpr (kFusedLoops<kMode, KS, kNW, kIters>) {
    const int nrb = static_cast<int>(gridDim.x) - f.workgroups;
    for (int t = wg - f.workgroups; t < a.grid_tiles; t += nrb) {
      rebuild_role<kMode, KS, IdxT, kNW, kIters>(a, t);
      __syncthreads();
    }
  } else {
    rebuild_role<kMode, KS, IdxT, kNW, kIters>(a, wg - f.workgroups);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Fetch workgroups of a fused launch with `waves`-wave workgroups: the target in 4-wave
// workgroups (the caller's f.workgroups when positive, else skv::kDeviceFetchWGs for a value
// store in device memory and skv::fused_fetch_workgroups_target for one in pinned host memory)
// scaled to the workgroup size, then as few as give every workgroup the same number of tiles (the
// launch lasts as long as its busiest fetch workgroup), rounded up to a multiple of 8 for the
// rebuild tiles' XCD map.
int fused_fetch_workgroups(const skv::FetchArgs<int32_t>& f, int waves) {
  const int tiles = std::max(f.rows * f.tiles, 1);
  const int t4 = f.workgroups > 0              ? f.workgroups
                 : skv::is_device_memory(f.src) ? skv::kDeviceFetchWGs
                                                : skv::fused_fetch_workgroups_target();
  const int target = std::max(1, t4 * 4 / waves);
  const int per = (tiles + target - 1) / target;  // tiles per workgroup
  const int want = (tiles + per - 1) / per;
  return (want + kXcds - 1) / kXcds * kXcds;
}

template <int kMode, int KS, typename IdxT, int kNW, int kIters, bool kFused>
int launch_ks(dim3 grid, size_t lds, hipStream_t stream, const RebuildArgs& a, const skv::FetchArgs<int32_t>* f) {
  // Ranks above 176 need more than 64 KiB of dynamic LDS (gfx950 has 160 KiB per CU): raise the
  // kernel's limit once.
  const int max_lds = static_cast<int>(kHeadDim * (kMaxRank + 8) * sizeof(uint16_t) + 2 * kMaxTileRows * sizeof(int32_t) +
                                       kMaxWaves * 16 * kStLd * sizeof(uint16_t));
  if constexpr (KS == 6 && kIters == 2) {
    // Not instantiated: ranks above 160 with 256-row tiles spill, so launch_rebuild gives that
    // rank 128-row tiles. Reaching this is a bug in that choice: fail instead of leaving the key
    // buffer stale.
    (void)grid, (void)lds, (void)stream, (void)a, (void)f;
    skv_set_error("rebuild_k_rope: no kernel for rank %d with 256-row tiles", a.rank);
    return SKV_EUNSUPPORTED;
  } else if constexpr (kFused) {
    if (lds > 65536) {
      static const hipError_t raised = hipFuncSetAttribute(
          reinterpret_cast<const void*>(&fetch_rebuild_kernel<kMode, KS, IdxT, kNW, kIters>),
          hipFuncAttributeMaxDynamicSharedMemorySize, max_lds);
      (void)raised;
    }
    skv::FetchArgs<int32_t> ff = *f;
    ff.workgroups = fused_fetch_workgroups(ff, kNW);
    // rebuild workgroups: the caller's cap (a multiple of 8) where the instance loops over tiles
    const int cap = (a.rebuild_wgs + kXcds - 1) / kXcds * kXcds;
    const int rb = cap > 0 && kFusedLoops<kMode, KS, kNW, kIters> ? std::min(static_cast<int>(grid.x), cap)
                                                                   : static_cast<int>(grid.x);
    hipLaunchKernelGGL((fetch_rebuild_kernel<kMode, KS, IdxT, kNW, kIters>), dim3(rb + ff.workgroups),
                       dim3(kNW * 64), lds, stream, a, ff);
    return SKV_OK;
  } else {
    (void)f;
    if (lds > 65536) {
      static const hipError_t raised = hipFuncSetAttribute(
          reinterpret_cast<const void*>(&rebuild_kernel<kMode, KS, IdxT, kNW, kIters>),
          hipFuncAttributeMaxDynamicSharedMemorySize, max_lds);
      (void)raised;
    }
    hipLaunchKernelGGL((rebuild_kernel<kMode, KS, IdxT, kNW, kIters>), grid, dim3(kNW * 64), lds, stream, a);
    return SKV_OK;
  }
}

template <int kMode, typename IdxT, int kNW, int kIters, bool kFused>
int launch_tile(int ks, dim3 grid, size_t lds, hipStream_t stream, const RebuildArgs& a,
                const skv::FetchArgs<int32_t>* f) {
  switch (ks) {
    case 1: return launch_ks<kMode, 1, IdxT, kNW, kIters, kFused>(grid, lds, stream, a, f);
    case 2: return launch_ks<kMode, 2, IdxT, kNW, kIters, kFused>(grid, lds, stream, a, f);
    case 3: return launch_ks<kMode, 3, IdxT, kNW, kIters, kFused>(grid, lds, stream, a, f);
    case 4: return launch_ks<kMode, 4, IdxT, kNW, kIters, kFused>(grid, lds, stream, a, f);
    case 5: return launch_ks<kMode, 5, IdxT, kNW, kIters, kFused>(grid, lds, stream, a, f);
    default: return launch_ks<kMode, 6, IdxT, kNW, kIters, kFused>(grid, lds, stream, a, f);
  }
}

// tile_rows: 256 (4 waves x 2 iterations), 128 (4 x 1) or 64 (2 x 1). kFused: the launch also
// takes the value fetch's workgroups (fetch_rebuild_kernel).
template <int kMode, typename IdxT, bool kFused = false>
int launch_mode(int tile_rows, int ks, dim3 grid, size_t lds, hipStream_t stream, const RebuildArgs& a,
                const skv::FetchArgs<int32_t>* f = nullptr, bool wide = false) {
  if constexpr (!kFused) {
    if (wide) return launch_tile<kMode, IdxT, 8, 1, false>(ks, grid, lds, stream, a, f);
  }
  if (tile_rows == 256) return launch_tile<kMode, IdxT, 4, 2, kFused>(ks, grid, lds, stream, a, f);
  if (tile_rows == 128) return launch_tile<kMode, IdxT, 4, 1, kFused>(ks, grid, lds, stream, a, f);
  return launch_tile<kMode, IdxT, 2, 1, kFused>(ks, grid, lds, stream, a, f);
}

// Workgroup shape: the largest tile that still gives the grid about 1.5 workgroups per CU (256
// CUs), so few (b, h) rows - GLM's 2 kv heads, a batch lane of 4 sequences - spread over the GPU
// instead of leaving most CUs idle: 256 rows (4 waves x 2), 128 (4 x 1) or 64 (2 x 1). Where
// 256-row tiles give about one workgroup per CU, 256 rows of 8 waves x 1 instead (*wide): the
// waves per CU of two 128-row workgroups, SV staged half as often (MI355X, 32 heads x 2048 rows:
// 15.1 vs 15.3 us without hits, 9.6 vs 10.9 us with 154 of 256 chunks hit; with the fetch in the
// same launch never). SKV_REBUILD_TILE=64/128/256/w256 forces one.
int choose_tile_rows(int BH, int rows, bool allow_wide, bool* wide) {
  *wide = false;
  const char* e = getenv("SKV_REBUILD_TILE");
  if (e && e[0] == 'w' && allow_wide) {
    *wide = true;
    return 256;
  }
  const int forced = e ? atoi(e) : 0;
  if (forced == 64 || forced == 128 || forced == 256) return forced;
  constexpr int kFill = 384;
  const int64_t t256 = static_cast<int64_t>(BH) * ((rows + 255) / 256);
  if (t256 >= kFill) return 256;
  if (allow_wide && t256 >= 256) {
    *wide = true;
    return 256;
  }
  if (static_cast<int64_t>(BH) * ((rows + 127) / 128) >= kFill) return 128;
  return 64;
}

int launch_rebuild(const char* what, int mode, bool ids64, RebuildArgs a, hipStream_t stream,
                   const skv::FetchArgs<int32_t>* fetch = nullptr) {
  if (!a.u || !a.sv || !a.ids || !a.cnts || !a.out || (mode != kPlain && !a.cs)) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (a.B <= 0 || a.H <= 0 || a.S <= 0 || a.chunk <= 0) {
    skv_set_error("%s: invalid shape batch=%d heads=%d chunks=%d chunk=%d", what, a.B, a.H, a.S, a.chunk);
    return SKV_EINVAL;
  }
  if (a.rank < 8 || a.rank > kMaxRank || a.rank % 8) {
    skv_set_error("%s: rank=%d must be a multiple of 8 in [8, %d]", what, a.rank, kMaxRank);
    return SKV_EUNSUPPORTED;
  }
  if (!aligned16(a.u) || !aligned16(a.sv) || a.u_sb % 8 || a.u_sh % 8 || a.u_sr % 8 || a.sv_sb % 8 || a.sv_sh % 8 ||
      a.sv_sn % 8) {
    skv_set_error("%s: U and SV rows must be 16-byte aligned (strides multiples of 8 elements)", what);
    return SKV_EINVAL;
  }
  if (a.u_rows < 1 || (mode != kPlain && a.cs_rows < 1)) {
    skv_set_error("%s: empty U (%lld rows) or cos/sin table (%lld rows)", what, (long long)a.u_rows,
                  (long long)a.cs_rows);
    return SKV_EINVAL;
  }
  if (!aligned16(a.out) || a.o_sb % 8 || a.o_sh % 8 || a.o_ss % 8 ||
      (mode != kPlain && (!aligned16(a.cs) || a.cs_stride % 8))) {
    skv_set_error("%s: output and cos/sin rows must be 16-byte aligned (strides multiples of 8 elements)", what);
    return SKV_EINVAL;
  }
  if (static_cast<int64_t>(a.S) * a.chunk > (int64_t{1} << 30)) {
    skv_set_error("%s: %d chunks of %d rows is too many", what, a.S, a.chunk);
    return SKV_EUNSUPPORTED;
  }
  const int BH = a.B * a.H;
  bool wide = false;
  int tile_rows = choose_tile_rows(BH, a.S * a.chunk, fetch == nullptr, &wide);
  if (!wide && tile_rows == 256 && a.rank > 160) tile_rows = 128;  // (no spill-free 4 x 2 kernel there)
  const int waves = wide ? 8 : tile_rows == 64 ? 2 : 4;
  a.tiles = (a.S * a.chunk + tile_rows - 1) / tile_rows;
  // Deal the miss rows over every tile while the grid is at most ~4 workgroups per CU (all of it
  // in flight at once: hits then shorten each workgroup; MI355X, batch 8 with 154 of 256 chunks
  // hit, 18.2 -> 13.5 us); larger grids keep whole tiles, which stage SV once per 256 rows
  // (batch 32: 39.6 vs 45.3 us). SKV_REBUILD_SPREAD=0/1 forces either.
  {
    const char* e = getenv("SKV_REBUILD_SPREAD");
    a.spread = e ? (e[0] == '1') : (static_cast<int64_t>(BH) * a.tiles <= 1024);
  }
  const int heads_padded = (BH + kXcds - 1) / kXcds * kXcds;
  const dim3 grid(static_cast<unsigned>(heads_padded * a.tiles));
  a.grid_tiles = static_cast<int>(grid.x);
  const size_t lds = static_cast<size_t>(kHeadDim) * (a.rank + 8) * sizeof(uint16_t) + 2 * tile_rows * sizeof(int32_t) +
                     static_cast<size_t>(waves) * 16 * kStLd * sizeof(uint16_t);
  const int ks = (a.rank + 31) / 32;
  int rc;
  if (fetch) {  // (the fused launch: the RoPE modes, with the int64 chunk ids of skv_rebuild_k_rope or
                // the int32 miss ids of skv_rebuild_k_rope_slots)
    if (ids64) {
      if (mode == kRopeHalf) rc = launch_mode<kRopeHalf, int64_t, true>(tile_rows, ks, grid, lds, stream, a, fetch);
      else rc = launch_mode<kRopeGlm, int64_t, true>(tile_rows, ks, grid, lds, stream, a, fetch);
    } else {
      if (mode == kRopeHalf) rc = launch_mode<kRopeHalf, int32_t, true>(tile_rows, ks, grid, lds, stream, a, fetch);
      else rc = launch_mode<kRopeGlm, int32_t, true>(tile_rows, ks, grid, lds, stream, a, fetch);
    }
  } else if (ids64) {
    if (mode == kPlain) rc = launch_mode<kPlain, int64_t>(tile_rows, ks, grid, lds, stream, a, nullptr, wide);
    else if (mode == kRopeHalf) rc = launch_mode<kRopeHalf, int64_t>(tile_rows, ks, grid, lds, stream, a, nullptr, wide);
    else rc = launch_mode<kRopeGlm, int64_t>(tile_rows, ks, grid, lds, stream, a, nullptr, wide);
  } else {
    if (mode == kPlain) rc = launch_mode<kPlain, int32_t>(tile_rows, ks, grid, lds, stream, a, nullptr, wide);
    else if (mode == kRopeHalf) rc = launch_mode<kRopeHalf, int32_t>(tile_rows, ks, grid, lds, stream, a, nullptr, wide);
    else rc = launch_mode<kRopeGlm, int32_t>(tile_rows, ks, grid, lds, stream, a, nullptr, wide);
  }
  if (rc) return rc;
  return skv_check_launch(what);
}

}  // namespace

extern "C" int skv_batch_gather_gemm(const uint16_t* a, const uint16_t* b, const int32_t* position_ids,
                                     uint16_t* output, int batch_size, int heads, int seq_len, int embed_dim, int rank,
                                     int sparse_budget, int max_seq_len, int chunk_size, const int32_t* offset_array,
                                     void* stream) {
  (void)max_seq_len;  // only sized the reference's unused RoPE epilogue operands
  const char* what = "batch_gather_gemm";
  if (embed_dim != kHeadDim || chunk_size <= 0 || sparse_budget % chunk_size != 0 || seq_len <= 0) {
    skv_set_error("%s: embed_dim=%d (must be 128), sparse_budget=%d, chunk_size=%d, seq_len=%d", what, embed_dim,
                  sparse_budget, chunk_size, seq_len);
    return SKV_EUNSUPPORTED;
  }
  RebuildArgs r{};
  r.u = a;
  r.u_sb = static_cast<int64_t>(seq_len) * rank;
  r.u_sh = 0;
  r.u_sr = rank;
  r.u_rows = seq_len;
  r.sv = b;
  r.sv_sh = static_cast<int64_t>(embed_dim) * rank;
  r.sv_sb = r.sv_sh * heads;
  r.sv_sn = rank;
  r.ids = position_ids;
  r.id_sh = sparse_budget / chunk_size;
  r.id_sb = r.id_sh * heads;
  r.cnts = offset_array;
  r.cs = nullptr;
  r.out = output;
  r.o_ss = embed_dim;
  r.o_sh = static_cast<int64_t>(sparse_budget) * embed_dim;
  r.o_sb = r.o_sh * heads;
  r.o_start = 0;
  r.B = batch_size;
  r.H = heads;
  r.S = sparse_budget / chunk_size;
  r.chunk = chunk_size;
  r.rank = rank;
  return launch_rebuild(what, kPlain, false, r, static_cast<hipStream_t>(stream));
}

extern "C" int skv_rebuild_k_rope(const uint16_t* u, int64_t u_stride_b, int64_t u_stride_h, int64_t u_stride_row,
                                  int64_t u_rows, const uint16_t* sv, int64_t sv_stride_b, int64_t sv_stride_h, int64_t sv_stride_n,
                                  const int64_t* position_ids, int64_t pid_stride_b, int64_t pid_stride_h,
                                  const int32_t* cnts, const uint16_t* cos_sin, int64_t stride_cos_sin,
                                  int64_t cos_sin_rows, int rope_mode, uint16_t* cache, int64_t stride_cache_b, int64_t stride_cache_h,
                                  int64_t stride_cache_s, int sparse_start, int batch_size, int heads, int num_chunks,
                                  int chunk_size, int rank, int head_dim, void* stream) {
  const char* what = "rebuild_k_rope";
  if (head_dim != kHeadDim || (rope_mode != 0 && rope_mode != 1)) {
    skv_set_error("%s: head_dim=%d (must be 128), rope_mode=%d (0 half-split, 1 GLM)", what, head_dim, rope_mode);
    return SKV_EUNSUPPORTED;
  }
  RebuildArgs r{};
  r.u = u;
  r.u_sb = u_stride_b;
  r.u_sh = u_stride_h;
  r.u_sr = u_stride_row;
  r.u_rows = u_rows;
  r.sv = sv;
  r.sv_sb = sv_stride_b;
  r.sv_sh = sv_stride_h;
  r.sv_sn = sv_stride_n;
  r.ids = position_ids;
  r.id_sb = pid_stride_b;
  r.id_sh = pid_stride_h;
  r.cnts = cnts;
  r.cs = cos_sin;
  r.cs_stride = stride_cos_sin;
  r.cs_rows = cos_sin_rows;
  r.out = cache;
  r.o_sb = stride_cache_b;
  r.o_sh = stride_cache_h;
  r.o_ss = stride_cache_s;
  r.o_start = sparse_start;
  r.B = batch_size;
  r.H = heads;
  r.S = num_chunks;
  r.chunk = chunk_size;
  r.rank = rank;
  return launch_rebuild(what, rope_mode == 0 ? kRopeHalf : kRopeGlm, true, r, static_cast<hipStream_t>(stream));
}

// The value fetch of the misses (skv_gather_copy_misses_with_offsets) and the key rebuild
// (skv_rebuild_k_rope) in one launch, for a selection that already moved the hits of both buffers.
extern "C" int skv_fetch_misses_rebuild_k_rope(
    const void* values, void* v_cache_buffer, const int32_t* offsets, int64_t cpu_v_length, int64_t gpu_v_offset,
    int64_t gpu_v_stride, const uint16_t* u, int64_t u_stride_b, int64_t u_stride_h, int64_t u_stride_row,
    int64_t u_rows, const uint16_t* sv, int64_t sv_stride_b, int64_t sv_stride_h, int64_t sv_stride_n,
    const int64_t* position_ids, int64_t pid_stride_b, int64_t pid_stride_h, const int32_t* cnts,
    const uint16_t* cos_sin, int64_t stride_cos_sin, int64_t cos_sin_rows, int rope_mode, uint16_t* cache,
    int64_t stride_cache_b, int64_t stride_cache_h, int64_t stride_cache_s, int sparse_start, int batch_size,
    int heads, int num_chunks, int chunk_size, int rank, int head_dim, int fetch_workgroups, int rebuild_workgroups,
    void* stream) {
  const char* what = "fetch_misses_rebuild_k_rope";
  if (fetch_workgroups < 0 || fetch_workgroups > 65536 || rebuild_workgroups < 0 || rebuild_workgroups > 65536) {
    skv_set_error("%s: fetch_workgroups=%d rebuild_workgroups=%d (0 for the default, at most 65536)", what,
                  fetch_workgroups, rebuild_workgroups);
    return SKV_EINVAL;
  }
  if (head_dim != kHeadDim || (rope_mode != 0 && rope_mode != 1)) {
    skv_set_error("%s: head_dim=%d (must be 128), rope_mode=%d (0 half-split, 1 GLM)", what, head_dim, rope_mode);
    return SKV_EUNSUPPORTED;
  }
  if (!values || !v_cache_buffer || !offsets || !cnts) {
    skv_set_error("%s: null value-fetch pointer", what);
    return SKV_EINVAL;
  }
  const int64_t chunk_elems = static_cast<int64_t>(chunk_size) * head_dim;
  if (!aligned16(values) || !aligned16(v_cache_buffer) || cpu_v_length % 8 || gpu_v_offset % 8 || gpu_v_stride % 8 ||
      cpu_v_length < chunk_elems || gpu_v_offset < 0 ||
      gpu_v_stride < gpu_v_offset + static_cast<int64_t>(num_chunks) * chunk_elems) {
    skv_set_error("%s: value rows must be 16-byte aligned and hold the selected region (cpu_v_length=%lld "
                  "offset=%lld stride=%lld)", what, (long long)cpu_v_length, (long long)gpu_v_offset,
                  (long long)gpu_v_stride);
    return SKV_EINVAL;
  }
  if (batch_size <= 0 || heads <= 0 || num_chunks <= 0 || chunk_size <= 0 ||
      static_cast<int64_t>(num_chunks) * chunk_elems > (int64_t{1} << 31)) {
    skv_set_error("%s: invalid shape batch=%d heads=%d chunks=%d chunk=%d", what, batch_size, heads, num_chunks,
                  chunk_size);
    return SKV_EINVAL;
  }
  skv::FetchArgs<int32_t> f{};
  f.src = static_cast<const u32x4*>(values);
  f.src_row_vec = cpu_v_length / 8;
  f.dst = static_cast<u32x4*>(v_cache_buffer);
  f.dst_row_vec = gpu_v_stride / 8;
  f.dst_offset_vec = gpu_v_offset / 8;
  f.ids = offsets;
  f.cnts = cnts;
  f.S = num_chunks;
  f.chunk_vec = static_cast<int>(chunk_elems / 8);
  f.src_chunks = cpu_v_length / chunk_elems;
  f.rows = batch_size * heads;
  f.tiles = (num_chunks + skv::kChunksPerFetchWG - 1) / skv::kChunksPerFetchWG;
  f.workgroups = fetch_workgroups;  // the target (0: default); the launch sets the count
  RebuildArgs r{};
  r.u = u;
  r.u_sb = u_stride_b;
  r.u_sh = u_stride_h;
  r.u_sr = u_stride_row;
  r.u_rows = u_rows;
  r.sv = sv;
  r.sv_sb = sv_stride_b;
  r.sv_sh = sv_stride_h;
  r.sv_sn = sv_stride_n;
  r.ids = position_ids;
  r.id_sb = pid_stride_b;
  r.id_sh = pid_stride_h;
  r.cnts = cnts;
  r.cs = cos_sin;
  r.cs_stride = stride_cos_sin;
  r.cs_rows = cos_sin_rows;
  r.out = cache;
  r.o_sb = stride_cache_b;
  r.o_sh = stride_cache_h;
  r.o_ss = stride_cache_s;
  r.o_start = sparse_start;
  r.B = batch_size;
  r.H = heads;
  r.S = num_chunks;
  r.chunk = chunk_size;
  r.rank = rank;
  r.rebuild_wgs = rebuild_workgroups;
  return launch_rebuild(what, rope_mode == 0 ? kRopeHalf : kRopeGlm, true, r, static_cast<hipStream_t>(stream), &f);
}

extern "C" int skv_rebuild_k_rope_slots(const uint16_t* u, int64_t u_stride_b, int64_t u_stride_h,
                                        int64_t u_stride_row, int64_t u_rows, const uint16_t* sv, int64_t sv_stride_b,
                                        int64_t sv_stride_h, int64_t sv_stride_n, const int32_t* miss_ids,
                                        const int32_t* miss_slot, const int32_t* cnts, const uint16_t* cos_sin,
                                        int64_t stride_cos_sin, int64_t cos_sin_rows, int rope_mode, uint16_t* cache,
                                        int64_t stride_cache_b, int64_t stride_cache_h, int64_t stride_cache_s,
                                        int pool_start, int pool_slots, int batch_size, int heads, int num_chunks,
                                        int chunk_size, int rank, int head_dim, void* stream) {
  const char* what = "rebuild_k_rope_slots";
  if (head_dim != kHeadDim || (rope_mode != 0 && rope_mode != 1)) {
    skv_set_error("%s: head_dim=%d (must be 128), rope_mode=%d (0 half-split, 1 GLM)", what, head_dim, rope_mode);
    return SKV_EUNSUPPORTED;
  }
  if (!miss_slot || pool_slots < 1) {
    skv_set_error("%s: miss_slot=%p pool_slots=%d", what, static_cast<const void*>(miss_slot), pool_slots);
    return SKV_EINVAL;
  }
  RebuildArgs r{};
  r.u = u;
  r.u_sb = u_stride_b;
  r.u_sh = u_stride_h;
  r.u_sr = u_stride_row;
  r.u_rows = u_rows;
  r.sv = sv;
  r.sv_sb = sv_stride_b;
  r.sv_sh = sv_stride_h;
  r.sv_sn = sv_stride_n;
  r.ids = miss_ids;
  r.id_sh = num_chunks;
  r.id_sb = static_cast<int64_t>(num_chunks) * heads;
  r.cnts = cnts;
  r.cs = cos_sin;
  r.cs_stride = stride_cos_sin;
  r.cs_rows = cos_sin_rows;
  r.out = cache;
  r.o_sb = stride_cache_b;
  r.o_sh = stride_cache_h;
  r.o_ss = stride_cache_s;
  r.o_start = pool_start;
  r.B = batch_size;
  r.H = heads;
  r.S = num_chunks;
  r.chunk = chunk_size;
  r.rank = rank;
  r.dst_slot = miss_slot;
  r.ds_sh = num_chunks;
  r.ds_sb = static_cast<int64_t>(num_chunks) * heads;
  r.pool_slots = pool_slots;
  return launch_rebuild(what, rope_mode == 0 ? kRopeHalf : kRopeGlm, false, r, static_cast<hipStream_t>(stream));
}

// The chunk pool's value fetch of the misses (skv_gather_copy_misses_to_slots) and key rebuild
// (skv_rebuild_k_rope_slots) in one launch, their workgroups side by side: entries i >= cnts[r] of
// row r, chunk miss_ids[i] into slot miss_slot[i] of the value buffer (from the pinned host store)
// and of the key cache (rebuilt + RoPE). The pool's hits stay in their slots, so nothing moves first.
extern "C" int skv_fetch_misses_rebuild_k_rope_slots(
    const void* values, void* v_cache_buffer, int64_t cpu_v_length, int64_t gpu_v_offset, int64_t gpu_v_stride,
    const uint16_t* u, int64_t u_stride_b, int64_t u_stride_h, int64_t u_stride_row, int64_t u_rows,
    const uint16_t* sv, int64_t sv_stride_b, int64_t sv_stride_h, int64_t sv_stride_n, const int32_t* miss_ids,
    const int32_t* miss_slot, const int32_t* cnts, const uint16_t* cos_sin, int64_t stride_cos_sin,
    int64_t cos_sin_rows, int rope_mode, uint16_t* cache, int64_t stride_cache_b, int64_t stride_cache_h,
    int64_t stride_cache_s, int pool_start, int pool_slots, int batch_size, int heads, int num_chunks,
    int chunk_size, int rank, int head_dim, int fetch_workgroups, int rebuild_workgroups, void* stream) {
  const char* what = "fetch_misses_rebuild_k_rope_slots";
  if (fetch_workgroups < 0 || fetch_workgroups > 65536 || rebuild_workgroups < 0 || rebuild_workgroups > 65536) {
    skv_set_error("%s: fetch_workgroups=%d rebuild_workgroups=%d (0 for the default, at most 65536)", what,
                  fetch_workgroups, rebuild_workgroups);
    return SKV_EINVAL;
  }
  if (head_dim != kHeadDim || (rope_mode != 0 && rope_mode != 1)) {
    skv_set_error("%s: head_dim=%d (must be 128), rope_mode=%d (0 half-split, 1 GLM)", what, head_dim, rope_mode);
    return SKV_EUNSUPPORTED;
  }
  if (!values || !v_cache_buffer || !miss_ids || !miss_slot || !cnts) {
    skv_set_error("%s: null value-fetch pointer", what);
    return SKV_EINVAL;
  }
  if (batch_size <= 0 || heads <= 0 || num_chunks <= 0 || chunk_size <= 0 || pool_slots < num_chunks ||
      static_cast<int64_t>(pool_slots) * chunk_size * head_dim > (int64_t{1} << 31)) {
    skv_set_error("%s: invalid shape batch=%d heads=%d chunks=%d chunk=%d pool_slots=%d", what, batch_size, heads,
                  num_chunks, chunk_size, pool_slots);
    return SKV_EINVAL;
  }
  const int64_t chunk_elems = static_cast<int64_t>(chunk_size) * head_dim;
  if (!aligned16(values) || !aligned16(v_cache_buffer) || cpu_v_length % 8 || gpu_v_offset % 8 || gpu_v_stride % 8 ||
      cpu_v_length < chunk_elems || gpu_v_offset < 0 ||
      gpu_v_stride < gpu_v_offset + static_cast<int64_t>(pool_slots) * chunk_elems) {
    skv_set_error("%s: value rows must be 16-byte aligned and hold the pool (cpu_v_length=%lld offset=%lld "
                  "stride=%lld)", what, (long long)cpu_v_length, (long long)gpu_v_offset, (long long)gpu_v_stride);
    return SKV_EINVAL;
  }
  skv::FetchArgs<int32_t> f{};
  f.src = static_cast<const u32x4*>(values);
  f.src_row_vec = cpu_v_length / 8;
  f.dst = static_cast<u32x4*>(v_cache_buffer);
  f.dst_row_vec = gpu_v_stride / 8;
  f.dst_offset_vec = gpu_v_offset / 8;
  f.ids = miss_ids;
  f.cnts = cnts;
  f.dst_slot = miss_slot;
  f.pool_slots = pool_slots;
  f.S = num_chunks;
  f.chunk_vec = static_cast<int>(chunk_elems / 8);
  f.src_chunks = cpu_v_length / chunk_elems;
  f.rows = batch_size * heads;
  f.tiles = (num_chunks + skv::kChunksPerFetchWG - 1) / skv::kChunksPerFetchWG;
  f.workgroups = fetch_workgroups;  // the target (0: default); the launch sets the count
  RebuildArgs r{};
  r.u = u;
  r.u_sb = u_stride_b;
  r.u_sh = u_stride_h;
  r.u_sr = u_stride_row;
  r.u_rows = u_rows;
  r.sv = sv;
  r.sv_sb = sv_stride_b;
  r.sv_sh = sv_stride_h;
  r.sv_sn = sv_stride_n;
  r.ids = miss_ids;
  r.id_sh = num_chunks;
  r.id_sb = static_cast<int64_t>(num_chunks) * heads;
  r.cnts = cnts;
  r.cs = cos_sin;
  r.cs_stride = stride_cos_sin;
  r.cs_rows = cos_sin_rows;
  r.out = cache;
  r.o_sb = stride_cache_b;
  r.o_sh = stride_cache_h;
  r.o_ss = stride_cache_s;
  r.o_start = pool_start;
  r.B = batch_size;
  r.H = heads;
  r.S = num_chunks;
  r.chunk = chunk_size;
  r.rank = rank;
  r.dst_slot = miss_slot;
  r.ds_sh = num_chunks;
  r.ds_sb = static_cast<int64_t>(num_chunks) * heads;
  r.pool_slots = pool_slots;
  r.rebuild_wgs = rebuild_workgroups;
  return launch_rebuild(what, rope_mode == 0 ? kRopeHalf : kRopeGlm, false, r, static_cast<hipStream_t>(stream), &f);
}
