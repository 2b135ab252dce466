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
//   * workgroup = 4 waves, owns kTileRows consecutive rows of one head; SV of that head
//     (128 x rank bf16, 40 KB at rank 160) is staged once into LDS;
//   * a wave computes 32 rows x 128 columns per iteration with v_mfma_f32_16x16x32_bf16:
//     A = 16 gathered U rows (16-byte loads straight from HBM, 4 lanes per 64-byte k-slab),
//     B = SV from LDS, 8 column tiles x ceil(rank/32) k-steps, fp32 accumulation;
//   * the epilogue rounds to bf16 and applies the rotation lane-locally: columns d and d+64
//     live in column tiles t and t+4 of the same lane (GLM pairs use a 1-lane shuffle).
//   * blockIdx -> (head, tile) is XCD-aware: all tiles of a head land on the same XCD
//     (workgroups are dealt round-robin over the 8 XCDs), so SV is fetched from HBM once per
//     head and re-read from that XCD's L2.
#include "rope_math.h"

namespace {

using skv::u32x4;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kTileRows = 256;  // rows per workgroup: 4 waves x 2 iterations x 32 rows
constexpr int kHeadDim = 128;
constexpr int kMaxRank = 192;
constexpr int kXcds = 8;

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
};

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8_t, v); }

template <typename IdxT>
__device__ __forceinline__ int64_t row_pos(const RebuildArgs& a, const IdxT* ids, int row) {
  return static_cast<int64_t>(ids[row / a.chunk]) * a.chunk + row % a.chunk;
}

template <int kMode, typename IdxT>
__global__ void __launch_bounds__(kThreads) rebuild_kernel(RebuildArgs a) {
  extern __shared__ __align__(16) uint16_t sv_lds[];  // [128][rank + 8]

  const int bid = blockIdx.x;
  const int xcd = bid % kXcds;
  const int local = bid / kXcds;
  const int head = xcd + kXcds * (local / a.tiles);
  const int tile = local % a.tiles;
  const int BH = a.B * a.H;
  if (head >= BH) return;
  const int b = head / a.H;
  const int h = head - b * a.H;

  const int total_rows = a.S * a.chunk;
  const int miss_begin = min(a.cnts[head], a.S) * a.chunk;
  const int row_begin = tile * kTileRows;
  const int row_end = min(row_begin + kTileRows, total_rows);
  if (row_end <= miss_begin || row_begin >= row_end) return;

  const int ldr = a.rank + 8;  // padded LDS row (elements) against bank conflicts
  const int k8 = a.rank / 8;
  const uint16_t* svp = a.sv + b * a.sv_sb + h * a.sv_sh;
  for (int idx = threadIdx.x; idx < kHeadDim * k8; idx += kThreads) {
    int n = idx / k8, kk = (idx - n * k8) * 8;
    *reinterpret_cast<u32x4*>(&sv_lds[n * ldr + kk]) = *reinterpret_cast<const u32x4*>(&svp[n * a.sv_sn + kk]);
  }
  __syncthreads();

  const IdxT* ids = static_cast<const IdxT*>(a.ids) + b * a.id_sb + h * a.id_sh;
  const uint16_t* ubase = a.u + b * a.u_sb + h * a.u_sh;
  uint16_t* obase = a.out + b * a.o_sb + h * a.o_sh;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;  // A row / B column / D column within a 16x16 tile
  const int lk = lane >> 4;  // k-slab (A/B) and row quad (D)
  const int ksteps = (a.rank + 31) / 32;
  const u32x4 zero4 = {0u, 0u, 0u, 0u};

  for (int it = 0; it < 2; ++it) {
    const int rb = row_begin + (wave + 4 * it) * 32;
    if (rb >= row_end || rb + 32 <= miss_begin) continue;  // wave-uniform

    // A fragments for the two 16-row halves.
    bf16x8_t afrag[2][kMaxRank / 32];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int row = rb + m * 16 + li;
      bool valid = row >= miss_begin && row < row_end;
      int64_t pos = valid ? row_pos(a, ids, row) : 0;
      valid = valid && pos >= 0 && pos < a.u_rows;
      const uint16_t* up = ubase + pos * a.u_sr;
#pragma unroll
      for (int ks = 0; ks < kMaxRank / 32; ++ks) {
        const int kk = ks * 32 + lk * 8;
        u32x4 v = zero4;
        if (ks < ksteps && valid && kk < a.rank) v = *reinterpret_cast<const u32x4*>(up + kk);
        afrag[m][ks] = as_bf16x8(v);
      }
    }

    f32x4_t acc[2][8];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[m][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int ks = 0; ks < kMaxRank / 32; ++ks) {
      if (ks >= ksteps) break;
      const int kk = ks * 32 + lk * 8;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        u32x4 bv = zero4;
        if (kk < a.rank) bv = *reinterpret_cast<const u32x4*>(&sv_lds[(t * 16 + li) * ldr + kk]);
        const bf16x8_t bfrag = as_bf16x8(bv);
        acc[0][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag[0][ks], bfrag, acc[0][t], 0, 0, 0);
        acc[1][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag[1][ks], bfrag, acc[1][t], 0, 0, 0);
      }
    }

    // Epilogue: lane holds rows rb + m*16 + lk*4 + v, column t*16 + li of tile t.
#pragma unroll
    for (int m = 0; m < 2; ++m) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = rb + m * 16 + lk * 4 + v;
        bool valid = row >= miss_begin && row < row_end;
        int64_t pos = valid ? row_pos(a, ids, row) : 0;
        if (kMode != kPlain) valid = valid && pos >= 0 && pos < a.cs_rows;
        uint16_t* orow = obase + static_cast<int64_t>(a.o_start + row) * a.o_ss;
        const uint16_t* c = a.cs + pos * a.cs_stride;
        if (kMode == kPlain) {
          if (valid) {
#pragma unroll
            for (int t = 0; t < 8; ++t) orow[t * 16 + li] = skv::f2bf(acc[m][t][v]);
          }
        } else if (kMode == kRopeHalf) {
          if (valid) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const int d = t * 16 + li;
              uint16_t y1, y2;
              skv::rope_half_split(skv::f2bf(acc[m][t][v]), skv::f2bf(acc[m][t + 4][v]), c[d], c[d + 64], y1, y2);
              orow[d] = y1;
              orow[d + 64] = y2;
            }
          }
        } else {  // GLM: interleaved pairs on dims 0..63, dims 64..127 unchanged
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int d = t * 16 + li;
            const uint16_t x = skv::f2bf(acc[m][t][v]);
            const uint16_t other = static_cast<uint16_t>(__shfl_xor(static_cast<int>(x), 1, 64));
            if (valid) {
              const int pair = d >> 1;
              const uint16_t xe = (d & 1) ? other : x;
              const uint16_t xo = (d & 1) ? x : other;
              uint16_t ye, yo;
              skv::rope_half_split(xe, xo, c[pair], c[pair + 32], ye, yo);
              orow[d] = (d & 1) ? yo : ye;
            }
          }
          if (valid) {
#pragma unroll
            for (int t = 4; t < 8; ++t) orow[t * 16 + li] = skv::f2bf(acc[m][t][v]);
          }
        }
      }
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch_rebuild(const char* what, int mode, bool ids64, RebuildArgs a, hipStream_t stream) {
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
  a.tiles = (a.S * a.chunk + kTileRows - 1) / kTileRows;
  const int BH = a.B * a.H;
  const int heads_padded = (BH + kXcds - 1) / kXcds * kXcds;
  const dim3 grid(static_cast<unsigned>(heads_padded * a.tiles));
  const size_t lds = static_cast<size_t>(kHeadDim) * (a.rank + 8) * sizeof(uint16_t);
#define SKV_LAUNCH(M, T) hipLaunchKernelGGL((rebuild_kernel<M, T>), grid, dim3(kThreads), lds, stream, a)
  if (ids64) {
    if (mode == kPlain) SKV_LAUNCH(kPlain, int64_t);
    else if (mode == kRopeHalf) SKV_LAUNCH(kRopeHalf, int64_t);
    else SKV_LAUNCH(kRopeGlm, int64_t);
  } else {
    if (mode == kPlain) SKV_LAUNCH(kPlain, int32_t);
    else if (mode == kRopeHalf) SKV_LAUNCH(kRopeHalf, int32_t);
    else SKV_LAUNCH(kRopeGlm, int32_t);
  }
#undef SKV_LAUNCH
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
