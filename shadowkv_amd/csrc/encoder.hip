// f1: the prefill-side encoder of the offload cache (models/kvcache/shadow.py:463-544), on the GPU.
//
//   chunk_stats_kernel    per (b, h, chunk) of the post-RoPE keys: the chunk mean (the landmark
//                         candidate, fp32 sum / c rounded once to bf16, shadow.py:486-488) and the
//                         minimum over the chunk's rows of cos(candidate, row) in fp32
//                         (shadow.py:489-490);
//   select_outliers_kernel one workgroup per (b, h): the outlier_chunk chunks of smallest minimum
//                         cosine (torch.topk(largest=False), shadow.py:490) by a 4-pass radix
//                         select over order-preserving 32-bit keys, ties to the lowest chunk id,
//                         written in ascending (cosine, id) order; then the ids of every other
//                         chunk, ascending (the landmark ids, shadow.py:513-516);
//   gather_rows_kernel    landmarks[r][j] = candidates[r][landmark_idx[r][j]] (shadow.py:517-519).
//
// The rest of the encoder is library work or other entry points: the rank-R factors come from the
// Gram matrix K^T K (hipBLASLt) and its eigendecomposition (rocSOLVER), the outlier and initially
// selected K/V chunks are copied by the chunk-gather kernel, the initial selection is the decode
// path's scoring + GQA max + top-k.
#include "skv_common.h"

namespace {

using skv::u32x4;

constexpr int kHeadDim = 128;
constexpr int kThreads = 256;
constexpr int kMaxChunks = 131072;  // 1M-token prompts at chunk 8 (LDS bitmap of 16 KB)
constexpr int kMaxOutliers = 512;
constexpr int kMaxChunkRows = 32;  // rows per chunk held in registers by chunk_stats (8 per lane)

// One wave per chunk, 16 lanes per row (8 dims each), 4 rows per load instruction; RPL rows per
// lane (chunk size <= 4 * RPL).
template <int kRowsPerLane>
__global__ void __launch_bounds__(kThreads) chunk_stats_kernel(const uint16_t* __restrict__ k, int64_t k_sb,
                                                               int64_t k_sh, int64_t k_ss, int H, int chunks,
                                                               int c, uint16_t* __restrict__ cand,
                                                               float* __restrict__ min_cos, int total) {
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (item >= total) return;  // wave-uniform
  const int bh = item / chunks;
  const int ch = item - bh * chunks;
  const int b = bh / H, h = bh - b * H;
  const int li = lane & 15, grp = lane >> 4;
  const uint16_t* base = k + b * k_sb + h * k_sh + static_cast<int64_t>(ch) * c * k_ss + 8 * li;
  // Sum of the chunk's rows for this lane's 8 dims (rows grp, grp+4, ...), then across the 4 row
  // groups (lanes li, li+16, li+32, li+48): v_permlane32_swap / v_permlane16_swap of a value with
  // itself hand each lane its own value and its partner's (lane ^ 32, then lane ^ 16).
  // The lane's rows (grp, grp+4, ...; at most kRowsPerLane) stay in registers for both passes; all
  // are requested before the first is used.
  u32x4 rv[kRowsPerLane];
#pragma unroll
  for (int j = 0; j < kRowsPerLane; ++j) {
    const int r = grp + 4 * j;
    rv[j] = skv::load16_or_zero(base + static_cast<int64_t>(min(r, c - 1)) * k_ss, r < c);
  }
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < kRowsPerLane; ++j) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s[2 * e] += skv::bf_lo(rv[j][e]);
      s[2 * e + 1] += skv::bf_hi(rv[j][e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(s[e]), __float_as_uint(s[e]), false, false);
    s[e] = __uint_as_float(x[0]) + __uint_as_float(x[1]);  // lower-half lane's value + upper-half lane's
    const auto y = __builtin_amdgcn_permlane16_swap(__float_as_uint(s[e]), __float_as_uint(s[e]), false, false);
    s[e] = __uint_as_float(y[0]) + __uint_as_float(y[1]);
  }
  // Candidate = bf16(sum / c); every row group holds the same values, group 0 stores them.
  float m[8];
  const float cf = static_cast<float>(c);
#pragma unroll
  for (int e = 0; e < 8; ++e) m[e] = skv::bf2f(skv::f2bf(s[e] / cf));
  if (grp == 0) {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = skv::f2bf2(m[2 * e], m[2 * e + 1]);
    *reinterpret_cast<u32x4*>(cand + static_cast<int64_t>(item) * kHeadDim + 8 * li) = o;
  }
  // ||candidate||: sum over the 16 lanes of a row group (all groups hold the candidate).
  float mm = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) mm = fmaf(m[e], m[e], mm);
  mm += skv::row_ror<8>(mm);
  mm += skv::row_ror<4>(mm);
  mm += skv::row_ror<2>(mm);
  mm += skv::row_ror<1>(mm);
  const float nm = fmaxf(sqrtf(mm), 1e-8f);
  // cos(candidate, row) for every row; the minimum over the chunk.
  float mn = INFINITY;
#pragma unroll
  for (int j = 0; j < kRowsPerLane; ++j) {
    const int r = grp + 4 * j;
    float dot = 0.f, rr = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = skv::bf_lo(rv[j][e]), bq = skv::bf_hi(rv[j][e]);
      dot = fmaf(m[2 * e], a, fmaf(m[2 * e + 1], bq, dot));
      rr = fmaf(a, a, fmaf(bq, bq, rr));
    }
    dot += skv::row_ror<8>(dot);
    dot += skv::row_ror<4>(dot);
    dot += skv::row_ror<2>(dot);
    dot += skv::row_ror<1>(dot);
    rr += skv::row_ror<8>(rr);
    rr += skv::row_ror<4>(rr);
    rr += skv::row_ror<2>(rr);
    rr += skv::row_ror<1>(rr);
    if (r < c) mn = fminf(mn, dot / (nm * fmaxf(sqrtf(rr), 1e-8f)));
  }
  mn = fminf(fminf(skv::lane_value(mn, 0), skv::lane_value(mn, 16)),
             fminf(skv::lane_value(mn, 32), skv::lane_value(mn, 48)));
  if (lane == 0) min_cos[item] = mn;
}

// Order-preserving unsigned key of a float (ascending floats -> ascending keys; NaN last).
__device__ __forceinline__ uint32_t float_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (f != f) return 0xffffffffu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ void __launch_bounds__(kThreads) select_outliers_kernel(const float* __restrict__ min_cos, int chunks,
                                                                   int k_out, int64_t* __restrict__ outlier_idx,
                                                                   int64_t* __restrict__ landmark_idx) {
  __shared__ int hist[256];
  __shared__ int scan[kThreads / 64 + 1];
  __shared__ uint32_t sel_key[kMaxOutliers];
  __shared__ int sel_id[kMaxOutliers];
  __shared__ uint32_t is_out[kMaxChunks / 32];
  __shared__ int bin_sh, need_sh;
  __shared__ int count_sh;
  const int row = blockIdx.x;
  const float* key_row = min_cos + static_cast<int64_t>(row) * chunks;
  const int per = (chunks + kThreads - 1) / kThreads;  // contiguous range per thread (id order)
  const int i0 = min(chunks, threadIdx.x * per), i1 = min(chunks, i0 + per);

  // Radix select of the k_out-th smallest key, 8 bits per pass from the top.
  uint32_t prefix = 0, mask = 0;
  int need = k_out;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = threadIdx.x; i < 256; i += kThreads) hist[i] = 0;
    __syncthreads();
    for (int i = i0; i < i1; ++i) {
      const uint32_t kk = float_key(key_row[i]);
      if ((kk & mask) == prefix) atomicAdd(&hist[(kk >> shift) & 255], 1);
    }
    __syncthreads();
    if (threadIdx.x < 64) {  // wave 0: cumulative counts over the 256 bins, 4 per lane
      int c4[4], t = 0;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        c4[u] = hist[threadIdx.x * 4 + u];
        t += c4[u];
      }
      const int incl = skv::wave_inclusive_scan(t);
      int before = incl - t;
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
  // prefix = exact key of the k_out-th smallest; `need` of the chunks equal to it are taken, lowest
  // ids first: a block scan of per-thread equal counts over the id-ordered ranges.
  for (int w = threadIdx.x; w < (chunks + 31) / 32; w += kThreads) is_out[w] = 0u;
  if (threadIdx.x == 0) count_sh = 0;
  int eq = 0;
  for (int i = i0; i < i1; ++i) eq += float_key(key_row[i]) == prefix;
  int eq_total;
  int eq_before = skv::block_exclusive_scan(eq, scan, &eq_total);
  for (int i = i0; i < i1; ++i) {
    const uint32_t kk = float_key(key_row[i]);
    bool take = kk < prefix;
    if (kk == prefix) take = eq_before++ < need;
    if (take) {
      const int slot = atomicAdd(&count_sh, 1);
      sel_key[slot] = kk;
      sel_id[slot] = i;
      atomicOr(&is_out[i >> 5], 1u << (i & 31));
    }
  }
  __syncthreads();
  // Ascending (key, id) order of the selected chunks: rank of each by counting (k_out <= 512).
  for (int j = threadIdx.x; j < k_out; j += kThreads) {
    const uint32_t kj = sel_key[j];
    const int ij = sel_id[j];
    int rank = 0;
    for (int t = 0; t < k_out; ++t) rank += (sel_key[t] < kj) || (sel_key[t] == kj && sel_id[t] < ij);
    outlier_idx[static_cast<int64_t>(row) * k_out + rank] = ij;
  }
  // Landmark ids: every other chunk, ascending.
  int keep = 0;
  for (int i = i0; i < i1; ++i) keep += !((is_out[i >> 5] >> (i & 31)) & 1u);
  int keep_total;
  int pos = skv::block_exclusive_scan(keep, scan, &keep_total);
  int64_t* lrow = landmark_idx + static_cast<int64_t>(row) * (chunks - k_out);
  for (int i = i0; i < i1; ++i)
    if (!((is_out[i >> 5] >> (i & 31)) & 1u)) lrow[pos++] = i;
}

// dst[r][j] = src[r][idx[r][j]] for 256-byte rows; one wave per 4 rows (16 lanes per row).
__global__ void __launch_bounds__(kThreads) gather_rows_kernel(const u32x4* __restrict__ src, int src_rows,
                                                               const int64_t* __restrict__ idx, u32x4* __restrict__ dst,
                                                               int dst_rows, int64_t total) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t row = t >> 4;  // global destination row (r * dst_rows + j)
  if (row >= total) return;
  const int64_t r = row / dst_rows;
  const int64_t s = idx[row];
  if (s < 0 || s >= src_rows) return;
  dst[row * 16 + (t & 15)] = src[(r * src_rows + s) * 16 + (t & 15)];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int skv_chunk_stats(const uint16_t* keys, int64_t stride_b, int64_t stride_h, int64_t stride_s,
                               int batch_size, int heads, int chunks, int chunk_size, uint16_t* candidates,
                               float* min_cos, void* stream) {
  const char* what = "chunk_stats";
  if (!keys || !candidates || !min_cos) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (batch_size < 1 || heads < 1 || chunks < 1 || chunk_size < 1) {
    skv_set_error("%s: batch=%d heads=%d chunks=%d chunk_size=%d", what, batch_size, heads, chunks, chunk_size);
    return SKV_EINVAL;
  }
  if (chunk_size > kMaxChunkRows) {
    skv_set_error("%s: chunk_size=%d (at most %d)", what, chunk_size, kMaxChunkRows);
    return SKV_EUNSUPPORTED;
  }
  if (!aligned16(keys) || !aligned16(candidates) || stride_b % 8 || stride_h % 8 || stride_s % 8) {
    skv_set_error("%s: key rows must be 16-byte aligned", what);
    return SKV_EINVAL;
  }
  const int64_t total = static_cast<int64_t>(batch_size) * heads * chunks;
  if (total > (int64_t{1} << 30)) {
    skv_set_error("%s: %lld chunks", what, (long long)total);
    return SKV_EUNSUPPORTED;
  }
  const int per_wg = kThreads / 64;
  const dim3 grid(static_cast<unsigned>((total + per_wg - 1) / per_wg));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, s, keys, stride_b, stride_h, stride_s, heads, chunks,
                       chunk_size, candidates, min_cos, static_cast<int>(total));
  };
  if (chunk_size <= 4) go(chunk_stats_kernel<1>);
  else if (chunk_size <= 8) go(chunk_stats_kernel<2>);
  else if (chunk_size <= 16) go(chunk_stats_kernel<4>);
  else go(chunk_stats_kernel<8>);
  return skv_check_launch(what);
}

extern "C" int skv_select_outliers(const float* min_cos, int rows, int chunks, int outliers, int64_t* outlier_idx,
                                   int64_t* landmark_idx, void* stream) {
  const char* what = "select_outliers";
  if (!min_cos || !outlier_idx || !landmark_idx) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (rows < 1 || chunks < 1 || chunks > kMaxChunks || outliers < 1 || outliers > kMaxOutliers ||
      outliers >= chunks) {
    skv_set_error("%s: rows=%d chunks=%d outliers=%d (chunks <= %d, 1 <= outliers <= %d, outliers < chunks)", what,
                  rows, chunks, outliers, kMaxChunks, kMaxOutliers);
    return SKV_EUNSUPPORTED;
  }
  hipLaunchKernelGGL(select_outliers_kernel, dim3(rows), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     min_cos, chunks, outliers, outlier_idx, landmark_idx);
  return skv_check_launch(what);
}

extern "C" int skv_gather_rows(const uint16_t* src, int rows, int src_rows, const int64_t* idx, int dst_rows,
                               uint16_t* dst, void* stream) {
  const char* what = "gather_rows";
  if (!src || !idx || !dst) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (rows < 1 || src_rows < 1 || dst_rows < 1) {
    skv_set_error("%s: rows=%d src_rows=%d dst_rows=%d", what, rows, src_rows, dst_rows);
    return SKV_EINVAL;
  }
  if (!aligned16(src) || !aligned16(dst)) {
    skv_set_error("%s: rows must be 16-byte aligned", what);
    return SKV_EINVAL;
  }
  const int64_t total = static_cast<int64_t>(rows) * dst_rows;
  const int64_t threads = total * 16;
  hipLaunchKernelGGL(gather_rows_kernel, dim3(static_cast<unsigned>((threads + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream), reinterpret_cast<const u32x4*>(src), src_rows,
                     idx, reinterpret_cast<u32x4*>(dst), dst_rows, total);
  return skv_check_launch(what);
}
