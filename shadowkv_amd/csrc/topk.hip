// a2: per-row top-k chunk selection over bf16 scores, fused with the landmark-id gather.
//
// Replaces torch.topk(scores, k).indices followed by k_landmark_idx.gather
// (models/kvcache/shadow.py:571-573). torch leaves the choice among equal scores to the
// implementation; this kernel fixes a total order — value descending, then index ascending —
// and emits the k winners in that order.
//
// One workgroup (16 wave64) per row, radix select on the 16-bit order-preserving key:
//   pass 1: LDS histogram of the high byte -> bin holding the k-th largest key;
//   pass 2: histogram of the low byte inside that bin -> the exact threshold key T and the
//           number of keys strictly above it;
//   pass 3: an order-preserving compaction in blocks of 1024 elements (one block scan per
//           block) collects every key > T and the first (k - #above) keys == T by index;
//   the k survivors are bitonic-sorted in LDS on (~key, index) and mapped through the
//   landmark-id table.
#include "skv_common.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kMaxK = 4096;

// Wave 0 finds bin b with above(b) < want <= above(b) + hist[b], where above(b) counts the
// entries in bins > b. Results go to out[0] = b, out[1] = above(b).
__device__ void select_bin(const uint32_t* hist, int want, int* out) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    uint32_t h[4];
    int local = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      h[u] = hist[255 - 4 * lane - u];
      local += static_cast<int>(h[u]);
    }
    int incl = skv::wave_inclusive_scan(local);
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

__global__ void __launch_bounds__(kThreads) topk_kernel(const uint16_t* __restrict__ scores, int64_t sstride,
                                                        const int64_t* __restrict__ lidx, int64_t istride, int n, int k,
                                                        int P, int64_t* __restrict__ out) {
  extern __shared__ __align__(16) uint64_t sel[];  // P
  __shared__ uint32_t hist[256];
  __shared__ int found[2];
  __shared__ int scan_tmp[kThreads / 64 + 1];

  const int row = blockIdx.x;
  const uint16_t* sr = scores + static_cast<int64_t>(row) * sstride;

  for (int i = threadIdx.x; i < 256; i += kThreads) hist[i] = 0;
  __syncthreads();
  for (int j = threadIdx.x; j < n; j += kThreads) atomicAdd(&hist[skv::bf16_order_key(sr[j]) >> 8], 1u);
  __syncthreads();
  select_bin(hist, k, found);
  const uint32_t b1 = static_cast<uint32_t>(found[0]);
  const int above1 = found[1];
  __syncthreads();

  for (int i = threadIdx.x; i < 256; i += kThreads) hist[i] = 0;
  __syncthreads();
  for (int j = threadIdx.x; j < n; j += kThreads) {
    const uint32_t key = skv::bf16_order_key(sr[j]);
    if ((key >> 8) == b1) atomicAdd(&hist[key & 255u], 1u);
  }
  __syncthreads();
  select_bin(hist, k - above1, found);
  const uint32_t T = (b1 << 8) | static_cast<uint32_t>(found[0]);
  const int c_gt = above1 + found[1];
  const int need_eq = k - c_gt;

  int gt_base = 0, eq_base = 0;
  for (int blk = 0; blk * kThreads < n; ++blk) {
    const int j = blk * kThreads + threadIdx.x;
    uint32_t key = 0;
    bool gt = false, eq = false;
    if (j < n) {
      key = skv::bf16_order_key(sr[j]);
      gt = key > T;
      eq = key == T;
    }
    int total = 0;
    const int excl = skv::block_exclusive_scan(static_cast<int>(gt) | (static_cast<int>(eq) << 16), scan_tmp, &total);
    const uint64_t composite = (static_cast<uint64_t>(0xffffu - key) << 32) | static_cast<uint32_t>(j);
    if (gt) sel[gt_base + (excl & 0xffff)] = composite;
    if (eq) {
      const int r = eq_base + (excl >> 16);
      if (r < need_eq) sel[c_gt + r] = composite;
    }
    gt_base += total & 0xffff;
    eq_base += total >> 16;
    if (gt_base >= c_gt && eq_base >= need_eq) break;  // workgroup-uniform
  }
  for (int i = k + threadIdx.x; i < P; i += kThreads) sel[i] = ~0ull;
  __syncthreads();

  for (int kk = 2; kk <= P; kk <<= 1) {
    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
      for (int i = threadIdx.x; i < P; i += kThreads) {
        const int ixj = i ^ jj;
        if (ixj > i) {
          const uint64_t x = sel[i], y = sel[ixj];
          if ((x > y) == ((i & kk) == 0)) {
            sel[i] = y;
            sel[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  const int64_t* lrow = lidx + static_cast<int64_t>(row) * istride;
  for (int t = threadIdx.x; t < k; t += kThreads) {
    const uint32_t j = static_cast<uint32_t>(sel[t]);
    out[static_cast<int64_t>(row) * k + t] = (j < static_cast<uint32_t>(n)) ? lrow[j] : -1;
  }
}

}  // namespace

extern "C" int skv_topk_gather(const uint16_t* scores, int64_t score_stride, const int64_t* landmark_idx,
                               int64_t idx_stride, int rows, int n, int k, int64_t* out_ids, void* stream) {
  const char* what = "topk_gather";
  if (!scores || !landmark_idx || !out_ids) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (rows < 1 || n < 1 || k < 1 || k > n || score_stride < n || idx_stride < n) {
    skv_set_error("%s: invalid shape rows=%d n=%d k=%d strides=%lld/%lld", what, rows, n, k, (long long)score_stride,
                  (long long)idx_stride);
    return SKV_EINVAL;
  }
  if (k > kMaxK) {
    skv_set_error("%s: k=%d above the supported maximum %d", what, k, kMaxK);
    return SKV_EUNSUPPORTED;
  }
  int P = 64;
  while (P < k) P <<= 1;
  hipLaunchKernelGGL(topk_kernel, dim3(rows), dim3(kThreads), static_cast<size_t>(P) * sizeof(uint64_t),
                     static_cast<hipStream_t>(stream), scores, score_stride, landmark_idx, idx_stride, n, k, P, out_ids);
  return skv_check_launch(what);
}
