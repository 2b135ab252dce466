// a2: per-row top-k chunk selection over bf16 scores, fused with the landmark-id gather.
//
// Replaces torch.topk(scores, k).indices followed by k_landmark_idx.gather
// (models/kvcache/shadow.py:571-573). torch leaves the choice among equal scores to the
// implementation; this kernel fixes a total order — value descending, then index ascending —
// and emits the k winners in that order.
//
// One workgroup (16 wave64) per row, radix select on the 16-bit order-preserving key
// (select_core.h): a high-byte then a low-byte LDS histogram locate the k-th key T, an
// order-preserving block-scan compaction collects every key > T and the first keys == T by
// index, and the survivors are bitonic-sorted in LDS and mapped through the landmark ids.
#include "select_core.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kMaxK = 4096;

__global__ void __launch_bounds__(kThreads) topk_kernel(const uint16_t* __restrict__ scores, int64_t sstride,
                                                        const int64_t* __restrict__ lidx, int64_t istride, int n, int k,
                                                        int P, int64_t* __restrict__ out) {
  extern __shared__ __align__(16) uint64_t sel[];  // P
  __shared__ skv::TopkShared sh;
  const int row = blockIdx.x;
  const uint16_t* sr = scores + static_cast<int64_t>(row) * sstride;
  skv::radix_topk([&](int j) { return skv::bf16_order_key(sr[j]); }, n, k, P, sel, sh, false);
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
