// a1 tail + a2 + a3 fused: chunk selection for one decode step in one launch.
//
// Replaces the sequence of models/kvcache/shadow.py:553-574 after the scoring GEMM:
// the softmax normalisation of batch_gemm_softmax (kernels/batch_gemm_softmax.h:66-242),
// torch.max over the query-head group, torch.topk, the landmark-id gather, and
// reorder_keys_and_compute_offsets (kernels/gather_copy.cu:189-235).
//
// One workgroup (16 wave64) per (batch, kv-head) row; thread t owns the contiguous landmarks
// [t*E, t*E+E):
//   1. merge the per-256-column (max, sum exp) partials of every query row;
//   2. p_j = max_i bf16(exp(D[i,j] - max_i) / sum_i), kept as 16-bit order keys in LDS (or in
//      global scratch when n is too large), high-byte histogram with run-length-merged atomics;
//   3. radix threshold: the k-th key T and the count of keys above it (two histogram passes);
//   4. winners = keys > T plus the lowest-index keys == T (one block scan ranks the ties); each
//      winner's chunk id is set in a chunk-id bitmap `sel`, the previous slots' ids in `old`;
//   5. hits: a scan over the previous slots whose id is in `sel` emits them in old-slot order;
//      misses: a popcount scan over the words of `sel & ~old` emits them in ascending id order.
// With out_selected requested, the winners are additionally bitonic-sorted (value desc, index
// asc) to emit the ids in top-k order. The arithmetic of step 2 and the selection rule are those
// of score.hip softmax_kernel and topk.hip, so the result is bit-identical to the unfused path.
#include "select_core.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kMaxM = 16;
constexpr int kMaxS = 2048;
constexpr size_t kLdsBudget = 60 * 1024;  // dynamic LDS cap (static LDS adds ~1.4 KB)

struct SelectArgs {
  const uint16_t* D;
  const float* norm;
  const float* sum;
  int m, n, tiles;
  const int64_t* lidx;
  int64_t lstride;
  int S, P, n_lds, words;  // words = bitmap words covering chunk ids [0, 32*words)
  int64_t* pos;
  int32_t* offsets;
  int32_t* cnts;
  uint16_t* out_scores;  // [rows][n], required when n_lds == 0
  int64_t* out_sel;      // [rows][S] ids in top-k order, optional
};

__device__ __forceinline__ int scan_excl(int v, int* scratch, int* total) {
  return skv::block_exclusive_scan(v, scratch, total);
}

__global__ void __launch_bounds__(kThreads) select_kernel(SelectArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint32_t* selmap = reinterpret_cast<uint32_t*>(smem);   // words
  uint32_t* oldmap = selmap + a.words;                     // words
  uint64_t* sorted = reinterpret_cast<uint64_t*>(oldmap + a.words);  // P, only with out_sel (8-byte aligned)
  uint16_t* keys = reinterpret_cast<uint16_t*>(sorted + (a.out_sel ? a.P : 0));      // n_lds
  __shared__ skv::TopkShared sh;
  __shared__ float gmax[kMaxM], ginv[kMaxM];
  __shared__ int sel_count;

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int m = a.m, n = a.n, S = a.S;
  const int64_t base = static_cast<int64_t>(row) * S;
  int64_t* prow = a.pos + base;

  for (int i = wave; i < m; i += kThreads / 64) {
    const float* nr = a.norm + (static_cast<int64_t>(row) * m + i) * a.tiles;
    const float* sr = a.sum + (static_cast<int64_t>(row) * m + i) * a.tiles;
    float mx = -INFINITY;
    for (int t = lane; t < a.tiles; t += 64) mx = fmaxf(mx, nr[t]);
    mx = skv::wave_max(mx);
    float s = 0.f;
    for (int t = lane; t < a.tiles; t += 64) s += sr[t] * expf(nr[t] - mx);
    s = skv::wave_sum(s);
    if (lane == 0) {
      gmax[i] = mx;
      ginv[i] = 1.f / s;
    }
  }
  for (int i = tid; i < 256; i += kThreads) sh.hist[i] = 0;
  for (int w = tid; w < 2 * a.words; w += kThreads) selmap[w] = 0;  // selmap and oldmap
  if (tid == 0) sel_count = 0;
  __syncthreads();
  // previous slots into the old-id bitmap (ids outside the bitmap can never be hits)
  for (int j = tid; j < S; j += kThreads) {
    const int64_t id = prow[j];
    if (id >= 0 && id < 32ll * a.words) atomicOr(&oldmap[id >> 5], 1u << (id & 31));
  }

  const int E = (n + kThreads - 1) / kThreads;
  const int lo = min(tid * E, n), hi = min(lo + E, n);
  const uint16_t* Drow = a.D + static_cast<int64_t>(row) * m * n;
  uint16_t* srow = a.out_scores ? a.out_scores + static_cast<int64_t>(row) * n : nullptr;
  {
    uint32_t run_bin = 0xffffffffu, run = 0;
    for (int j = lo; j < hi; ++j) {
      float best = -INFINITY;
      for (int i = 0; i < m; ++i) {
        const uint16_t p = skv::f2bf(expf(skv::bf2f(Drow[static_cast<int64_t>(i) * n + j]) - gmax[i]) * ginv[i]);
        best = fmaxf(best, skv::bf2f(p));
      }
      const uint16_t b = skv::f2bf(best);
      const uint32_t key = skv::bf16_order_key(b);
      if (a.n_lds) keys[j] = static_cast<uint16_t>(key);
      if (srow) srow[j] = b;
      if ((key >> 8) != run_bin) {
        if (run) atomicAdd(&sh.hist[run_bin], run);
        run_bin = key >> 8;
        run = 0;
      }
      ++run;
    }
    if (run) atomicAdd(&sh.hist[run_bin], run);
  }
  __syncthreads();
  auto key_of = [&](int j) -> uint32_t {
    return a.n_lds ? static_cast<uint32_t>(keys[j]) : skv::bf16_order_key(srow[j]);
  };

  skv::select_bin(sh.hist, S, sh.found);
  const uint32_t b1 = static_cast<uint32_t>(sh.found[0]);
  const int above1 = sh.found[1];
  __syncthreads();
  for (int i = tid; i < 256; i += kThreads) sh.hist[i] = 0;
  __syncthreads();
  {
    uint32_t run_bin = 0xffffffffu, run = 0;
    for (int j = lo; j < hi; ++j) {
      const uint32_t kj = key_of(j);
      if ((kj >> 8) != b1) continue;
      if ((kj & 255u) != run_bin) {
        if (run) atomicAdd(&sh.hist[run_bin], run);
        run_bin = kj & 255u;
        run = 0;
      }
      ++run;
    }
    if (run) atomicAdd(&sh.hist[run_bin], run);
  }
  __syncthreads();
  skv::select_bin(sh.hist, S - above1, sh.found);
  const uint32_t T = (b1 << 8) | static_cast<uint32_t>(sh.found[0]);
  const int need_eq = S - above1 - sh.found[1];

  // Rank the ties in index order (blocked ownership makes the scan order the index order).
  int my_eq = 0;
  for (int j = lo; j < hi; ++j) my_eq += key_of(j) == T;
  int total_eq = 0;
  int eq_rank = scan_excl(my_eq, sh.scan, &total_eq);
  const int64_t* lrow = a.lidx + static_cast<int64_t>(row) * a.lstride;
  for (int j = lo; j < hi; ++j) {
    const uint32_t kj = key_of(j);
    bool win = kj > T;
    if (kj == T) win = eq_rank++ < need_eq;
    if (!win) continue;
    const int64_t id = lrow[j];
    if (id >= 0 && id < 32ll * a.words) atomicOr(&selmap[id >> 5], 1u << (id & 31));
    if (a.out_sel) sorted[atomicAdd(&sel_count, 1)] = (static_cast<uint64_t>(0xffffu - kj) << 32) | static_cast<uint32_t>(j);
  }
  __syncthreads();

  // Hits in previous-slot order.
  const int Es = (S + kThreads - 1) / kThreads;
  const int slo = min(tid * Es, S), shi = min(slo + Es, S);
  int my_hits = 0;
  for (int j = slo; j < shi; ++j) {
    const int64_t id = prow[j];
    my_hits += id >= 0 && id < 32ll * a.words && ((selmap[id >> 5] >> (id & 31)) & 1u);
  }
  // Misses in ascending id order.
  const int Ew = (a.words + kThreads - 1) / kThreads;
  const int wlo = min(tid * Ew, a.words), whi = min(wlo + Ew, a.words);
  int my_miss = 0;
  for (int w = wlo; w < whi; ++w) my_miss += __popc(selmap[w] & ~oldmap[w]);
  int total_hits = 0, total_miss = 0;
  int hrank = scan_excl(my_hits, sh.scan, &total_hits);
  int mrank = scan_excl(my_miss, sh.scan, &total_miss);
  // All previous-slot ids were read above (scan barriers separate reads from these writes).
  int64_t hit_ids[kMaxS / kThreads + 1];
  int nh = 0;
  for (int j = slo; j < shi; ++j) {
    const int64_t id = prow[j];
    if (id >= 0 && id < 32ll * a.words && ((selmap[id >> 5] >> (id & 31)) & 1u)) hit_ids[nh++] = id | (static_cast<int64_t>(j) << 40);
  }
  __syncthreads();
  for (int h = 0; h < nh; ++h) {
    const int64_t id = hit_ids[h] & ((1ll << 40) - 1);
    const int j = static_cast<int>(hit_ids[h] >> 40);
    prow[hrank] = id;
    a.offsets[base + hrank] = j;
    ++hrank;
  }
  for (int w = wlo; w < whi; ++w) {
    uint32_t bits = selmap[w] & ~oldmap[w];
    while (bits) {
      const int b = __ffs(bits) - 1;
      bits &= bits - 1;
      const int id = w * 32 + b;
      prow[total_hits + mrank] = id;
      a.offsets[base + total_hits + mrank] = id;
      ++mrank;
    }
  }
  if (tid == 0) a.cnts[row] = total_hits;

  if (a.out_sel) {
    for (int i = S + tid; i < a.P; i += kThreads) sorted[i] = ~0ull;
    __syncthreads();
    skv::block_bitonic_sort(sorted, a.P);
    for (int t = tid; t < S; t += kThreads) {
      const uint32_t j = static_cast<uint32_t>(sorted[t]);
      a.out_sel[base + t] = (j < static_cast<uint32_t>(n)) ? lrow[j] : -1;
    }
  }
}

}  // namespace

extern "C" int skv_select_chunks(const uint16_t* D, const float* norm, const float* sum, int rows, int m, int n,
                                 const int64_t* landmark_idx, int64_t idx_stride, int select_sets, int num_chunks,
                                 int64_t* position_ids, int32_t* offsets, int32_t* cnts, uint16_t* out_scores,
                                 int64_t* out_selected, void* stream) {
  const char* what = "select_chunks";
  if (!D || !norm || !sum || !landmark_idx || !position_ids || !offsets || !cnts) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (rows < 1 || m < 1 || m > kMaxM || n < 1 || idx_stride < n || select_sets < 1 || select_sets > n ||
      num_chunks < 1) {
    skv_set_error("%s: invalid shape rows=%d m=%d n=%d select_sets=%d num_chunks=%d idx_stride=%lld", what, rows, m, n,
                  select_sets, num_chunks, (long long)idx_stride);
    return SKV_EINVAL;
  }
  if (select_sets > kMaxS) {
    skv_set_error("%s: select_sets=%d above the supported maximum %d", what, select_sets, kMaxS);
    return SKV_EUNSUPPORTED;
  }
  int P = 64;
  while (P < select_sets) P <<= 1;
  const int words = (num_chunks + 31) / 32;
  const size_t fixed = static_cast<size_t>(words) * 8 + (out_selected ? static_cast<size_t>(P) * 8 : 0);
  if (fixed > kLdsBudget) {
    skv_set_error("%s: %d chunks need %zu bytes of bitmap, above the LDS budget", what, num_chunks, fixed);
    return SKV_EUNSUPPORTED;
  }
  const int n_lds = (fixed + static_cast<size_t>(n) * 2 <= kLdsBudget) ? n : 0;
  if (!n_lds && !out_scores) {
    skv_set_error("%s: n=%d landmarks do not fit LDS; pass out_scores as staging", what, n);
    return SKV_EINVAL;
  }
  SelectArgs a{};
  a.D = D;
  a.norm = norm;
  a.sum = sum;
  a.m = m;
  a.n = n;
  a.tiles = (n + 255) / 256;
  a.lidx = landmark_idx;
  a.lstride = idx_stride;
  a.S = select_sets;
  a.P = P;
  a.n_lds = n_lds;
  a.words = words;
  a.pos = position_ids;
  a.offsets = offsets;
  a.cnts = cnts;
  a.out_scores = out_scores;
  a.out_sel = out_selected;
  const size_t lds = fixed + static_cast<size_t>(n_lds) * 2;
  hipLaunchKernelGGL(select_kernel, dim3(rows), dim3(kThreads), (lds + 15) / 16 * 16, static_cast<hipStream_t>(stream),
                     a);
  return skv_check_launch(what);
}
