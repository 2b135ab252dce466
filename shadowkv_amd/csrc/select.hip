// a1 tail + a2 + a3 fused: chunk selection for one decode step in one launch.
//
// Replaces the sequence of models/kvcache/shadow.py:553-574 after the scoring GEMM:
// the softmax normalisation of batch_gemm_softmax (kernels/batch_gemm_softmax.h:66-242),
// torch.max over the query-head group, torch.topk, the landmark-id gather, and
// reorder_keys_and_compute_offsets (kernels/gather_copy.cu:189-235).
//
// Few rows (rows <= 32, m*n >= 2^15): step 2's probabilities come from the many-workgroup
// softmax + GQA-max kernel (score.hip) into out_scores first, and this kernel starts from them.
//
// One workgroup (16 wave64) per (batch, kv-head) row; thread t owns a contiguous block of
// landmarks (whole 8-landmark units when n % 8 == 0, so the logits of all m query rows arrive as
// 16-byte vectors requested together, and keys move as 16-byte vectors):
//   1. merge the per-256-column (max, sum exp) partials of every query row;
//   2. p_j = max_i bf16(exp(D[i,j] - max_i) / sum_i), kept as 16-bit order keys in LDS (or in
//      global scratch when n is too large), high-byte histogram with run-length-merged atomics;
//   3. radix threshold: the k-th key T and the count of keys above it (two histogram passes);
//   4. winners = keys > T plus the lowest-index keys == T (one block scan ranks the ties) are
//      listed in LDS; then every winner's chunk id is loaded at once and set in a chunk-id bitmap
//      `sel`, the previous slots' ids in `old`;
//   5. hits: a scan over the previous slots whose id is in `sel` emits them in old-slot order;
//      misses: a popcount scan over the words of `sel & ~old` emits them in ascending id order.
// With out_selected requested, the winners are additionally bitonic-sorted (value desc, index
// asc) to emit the ids in top-k order. Without previous slots (position_ids null: the selection
// of a chunk pool, which does its own hit lookup) steps 4's bitmaps and 5 are skipped and only the
// ids in top-k order are written. The arithmetic of step 2 and the selection rule are those
// of score.hip softmax_kernel and topk.hip, so the result is bit-identical to the unfused path.
#include <algorithm>
#include <cstdlib>

#include "select_core.h"
#include "softmax_keys.h"

namespace {

using skv::u32x4;

constexpr int kThreads = 1024;
constexpr int kMaxM = 16;
constexpr int kMaxS = 2048;
constexpr size_t kLdsBudget = 150 * 1024;  // dynamic LDS cap (static LDS adds ~1.4 KB; 160 KB per CU)

struct SelectArgs {
  int vec;  // n % 8 == 0: 8-landmark units
  const uint16_t* D;
  const float* norm;
  const float* sum;
  int m, n, tiles;
  const int64_t* lidx;
  int64_t lstride;
  int S, P, n_lds, words;  // words = bitmap words covering chunk ids [0, 32*words)
  int keys_off;            // byte offset of the LDS key array
  int64_t* pos;  // previous slots, reordered in place; null: selection only (out_sel required)
  int32_t* offsets;
  int32_t* cnts;
  uint16_t* out_scores;  // [rows][n], required when n_lds == 0
  int pre;               // out_scores already holds the GQA-max probabilities (split path)
  int64_t* out_sel;      // [rows][S] ids in top-k order, optional
  // Hit moves folded into the selection (optional): after the reorder, row r's hit chunks of each
  // non-null buffer are compacted in place, slot i <- slot offsets[i] for i < cnt, where slot i of
  // row r is at mv_buf[k] + r * mv_stride + mv_offset + i * mv_chunk (bf16 elements).
  uint16_t* mv_buf[2];
  int64_t mv_stride, mv_offset;
  int mv_chunk;
  int hit_src_off;  // byte offset of the LDS list of the hits' old slots (S int32), when moving
  // Split path: the softmax kernel's per-workgroup histograms of the keys' high bytes
  // ([rows][h1_parts][256]), summed here instead of counting the keys again; null: count them.
  const uint32_t* h1;
  int h1_parts;
  // With h1, the keys whose high byte is at least the threshold bin's are first compacted (index
  // order) into an LDS candidate list of at most cand_cap entries at byte offset cand_off (keys,
  // then 16-byte aligned indices), and every later pass runs over the list; more candidates than
  // that (e.g. all keys tied) fall back to the passes over all keys. cand_cap 0: no list.
  int cand_off, cand_cap;
};

__device__ __forceinline__ int scan_excl(int v, int* scratch, int* total) {
  return skv::block_exclusive_scan(v, scratch, total);
}

// Largest of the 8 raw 16-bit halves of v (written on 32-bit operations: this compiler reduced a
// max over ext_vector_type(2) unsigned shorts of the four words to one word's halves).
__device__ __forceinline__ uint32_t unit_max_raw(const u32x4& v) {
  const uint32_t a = max(v.x & 0xffffu, v.x >> 16), b = max(v.y & 0xffffu, v.y >> 16);
  const uint32_t c = max(v.z & 0xffffu, v.z >> 16), d = max(v.w & 0xffffu, v.w >> 16);
  return max(max(a, b), max(c, d));
}

__device__ __forceinline__ uint16_t half_of(const u32x4& v, int e) {
  const uint32_t w = v[e >> 1];
  return static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
}

// Hits in previous-slot order, then misses in ascending id order, from the selection bitmap
// `selmap` (every winner's chunk id) and `oldmap` (the previous slots' ids), both in LDS:
// prow[0, S) and offs[0, S) rewritten in place, *cnt = number of hits, also returned (the reorder of
// kernels/map.cuh:475-516); hit_src, when given, receives the hits' old slots. Called by every
// thread of a kThreads workgroup.
__device__ __forceinline__ int reorder_from_bitmaps(const uint32_t* selmap, const uint32_t* oldmap, int words,
                                                    int64_t* prow, int32_t* offs, int32_t* cnt, int S, int* scan,
                                                    int32_t* hit_src = nullptr) {
  const int tid = threadIdx.x;
  const int Es = (S + kThreads - 1) / kThreads;
  const int slo = min(tid * Es, S), shi = min(slo + Es, S);
  int my_hits = 0;
  for (int j = slo; j < shi; ++j) {
    const int64_t id = prow[j];
    my_hits += id >= 0 && id < 32ll * words && ((selmap[id >> 5] >> (id & 31)) & 1u);
  }
  const int Ew = (words + kThreads - 1) / kThreads;
  const int wlo = min(tid * Ew, words), whi = min(wlo + Ew, words);
  int my_miss = 0;
  for (int w = wlo; w < whi; ++w) my_miss += __popc(selmap[w] & ~oldmap[w]);
  int total_hits = 0, total_miss = 0;
  int hrank = scan_excl(my_hits, scan, &total_hits);
  int mrank = scan_excl(my_miss, scan, &total_miss);
  // All previous-slot ids were read above (scan barriers separate reads from these writes).
  int64_t hit_ids[kMaxS / kThreads + 1];
  int nh = 0;
  for (int j = slo; j < shi; ++j) {
    const int64_t id = prow[j];
    if (id >= 0 && id < 32ll * words && ((selmap[id >> 5] >> (id & 31)) & 1u)) hit_ids[nh++] = id | (static_cast<int64_t>(j) << 40);
  }
  __syncthreads();
  for (int h = 0; h < nh; ++h) {
    const int64_t id = hit_ids[h] & ((1ll << 40) - 1);
    const int j = static_cast<int>(hit_ids[h] >> 40);
    prow[hrank] = id;
    offs[hrank] = j;
    if (hit_src) hit_src[hrank] = j;
    ++hrank;
  }
  for (int w = wlo; w < whi; ++w) {
    uint32_t bits = selmap[w] & ~oldmap[w];
    while (bits) {
      const int b = __ffs(bits) - 1;
      bits &= bits - 1;
      const int id = w * 32 + b;
      prow[total_hits + mrank] = id;
      offs[total_hits + mrank] = id;
      ++mrank;
    }
  }
  if (tid == 0) *cnt = total_hits;
  return total_hits;  // the same value in every thread
}

// The folded hit moves of one row: in each buffer the call names, in-place forward compaction
// of the row's hit chunks, slot i <- slot src[i] for i < hits (src = the reorder's hit offsets, in
// LDS, strictly ascending with src[i] >= i). src[i] - i never decreases, so the moves with
// src[i] == i form a prefix [0, p), found by a binary search every thread makes alike, and are
// skipped; every later move has src[i] > i. The rest go in ascending batches of kPer 16-byte
// vectors per thread and buffer, every load of a batch completing (barrier) before any of its
// stores. A batch never reads what an earlier batch wrote (it reads slots src[i] > i >= every
// slot written before), and a slot a batch writes was read, if at all, by an earlier move: in an
// earlier batch, whose loads every thread consumed (stored) before reaching this batch's barrier,
// or in this batch, before the barrier. Called by every thread of the workgroup.
__device__ __forceinline__ void move_row_hits(const SelectArgs& a, int row, const int32_t* src, int hits) {
  constexpr int kPer = 4;
  __syncthreads();  // src complete
  int lo = 0, hi = hits;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (src[mid] == mid) lo = mid + 1;
    else hi = mid;
  }
  const int p = lo;
  if (p == hits) return;  // nothing to move (uniform)
  const int tid = threadIdx.x;
  const int vecs = a.mv_chunk / 8;
  const int64_t total = static_cast<int64_t>(hits - p) * vecs;
  const int64_t roff = static_cast<int64_t>(row) * a.mv_stride + a.mv_offset;
  uint16_t* const bv = a.mv_buf[0] ? a.mv_buf[0] + roff : nullptr;
  uint16_t* const bk = a.mv_buf[1] ? a.mv_buf[1] + roff : nullptr;
  for (int64_t v0 = 0; v0 < total; v0 += static_cast<int64_t>(kThreads) * kPer) {
    u32x4 dv[kPer], dk[kPer];
    int64_t from[kPer], to[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int64_t v = v0 + static_cast<int64_t>(k) * kThreads + tid;
      to[k] = -1;
      from[k] = 0;
      if (v < total) {
        const int i = p + static_cast<int>(v / vecs);
        const int e = static_cast<int>(v - static_cast<int64_t>(i - p) * vecs) * 8;
        from[k] = static_cast<int64_t>(src[i]) * a.mv_chunk + e;
        to[k] = static_cast<int64_t>(i) * a.mv_chunk + e;
      }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      if (to[k] < 0) continue;
      if (bv) dv[k] = *reinterpret_cast<const u32x4*>(bv + from[k]);
      if (bk) dk[k] = *reinterpret_cast<const u32x4*>(bk + from[k]);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      if (to[k] < 0) continue;
      if (bv) *reinterpret_cast<u32x4*>(bv + to[k]) = dv[k];
      if (bk) *reinterpret_cast<u32x4*>(bk + to[k]) = dk[k];
    }
  }
}

template <int MP>
__global__ void __launch_bounds__(kThreads) select_kernel(SelectArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint32_t* selmap = reinterpret_cast<uint32_t*>(smem);   // words
  uint32_t* oldmap = selmap + a.words;                     // words
  uint64_t* sorted = reinterpret_cast<uint64_t*>(oldmap + a.words);  // P winners (8-byte aligned)
  uint16_t* keys = reinterpret_cast<uint16_t*>(smem + a.keys_off);                   // n_lds, 16-byte aligned
  __shared__ skv::TopkShared sh;
  __shared__ float gmax[kMaxM], ginv[kMaxM];
  __shared__ int sel_count;

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int m = a.m, n = a.n, S = a.S;
  const int64_t base = static_cast<int64_t>(row) * S;
  int64_t* prow = a.pos ? a.pos + base : nullptr;
  // Candidate-list path with at most kRegU 8-key units per thread (the MP = 4 instance, which the
  // launcher uses for every split-path call): the thread's keys are requested here, at entry, and
  // tested from registers once the threshold bin is known.
  constexpr int kRegU = MP == 4 ? 8 : 1;
  const int reg_eu = (n / 8 + kThreads - 1) / kThreads;
  const bool regs = MP == 4 && a.h1 != nullptr && a.pre && a.vec && a.cand_cap > 0 && reg_eu <= kRegU;  // uniform
  u32x4 kr[kRegU];
  if (regs) {
    const int u0 = min(tid * reg_eu, n / 8), u1 = min(u0 + reg_eu, n / 8);
    const u32x4* sv = reinterpret_cast<const u32x4*>(a.out_scores + static_cast<int64_t>(row) * n);
#pragma unroll
    for (int u = 0; u < kRegU; ++u) {
      kr[u] = u32x4{0u, 0u, 0u, 0u};
      if (u0 + u < u1) kr[u] = sv[u0 + u];
    }
  }

  if (!a.pre) skv::merge_softmax_partials<kThreads / 64>(a.norm, a.sum, row, m, a.tiles, gmax, ginv);
  for (int i = tid; i < 256; i += kThreads) sh.hist[i] = 0;
  for (int w = tid; w < 2 * a.words; w += kThreads) selmap[w] = 0;  // selmap and oldmap
  if (tid == 0) sel_count = 0;
  __syncthreads();
  // previous slots into the old-id bitmap (ids outside the bitmap can never be hits)
  for (int j = tid; j < (a.pos ? S : 0); j += kThreads) {
    const int64_t id = prow[j];
    if (id >= 0 && id < 32ll * a.words) atomicOr(&oldmap[id >> 5], 1u << (id & 31));
  }

  // Blocked ownership in units of kU landmarks; index order is unit order is thread order.
  const int kU = a.vec ? 8 : 1;
  const int nu = (n + kU - 1) / kU;
  const int Eu = (nu + kThreads - 1) / kThreads;
  const int ulo = min(tid * Eu, nu), uhi = min(ulo + Eu, nu);
  const int lo = ulo * kU, hi = min(uhi * kU, n);
  const uint16_t* Drow = a.D + static_cast<int64_t>(row) * m * n;
  uint16_t* srow = a.out_scores ? a.out_scores + static_cast<int64_t>(row) * n : nullptr;
  // candidate list (see SelectArgs::cand_cap): set once the threshold bin is known
  const bool cand_try = a.h1 != nullptr && a.pre && a.vec && a.cand_cap > 0;  // uniform
  uint16_t* ck = reinterpret_cast<uint16_t*>(smem + a.cand_off);
  int32_t* ci = reinterpret_cast<int32_t*>(smem + a.cand_off + (static_cast<size_t>(a.cand_cap) * 2 + 15) / 16 * 16);
  bool cand = false;
  int nc = 0, clo = 0, chi = 0;
  auto prob_max = [&](float (&dv)[MP]) -> uint16_t {  // bf16 of max_i bf16(softmax_i)
    float best = -INFINITY;
#pragma unroll
    for (int i = 0; i < MP; ++i) {
      if (i < m) {
        const uint16_t p = skv::f2bf(expf(dv[i] - gmax[i]) * ginv[i]);
        best = fmaxf(best, skv::bf2f(p));
      }
    }
    return skv::f2bf(best);
  };
  // The keys of this thread's block, 8 at a time where the unit allows: f(j, key) for j in [lo, hi).
  auto for_keys = [&](auto&& f) {
    if (cand) {  // this thread's block of the candidate list (index order)
      for (int c = clo; c < chi; ++c) f(ci[c], static_cast<uint32_t>(ck[c]));
      return;
    }
    if (a.vec) {
      for (int u = ulo; u < uhi; ++u) {
        uint32_t k8[8];
        if (a.n_lds) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(&keys[8 * u]);
#pragma unroll
          for (int e = 0; e < 8; ++e) k8[e] = half_of(v, e);
        } else {
          const u32x4 v = *reinterpret_cast<const u32x4*>(&srow[8 * u]);
#pragma unroll
          for (int e = 0; e < 8; ++e) k8[e] = skv::bf16_order_key(half_of(v, e));
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) f(8 * u + e, k8[e]);
      }
    } else {
      for (int j = lo; j < hi; ++j) f(j, a.n_lds ? static_cast<uint32_t>(keys[j]) : skv::bf16_order_key(srow[j]));
    }
  };
  // The same keys in any order, for the histogram passes: with the keys in global memory the
  // workgroup reads the row interleaved (each wave load is 1 KB contiguous) with kB loads per lane
  // requested before the first is used, so a pass costs a few memory latencies, not one per unit.
  auto for_keys_global_any = [&](auto&& f) {
    constexpr int kB = 4;
    const u32x4* sv = reinterpret_cast<const u32x4*>(srow);
    for (int u0 = tid; u0 < nu; u0 += kThreads * kB) {
      u32x4 v[kB];
#pragma unroll
      for (int b = 0; b < kB; ++b) v[b] = sv[min(u0 + b * kThreads, nu - 1)];
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        if (u0 + b * kThreads < nu) {
#pragma unroll
          for (int e = 0; e < 8; ++e) f(8 * (u0 + b * kThreads) + e, skv::bf16_order_key(half_of(v[b], e)));
        }
      }
    }
  };
  auto for_keys_any = [&](auto&& f) {
    if (cand || a.n_lds || !a.vec) {
      for_keys(f);
      return;
    }
    for_keys_global_any(f);
  };
  {
    // Fused path: run-length-merged LDS atomics (a thread's consecutive keys often share a bin).
    // Split path: the keys are read in any order, so counts go to 8 per-thread registers for the
    // bins [wbase, wbase + 8) around the thread's first key, LDS atomics only outside that window
    // (softmax outputs crowd into a few adjacent high-byte (exponent) bins).
    uint32_t run_bin = 0xffffffffu, run = 0;
    auto count = [&](uint32_t bin) {
      if (bin != run_bin) {
        if (run) atomicAdd(&sh.hist[run_bin], run);
        run_bin = bin;
        run = 0;
      }
      ++run;
    };
    uint32_t wc[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    int wbase = -1;
    auto count_win = [&](uint32_t bin) {
      if (wbase < 0) wbase = max(0, static_cast<int>(bin) - 3);
      const uint32_t d = bin - static_cast<uint32_t>(wbase);
      if (d < 8u) {
#pragma unroll
        for (int k = 0; k < 8; ++k) wc[k] += d == static_cast<uint32_t>(k);
      } else {
        atomicAdd(&sh.hist[bin], 1u);
      }
    };
    const bool counted = a.h1 != nullptr;  // the softmax kernel counted the keys (uniform)
    if (a.pre && a.n_lds && !cand_try) {  // the keys staged in LDS on the way, for the later passes
      if (a.vec) {
        for_keys_global_any([&](int j, uint32_t kj) {
          keys[j] = static_cast<uint16_t>(kj);
          if (!counted) count_win(kj >> 8);
        });
      } else {
        for (int j = lo; j < hi; ++j) {
          const uint32_t kj = skv::bf16_order_key(srow[j]);
          keys[j] = static_cast<uint16_t>(kj);
          if (!counted) count_win(kj >> 8);
        }
      }
    } else if (a.pre) {
      if (!counted) for_keys_any([&](int, uint32_t kj) { count_win(kj >> 8); });
    } else if (a.vec) {
      for (int u = ulo; u < uhi; ++u) {
        u32x4 dv[MP];
#pragma unroll
        for (int i = 0; i < MP; ++i) {  // every query row's 8 logits requested before any math
          dv[i] = u32x4{0u, 0u, 0u, 0u};
          if (i < m) dv[i] = *reinterpret_cast<const u32x4*>(Drow + static_cast<int64_t>(i) * n + 8 * u);
        }
        uint32_t kw[4], bw[4];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float x[MP];
#pragma unroll
          for (int i = 0; i < MP; ++i) x[i] = skv::bf2f(half_of(dv[i], e));
          const uint16_t b = prob_max(x);
          const uint32_t key = skv::bf16_order_key(b);
          if (e & 1) {
            kw[e >> 1] |= key << 16;
            bw[e >> 1] |= static_cast<uint32_t>(b) << 16;
          } else {
            kw[e >> 1] = key;
            bw[e >> 1] = b;
          }
          count(key >> 8);
        }
        if (a.n_lds) *reinterpret_cast<u32x4*>(&keys[8 * u]) = u32x4{kw[0], kw[1], kw[2], kw[3]};
        if (srow) *reinterpret_cast<u32x4*>(&srow[8 * u]) = u32x4{bw[0], bw[1], bw[2], bw[3]};
      }
    } else {
      for (int j = lo; j < hi; ++j) {
        float x[MP];
#pragma unroll
        for (int i = 0; i < MP; ++i) x[i] = i < m ? skv::bf2f(Drow[static_cast<int64_t>(i) * n + j]) : 0.f;
        const uint16_t b = prob_max(x);
        const uint32_t key = skv::bf16_order_key(b);
        if (a.n_lds) keys[j] = static_cast<uint16_t>(key);
        if (srow) srow[j] = b;
        count(key >> 8);
      }
    }
    if (run) atomicAdd(&sh.hist[run_bin], run);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (wc[k]) atomicAdd(&sh.hist[wbase + k], wc[k]);
    if (counted) {
      // the row's partial histograms: thread t adds bin t % 256 of parts t / 256, t / 256 + 4, ...
      // (16 loads requested before the first is used), the 4 part groups meeting in sh.hist
      static_assert(kThreads % 256 == 0, "whole bins per thread group");
      constexpr int kG = kThreads / 256;
      const uint32_t* hr = a.h1 + static_cast<int64_t>(row) * a.h1_parts * 256;
      const int b = tid & 255;
      uint32_t acc = 0;
      for (int q0 = tid >> 8; q0 < a.h1_parts; q0 += kG * 16) {
        uint32_t v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int q = q0 + kG * u;
          v[u] = q < a.h1_parts ? hr[static_cast<int64_t>(q) * 256 + b] : 0u;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) acc += v[u];
      }
      if (acc) atomicAdd(&sh.hist[b], acc);
    }
  }
  __syncthreads();
  skv::select_bin(sh.hist, S, sh.found);
  const uint32_t b1 = static_cast<uint32_t>(sh.found[0]);
  const int above1 = sh.found[1];
  __syncthreads();
  for (int i = tid; i < 256; i += kThreads) sh.hist[i] = 0;
  if (cand_try) {
    // Keys with high byte >= b1 (every winner among them): count this thread's, scan, and, if
    // they fit, write them in index order to the candidate list (the row is read twice from
    // global memory, the second time from the L2); else stage all keys as the passes expect.
    const u32x4* sv = reinterpret_cast<const u32x4*>(srow);
    int my_c = 0;
    uint64_t hitmask = 0;  // regs: bit 8u + e marks key e of unit u as a candidate
    if (regs) {  // (ulo, uhi) are the units loaded into kr at entry
      // A unit whose 8 raw bf16 values are all below kraw (with the threshold bin non-negative,
      // raw order is value order for non-negative values) holds no candidate: one packed maximum
      // over the unit instead of 8 key tests (about 1 unit in 10 holds a candidate). A negative
      // value (sign bit set) fails the test and takes the per-key path.
      const uint32_t kraw = b1 >= 0x80u ? (b1 << 8) - 0x8000u : 0u;
#pragma unroll
      for (int u = 0; u < kRegU; ++u) {
        if (ulo + u < uhi) {
          if (b1 >= 0x80u && unit_max_raw(kr[u]) < kraw) continue;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            hitmask |= static_cast<uint64_t>((skv::bf16_order_key(half_of(kr[u], e)) >> 8) >= b1) << (8 * u + e);
        }
      }
      my_c = __popcll(hitmask);
    } else {
      for (int u = ulo; u < uhi; ++u) {
        const u32x4 v = sv[u];
#pragma unroll
        for (int e = 0; e < 8; ++e) my_c += (skv::bf16_order_key(half_of(v, e)) >> 8) >= b1;
      }
    }
    int pos = scan_excl(my_c, sh.scan, &nc);
    if (nc <= a.cand_cap) {
      if (regs) {
#pragma unroll
        for (int u = 0; u < kRegU; ++u) {
          uint32_t bits = static_cast<uint32_t>(hitmask >> (8 * u)) & 0xffu;
          while (bits) {
            const int e = __ffs(bits) - 1;
            bits &= bits - 1;
            ck[pos] = static_cast<uint16_t>(skv::bf16_order_key(half_of(kr[u], e)));
            ci[pos] = 8 * (ulo + u) + e;
            ++pos;
          }
        }
      } else {
        for (int u = ulo; u < uhi; ++u) {
          const u32x4 v = sv[u];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t kj = skv::bf16_order_key(half_of(v, e));
            if ((kj >> 8) >= b1) {
              ck[pos] = static_cast<uint16_t>(kj);
              ci[pos] = 8 * u + e;
              ++pos;
            }
          }
        }
      }
      cand = true;
      const int Ec = (nc + kThreads - 1) / kThreads;
      clo = min(tid * Ec, nc);
      chi = min(clo + Ec, nc);
    } else if (a.n_lds) {
      for_keys_global_any([&](int j, uint32_t kj) { keys[j] = static_cast<uint16_t>(kj); });
    }
  }
  __syncthreads();
  {
    uint32_t run_bin = 0xffffffffu, run = 0;
    for_keys_any([&](int, uint32_t kj) {
      if ((kj >> 8) != b1) return;
      if ((kj & 255u) != run_bin) {
        if (run) atomicAdd(&sh.hist[run_bin], run);
        run_bin = kj & 255u;
        run = 0;
      }
      ++run;
    });
    if (run) atomicAdd(&sh.hist[run_bin], run);
  }
  __syncthreads();
  skv::select_bin(sh.hist, S - above1, sh.found);
  const uint32_t T = (b1 << 8) | static_cast<uint32_t>(sh.found[0]);
  const int need_eq = S - above1 - sh.found[1];

  // Winners at their positions without atomics: one pass counts each thread's keys above T and
  // equal to T, one scan gives every thread its first slot for each (blocked ownership makes the
  // scan order the index order, so ties are ranked by index), a second pass writes them:
  // keys > T at [0, c_gt), the first need_eq ties at [c_gt, S). The keys > T number fewer than S
  // (T is the S-th largest), so their prefix fits 12 bits; ties take the upper 20 bits when n
  // allows, else a scan of their own.
  int my_gt = 0, my_eq = 0;
  for_keys([&](int, uint32_t kj) {
    my_gt += kj > T;
    my_eq += kj == T;
  });
  int gt_pos, eq_rank, c_gt;
  if (n < (1 << 19)) {
    int total = 0;
    const int excl = scan_excl(my_gt | (my_eq << 12), sh.scan, &total);
    gt_pos = excl & 0xfff;
    eq_rank = excl >> 12;
    c_gt = total & 0xfff;
  } else {
    gt_pos = scan_excl(my_gt, sh.scan, &c_gt);
    int total_eq = 0;
    eq_rank = scan_excl(my_eq, sh.scan, &total_eq);
  }
  const int64_t* lrow = a.lidx + static_cast<int64_t>(row) * a.lstride;
  for_keys([&](int j, uint32_t kj) {
    const uint64_t comp = (static_cast<uint64_t>(0xffffu - kj) << 32) | static_cast<uint32_t>(j);
    if (kj > T) {
      sorted[gt_pos++] = comp;
    } else if (kj == T) {
      if (eq_rank < need_eq) sorted[c_gt + eq_rank] = comp;
      ++eq_rank;
    }
  });
  if (tid == 0) sel_count = S;
  __syncthreads();
  if (a.pos) {
    // The winners' chunk ids into the selection bitmap: every id load of the workgroup in flight
    // together (exactly S winners).
    for (int i = tid; i < sel_count; i += kThreads) {
      const int64_t id = lrow[static_cast<uint32_t>(sorted[i])];
      if (id >= 0 && id < 32ll * a.words) atomicOr(&selmap[id >> 5], 1u << (id & 31));
    }
    __syncthreads();
    int32_t* hit_src = a.hit_src_off ? reinterpret_cast<int32_t*>(smem + a.hit_src_off) : nullptr;
    const int hits = reorder_from_bitmaps(selmap, oldmap, a.words, prow, a.offsets + base, a.cnts + row, S, sh.scan, hit_src);
    if (hit_src) move_row_hits(a, row, hit_src, hits);
  }

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

// ---------------------------------------------------------------------------------------------
// Few rows over many workgroups (skv_select_chunks_ws): after the softmax kernel has written the
// GQA-max probabilities (keys) of every row, each row is cut into `parts` slices of part_len keys,
// one workgroup per (slice, row):
//   part_hist_kernel<1>: high-byte histogram of the slice            -> h1[row][part][256]
//   part_hist_kernel<2>: bin b1 of the S-th largest key from sum(h1); low-byte histogram of the
//                        slice's keys in bin b1, and its count of keys above bin b1
//                                                                    -> h2[row][part][256], cnt[row][part][0]
//   part_emit_kernel:    threshold T (S-th largest key) from sum(h1), sum(h2); the slice's first
//                        ranks from the earlier slices' counts above b1 and low-byte histograms
//                        (so no launch counts the slices' keys > T and == T first); the slice's
//                        winners (keys > T, and keys == T ranked by index among all ties, the
//                        lowest need_eq indices winning) at their rank positions
//                                                                    -> win[row][0, S)
//   select_finish_kernel (one workgroup per row): winners' chunk ids into the selection bitmap,
//                        the reorder, and the top-k order when requested.
// The selection rule, key order and outputs are those of select_kernel (bit-identical).
constexpr int kPartThreads = 256;
constexpr int kMaxPartLen = 4096;  // 16 keys per thread in part_emit_kernel

struct PartArgs {
  const uint16_t* scores;  // [rows][n] bf16 GQA-max probabilities
  int n, S, parts, part_len;
  uint32_t* h1;   // [rows][parts][256]
  uint32_t* h2;   // [rows][parts][256]
  int32_t* cnt;   // [rows][parts][2]: [0] the slice's keys above the threshold's high-byte bin
  int32_t* hb;    // [rows][4]: [0] the threshold's high-byte bin b1, [1] the row's keys above it
  uint64_t* win;  // [rows][S]: (0xffff - key) << 32 | landmark index
  int h1_parts;   // partial histograms per row in h1 (parts, or the softmax kernel's workgroups)
  int vec;        // rows of 16-byte aligned, multiple-of-8 length: keys loaded as 16-byte vectors
};

// Sums the rows' partial histograms h[parts][256] into tot and finds the bin of the want-th
// largest key: out[0] = bin, out[1] = keys in higher bins. Thread t adds bins [4(t%64), +4) of
// parts t/64, t/64 + 4, ... with 16-byte loads, 16 requested before the first is used; the four
// part groups meet in LDS (part_tot). Every thread of the kPartThreads workgroup calls it.
__device__ void sum_select(const uint32_t* h, int parts, int want, uint32_t* tot, uint32_t (*part_tot)[256],
                           int* out) {
  const int quad = threadIdx.x & 63, grp = threadIdx.x >> 6;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int q0 = grp; q0 < parts; q0 += 64) {
    u32x4 v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int q = min(q0 + 4 * u, parts - 1);
      v[u] = *reinterpret_cast<const u32x4*>(&h[q * 256 + 4 * quad]);
    }
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (q0 + 4 * u < parts) acc += v[u];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) part_tot[grp][4 * quad + e] = acc[e];
  __syncthreads();
  for (int b = threadIdx.x; b < 256; b += blockDim.x)
    tot[b] = (part_tot[0][b] + part_tot[1][b]) + (part_tot[2][b] + part_tot[3][b]);
  __syncthreads();
  skv::select_bin(tot, want, out);
}

constexpr int kPartE = kMaxPartLen / kPartThreads;  // keys per thread, at most

// This thread's block of the slice: keys [lo, lo + E) of the row (blocked ownership, index order),
// all requested before the first is used; entries past the slice are marked invalid (valid bit).
__device__ __forceinline__ void load_part_keys(const PartArgs& a, int row, int part, uint32_t (&kv)[kPartE],
                                               uint32_t* valid, int* lo_out) {
  const int j0 = part * a.part_len, j1 = min(a.n, j0 + a.part_len);
  const int E = (a.part_len + kPartThreads - 1) / kPartThreads;
  const int lo = min(j1, j0 + static_cast<int>(threadIdx.x) * E), hi = min(j1, lo + E);
  const uint16_t* sr = a.scores + static_cast<int64_t>(row) * a.n;
  uint32_t v = 0;
  if (a.vec && (E & 7) == 0) {
    // 16-byte vectors: j0, E and n are multiples of 8 here, so a vector is either wholly inside
    // [lo, hi) or wholly past it.
#pragma unroll
    for (int w = 0; w < kPartE / 8; ++w) {
      const int j = lo + 8 * w;
      const bool ok = 8 * w < E && j < hi;
      const u32x4 x = *reinterpret_cast<const u32x4*>(sr + (ok ? j : 0));
      const uint32_t words[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kv[8 * w + 2 * e] = skv::bf16_order_key(static_cast<uint16_t>(words[e] & 0xffffu));
        kv[8 * w + 2 * e + 1] = skv::bf16_order_key(static_cast<uint16_t>(words[e] >> 16));
      }
      v |= (ok ? 0xffu : 0u) << (8 * w);
    }
  } else {
#pragma unroll
    for (int u = 0; u < kPartE; ++u) {
      const bool ok = u < E && lo + u < hi;
      kv[u] = skv::bf16_order_key(sr[ok ? lo + u : 0]);
      v |= static_cast<uint32_t>(ok) << u;
    }
  }
  *valid = v;
  *lo_out = lo;
}

template <int kPass>
__global__ void __launch_bounds__(kPartThreads) part_hist_kernel(PartArgs a) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t tot[256];
  __shared__ uint32_t part_tot[kPartThreads / 64][256];
  __shared__ int found[2];
  __shared__ int scan[kPartThreads / 64 + 1];
  const int part = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  for (int b = tid; b < 256; b += kPartThreads) hist[b] = 0;
  uint32_t b1 = 0;
  if (kPass == 2) {
    sum_select(a.h1 + static_cast<int64_t>(row) * a.h1_parts * 256, a.h1_parts, a.S, tot, part_tot, found);
    b1 = static_cast<uint32_t>(found[0]);
    if (part == 0 && tid == 0) {  // for the emit pass, which then sums only the low-byte histograms
      a.hb[row * 4] = found[0];
      a.hb[row * 4 + 1] = found[1];
    }
  } else {
    __syncthreads();
  }
  uint32_t kv[kPartE], valid;
  int lo;
  load_part_keys(a, row, part, kv, &valid, &lo);
  // Pass 1 counts in 8 per-thread registers around the thread's first bin (keys crowd into a few
  // adjacent high-byte bins), LDS atomics outside that window; pass 2 spreads over 256 bins.
  uint32_t wc[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  int wbase = -1;
  int above = 0;  // pass 2: keys above bin b1
#pragma unroll
  for (int u = 0; u < kPartE; ++u) {
    if (!((valid >> u) & 1u)) continue;
    const uint32_t k = kv[u];
    if (kPass == 1) {
      const uint32_t bin = k >> 8;
      if (wbase < 0) wbase = max(0, static_cast<int>(bin) - 3);
      const uint32_t d = bin - static_cast<uint32_t>(wbase);
      if (d < 8u) {
#pragma unroll
        for (int q = 0; q < 8; ++q) wc[q] += d == static_cast<uint32_t>(q);
      } else {
        atomicAdd(&hist[bin], 1u);
      }
    } else if ((k >> 8) == b1) {
      atomicAdd(&hist[k & 255u], 1u);
    } else {
      above += (k >> 8) > b1;
    }
  }
  if (kPass == 1) {
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (wc[q]) atomicAdd(&hist[wbase + q], wc[q]);
  }
  __syncthreads();
  uint32_t* out = (kPass == 1 ? a.h1 : a.h2) + (static_cast<int64_t>(row) * a.parts + part) * 256;
  for (int b = tid; b < 256; b += kPartThreads) out[b] = hist[b];
  if (kPass == 2) {
    int total;
    skv::block_exclusive_scan(above, scan, &total);
    if (tid == 0) a.cnt[(static_cast<int64_t>(row) * a.parts + part) * 2] = total;
  }
}

// T, keys > T over the row (c_gt) and the ties that win (need_eq): the high-byte bin b1 as the
// histogram pass found it, the low byte from the summed low-byte histograms.
__device__ void row_threshold(const PartArgs& a, int row, uint32_t* tot, uint32_t (*part_tot)[256], int* found,
                              uint32_t* T, int* c_gt, int* need_eq) {
  const uint32_t b1 = static_cast<uint32_t>(a.hb[row * 4]);
  const int above1 = a.hb[row * 4 + 1];
  sum_select(a.h2 + static_cast<int64_t>(row) * a.parts * 256, a.parts, a.S - above1, tot, part_tot, found);
  *T = (b1 << 8) | static_cast<uint32_t>(found[0]);
  *c_gt = above1 + found[1];
  *need_eq = a.S - *c_gt;
}

__global__ void __launch_bounds__(kPartThreads) part_emit_kernel(PartArgs a) {
  __shared__ uint32_t tot[256];
  __shared__ uint32_t part_tot[kPartThreads / 64][256];
  __shared__ int found[2];
  __shared__ int scan[kPartThreads / 64 + 1];
  const int part = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  // Blocked ownership: thread t holds keys [lo, lo + E) of the slice in index order (requested
  // first, so their latency overlaps the threshold's histogram sums).
  uint32_t kv[kPartE], valid;
  int lo;
  load_part_keys(a, row, part, kv, &valid, &lo);
  uint32_t T;
  int c_gt, need_eq;
  row_threshold(a, row, tot, part_tot, found, &T, &c_gt, &need_eq);
  // This slice's first ranks: over the slices before it, the keys above bin b1 (counted by pass
  // 2) plus those of bin b1 above T's low byte, and the ties (low byte == T's), from their
  // low-byte histograms (thread t sums bin t).
  const uint32_t tl = T & 255u;
  int bin_sum = 0, hi_sum = 0;
  {
    const uint32_t* h2 = a.h2 + static_cast<int64_t>(row) * a.parts * 256 + tid;
    for (int q = 0; q < part; ++q) bin_sum += static_cast<int>(h2[q * 256]);
    const int32_t* c = a.cnt + static_cast<int64_t>(row) * a.parts * 2;
    for (int q = tid; q < part; q += kPartThreads) hi_sum += c[2 * q];
  }
  int base_gt, base_eq, hi_total;
  skv::block_exclusive_scan(static_cast<uint32_t>(tid) > tl ? bin_sum : 0, scan, &base_gt);
  skv::block_exclusive_scan(static_cast<uint32_t>(tid) == tl ? bin_sum : 0, scan, &base_eq);
  skv::block_exclusive_scan(hi_sum, scan, &hi_total);
  base_gt += hi_total;
  int gt = 0, eq = 0;
#pragma unroll
  for (int u = 0; u < kPartE; ++u) {
    const bool ok = (valid >> u) & 1u;
    gt += ok && kv[u] > T;
    eq += ok && kv[u] == T;
  }
  int gt_total, eq_total;
  int gr = skv::block_exclusive_scan(gt, scan, &gt_total);
  int er = skv::block_exclusive_scan(eq, scan, &eq_total);
  gr += base_gt;
  er += base_eq;
  uint64_t* w = a.win + static_cast<int64_t>(row) * a.S;
#pragma unroll
  for (int u = 0; u < kPartE; ++u) {
    const int j = lo + u;
    if (!((valid >> u) & 1u)) continue;
    const uint64_t comp = (static_cast<uint64_t>(0xffffu - kv[u]) << 32) | static_cast<uint32_t>(j);
    if (kv[u] > T) {
      if (gr < a.S) w[gr] = comp;  // gr < c_gt <= S by construction; the guard keeps a bad count in bounds
      ++gr;
    } else if (kv[u] == T) {
      if (er < need_eq && c_gt + er < a.S) w[c_gt + er] = comp;
      ++er;
    }
  }
}

__global__ void __launch_bounds__(kThreads) select_finish_kernel(SelectArgs a, PartArgs pa) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint32_t* selmap = reinterpret_cast<uint32_t*>(smem);
  uint32_t* oldmap = selmap + a.words;
  uint64_t* sorted = reinterpret_cast<uint64_t*>(oldmap + a.words);  // P
  __shared__ int scan[kThreads / 64 + 1];
  const int row = blockIdx.x, tid = threadIdx.x, S = a.S;
  const int64_t base = static_cast<int64_t>(row) * S;
  int64_t* prow = a.pos ? a.pos + base : nullptr;
  const int64_t* lrow = a.lidx + static_cast<int64_t>(row) * a.lstride;
  const bool reorder = a.pos != nullptr;
  for (int w = tid; w < 2 * a.words; w += kThreads) selmap[w] = 0;
  __syncthreads();
  for (int j = tid; j < (reorder ? S : 0); j += kThreads) {
    const int64_t id = prow[j];
    if (id >= 0 && id < 32ll * a.words) atomicOr(&oldmap[id >> 5], 1u << (id & 31));
  }
  const uint64_t* w = pa.win + base;
  for (int i = tid; i < S; i += kThreads) {
    const uint64_t c = w[i];
    sorted[i] = c;
    if (!reorder) continue;
    const int64_t id = lrow[min(static_cast<uint32_t>(c), static_cast<uint32_t>(a.n - 1))];
    if (id >= 0 && id < 32ll * a.words) atomicOr(&selmap[id >> 5], 1u << (id & 31));
  }
  __syncthreads();
  if (reorder) {
    int32_t* hit_src = a.hit_src_off ? reinterpret_cast<int32_t*>(smem + a.hit_src_off) : nullptr;
    const int hits = reorder_from_bitmaps(selmap, oldmap, a.words, prow, a.offsets + base, a.cnts + row, S, scan, hit_src);
    if (hit_src) move_row_hits(a, row, hit_src, hits);
  }
  if (a.out_sel) {
    for (int i = S + tid; i < a.P; i += kThreads) sorted[i] = ~0ull;
    __syncthreads();
    skv::block_bitonic_sort(sorted, a.P);
    for (int i = tid; i < S; i += kThreads) {
      const uint32_t j = static_cast<uint32_t>(sorted[i]);
      a.out_sel[base + i] = (j < static_cast<uint32_t>(a.n)) ? lrow[j] : -1;
    }
  }
}

// Slices of part_len keys (a multiple of 256, at most kMaxPartLen), about 256 / rows per row.
void part_plan(int rows, int n, int* parts, int* part_len) {
  const int target = std::max(1, std::min(64, 256 / std::max(1, rows)));
  int len = (n + target - 1) / target;
  len = std::max(256, std::min(kMaxPartLen, (len + 255) / 256 * 256));
  *part_len = len;
  *parts = (n + len - 1) / len;
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

// Workspace layout of skv_select_chunks_ws: h1, h2, cnt, hb, win, then the softmax kernel's
// per-workgroup key histograms (hs: [rows][softmax_hist_parts][256]; *hs_out when asked).
size_t part_workspace(int rows, int n, int S, PartArgs* pa, void* ws, uint32_t** hs_out = nullptr) {
  int parts, len;
  part_plan(rows, n, &parts, &len);
  const size_t h = align256(static_cast<size_t>(rows) * parts * 256 * 4);
  const size_t c = align256(static_cast<size_t>(rows) * parts * 2 * 4);
  const size_t t = align256(static_cast<size_t>(rows) * 4 * 4);
  const size_t wn = align256(static_cast<size_t>(rows) * S * 8);
  const size_t hs = align256(static_cast<size_t>(rows) * skv::softmax_hist_parts(rows, n) * 256 * 4);
  unsigned char* p = static_cast<unsigned char*>(ws);
  if (pa) {
    pa->parts = parts;
    pa->part_len = len;
    pa->h1 = reinterpret_cast<uint32_t*>(p);
    pa->h1_parts = parts;
    pa->h2 = reinterpret_cast<uint32_t*>(p + h);
    pa->cnt = reinterpret_cast<int32_t*>(p + 2 * h);
    pa->hb = reinterpret_cast<int32_t*>(p + 2 * h + c);
    pa->win = reinterpret_cast<uint64_t*>(p + 2 * h + c + t);
  }
  if (hs_out) *hs_out = hs ? reinterpret_cast<uint32_t*>(p + 2 * h + c + t + wn) : nullptr;
  return 2 * h + c + t + wn + hs;
}

// Path of a selection call. kFused: the selection kernel computes the keys itself (one workgroup
// per row). kSplit: few rows (at most 32, or 64 with a workspace) and m*n >= 2^15, so the keys
// come from the many-workgroup softmax kernel first. kParts: as kSplit, and long rows (n >= kPartsMinKeys) with a
// workspace, so the selection passes also run over many workgroups per row. Environment
// SKV_SELECT_SPLIT=0/1/2 forces fused / split / parts (parts only with a workspace), read per call.
enum SelectPath { kFused = 0, kSplitPath = 1, kParts = 2 };
// Row length from which the few-row selection runs its radix passes over many workgroups per row.
// Measured at 8 rows, keys-first vs many workgroups: 15304 keys 17.9 vs 23.6 µs; 32712 keys 32.5
// vs 30.4 µs alone, but the GLM-4-9B decode step is slower with the six launches (387 vs 394
// tokens/s); 130680 keys 93 vs 45 µs.
constexpr int kPartsMinKeys = 65536;

SelectPath select_path(int rows, int m, int n, bool has_scores, bool has_ws) {
  if (!has_scores) return kFused;
  const char* e = getenv("SKV_SELECT_SPLIT");
  if (e && e[0] >= '0' && e[0] <= '2' && e[1] == 0) {
    const int v = e[0] - '0';
    return v == 2 ? (has_ws ? kParts : kSplitPath) : static_cast<SelectPath>(v);
  }
  // With a workspace the keys-first selection works on a candidate list and stays ahead of the
  // fused kernel up to 64 rows (measured at 64 x 4 x 15304: 16.9 vs 21.2 µs; 192 rows: 29.6 vs 23.3).
  if (rows > (has_ws ? 64 : 32) || static_cast<int64_t>(m) * n < (int64_t{1} << 15)) return kFused;
  return (has_ws && n >= kPartsMinKeys) ? kParts : kSplitPath;
}

int select_impl(const char* what, const uint16_t* D, const float* norm, const float* sum, int rows, int m, int n,
                const int64_t* landmark_idx, int64_t idx_stride, int select_sets, int num_chunks, int64_t* position_ids,
                int32_t* offsets, int32_t* cnts, uint16_t* out_scores, int64_t* out_selected, void* workspace,
                int64_t workspace_bytes, void* stream, uint16_t* mv_v = nullptr, uint16_t* mv_k = nullptr,
                int64_t mv_offset = 0, int64_t mv_stride = 0, int mv_chunk = 0) {
  // No previous slots: selection only, the ids in top-k order into out_selected.
  const bool reorder = position_ids != nullptr;
  const bool move = mv_v || mv_k;
  if (move && (!reorder || mv_chunk < 8 || mv_chunk % 8 || mv_offset < 0 || mv_offset % 8 ||
               mv_stride < mv_offset + static_cast<int64_t>(select_sets) * mv_chunk || mv_stride % 8 ||
               (reinterpret_cast<uintptr_t>(mv_v) & 15u) || (reinterpret_cast<uintptr_t>(mv_k) & 15u))) {
    skv_set_error("%s: hit moves need previous slots, a chunk of a multiple of 8 elements, 16-byte aligned "
                  "buffers and a row stride holding the selected region (chunk=%d offset=%lld stride=%lld)",
                  what, mv_chunk, (long long)mv_offset, (long long)mv_stride);
    return SKV_EINVAL;
  }
  if (!D || !norm || !sum || !landmark_idx || (reorder && (!offsets || !cnts)) || (!reorder && !out_selected)) {
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
  const int words = reorder ? (num_chunks + 31) / 32 : 0;
  const size_t base_lds = (static_cast<size_t>(words) * 8 + static_cast<size_t>(P) * 8 + 15) / 16 * 16;
  // the hits' old slots, for the folded hit moves
  const size_t fixed = base_lds + (move ? (static_cast<size_t>(select_sets) * 4 + 15) / 16 * 16 : 0);
  if (fixed > kLdsBudget) {
    skv_set_error("%s: %d chunks need %zu bytes of bitmap, above the LDS budget", what, num_chunks, fixed);
    return SKV_EUNSUPPORTED;
  }
  // Few rows: the per-row key computation (m*n exponentials) would run on as many workgroups as
  // rows, so it moves to the many-workgroup softmax + GQA-max kernel, which writes the keys
  // (bit-identical) into out_scores; the selection kernel then starts from them.
  const SelectPath path = select_path(rows, m, n, out_scores != nullptr, workspace != nullptr);
  const bool split = path != kFused;
  const bool parts = path == kParts;
  if (parts) {
    const size_t need = part_workspace(rows, n, select_sets, nullptr, nullptr);
    if (workspace_bytes < static_cast<int64_t>(need)) {
      skv_set_error("%s: workspace of %lld bytes, %zu needed", what, (long long)workspace_bytes, need);
      return SKV_EINVAL;
    }
  }
  const int n_lds = (fixed + static_cast<size_t>(n) * 2 <= kLdsBudget) ? n : 0;
  if (!n_lds && !out_scores) {
    skv_set_error("%s: n=%d landmarks do not fit LDS; pass out_scores as staging", what, n);
    return SKV_EINVAL;
  }
  SelectArgs a{};
  a.vec = (n % 8 == 0 && (reinterpret_cast<uintptr_t>(D) & 15u) == 0 &&
           (!out_scores || (reinterpret_cast<uintptr_t>(out_scores) & 15u) == 0));
  a.keys_off = static_cast<int>(fixed);
  a.hit_src_off = move ? static_cast<int>(base_lds) : 0;
  a.mv_buf[0] = mv_v;
  a.mv_buf[1] = mv_k;
  a.mv_offset = mv_offset;
  a.mv_stride = mv_stride;
  a.mv_chunk = mv_chunk;
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
  a.pre = split ? 1 : 0;
  size_t lds = fixed + static_cast<size_t>(n_lds) * 2;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  // With the full workspace the softmax kernel also counts the keys' high bytes per workgroup,
  // and the selection sums those counts instead of counting every key again.
  uint32_t* hs = nullptr;
  if (split && workspace && n % 8 == 0 && ((reinterpret_cast<uintptr_t>(D) | reinterpret_cast<uintptr_t>(out_scores)) & 15u) == 0 &&
      workspace_bytes >= static_cast<int64_t>(part_workspace(rows, n, select_sets, nullptr, nullptr)))
    part_workspace(rows, n, select_sets, nullptr, workspace, &hs);
  a.h1 = hs;
  a.h1_parts = hs ? skv::softmax_hist_parts(rows, n) : 0;
  // The candidate list: in the keys' LDS region when the row fits LDS (free until the keys would
  // be staged, which only the fallback does), else in what the budget leaves after the fixed part.
  a.cand_off = 0;
  a.cand_cap = 0;
  if (hs && !parts && a.vec) {
    const size_t room = n_lds ? static_cast<size_t>(n_lds) * 2 : std::min<size_t>(kLdsBudget - fixed, 96 * 1024);
    const size_t cap = room >= 32 ? (room - 16) / 6 : 0;
    if (cap >= static_cast<size_t>(select_sets)) {
      a.cand_off = static_cast<int>(fixed);
      a.cand_cap = static_cast<int>(cap);
      if (!n_lds) lds = fixed + room;
    }
  }
  const size_t ldsb = (lds + 15) / 16 * 16;
  if (split) {
    const int rc = hs ? skv::softmax_keys_hist(D, norm, sum, out_scores, hs, rows, m, n, st)
                      : skv_softmax_gqa_max(D, norm, sum, nullptr, out_scores, rows, m, n, stream);
    if (rc) return rc;
  }
  if (parts) {
    PartArgs pa{};
    pa.scores = out_scores;
    pa.n = n;
    pa.S = select_sets;
    pa.vec = n % 8 == 0 && (reinterpret_cast<uintptr_t>(out_scores) & 15u) == 0;
    part_workspace(rows, n, select_sets, &pa, workspace);
    const dim3 pg(pa.parts, rows);
    if (hs) {  // the high-byte histograms are the softmax kernel's
      pa.h1 = hs;
      pa.h1_parts = a.h1_parts;
    } else {
      hipLaunchKernelGGL(part_hist_kernel<1>, pg, dim3(kPartThreads), 0, st, pa);
    }
    hipLaunchKernelGGL(part_hist_kernel<2>, pg, dim3(kPartThreads), 0, st, pa);
    hipLaunchKernelGGL(part_emit_kernel, pg, dim3(kPartThreads), 0, st, pa);
    const size_t fb = (fixed + 15) / 16 * 16;
    hipLaunchKernelGGL(select_finish_kernel, dim3(rows), dim3(kThreads), fb, st, a, pa);
    return skv_check_launch(what);
  }
  // (keys precomputed: the query count plays no part, and the MP = 4 instance keeps them in registers)
  if (m <= 4 || split) hipLaunchKernelGGL(select_kernel<4>, dim3(rows), dim3(kThreads), ldsb, st, a);
  else if (m <= 8) hipLaunchKernelGGL(select_kernel<8>, dim3(rows), dim3(kThreads), ldsb, st, a);
  else hipLaunchKernelGGL(select_kernel<16>, dim3(rows), dim3(kThreads), ldsb, st, a);
  return skv_check_launch(what);
}

}  // namespace

extern "C" int skv_select_chunks(const uint16_t* D, const float* norm, const float* sum, int rows, int m, int n,
                                 const int64_t* landmark_idx, int64_t idx_stride, int select_sets, int num_chunks,
                                 int64_t* position_ids, int32_t* offsets, int32_t* cnts, uint16_t* out_scores,
                                 int64_t* out_selected, void* stream) {
  return select_impl("select_chunks", D, norm, sum, rows, m, n, landmark_idx, idx_stride, select_sets, num_chunks,
                     position_ids, offsets, cnts, out_scores, out_selected, nullptr, 0, stream);
}

extern "C" int64_t skv_select_workspace_bytes(int rows, int n, int select_sets) {
  if (rows < 1 || n < 1 || select_sets < 1) return 0;
  return static_cast<int64_t>(part_workspace(rows, n, select_sets, nullptr, nullptr));
}

extern "C" int skv_select_chunks_ws(const uint16_t* D, const float* norm, const float* sum, int rows, int m, int n,
                                    const int64_t* landmark_idx, int64_t idx_stride, int select_sets, int num_chunks,
                                    int64_t* position_ids, int32_t* offsets, int32_t* cnts, uint16_t* out_scores,
                                    int64_t* out_selected, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!workspace) {
    skv_set_error("select_chunks_ws: null workspace");
    return SKV_EINVAL;
  }
  return select_impl("select_chunks_ws", D, norm, sum, rows, m, n, landmark_idx, idx_stride, select_sets, num_chunks,
                     position_ids, offsets, cnts, out_scores, out_selected, workspace, workspace_bytes, stream);
}

extern "C" int skv_select_chunks_compact(const uint16_t* D, const float* norm, const float* sum, int rows, int m, int n,
                                         const int64_t* landmark_idx, int64_t idx_stride, int select_sets,
                                         int num_chunks, int64_t* position_ids, int32_t* offsets, int32_t* cnts,
                                         uint16_t* out_scores, int64_t* out_selected, void* workspace,
                                         int64_t workspace_bytes, void* v_buffer, void* k_buffer, int64_t buf_offset,
                                         int64_t buf_stride, int chunk_elems, void* stream) {
  if (!v_buffer && !k_buffer) {
    skv_set_error("select_chunks_compact: no buffer to compact (use skv_select_chunks_ws)");
    return SKV_EINVAL;
  }
  return select_impl("select_chunks_compact", D, norm, sum, rows, m, n, landmark_idx, idx_stride, select_sets,
                     num_chunks, position_ids, offsets, cnts, out_scores, out_selected, workspace, workspace_bytes,
                     stream, static_cast<uint16_t*>(v_buffer), static_cast<uint16_t*>(k_buffer), buf_offset,
                     buf_stride, chunk_elems);
}
