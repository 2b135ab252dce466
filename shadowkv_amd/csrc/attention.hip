// a8: sparse decode attention of one query token over the assembled K/V buffers.
//
// Replaces flash_attn_with_kvcache(q, k, v, causal=True) at models/attention/shadow.py:48
// (q_len = 1, so causality masks nothing). Split-L flash decoding for CDNA4:
//   attn_split_kernel: workgroup = (kv head, split of 64 or 128 keys); all G query heads that
//     share the kv head are served by one pass over its K and V rows, so every K/V byte is read
//     once from HBM. Scores on MFMA: v_mfma_f32_16x16x32_bf16 with the (up to 16) query heads as
//     the A rows and 16 keys as the B columns, so each lane ends up holding finished scores (no
//     cross-lane reduction); split softmax per query head with DPP/readlane wave reductions;
//     P.V on MFMA for 9..16 query heads (P in bf16 as the A operand, the V tile read transposed
//     from LDS as B, each wave owning 32 dims), in fp32 for 1..8 (16 key streams x 8 dims per
//     lane, the streams summed through LDS).
//   Merge of the splits, one of two ways:
//   - fused (on request; rows of at most 64 splits): every split of a (sequence, kv head) row runs on one XCD
//     (the grid is ordered so that they share blockIdx mod 8, and the dispatcher hands workgroup w
//     to XCD w mod 8; a probe kernel checks that mapping once per device, and every workgroup
//     checks its own XCC id against it). The split partials then meet in that XCD's L2: each
//     workgroup waits for its partial stores to reach the L2, counts itself in on the row's
//     arrival counter (a wrapping atomic increment in the L2, so the last arrival leaves it at
//     zero for the next call or graph replay), and the last one merges the row's splits, reading
//     the partials with L1-bypassing loads. One launch, and no cross-XCD write-back or
//     invalidation of the L2s (the agent-scope fence such a hand-off would otherwise need cost
//     ten times the kernel on MI355X).
//   - attn_combine_kernel (the default): a second launch,
//     a log-sum-exp merge of the splits in one pass (running maximum), every load of a 32-split
//     chunk issued before the first is used; bf16 output.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "wave_reduce.h"

namespace {

using skv::u32x4;

constexpr int kThreads = 256;
// Keys per split workgroup: 128 (rather than 256: twice the workgroups in flight at decode batch
// sizes; MI355X, cold K/V, Llama-3-8B shape batch 8: 24 vs 29 us; GLM-4-9B batch 4: 19 vs 27 us),
// or 64 for grids that would otherwise give fewer than two workgroups per CU.
constexpr int kSplitLong = 128;
constexpr int kSplitShort = 64;
constexpr int kHeadDim = 128;
constexpr int kMaxKvLen = 262144;
// Fused merge: rows of at most kMaxFusedSplits splits, at most kMaxFusedRows (sequence, kv head)
// rows per call (their arrival counters sit at the head of the workspace).
constexpr int kMaxFusedSplits = 64;
constexpr int kMaxFusedRows = 4096;
constexpr int64_t kArrivalBytes = kMaxFusedRows * sizeof(uint32_t);
constexpr int kXcds = 8;
// s_getreg_b32 hwreg(HW_REG_XCC_ID, 0, 4): the XCC (XCD) the wave runs on.
constexpr int kHwRegXccId = (3 << 11) | (0 << 6) | 20;

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(w[e] << 16);
    f[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
  }
}

struct AttnArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  int64_t kv_sb, kv_sh, kv_ss;
  int Hkv, G, L, splits;  // L: maximum length (grid sizing)
  int split_keys;         // keys per split workgroup
  const int32_t* L_dev;   // optional device-resident length, clamped to [1, L]
  float scale;
  float* ws_o;   // [B*Hq][splits][128]
  float* ws_ml;  // [B*Hq][splits][2]
  uint16_t* out;
  int64_t o_sb, o_sh;
  // Paged selected region (chunk pool): virtual keys [sp0, sp0 + sel*chunk) are chunk j of the
  // selection at physical rows sp0 + slot[(b*Hkv + h)*sel + j]*chunk + ...; virtual keys past the
  // selection sit `delta` rows further (after the pool's pool_slots chunks).
  const int32_t* slot;
  int sp0, sel, chunk, pool_slots, delta;
  // Values read in place (a value store in device memory): the selected region's value rows
  // [sp0, sp0 + sel*chunk) come from row cid*chunk + r of (b, h) in the store, cid = vids[(b*Hkv +
  // h)*sel + j] the chunk id of slot j (clamped to [0, vs_chunks)); the keys and every other value
  // row come from k / v as usual.
  const uint16_t* vs;
  int64_t vs_sb, vs_sh, vs_chunks;
  const int64_t* vids;
  // Fused merge: one arrival counter per (b, kv head) row (zero between calls), the row count,
  // the XCC id the mapping probe saw for each blockIdx class mod 8 (4 bits each), and a flag set
  // by any workgroup that finds itself elsewhere.
  uint32_t* arrivals;
  int rows;
  uint32_t xcc_map;
  uint32_t* misplaced;
};

__device__ __forceinline__ int live_length(const AttnArgs& a) {
  return a.L_dev ? min(max(*a.L_dev, 1), a.L) : a.L;
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Fused-merge thread layout: units of (query head, 4 dims), each summed over a share of the
// splits (kParts threads per unit when the units do not fill the workgroup) or, for 16 heads,
// two units per thread.
template <int GP>
struct MergeShape {
  static constexpr int kUnits = GP * 32;
  static constexpr int kParts = kUnits >= kThreads ? 1 : kThreads / kUnits;
  static constexpr int kPerThread = kUnits > kThreads ? kUnits / kThreads : 1;
  static constexpr int kBytes = (kParts - 1) * kUnits * 16;  // the parts' float4 sums
};

// The last workgroup of row bh merges its `used` splits (used <= kMaxFusedSplits): weights
// w[g][s] = exp(m[g][s] - M_g) and denominators from the (m, l) pairs, then each unit's
// sum_s w[g][s] o[g][s][4 dims], every partial read with buffer loads that bypass the L1 (sc1;
// served by the XCD's L2, where the row's other workgroups left them).
template <int GP>
__device__ __forceinline__ void fused_merge(const AttnArgs& a, int bh, int used, float (*wt)[kMaxFusedSplits],
                                            float* lsum, unsigned char* part_lds) {
  using MS = MergeShape<GP>;
  const int G = a.G;
  const int Hq = a.Hkv * G;
  const int b = bh / a.Hkv;
  const int h = bh - b * a.Hkv;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row0 = static_cast<int64_t>(b) * Hq + h * G;  // first (b, query head) row of the kv head
  constexpr uint32_t kSc1 = 16;                               // cache policy: device scope, L1 miss
  constexpr int kDw3 = 0x00020000;                            // buffer resource word 3 (gfx9)
  const __amdgpu_buffer_rsrc_t mlr = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_ml + row0 * a.splits * 2, 0, static_cast<int>(G * a.splits * 8), kDw3);
  const __amdgpu_buffer_rsrc_t orr = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_o + row0 * a.splits * kHeadDim, 0, static_cast<int>(G * a.splits * kHeadDim * 4), kDw3);
  constexpr int kHeadsPerWave = (GP + 3) / 4;
  float mv[kHeadsPerWave], lv[kHeadsPerWave];
#pragma unroll
  for (int t = 0; t < kHeadsPerWave; ++t) {
    const int g = wave + 4 * t;
    const bool ok = g < G && lane < used;
    const auto p = __builtin_amdgcn_raw_buffer_load_b64(mlr, ((min(g, G - 1) * a.splits + min(lane, used - 1)) * 8),
                                                        0, kSc1);
    mv[t] = ok ? __uint_as_float(p[0]) : -INFINITY;
    lv[t] = ok ? __uint_as_float(p[1]) : 0.f;
  }
#pragma unroll
  for (int t = 0; t < kHeadsPerWave; ++t) {
    const int g = wave + 4 * t;
    if (g < G) {  // wave-uniform
      const float M = skv::wave_max_dpp(mv[t]);  // every live split has a finite maximum
      const float w = lane < used ? expf(mv[t] - M) : 0.f;
      const float l = skv::wave_sum_dpp(w * lv[t]);
      wt[g][lane] = w;
      if (lane == 0) lsum[g] = l;
    }
  }
  __syncthreads();
  float4* parts = reinterpret_cast<float4*>(part_lds);
#pragma unroll
  for (int k = 0; k < MS::kPerThread; ++k) {
    const int u = MS::kPerThread > 1 ? threadIdx.x + k * kThreads : threadIdx.x % MS::kUnits;
    const int p = MS::kParts > 1 ? threadIdx.x / MS::kUnits : 0;
    const int g = u >> 5, d4 = u & 31;
    float4 acc = {0.f, 0.f, 0.f, 0.f};
    if (g < G) {
      constexpr int kBatch = 8;
      for (int s0 = p; s0 < used; s0 += kBatch * MS::kParts) {
        uint32_t __attribute__((ext_vector_type(4))) v[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
          const int sp = min(s0 + i * MS::kParts, used - 1);
          v[i] = __builtin_amdgcn_raw_buffer_load_b128(orr, ((g * a.splits + sp) * kHeadDim + 4 * d4) * 4, 0, kSc1);
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
          const int sp = s0 + i * MS::kParts;
          const float w = sp < used ? wt[g][sp] : 0.f;
          acc.x = fmaf(w, __uint_as_float(v[i][0]), acc.x);
          acc.y = fmaf(w, __uint_as_float(v[i][1]), acc.y);
          acc.z = fmaf(w, __uint_as_float(v[i][2]), acc.z);
          acc.w = fmaf(w, __uint_as_float(v[i][3]), acc.w);
        }
      }
    }
    if constexpr (MS::kParts > 1) {
      if (p > 0) parts[(p - 1) * MS::kUnits + u] = acc;
      __syncthreads();
      if (p > 0) continue;  // (kPerThread == 1 here)
#pragma unroll
      for (int q = 1; q < MS::kParts; ++q) {
        const float4 o = parts[(q - 1) * MS::kUnits + u];
        acc.x += o.x;
        acc.y += o.y;
        acc.z += o.z;
        acc.w += o.w;
      }
    }
    if (g < G) {
      const float inv = 1.f / lsum[g];
      uint16_t* dst = a.out + b * a.o_sb + (h * G + g) * a.o_sh + 4 * d4;
      *reinterpret_cast<uint32_t __attribute__((ext_vector_type(2)))*>(dst) = {skv::f2bf2(acc.x * inv, acc.y * inv),
                                                                              skv::f2bf2(acc.z * inv, acc.w * inv)};
    }
  }
}

// kSplit keys per workgroup; the split's V rows are requested right after the scores, so their
// latency overlaps the softmax (requesting them with K, at entry, measured no faster and holds
// more registers). kFused: blockIdx.x enumerates (row, split) so that a row's splits share
// blockIdx mod 8 (one XCD), and the last split of each row merges them (fused_merge).
// kMap: 0 keys and values at their rows; 1 the selected region through the chunk pool's slot list
// (a.slot); 2 the selected region's values in place in the value store (a.vs).
template <int GP, int kMap, int kSplit, bool kFused>
__global__ void __launch_bounds__(kThreads) attn_split_kernel(AttnArgs a) {
  constexpr int kRows = kSplit / 16;        // keys per P.V stream
  constexpr int kGroups = kSplit / 4 / 16;  // 16-key MFMA groups per wave
  constexpr int kPerLane = kSplit / 64;     // softmax entries per lane
  constexpr int kVals = GP * 8;              // P.V partial sums per lane: [head][8 dims]
  constexpr int kKept = kVals / 4;           // per lane after the in-wave stream fold
  static_assert(kSplit == 64 || kSplit == 128, "64 or 128 keys per split");
  __shared__ float p_lds[GP][kSplit];
  // [wave][lane][value] for the fp32 P.V path; the MFMA P.V path (GP == 16) stages the V tile here
  // instead ([key][kVtLd] bf16, rows padded so the 4 key groups of an operand read hit disjoint
  // banks).
  constexpr int kVtLd = kHeadDim + 4;
  constexpr int kRedBytes = 4 * 64 * kKept * 4;
  constexpr int kVtBytes = GP == 16 ? kSplit * kVtLd * 2 : 0;
  constexpr int kMergeBytes = kFused ? MergeShape<GP>::kBytes : 0;
  constexpr int kBigBytes = kRedBytes > kVtBytes ? (kRedBytes > kMergeBytes ? kRedBytes : kMergeBytes)
                                                 : (kVtBytes > kMergeBytes ? kVtBytes : kMergeBytes);
  __shared__ __align__(16) unsigned char big[kBigBytes];
  float (*red)[64][kKept] = reinterpret_cast<float (*)[64][kKept]>(big);
  __shared__ float ml[GP][2];
  __shared__ int prow[kMap == 1 ? kSplit : 1];  // physical row of each key of the split (pool)
  __shared__ const uint16_t* vrow[kMap == 2 ? kSplit : 1];  // value row of each key (values in place)

  int split, bh;
  if constexpr (kFused) {
    // w = x + 8 j: XCD x takes rows x, x + 8, ... and their splits in order.
    const int w = blockIdx.x;
    const int x = w & (kXcds - 1), j = w >> 3;
    const int i = j / a.splits;
    split = j - i * a.splits;
    bh = x + kXcds * i;
    if (bh >= a.rows) return;  // workgroup-uniform: padding of the last row group
    if (threadIdx.x == 0) {
      const uint32_t xcc = __builtin_amdgcn_s_getreg(kHwRegXccId) & 15u;
      if (xcc != ((a.xcc_map >> (4 * x)) & 15u)) *a.misplaced = 1u;  // (never seen: the probe confirmed the map)
    }
  } else {
    split = blockIdx.x;
    bh = blockIdx.y;
  }
  const int b = bh / a.Hkv;
  const int h = bh - b * a.Hkv;
  const int L = live_length(a);
  const int s0 = split * kSplit;
  if (s0 >= L) return;  // workgroup-uniform: splits past the live length do nothing (nor count)
  const int s1 = min(s0 + kSplit, L);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int grp = lane >> 4;
  const int G = a.G;
  const uint16_t* kh = a.k + b * a.kv_sb + h * a.kv_sh;
  const uint16_t* vh = a.v + b * a.kv_sb + h * a.kv_sh;

  // Q as MFMA A operand: lane (li, grp) holds query head li (zero rows past G), dims
  // [32*ks + 8*grp, +8). Loaded first; every load below is unconditional (clamped index, value
  // zeroed), so a batch of loads is issued before any is waited on.
  u32x4 qf[4];
  const uint16_t* qrow = a.q + b * a.q_sb + (h * G + min(li, G - 1)) * a.q_sh + 8 * grp;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) qf[ks] = skv::load16_or_zero(qrow + 32 * ks, li < G);
  // Key jl of the split (clamped to the live keys) lives at row key_row(jl).
  if (kMap == 1) {
    for (int jl = threadIdx.x; jl < kSplit; jl += kThreads) {
      const int sk = min(s0 + jl, s1 - 1);
      int r = sk;
      if (sk >= a.sp0) {
        const int j = sk - a.sp0;
        if (j < a.sel * a.chunk) {
          const int sl = a.slot[static_cast<int64_t>(bh) * a.sel + j / a.chunk];
          r = a.sp0 + min(max(sl, 0), a.pool_slots - 1) * a.chunk + j % a.chunk;
        } else {
          r = sk + a.delta;
        }
      }
      prow[jl] = r;
    }
    __syncthreads();
  }
  auto key_row = [&](int jl) -> int64_t { return kMap == 1 ? prow[jl] : min(s0 + jl, s1 - 1); };
  // K as MFMA B operand: lane (li, grp) holds key (wave*64 + 16*kg + li), same dims.
  u32x4 kf[kGroups][4];
#pragma unroll
  for (int kg = 0; kg < kGroups; ++kg) {
    const int s = s0 + wave * (kSplit / 4) + 16 * kg + li;
    const uint16_t* krow = kh + key_row(s - s0) * a.kv_ss + 8 * grp;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) kf[kg][ks] = skv::load16_or_zero(krow + 32 * ks, s < s1);
  }
  // Values in place: the wave's own V keys (stream 4*wave + grp of every 16, see load_v) get their
  // rows from lanes t < kRows * 4 of the wave, key (t / 4) * 16 + 4 * wave + t % 4, each lane's
  // chunk id requested here, after the K loads; the wave reads them back from LDS after its scores,
  // so no workgroup barrier is needed.
  const int vkey = ((lane >> 2) * 16 + 4 * wave + (lane & 3));  // (lanes below kRows * 4)
  const uint16_t* vself = nullptr;
  int64_t vcid = 0;
  bool vin = false;
  if (kMap == 2 && lane < kRows * 4) {
    const int sk = min(s0 + vkey, s1 - 1);
    const int j = sk - a.sp0;
    vself = vh + sk * a.kv_ss;
    vin = j >= 0 && j < a.sel * a.chunk;
    if (vin) vcid = a.vids[static_cast<int64_t>(bh) * a.sel + j / a.chunk];
  }
  // V for P.V: stream (wave, grp) takes keys s0 + 16*i + stream, lane li its dims [8*li, +8), so
  // each wave load reads 4 consecutive rows (1 KB when rows are contiguous). Non-temporal loads:
  // in this order they stream faster than plain ones (MI355X, Llama-3-8B shape batch 24: 49.6 vs
  // 52.7 us per call), while K, read in the MFMA operand order (64 bytes of 16 rows per load),
  // gains nothing from the hint.
  const int stream = wave * 4 + grp;
  u32x4 vr[kRows];
  auto load_v = [&]() {
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const int s = s0 + i * 16 + stream;
      const uint16_t* vp = kMap == 2 ? vrow[i * 16 + stream] : vh + key_row(i * 16 + stream) * a.kv_ss;
      const u32x4 x = skv::load_nt(reinterpret_cast<const u32x4*>(vp + li * 8));
      vr[i] = s < s1 ? x : u32x4{0u, 0u, 0u, 0u};
    }
  };
#pragma unroll
  for (int kg = 0; kg < kGroups; ++kg) {
    f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, qf[ks]),
                                                  __builtin_bit_cast(bf16x8_t, kf[kg][ks]), d, 0, 0, 0);
    // D[head 4*grp + v][key li]
    const int jl = wave * (kSplit / 4) + 16 * kg + li;
    const bool live = s0 + jl < s1;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int g = 4 * grp + v;
      if (g < G) p_lds[g][jl] = live ? d[v] * a.scale : -INFINITY;
    }
  }
  if (kMap == 2) {
    if (lane < kRows * 4) {
      if (vin) {
        const int j = min(s0 + vkey, s1 - 1) - a.sp0;
        const int64_t cid = min(max(vcid, int64_t{0}), a.vs_chunks - 1);
        vself = a.vs + b * a.vs_sb + h * a.vs_sh + (cid * a.chunk + j % a.chunk) * kHeadDim;
      }
      vrow[vkey] = vself;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's rows are in LDS
    __builtin_amdgcn_wave_barrier();
  }
  load_v();
  __syncthreads();

  for (int g = wave; g < G; g += 4) {
    float x[kPerLane];
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < kPerLane; ++u) {
      x[u] = p_lds[g][lane * kPerLane + u];
      mx = fmaxf(mx, x[u]);
    }
    mx = skv::wave_max_dpp(mx);
    float l = 0.f;
#pragma unroll
    for (int u = 0; u < kPerLane; ++u) {
      const float e = (x[u] == -INFINITY) ? 0.f : expf(x[u] - mx);
      p_lds[g][lane * kPerLane + u] = e;
      l += e;
    }
    l = skv::wave_sum_dpp(l);
    if (lane == 0) {
      ml[g][0] = mx;
      ml[g][1] = l;
    }
  }
  __syncthreads();

  if constexpr (GP == 16) {
    // P.V on MFMA (9..16 query heads per kv head): O[head][dim] += P[head][32 keys] . V[32 keys][dim]
    // with P as the A operand (rows past G zero; rounded to bf16, as flash attention does for its
    // second product) and V as B, read transposed from an LDS copy of the split's V tile. Wave w
    // owns dims [32w, 32w + 32) for every head, so no cross-wave sum is needed (MI355X, GLM-4-9B
    // batch 4: 10.9 vs 18.5 us with fp32 P.V). For 4 query heads the same path measured faster
    // alone (22.2 vs 23.6 us at Llama-3-8B batch 8) but slowed the pipelined decode step (373 vs
    // 382 tokens/s: the V tile's 34 KB of LDS per workgroup), so 1..8 heads keep fp32 P.V.
    uint16_t* vt = reinterpret_cast<uint16_t*>(big);
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      uint16_t* dst = vt + (i * 16 + stream) * kVtLd + li * 8;
      *reinterpret_cast<uint32_t __attribute__((ext_vector_type(2)))*>(dst) = {vr[i].x, vr[i].y};
      *reinterpret_cast<uint32_t __attribute__((ext_vector_type(2)))*>(dst + 4) = {vr[i].z, vr[i].w};
    }
    __syncthreads();
    const int qh = lane & 15;    // A row: query head of the group; B column: dim within the tile
    const int slab = lane >> 4;  // k-slab: keys [8*slab, +8) of each 32-key step
    f32x4_t o[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ks = 0; ks < kSplit / 32; ++ks) {
      const int k0 = ks * 32 + 8 * slab;
      u32x4 pa = {0u, 0u, 0u, 0u};
      if (qh < G) {
        const float* pr = &p_lds[qh][k0];
        pa = u32x4{skv::f2bf2(pr[0], pr[1]), skv::f2bf2(pr[2], pr[3]), skv::f2bf2(pr[4], pr[5]),
                   skv::f2bf2(pr[6], pr[7])};
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int dim = wave * 32 + t * 16 + qh;
        const uint16_t* vc = vt + k0 * kVtLd + dim;
        uint16_t e[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) e[u] = vc[u * kVtLd];
        const u32x4 vb = {static_cast<uint32_t>(e[0]) | (static_cast<uint32_t>(e[1]) << 16),
                          static_cast<uint32_t>(e[2]) | (static_cast<uint32_t>(e[3]) << 16),
                          static_cast<uint32_t>(e[4]) | (static_cast<uint32_t>(e[5]) << 16),
                          static_cast<uint32_t>(e[6]) | (static_cast<uint32_t>(e[7]) << 16)};
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, pa),
                                                       __builtin_bit_cast(bf16x8_t, vb), o[t], 0, 0, 0);
      }
    }
    // D[head 4*slab + v][dim]: this lane holds 4 heads of one dim per tile.
    const int Hq = a.Hkv * G;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int dim = wave * 32 + t * 16 + qh;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int g = 4 * slab + v;
        if (g < G) {
          const int64_t r = (static_cast<int64_t>(b) * Hq + h * G + g) * a.splits + split;
          a.ws_o[r * kHeadDim + dim] = o[t][v];
        }
      }
    }
    if (threadIdx.x < G) {
      const int g = threadIdx.x;
      const int64_t r = (static_cast<int64_t>(b) * Hq + h * G + g) * a.splits + split;
      a.ws_ml[r * 2] = ml[g][0];
      a.ws_ml[r * 2 + 1] = ml[g][1];
    }
  } else {
    float acc[GP][8];
#pragma unroll
    for (int g = 0; g < GP; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const int jl = i * 16 + stream;
      if (s0 + jl < s1) {
        float vf[8];
        unpack8(vr[i], vf);
#pragma unroll
        for (int g = 0; g < GP; ++g) {
          if (g < G) {
            const float p = p_lds[g][jl];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
          }
        }
      }
    }

    // Sum the 16 key streams. The 4 streams of a wave (lane bits 5 and 4) fold in registers:
    // v_permlane32_swap / v_permlane16_swap with the lower half of the values as one operand and
    // the upper half as the other hand every lane its own kept value and its partner's copy of
    // it, so each step is a swap and an add and halves the values a lane holds. Lane (grp, li)
    // then holds flattened values [grp*kKept, +kKept) of [head][8 dims] for dims li*8..+8; the 4
    // waves are summed through LDS.
    float v[kVals];
#pragma unroll
    for (int g = 0; g < GP; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) v[g * 8 + e] = acc[g][e];
#pragma unroll
    for (int j = 0; j < kVals / 2; ++j) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[j]), __float_as_uint(v[kVals / 2 + j]),
                                                      false, false);
      v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int j = 0; j < kKept; ++j) {
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[j]), __float_as_uint(v[kKept + j]), false,
                                                      false);
      v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int j = 0; j < kKept; ++j) red[wave][lane][j] = v[j];
    __syncthreads();
    const int Hq = a.Hkv * G;
    for (int idx = threadIdx.x; idx < G * kHeadDim; idx += kThreads) {
      const int g = idx / kHeadDim, d = idx - g * kHeadDim;
      const int f = g * 8 + (d & 7);                        // flattened value index
      const int src = (f / kKept) * 16 + (d >> 3);           // lane (grp, li) that holds it
      const int j = f % kKept;
      const float o = (red[0][src][j] + red[1][src][j]) + (red[2][src][j] + red[3][src][j]);
      const int64_t r = (static_cast<int64_t>(b) * Hq + h * G + g) * a.splits + split;
      a.ws_o[r * kHeadDim + d] = o;
      if (d == 0) {
        a.ws_ml[r * 2] = ml[g][0];
        a.ws_ml[r * 2 + 1] = ml[g][1];
      }
    }
  }
  if constexpr (kFused) {
    // This workgroup's partials must be in the L2 before it counts itself in: every thread waits
    // for its own stores (a workgroup-scope release does not wait for them), then one arrival.
    __shared__ int last;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    const int used = (L + kSplit - 1) / kSplit;  // live splits of the row, each counted once
    if (threadIdx.x == 0) {
      // Wrapping increment: the used-th arrival sees used - 1 and leaves 0 behind.
      const uint32_t seen = __builtin_amdgcn_atomic_inc32(a.arrivals + bh, static_cast<uint32_t>(used - 1),
                                                          __ATOMIC_RELAXED, "workgroup");
      last = seen == static_cast<uint32_t>(used - 1);
    }
    __syncthreads();
    if (!last) return;
    fused_merge<GP>(a, bh, used, reinterpret_cast<float (*)[kMaxFusedSplits]>(&p_lds[0][0]), &ml[0][0], big);
  }
}

// One workgroup per (b, query head): `groups` groups of 128 threads (one lane per dim), group g
// merging chunks g, g + groups, ... of kChunk splits. Online merge per chunk: each thread first
// requests its dim of the chunk's kChunk partial outputs, lanes 0..kChunk-1 of the group's first
// wave request one split's (m, l) each (vector loads, so no scalar-load waits), and the chunk's
// maximum and weights go through LDS; the running maximum M, denominator l and accumulator acc
// are rescaled when M grows. The groups' (M, l, acc) are merged the same way at the end. Several
// groups serve long rows (many splits), whose chunks would otherwise be merged one after another:
// up to 8 (256 splits in one round; the 1M shape's 154 splits per row: 23.1 vs 24.4 us with 4).
constexpr int kMaxCombineGroups = 8;

__global__ void __launch_bounds__(kHeadDim * kMaxCombineGroups) attn_combine_kernel(AttnArgs a) {
  constexpr int kChunk = 32;
  __shared__ float w_s[kMaxCombineGroups][kChunk];
  __shared__ float m_s[kMaxCombineGroups], l_s[kMaxCombineGroups];
  __shared__ float acc_s[kMaxCombineGroups][kHeadDim];
  const int groups = blockDim.x / kHeadDim;
  const int g = threadIdx.x / kHeadDim;
  const int row = blockIdx.x;  // b*Hq + hq
  const int Hq = a.Hkv * a.G;
  const int b = row / Hq;
  const int hq = row - b * Hq;
  const int d = threadIdx.x - g * kHeadDim;
  const float2* ml = reinterpret_cast<const float2*>(a.ws_ml) + static_cast<int64_t>(row) * a.splits;
  const float* o = a.ws_o + static_cast<int64_t>(row) * a.splits * kHeadDim + d;
  const int used = (live_length(a) + a.split_keys - 1) / a.split_keys;  // >= 1
  // Groups in use follow the live split count only (not the launch), so a device length and the
  // same host length merge in the same order; groups beyond it stay idle.
  const int eg = min(groups, (used + kChunk - 1) / kChunk);
  const int iters = (used + kChunk * eg - 1) / (kChunk * eg);  // the same for every group
  float M = -INFINITY, l = 0.f, acc = 0.f;
  for (int it = 0; it < iters; ++it) {
    const int s0 = (it * eg + g) * kChunk;
    const bool live = g < eg && s0 < used;  // group-uniform: this group has a chunk this round
    float x[kChunk];
#pragma unroll
    for (int u = 0; u < kChunk; ++u) x[u] = o[static_cast<int64_t>(min(s0 + u, used - 1)) * kHeadDim];
    const bool own = d < kChunk && s0 + d < used;  // this lane's split of the chunk
    const float2 p = ml[min(s0 + d, used - 1)];
    const float cm = skv::wave_max_dpp(own ? p.x : -INFINITY);  // the group's first wave holds the chunk
    if (d == 0) m_s[g] = cm;
    __syncthreads();
    const float Mn = live ? fmaxf(M, m_s[g]) : M;
    const float w = own ? expf(p.x - Mn) : 0.f;
    const float lw = skv::wave_sum_dpp(own ? p.y * w : 0.f);
    if (d < kChunk) w_s[g][d] = w;
    if (d == 0) l_s[g] = lw;
    __syncthreads();
    if (live) {
      const float r = expf(M - Mn);  // 0 on the group's first chunk (M = -inf)
      float sum = 0.f;
#pragma unroll
      for (int u = 0; u < kChunk; ++u) sum = fmaf(w_s[g][u], x[u], sum);
      acc = fmaf(acc, r, sum);
      l = fmaf(l, r, l_s[g]);
      M = Mn;
    }
    __syncthreads();  // w_s, m_s, l_s are rewritten by the next round
  }
  if (groups > 1) {
    acc_s[g][d] = acc;
    if (d == 0) {
      m_s[g] = M;
      l_s[g] = l;
    }
    __syncthreads();
    if (g != 0) return;
    float Mt = m_s[0];
    for (int q = 1; q < groups; ++q) Mt = fmaxf(Mt, m_s[q]);  // group 0 always merged a chunk
    l = 0.f;
    acc = 0.f;
    for (int q = 0; q < groups; ++q) {
      const float r = expf(m_s[q] - Mt);  // 0 for a group without chunks (M = -inf)
      l = fmaf(l_s[q], r, l);
      acc = fmaf(acc_s[q][d], r, acc);
    }
  }
  a.out[b * a.o_sb + hq * a.o_sh + d] = skv::f2bf(acc / l);
}

int splits_for(int kv_len, int split_keys) { return (kv_len + split_keys - 1) / split_keys; }

constexpr int kMaxDevices = 64;

// XCD mapping probe: workgroup w of a 1-D grid records the XCC id it runs on.
constexpr int kProbeWorkgroups = 4096;

__global__ void xcc_probe_kernel(uint32_t* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = __builtin_amdgcn_s_getreg(kHwRegXccId) & 15u;
}

}  // namespace

static __device__ uint32_t xcc_probe_out[kProbeWorkgroups];
static __device__ uint32_t xcc_misplaced;  // set by a fused attention workgroup off its expected XCD

namespace {

struct XccMap {
  int state = 0;      // 0 not probed, 1 confirmed, -1 not confirmed
  uint32_t map = 0;   // XCC id of blockIdx class x (mod 8) in bits [4x, 4x + 4)
  uint32_t* misplaced = nullptr;
};
std::mutex g_xcc_mu;
XccMap g_xcc[kMaxDevices];

// Whether this device's dispatcher hands every workgroup of a 1-D grid with the same blockIdx mod
// 8 to one XCC (probed once per device with kProbeWorkgroups workgroups; on MI355X workgroup w
// runs on XCD w mod 8). Not probed while `stream` is capturing a graph (the probe waits for its
// result): such a call takes the two-launch merge.
bool fused_mapping(hipStream_t stream, uint32_t* map, uint32_t** misplaced) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lock(g_xcc_mu);
  XccMap& m = g_xcc[dev];
  if (m.state == 0) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
    void* out = nullptr;
    void* mis = nullptr;
    uint32_t h[kProbeWorkgroups];
    bool ok = hipGetSymbolAddress(&out, HIP_SYMBOL(xcc_probe_out)) == hipSuccess &&
              hipGetSymbolAddress(&mis, HIP_SYMBOL(xcc_misplaced)) == hipSuccess && out && mis;
    if (ok) {
      hipLaunchKernelGGL(xcc_probe_kernel, dim3(kProbeWorkgroups), dim3(64), 0, stream, static_cast<uint32_t*>(out));
      ok = hipGetLastError() == hipSuccess &&
           hipMemcpyAsync(h, out, sizeof(h), hipMemcpyDeviceToHost, stream) == hipSuccess &&
           hipStreamSynchronize(stream) == hipSuccess;
    }
    uint32_t packed = 0;
    for (int x = 0; ok && x < kXcds; ++x) packed |= (h[x] & 15u) << (4 * x);
    for (int w = 0; ok && w < kProbeWorkgroups; ++w) ok = h[w] == h[w % kXcds];
    m.state = ok ? 1 : -1;
    m.map = packed;
    m.misplaced = static_cast<uint32_t*>(mis);
  }
  *map = m.map;
  *misplaced = m.misplaced;
  return m.state == 1;
}

}  // namespace

extern "C" int skv_sparse_attn_xcd_check(int32_t* state, uint32_t* xcc_map, uint32_t* misplaced) {
  int dev = -1;
  if (!state || !xcc_map || !misplaced) {
    skv_set_error("sparse_attn_xcd_check: null pointer");
    return SKV_EINVAL;
  }
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    skv_set_error("sparse_attn_xcd_check: no usable current device");
    return SKV_ELAUNCH;
  }
  {
    std::lock_guard<std::mutex> lock(g_xcc_mu);
    *state = g_xcc[dev].state;
    *xcc_map = g_xcc[dev].map;
  }
  *misplaced = 0;
  const hipError_t e = hipMemcpyFromSymbol(misplaced, HIP_SYMBOL(xcc_misplaced), sizeof(uint32_t), 0,
                                           hipMemcpyDeviceToHost);
  if (e != hipSuccess) {
    skv_set_error("sparse_attn_xcd_check: %s", hipGetErrorString(e));
    return SKV_ELAUNCH;
  }
  return SKV_OK;
}

extern "C" int64_t skv_sparse_attn_workspace_bytes(int batch_size, int q_heads, int kv_len) {
  if (batch_size < 1 || q_heads < 1 || kv_len < 1) return 0;
  // Arrival counters, then the partials of the shorter split (the launch may choose either).
  return kArrivalBytes +
         static_cast<int64_t>(batch_size) * q_heads * splits_for(kv_len, kSplitShort) * (kHeadDim + 2) * sizeof(float);
}

namespace {

// Keys per split: 128. SKV_ATTN_SPLIT=64 forces 64-key splits (twice the workgroups; measured
// slower at every decode shape on MI355X: Llama-3-8B batch 4 23.1 vs 15.5 us, GLM-4-9B batch 4
// 11.7 vs 10.8 us with the two-launch merge).
int choose_split_keys(int rows, int kv_len) {
  (void)rows, (void)kv_len;
  const char* e = getenv("SKV_ATTN_SPLIT");
  const int forced = e ? atoi(e) : 0;
  if (forced == kSplitShort || forced == kSplitLong) return forced;
  return kSplitLong;
}

template <int kMap, int kSplit, bool kFused>
void launch_split(int G, dim3 grid, hipStream_t s, const AttnArgs& a) {
  if (G == 1) hipLaunchKernelGGL((attn_split_kernel<1, kMap, kSplit, kFused>), grid, dim3(kThreads), 0, s, a);
  else if (G == 2) hipLaunchKernelGGL((attn_split_kernel<2, kMap, kSplit, kFused>), grid, dim3(kThreads), 0, s, a);
  else if (G <= 4) hipLaunchKernelGGL((attn_split_kernel<4, kMap, kSplit, kFused>), grid, dim3(kThreads), 0, s, a);
  else if (G <= 8) hipLaunchKernelGGL((attn_split_kernel<8, kMap, kSplit, kFused>), grid, dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL((attn_split_kernel<16, kMap, kSplit, kFused>), grid, dim3(kThreads), 0, s, a);
}

template <int kMap, bool kFused>
void launch_split_keys(int G, dim3 grid, hipStream_t s, const AttnArgs& a) {
  if (a.split_keys == kSplitShort) launch_split<kMap, kSplitShort, kFused>(G, grid, s, a);
  else launch_split<kMap, kSplitLong, kFused>(G, grid, s, a);
}

// The selected region's values read in place from a value store (skv_sparse_attn_decode_vstore).
struct VStore {
  const uint16_t* store;
  int64_t stride_b, stride_h, chunks;
  const int64_t* ids;
};

int attn_decode(const char* what, const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t* k_cache,
                const uint16_t* v_cache, int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_s, int batch_size,
                int q_heads, int kv_heads, int head_dim, int kv_len, const int32_t* kv_len_dev, float scale,
                void* workspace, int64_t workspace_bytes, uint16_t* out, int64_t o_stride_b, int64_t o_stride_h,
                const int32_t* slot, int sparse_start, int select_sets, int chunk, int pool_slots, void* stream,
                const VStore* vsm = nullptr) {
  if (!q || !k_cache || !v_cache || !workspace || !out) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (head_dim != kHeadDim || batch_size < 1 || kv_heads < 1 || q_heads < kv_heads || q_heads % kv_heads || kv_len < 1) {
    skv_set_error("%s: unsupported shape batch=%d q_heads=%d kv_heads=%d head_dim=%d kv_len=%d", what, batch_size,
                  q_heads, kv_heads, head_dim, kv_len);
    return SKV_EUNSUPPORTED;
  }
  const int G = q_heads / kv_heads;
  if (G > 16) {
    skv_set_error("%s: %d query heads per kv head (max 16)", what, G);
    return SKV_EUNSUPPORTED;
  }
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache) |
       reinterpret_cast<uintptr_t>(workspace)) &
          15u ||
      q_stride_b % 8 || q_stride_h % 8 || kv_stride_b % 8 || kv_stride_h % 8 || kv_stride_s % 8) {
    skv_set_error("%s: q/K/V rows and the workspace must be 16-byte aligned", what);
    return SKV_EINVAL;
  }
  if (kv_len > kMaxKvLen) {
    skv_set_error("%s: kv_len=%d exceeds %d", what, kv_len, kMaxKvLen);
    return SKV_EUNSUPPORTED;
  }
  if (slot && (sparse_start < 0 || select_sets < 1 || chunk < 1 || pool_slots < select_sets)) {
    skv_set_error("%s: paged region sparse_start=%d select_sets=%d chunk=%d pool_slots=%d", what, sparse_start,
                  select_sets, chunk, pool_slots);
    return SKV_EINVAL;
  }
  if (vsm && (!vsm->store || !vsm->ids || sparse_start < 0 || select_sets < 1 || chunk < 1 || vsm->chunks < 1 ||
              (reinterpret_cast<uintptr_t>(vsm->store) & 15u) || vsm->stride_b % 8 || vsm->stride_h % 8)) {
    skv_set_error("%s: value store (16-byte aligned, strides multiples of 8 elements, ids) and region "
                  "sparse_start=%d select_sets=%d chunk=%d store_chunks=%lld", what, sparse_start, select_sets, chunk,
                  (long long)(vsm ? vsm->chunks : 0));
    return SKV_EINVAL;
  }
  const int64_t need = skv_sparse_attn_workspace_bytes(batch_size, q_heads, kv_len);
  if (workspace_bytes < need) {
    skv_set_error("%s: workspace of %lld bytes, %lld needed", what, (long long)workspace_bytes, (long long)need);
    return SKV_EINVAL;
  }
  const int rows = batch_size * kv_heads;
  AttnArgs a{};
  a.q = q;
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.k = k_cache;
  a.v = v_cache;
  a.kv_sb = kv_stride_b;
  a.kv_sh = kv_stride_h;
  a.kv_ss = kv_stride_s;
  a.Hkv = kv_heads;
  a.G = G;
  a.L = kv_len;
  a.L_dev = kv_len_dev;
  a.split_keys = choose_split_keys(rows, kv_len);
  a.splits = splits_for(kv_len, a.split_keys);
  a.scale = scale;
  a.arrivals = static_cast<uint32_t*>(workspace);
  a.ws_o = reinterpret_cast<float*>(static_cast<unsigned char*>(workspace) + kArrivalBytes);
  a.ws_ml = a.ws_o + static_cast<int64_t>(batch_size) * q_heads * a.splits * kHeadDim;
  a.out = out;
  a.o_sb = o_stride_b;
  a.o_sh = o_stride_h;
  a.slot = slot;
  a.sp0 = sparse_start;
  a.sel = select_sets;
  a.chunk = chunk;
  a.pool_slots = pool_slots;
  a.delta = (pool_slots - select_sets) * chunk;
  a.rows = rows;
  if (vsm) {
    a.vs = vsm->store;
    a.vs_sb = vsm->stride_b;
    a.vs_sh = vsm->stride_h;
    a.vs_chunks = vsm->chunks;
    a.vids = vsm->ids;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The merge folded into the split launch, on request (SKV_ATTN_FUSED=1): rows of at most 64
  // splits, at least one row per XCD (the rows of one XCD share its 32 CUs), the XCD mapping
  // confirmed on this device. Not the default: on MI355X it measured even with the second launch
  // alone (Llama-3-8B shape batch 4: 15.5 vs 15.8 us; batch 8: 23.8 vs 23.6; GLM-4-9B batch 4,
  // 16 heads merged by one workgroup: 12.2 vs 10.8) and slower inside the pipelined decode step,
  // beside the other lane's host-link fetch (36.7 vs 23.5 + 10.0 us per lane-layer).
  const char* fe = getenv("SKV_ATTN_FUSED");
  bool fused = !vsm && fe && fe[0] == '1' && rows >= kXcds && rows <= kMaxFusedRows && a.splits <= kMaxFusedSplits &&
               (reinterpret_cast<uintptr_t>(out) & 7u) == 0 && o_stride_b % 4 == 0 && o_stride_h % 4 == 0;  // 8-byte stores
  if (fused) fused = fused_mapping(s, &a.xcc_map, &a.misplaced);
  if (fused) {
    const dim3 grid(static_cast<unsigned>(kXcds * ((rows + kXcds - 1) / kXcds) * a.splits));
    if (slot) launch_split_keys<1, true>(G, grid, s, a);
    else launch_split_keys<0, true>(G, grid, s, a);
    return skv_check_launch(what);
  }
  const dim3 grid(a.splits, rows);
  if (vsm) launch_split_keys<2, false>(G, grid, s, a);
  else if (slot) launch_split_keys<1, false>(G, grid, s, a);
  else launch_split_keys<0, false>(G, grid, s, a);
  int rc = skv_check_launch(what);
  if (rc) return rc;
  // Several merge groups only when there are chunks for them (the split count by the maximum length).
  const int groups = std::min(kMaxCombineGroups, (a.splits + 31) / 32);
  hipLaunchKernelGGL(attn_combine_kernel, dim3(batch_size * q_heads), dim3(kHeadDim * groups), 0, s, a);
  return skv_check_launch(what);
}

}  // namespace

extern "C" int skv_sparse_attn_decode(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t* k_cache,
                                      const uint16_t* v_cache, int64_t kv_stride_b, int64_t kv_stride_h,
                                      int64_t kv_stride_s, int batch_size, int q_heads, int kv_heads, int head_dim,
                                      int kv_len, const int32_t* kv_len_dev, float scale, void* workspace,
                                      int64_t workspace_bytes, uint16_t* out,
                                      int64_t o_stride_b, int64_t o_stride_h, void* stream) {
  return attn_decode("sparse_attn_decode", q, q_stride_b, q_stride_h, k_cache, v_cache, kv_stride_b, kv_stride_h,
                     kv_stride_s, batch_size, q_heads, kv_heads, head_dim, kv_len, kv_len_dev, scale, workspace,
                     workspace_bytes, out, o_stride_b, o_stride_h, nullptr, 0, 0, 0, 0, stream);
}

extern "C" int skv_sparse_attn_decode_paged(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h,
                                            const uint16_t* k_cache, const uint16_t* v_cache, int64_t kv_stride_b,
                                            int64_t kv_stride_h, int64_t kv_stride_s, int batch_size, int q_heads,
                                            int kv_heads, int head_dim, int kv_len, const int32_t* kv_len_dev,
                                            float scale, void* workspace, int64_t workspace_bytes, uint16_t* out,
                                            int64_t o_stride_b, int64_t o_stride_h, const int32_t* slot_list,
                                            int sparse_start, int select_sets, int chunk_size, int pool_slots,
                                            void* stream) {
  if (!slot_list) {
    skv_set_error("sparse_attn_decode_paged: null slot_list");
    return SKV_EINVAL;
  }
  return attn_decode("sparse_attn_decode_paged", q, q_stride_b, q_stride_h, k_cache, v_cache, kv_stride_b,
                     kv_stride_h, kv_stride_s, batch_size, q_heads, kv_heads, head_dim, kv_len, kv_len_dev, scale,
                     workspace, workspace_bytes, out, o_stride_b, o_stride_h, slot_list, sparse_start, select_sets,
                     chunk_size, pool_slots, stream);
}

extern "C" int skv_sparse_attn_decode_vstore(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h,
                                             const uint16_t* k_cache, const uint16_t* v_cache, int64_t kv_stride_b,
                                             int64_t kv_stride_h, int64_t kv_stride_s, int batch_size, int q_heads,
                                             int kv_heads, int head_dim, int kv_len, const int32_t* kv_len_dev,
                                             float scale, void* workspace, int64_t workspace_bytes, uint16_t* out,
                                             int64_t o_stride_b, int64_t o_stride_h, const uint16_t* v_store,
                                             int64_t vs_stride_b, int64_t vs_stride_h, int64_t store_chunks,
                                             const int64_t* position_ids, int sparse_start, int select_sets,
                                             int chunk_size, void* stream) {
  const VStore vsm{v_store, vs_stride_b, vs_stride_h, store_chunks, position_ids};
  return attn_decode("sparse_attn_decode_vstore", q, q_stride_b, q_stride_h, k_cache, v_cache, kv_stride_b,
                     kv_stride_h, kv_stride_s, batch_size, q_heads, kv_heads, head_dim, kv_len, kv_len_dev, scale,
                     workspace, workspace_bytes, out, o_stride_b, o_stride_h, nullptr, sparse_start, select_sets,
                     chunk_size, select_sets, stream, &vsm);
}

// ---- allocation-free variant ---------------------------------------------------------------
// The split partials of skv_sparse_attn_decode_noalloc live in this file-scope device array, one
// copy per GPU, held until the process ends. Its device address is looked up once per device
// (hipGetSymbolAddress with that device current) and only that address is handed to kernels;
// the array's name is a host-side stand-in in host code. The partials need no clearing: every
// live split writes its own before the merge reads them, and the merge reads live splits only.
// The arrival counters at its head start at zero (the array is zero when the code object loads)
// and every fused call leaves them at zero.
namespace {

constexpr int64_t kNoallocScratchBytes = 32ll << 20;  // 32 MiB per GPU

std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace {

// Device address of this GPU's `scratch` (the current device's), looked up on first use.
int noalloc_scratch(const char* what, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    skv_set_error("%s: no usable current device (%s)", what, hipGetErrorString(e));
    return SKV_ELAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      skv_set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev, hipGetErrorString(e));
      return SKV_ELAUNCH;
    }
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return SKV_OK;
}

}  // namespace

extern "C" int64_t skv_sparse_attn_noalloc_max_bytes(void) { return kNoallocScratchBytes; }

extern "C" int skv_sparse_attn_decode_noalloc(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h,
                                              const uint16_t* k_cache, const uint16_t* v_cache, int64_t kv_stride_b,
                                              int64_t kv_stride_h, int64_t kv_stride_s, int batch_size, int q_heads,
                                              int kv_heads, int head_dim, int kv_len, const int32_t* kv_len_dev,
                                              float scale, uint16_t* out, int64_t o_stride_b, int64_t o_stride_h,
                                              void* stream) {
  const char* what = "sparse_attn_decode_noalloc";
  const int64_t need = skv_sparse_attn_workspace_bytes(batch_size, q_heads, kv_len);
  if (need > kNoallocScratchBytes) {
    skv_set_error("%s: batch %d x %d query heads x %d keys need %lld bytes of split partials, more than the %lld "
                  "of the library's scratch; use skv_sparse_attn_decode with a workspace", what, batch_size, q_heads,
                  kv_len, (long long)need, (long long)kNoallocScratchBytes);
    return SKV_EUNSUPPORTED;
  }
  void* ws = nullptr;
  if (int rc = noalloc_scratch(what, &ws)) return rc;
  return attn_decode(what, q, q_stride_b, q_stride_h, k_cache, v_cache, kv_stride_b, kv_stride_h, kv_stride_s,
                     batch_size, q_heads, kv_heads, head_dim, kv_len, kv_len_dev, scale, ws, kNoallocScratchBytes,
                     out, o_stride_b, o_stride_h, nullptr, 0, 0, 0, 0, stream);
}
