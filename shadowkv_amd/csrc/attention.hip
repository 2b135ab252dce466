// a8: sparse decode attention of one query token over the assembled K/V buffers.
//
// Replaces flash_attn_with_kvcache(q, k, v, causal=True) at models/attention/shadow.py:48
// (q_len = 1, so causality masks nothing). Split-L flash decoding for CDNA4:
//   attn_split_kernel: workgroup = (kv head, split of 128 keys); all G query heads that
//     share the kv head are served by one pass over its K and V rows, so every K/V byte is read
//     once from HBM. Scores on MFMA: v_mfma_f32_16x16x32_bf16 with the (up to 16) query heads as
//     the A rows and 16 keys as the B columns, so each lane ends up holding finished scores (no
//     cross-lane reduction); split softmax per query head with DPP/readlane wave reductions;
//     P.V on MFMA for 9..16 query heads (P in bf16 as the A operand, the V tile read transposed
//     from LDS as B, each wave owning 32 dims), in fp32 for 1..8 (16 key streams x 8 dims per
//     lane, the streams summed through LDS).
//   attn_combine_kernel: log-sum-exp merge of the splits in one pass (running maximum), every
//     load of a 32-split chunk issued before the first is used; bf16 output.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "wave_reduce.h"

namespace {

using skv::u32x4;

constexpr int kThreads = 256;
// Keys per split workgroup. 128 rather than 256: twice the workgroups in flight at decode batch
// sizes (MI355X, cold K/V, Llama-3-8B shape batch 8: 24 vs 29 us; GLM-4-9B batch 4: 19 vs 27 us).
constexpr int kSplit = 128;
constexpr int kHeadDim = 128;
constexpr int kMaxKvLen = 262144;

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
};

__device__ __forceinline__ int live_length(const AttnArgs& a) {
  return a.L_dev ? min(max(*a.L_dev, 1), a.L) : a.L;
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// kSplit keys per workgroup; the split's V rows are requested right after the scores, so their
// latency overlaps the softmax (requesting them with K, at entry, measured no faster and holds
// more registers).
template <int GP, bool kPaged>
__global__ void __launch_bounds__(kThreads) attn_split_kernel(AttnArgs a) {
  constexpr int kRows = kSplit / 16;        // keys per P.V stream
  constexpr int kGroups = kSplit / 4 / 16;  // 16-key MFMA groups per wave
  constexpr int kPerLane = kSplit / 64;     // softmax entries per lane
  constexpr int kVals = GP * 8;              // P.V partial sums per lane: [head][8 dims]
  constexpr int kKept = kVals / 4;           // per lane after the in-wave stream fold
  __shared__ float p_lds[GP][kSplit];
  // [wave][lane][value] for the fp32 P.V path; the MFMA P.V path (GP == 16) stages the V tile here
  // instead ([key][kVtLd] bf16, rows padded so the 4 key groups of an operand read hit disjoint
  // banks).
  constexpr int kVtLd = kHeadDim + 4;
  constexpr int kRedBytes = 4 * 64 * kKept * 4;
  constexpr int kVtBytes = GP == 16 ? kSplit * kVtLd * 2 : 0;
  __shared__ __align__(16) unsigned char big[kRedBytes > kVtBytes ? kRedBytes : kVtBytes];
  float (*red)[64][kKept] = reinterpret_cast<float (*)[64][kKept]>(big);
  __shared__ float ml[GP][2];
  __shared__ int prow[kPaged ? kSplit : 1];  // physical row of each key of the split (paged)

  const int split = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / a.Hkv;
  const int h = bh - b * a.Hkv;
  const int L = live_length(a);
  const int s0 = split * kSplit;
  if (s0 >= L) return;  // workgroup-uniform: splits past the live length do nothing
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
  if (kPaged) {
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
  auto key_row = [&](int jl) -> int64_t { return kPaged ? prow[jl] : min(s0 + jl, s1 - 1); };
  // K as MFMA B operand: lane (li, grp) holds key (wave*64 + 16*kg + li), same dims.
  u32x4 kf[kGroups][4];
#pragma unroll
  for (int kg = 0; kg < kGroups; ++kg) {
    const int s = s0 + wave * (kSplit / 4) + 16 * kg + li;
    const uint16_t* krow = kh + key_row(s - s0) * a.kv_ss + 8 * grp;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) kf[kg][ks] = skv::load16_or_zero(krow + 32 * ks, s < s1);
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
      const u32x4 x = skv::load_nt(reinterpret_cast<const u32x4*>(vh + key_row(i * 16 + stream) * a.kv_ss + li * 8));
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
    return;
  }

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
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[j]), __float_as_uint(v[kVals / 2 + j]), false,
                                                    false);
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

}  // namespace

extern "C" int64_t skv_sparse_attn_workspace_bytes(int batch_size, int q_heads, int kv_len) {
  if (batch_size < 1 || q_heads < 1 || kv_len < 1) return 0;
  return static_cast<int64_t>(batch_size) * q_heads * splits_for(kv_len, kSplit) * (kHeadDim + 2) * sizeof(float);
}

namespace {

int attn_decode(const char* what, const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t* k_cache,
                const uint16_t* v_cache, int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_s, int batch_size,
                int q_heads, int kv_heads, int head_dim, int kv_len, const int32_t* kv_len_dev, float scale,
                void* workspace, int64_t workspace_bytes, uint16_t* out, int64_t o_stride_b, int64_t o_stride_h,
                const int32_t* slot, int sparse_start, int select_sets, int chunk, int pool_slots, void* stream) {
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
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) &
          15u ||
      q_stride_b % 8 || q_stride_h % 8 || kv_stride_b % 8 || kv_stride_h % 8 || kv_stride_s % 8) {
    skv_set_error("%s: q/K/V rows must be 16-byte aligned", what);
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
  const int64_t need = skv_sparse_attn_workspace_bytes(batch_size, q_heads, kv_len);
  if (workspace_bytes < need) {
    skv_set_error("%s: workspace of %lld bytes, %lld needed", what, (long long)workspace_bytes, (long long)need);
    return SKV_EINVAL;
  }
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
  a.split_keys = kSplit;
  a.splits = splits_for(kv_len, a.split_keys);
  a.scale = scale;
  a.ws_o = static_cast<float*>(workspace);
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(a.splits, batch_size * kv_heads);
  auto go = [&](auto paged) {
    constexpr bool P = decltype(paged)::value;
    if (G == 1) hipLaunchKernelGGL((attn_split_kernel<1, P>), grid, dim3(kThreads), 0, s, a);
    else if (G == 2) hipLaunchKernelGGL((attn_split_kernel<2, P>), grid, dim3(kThreads), 0, s, a);
    else if (G <= 4) hipLaunchKernelGGL((attn_split_kernel<4, P>), grid, dim3(kThreads), 0, s, a);
    else if (G <= 8) hipLaunchKernelGGL((attn_split_kernel<8, P>), grid, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL((attn_split_kernel<16, P>), grid, dim3(kThreads), 0, s, a);
  };
  if (slot) go(std::true_type{});
  else go(std::false_type{});
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

// ---- allocation-free variant ---------------------------------------------------------------
// The split partials of skv_sparse_attn_decode_noalloc live in this file-scope device array, one
// copy per GPU, held until the process ends. Its device address is looked up once per device
// (hipGetSymbolAddress with that device current) and only that address is handed to kernels;
// the array's name is a host-side stand-in in host code. The partials need no clearing: every
// live split writes its own before the merge reads them, and the merge reads live splits only.
namespace {

constexpr int64_t kNoallocScratchBytes = 32ll << 20;  // 32 MiB per GPU
constexpr int kMaxDevices = 64;

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
