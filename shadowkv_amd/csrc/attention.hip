// a8: sparse decode attention of one query token over the assembled K/V buffers.
//
// Replaces flash_attn_with_kvcache(q, k, v, causal=True) at models/attention/shadow.py:48
// (q_len = 1, so causality masks nothing). Split-L flash decoding for CDNA4:
//   attn_split_kernel: workgroup = (kv head, split of kSplit keys); all G query heads that
//     share the kv head are served by one pass over its K and V rows, so every K/V byte is read
//     once from HBM. Scores on MFMA: v_mfma_f32_16x16x32_bf16 with the (up to 16) query heads as
//     the A rows and 16 keys as the B columns, so each lane ends up holding finished scores (no
//     cross-lane reduction); split softmax per query head with DPP/readlane wave reductions;
//     P.V in fp32: 16 key streams x 8 dims per lane, the streams summed through LDS.
//   attn_combine_kernel: log-sum-exp merge of the splits, bf16 output.
#include "wave_reduce.h"

namespace {

using skv::u32x4;

constexpr int kThreads = 256;
constexpr int kSplit = 256;
constexpr int kHeadDim = 128;

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
  const int32_t* L_dev;   // optional device-resident length, clamped to [1, L]
  float scale;
  float* ws_o;   // [B*Hq][splits][128]
  float* ws_ml;  // [B*Hq][splits][2]
  uint16_t* out;
  int64_t o_sb, o_sh;
};

__device__ __forceinline__ int live_length(const AttnArgs& a) {
  return a.L_dev ? min(max(*a.L_dev, 1), a.L) : a.L;
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <int GP>
__global__ void __launch_bounds__(kThreads) attn_split_kernel(AttnArgs a) {
  // Up to 4 query heads per kv head, the split's K and V rows are all requested at entry (one
  // memory latency per workgroup); with more, V is requested right after the scores, so its
  // latency overlaps the softmax instead.
  constexpr bool kEarlyV = false;
  constexpr int kRows = kSplit / 16;        // keys per P.V stream
  constexpr int kGroups = kSplit / 4 / 16;  // 16-key MFMA groups per wave
  constexpr int kPass = GP < 4 ? GP : 4;    // query heads per stream-reduction pass
  __shared__ float p_lds[GP][kSplit];
  __shared__ __align__(16) float red[16][kPass][kHeadDim];  // [key stream][head of the pass][dim]
  __shared__ float ml[GP][2];

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
  // K as MFMA B operand: lane (li, grp) holds key (wave*64 + 16*kg + li), same dims.
  u32x4 kf[kGroups][4];
#pragma unroll
  for (int kg = 0; kg < kGroups; ++kg) {
    const int s = s0 + wave * (kSplit / 4) + 16 * kg + li;
    const uint16_t* krow = kh + static_cast<int64_t>(min(s, s1 - 1)) * a.kv_ss + 8 * grp;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) kf[kg][ks] = skv::load16_or_zero(krow + 32 * ks, s < s1);
  }
  // V for P.V: stream (wave, grp) takes keys s0 + 16*i + stream, lane li its dims [8*li, +8).
  const int stream = wave * 4 + grp;
  u32x4 vr[kRows];
  auto load_v = [&]() {
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const int s = s0 + i * 16 + stream;
      vr[i] = skv::load16_or_zero(vh + static_cast<int64_t>(min(s, s1 - 1)) * a.kv_ss + li * 8, s < s1);
    }
  };
  if (kEarlyV) load_v();
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
  if (!kEarlyV) load_v();
  __syncthreads();

  for (int g = wave; g < G; g += 4) {
    float x[4];
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      x[u] = p_lds[g][lane * 4 + u];
      mx = fmaxf(mx, x[u]);
    }
    mx = skv::wave_max_dpp(mx);
    float l = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float e = (x[u] == -INFINITY) ? 0.f : expf(x[u] - mx);
      p_lds[g][lane * 4 + u] = e;
      l += e;
    }
    l = skv::wave_sum_dpp(l);
    if (lane == 0) {
      ml[g][0] = mx;
      ml[g][1] = l;
    }
  }
  __syncthreads();

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

  // Sum the 16 key streams through LDS, kPass query heads per pass.
  const int Hq = a.Hkv * G;
#pragma unroll
  for (int p0 = 0; p0 < GP; p0 += kPass) {
    if (p0 > 0) __syncthreads();  // the previous pass has read red
#pragma unroll
    for (int gp = 0; gp < kPass; ++gp) {
      float* dst = &red[stream][gp][li * 8];
      *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{acc[p0 + gp][0], acc[p0 + gp][1], acc[p0 + gp][2], acc[p0 + gp][3]};
      *reinterpret_cast<f32x4_t*>(dst + 4) = f32x4_t{acc[p0 + gp][4], acc[p0 + gp][5], acc[p0 + gp][6], acc[p0 + gp][7]};
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < kPass * kHeadDim; idx += kThreads) {
      const int gp = idx / kHeadDim, d = idx - gp * kHeadDim;
      const int g = p0 + gp;
      if (g >= G) continue;
      float o = 0.f;
#pragma unroll
      for (int st = 0; st < 16; ++st) o += red[st][gp][d];
      const int64_t r = (static_cast<int64_t>(b) * Hq + h * G + g) * a.splits + split;
      a.ws_o[r * kHeadDim + d] = o;
      if (d == 0) {
        a.ws_ml[r * 2] = ml[g][0];
        a.ws_ml[r * 2 + 1] = ml[g][1];
      }
    }
  }
}

constexpr int kMaxSplits = 1024;  // kv_len <= 262144

// Block-wide (two waves) max / sum through a 2-slot LDS exchange.
__device__ __forceinline__ float block2_max(float v, float* x) {
  v = skv::wave_max_dpp(v);
  if ((threadIdx.x & 63) == 0) x[threadIdx.x >> 6] = v;
  __syncthreads();
  v = fmaxf(x[0], x[1]);
  __syncthreads();
  return v;
}
__device__ __forceinline__ float block2_sum(float v, float* x) {
  v = skv::wave_sum_dpp(v);
  if ((threadIdx.x & 63) == 0) x[threadIdx.x >> 6] = v;
  __syncthreads();
  v = x[0] + x[1];
  __syncthreads();
  return v;
}

__global__ void __launch_bounds__(kHeadDim) attn_combine_kernel(AttnArgs a) {
  static_assert(kHeadDim == 128, "two waves per row");
  __shared__ float w_lds[kMaxSplits];
  __shared__ float xch[2];
  const int row = blockIdx.x;  // b*Hq + hq
  const int Hq = a.Hkv * a.G;
  const int b = row / Hq;
  const int hq = row - b * Hq;
  const int d = threadIdx.x;
  const float* ml = a.ws_ml + static_cast<int64_t>(row) * a.splits * 2;
  const float* o = a.ws_o + static_cast<int64_t>(row) * a.splits * kHeadDim;
  const int used = (live_length(a) + kSplit - 1) / kSplit;
  float m = -INFINITY;
  for (int s = d; s < used; s += kHeadDim) m = fmaxf(m, ml[2 * s]);
  const float M = block2_max(m, xch);
  float l = 0.f;
  for (int s = d; s < used; s += kHeadDim) {
    const float w = expf(ml[2 * s] - M);
    w_lds[s] = w;
    l += ml[2 * s + 1] * w;
  }
  const float inv = 1.f / block2_sum(l, xch);  // the barriers also publish w_lds
  float acc = 0.f;
  int s = 0;
  for (; s + 8 <= used; s += 8) {
    float x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = o[static_cast<int64_t>(s + u) * kHeadDim + d];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = fmaf(w_lds[s + u], x[u], acc);
  }
  for (; s < used; ++s) acc = fmaf(w_lds[s], o[static_cast<int64_t>(s) * kHeadDim + d], acc);
  a.out[b * a.o_sb + hq * a.o_sh + d] = skv::f2bf(acc * inv);
}

int splits_for(int kv_len) { return (kv_len + kSplit - 1) / kSplit; }

}  // namespace

extern "C" int64_t skv_sparse_attn_workspace_bytes(int batch_size, int q_heads, int kv_len) {
  if (batch_size < 1 || q_heads < 1 || kv_len < 1) return 0;
  return static_cast<int64_t>(batch_size) * q_heads * splits_for(kv_len) * (kHeadDim + 2) * sizeof(float);
}

extern "C" int skv_sparse_attn_decode(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t* k_cache,
                                      const uint16_t* v_cache, int64_t kv_stride_b, int64_t kv_stride_h,
                                      int64_t kv_stride_s, int batch_size, int q_heads, int kv_heads, int head_dim,
                                      int kv_len, const int32_t* kv_len_dev, float scale, void* workspace,
                                      int64_t workspace_bytes, uint16_t* out,
                                      int64_t o_stride_b, int64_t o_stride_h, void* stream) {
  const char* what = "sparse_attn_decode";
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
  if (splits_for(kv_len) > kMaxSplits) {
    skv_set_error("%s: kv_len=%d exceeds %d", what, kv_len, kMaxSplits * kSplit);
    return SKV_EUNSUPPORTED;
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
  a.splits = splits_for(kv_len);
  a.scale = scale;
  a.ws_o = static_cast<float*>(workspace);
  a.ws_ml = a.ws_o + static_cast<int64_t>(batch_size) * q_heads * a.splits * kHeadDim;
  a.out = out;
  a.o_sb = o_stride_b;
  a.o_sh = o_stride_h;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(a.splits, batch_size * kv_heads);
  if (G == 1) hipLaunchKernelGGL(attn_split_kernel<1>, grid, dim3(kThreads), 0, s, a);
  else if (G == 2) hipLaunchKernelGGL(attn_split_kernel<2>, grid, dim3(kThreads), 0, s, a);
  else if (G <= 4) hipLaunchKernelGGL(attn_split_kernel<4>, grid, dim3(kThreads), 0, s, a);
  else if (G <= 8) hipLaunchKernelGGL(attn_split_kernel<8>, grid, dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL(attn_split_kernel<16>, grid, dim3(kThreads), 0, s, a);
  int rc = skv_check_launch(what);
  if (rc) return rc;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(batch_size * q_heads), dim3(kHeadDim), 0, s, a);
  return skv_check_launch(what);
}
