// a8: sparse decode attention of one query token over the assembled K/V buffers.
//
// Replaces flash_attn_with_kvcache(q, k, v, causal=True) at models/attention/shadow.py:48
// (q_len = 1, so causality masks nothing). Split-L flash decoding for CDNA4:
//   attn_split_kernel: workgroup = (kv head, split of kSplit keys); all G query heads that
//     share the kv head are served by one pass over its K and V rows, so every K/V byte is read
//     once from HBM. Scores: 16 lanes per 256-byte key row (16-byte loads), G dots combined with
//     a 16-lane reduce-scatter, staged in LDS; split softmax (max, exp, sum) per query head;
//     P.V: 16 key streams x 8 dims per lane, fp32 accumulation, reduced across streams.
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

template <int GP>
__global__ void __launch_bounds__(kThreads) attn_split_kernel(AttnArgs a) {
  __shared__ float p_lds[GP][kSplit];
  __shared__ float red[4][GP][kHeadDim];
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

  const uint16_t* kb = a.k + b * a.kv_sb + h * a.kv_sh;
  const uint16_t* vb = a.v + b * a.kv_sb + h * a.kv_sh;

  {
    float q[GP][8];
#pragma unroll
    for (int g = 0; g < GP; ++g) {
      if (g < G) {
        const int hq = h * G + g;
        u32x4 v = *reinterpret_cast<const u32x4*>(a.q + b * a.q_sb + hq * a.q_sh + li * 8);
        unpack8(v, q[g]);
#pragma unroll
        for (int e = 0; e < 8; ++e) q[g][e] *= a.scale;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) q[g][e] = 0.f;
      }
    }
    const int owner = skv::rs16_owner<GP>(li);
    const bool writer = skv::rs16_writer<GP>(li) && owner < G;
    constexpr int kSteps = kSplit / 16;  // 4 waves x 4 key groups per step
    for (int st = 0; st < kSteps; st += 4) {
      u32x4 rows[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int s = s0 + (st + u) * 16 + wave * 4 + grp;
        rows[u] = u32x4{0u, 0u, 0u, 0u};
        if (s < s1) rows[u] = *reinterpret_cast<const u32x4*>(kb + static_cast<int64_t>(s) * a.kv_ss + li * 8);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int jl = (st + u) * 16 + wave * 4 + grp;
        float kf[8];
        unpack8(rows[u], kf);
        float d[GP];
#pragma unroll
        for (int g = 0; g < GP; ++g) {
          float acc = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc = fmaf(q[g][e], kf[e], acc);
          d[g] = acc;
        }
        const float dot = skv::reduce_scatter16<GP>(d, li);
        if (writer) p_lds[owner][jl] = (s0 + jl < s1) ? dot : -INFINITY;
      }
    }
  }
  __syncthreads();

  for (int g = wave; g < G; g += 4) {
    float x[4];
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      x[u] = p_lds[g][lane * 4 + u];
      mx = fmaxf(mx, x[u]);
    }
    mx = skv::wave_max(mx);
    float l = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float e = (x[u] == -INFINITY) ? 0.f : expf(x[u] - mx);
      p_lds[g][lane * 4 + u] = e;
      l += e;
    }
    l = skv::wave_sum(l);
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
  const int stream = wave * 4 + grp;  // 16 key streams
  for (int t = 0; t < kSplit / 16; t += 4) {
    u32x4 rows[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int s = s0 + (t + u) * 16 + stream;
      rows[u] = u32x4{0u, 0u, 0u, 0u};
      if (s < s1) rows[u] = *reinterpret_cast<const u32x4*>(vb + static_cast<int64_t>(s) * a.kv_ss + li * 8);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int jl = (t + u) * 16 + stream;
      if (s0 + jl < s1) {
        float vf[8];
        unpack8(rows[u], vf);
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
  }
  // Sum the 4 key streams of the wave (lane groups), then the 4 waves through LDS.
#pragma unroll
  for (int g = 0; g < GP; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = acc[g][e];
      x += __shfl_xor(x, 16, 64);
      x += __shfl_xor(x, 32, 64);
      acc[g][e] = x;
    }
  if (grp == 0) {
#pragma unroll
    for (int g = 0; g < GP; ++g)
      if (g < G)
#pragma unroll
        for (int e = 0; e < 8; ++e) red[wave][g][li * 8 + e] = acc[g][e];
  }
  __syncthreads();
  const int Hq = a.Hkv * G;
  for (int idx = threadIdx.x; idx < G * kHeadDim; idx += kThreads) {
    const int g = idx / kHeadDim, d = idx - g * kHeadDim;
    const float o = red[0][g][d] + red[1][g][d] + red[2][g][d] + red[3][g][d];
    const int64_t r = (static_cast<int64_t>(b) * Hq + h * G + g) * a.splits + split;
    a.ws_o[r * kHeadDim + d] = o;
    if (d == 0) {
      a.ws_ml[r * 2] = ml[g][0];
      a.ws_ml[r * 2 + 1] = ml[g][1];
    }
  }
}

__global__ void __launch_bounds__(kHeadDim) attn_combine_kernel(AttnArgs a) {
  const int row = blockIdx.x;  // b*Hq + hq
  const int Hq = a.Hkv * a.G;
  const int b = row / Hq;
  const int hq = row - b * Hq;
  const int d = threadIdx.x;
  const float* ml = a.ws_ml + static_cast<int64_t>(row) * a.splits * 2;
  const float* o = a.ws_o + static_cast<int64_t>(row) * a.splits * kHeadDim;
  const int used = (live_length(a) + kSplit - 1) / kSplit;
  float M = -INFINITY;
  for (int s = 0; s < used; ++s) M = fmaxf(M, ml[2 * s]);
  float l = 0.f, acc = 0.f;
  for (int s = 0; s < used; ++s) {
    const float w = expf(ml[2 * s] - M);
    l += ml[2 * s + 1] * w;
    acc += o[static_cast<int64_t>(s) * kHeadDim + d] * w;
  }
  a.out[b * a.o_sb + hq * a.o_sh + d] = skv::f2bf(acc / l);
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
