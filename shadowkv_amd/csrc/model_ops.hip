// The new-token operations around the sparse path, fused (next to the path: the decode step's
// QKV RoPE + KV append and the layer's norm / activation):
//   skv_rmsnorm        residual add + RMSNorm: h = bf16(x + r) (the reference's bf16 residual add,
//                      models/llama.py:204,215) and y = bf16(h * rsqrt(mean(h^2) + eps) * w) in fp32
//                      with one rounding (flashinfer rmsnorm through layer_norm, models/llama.py:191,206,
//                      models/base.py:94, models/tensor_op.py:39-44);
//   skv_silu_and_mul   y = bf16(bf16(silu(g)) * u) for the fused gate/up rows (vLLM silu_and_mul,
//                      models/llama.py:208-214, models/glm.py:193);
//   skv_rope_qk_append the new token's q and k rotated with the bf16 per-op rounding of the
//                      reference's rotary kernels (vLLM rotary_embedding, models/llama.py:149-150,
//                      models/glm.py:200-201), q written contiguous
//                      for the scoring kernel, rotated k and raw v appended to the key/value
//                      buffers at a device-resident row (models/kvcache/shadow.py:621-633).
#include "rope_math.h"

namespace {

using skv::u32x4;

constexpr int kThreads = 256;
constexpr int kHeadDim = 128;

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = skv::bf_lo(v[e]);
    f[2 * e + 1] = skv::bf_hi(v[e]);
  }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  return u32x4{skv::f2bf2(f[0], f[1]), skv::f2bf2(f[2], f[3]), skv::f2bf2(f[4], f[5]), skv::f2bf2(f[6], f[7])};
}

// One workgroup per row; each thread owns 8-element vectors strided by the workgroup.
template <bool kResidual>
__global__ void __launch_bounds__(kThreads) rmsnorm_kernel(const uint16_t* __restrict__ x, int64_t xs,
                                                           const uint16_t* __restrict__ r, int64_t rs,
                                                           uint16_t* __restrict__ ro, int64_t ros,
                                                           const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
                                                           int64_t os, int hidden, float eps) {
  constexpr int kMaxVec = 4;  // hidden <= 4 * 8 * 256 = 8192
  __shared__ float part[kThreads / 64];
  const int row = blockIdx.x;
  const int nv = hidden / 8;
  float h[kMaxVec][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxVec; ++k) {
    const int v = threadIdx.x + k * kThreads;
    if (v < nv) {
      const u32x4 xv = *reinterpret_cast<const u32x4*>(x + row * xs + 8 * v);
      unpack8(xv, h[k]);
      if (kResidual) {
        float rv[8];
        unpack8(*reinterpret_cast<const u32x4*>(r + row * rs + 8 * v), rv);
#pragma unroll
        for (int e = 0; e < 8; ++e) h[k][e] = skv::bf2f(skv::f2bf(h[k][e] + rv[e]));  // bf16 residual add
        *reinterpret_cast<u32x4*>(ro + row * ros + 8 * v) = pack8(h[k]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(h[k][e], h[k][e], ss);
    }
  }
  ss = skv::wave_sum_dpp(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) tot += part[i];
  const float inv = rsqrtf(tot / static_cast<float>(hidden) + eps);
#pragma unroll
  for (int k = 0; k < kMaxVec; ++k) {
    const int v = threadIdx.x + k * kThreads;
    if (v < nv) {
      float wv[8], y[8];
      unpack8(*reinterpret_cast<const u32x4*>(w + 8 * v), wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = h[k][e] * inv * wv[e];
      *reinterpret_cast<u32x4*>(out + row * os + 8 * v) = pack8(y);
    }
  }
}

__global__ void __launch_bounds__(kThreads) silu_mul_kernel(const uint16_t* __restrict__ x, int64_t xs,
                                                            uint16_t* __restrict__ out, int64_t os, int d, int nvec) {
  const int row = blockIdx.y;
  const int v = blockIdx.x * kThreads + threadIdx.x;
  if (v >= nvec) return;
  float g[8], u[8], y[8];
  unpack8(*reinterpret_cast<const u32x4*>(x + row * xs + 8 * v), g);
  unpack8(*reinterpret_cast<const u32x4*>(x + row * xs + d + 8 * v), u);
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = skv::silu_mul(g[e], u[e]);
  *reinterpret_cast<u32x4*>(out + row * os + 8 * v) = pack8(y);
}

struct RopeAppendArgs {
  const uint16_t* qkv;
  int64_t qkv_sb;
  int Hq, Hkv;
  const int64_t* pos;
  const uint16_t* cs;
  int64_t cs_stride, cs_rows;
  int glm;
  uint16_t* q_out;
  int64_t qo_sb;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t kv_sb, kv_sh, kv_ss;
  const int64_t* row_dev;
  int64_t buf_len;
};

// Workgroup (b, head) of 64 threads over the Hq + 2*Hkv heads of the fused QKV row: q heads are
// rotated into q_out, k heads rotated into the key buffer row, v heads copied into the value
// buffer row. Half-split: thread t < 64 rotates the pair (t, t+64); GLM: threads t < 32 rotate
// the interleaved pair (2t, 2t+1) and the upper 64 dims pass through.
__global__ void __launch_bounds__(64) rope_qk_append_kernel(RopeAppendArgs a) {
  const int b = blockIdx.y;
  const int head = blockIdx.x;
  const int t = threadIdx.x;
  const uint16_t* src = a.qkv + b * a.qkv_sb + static_cast<int64_t>(head) * kHeadDim;
  const int64_t row = *a.row_dev;
  uint16_t* dst;
  if (head < a.Hq) {
    dst = a.q_out + b * a.qo_sb + static_cast<int64_t>(head) * kHeadDim;
  } else {
    if (row < 0 || row >= a.buf_len) return;  // beyond the buffer: nothing appended
    const int h = head < a.Hq + a.Hkv ? head - a.Hq : head - a.Hq - a.Hkv;
    uint16_t* cache = head < a.Hq + a.Hkv ? a.k_cache : a.v_cache;
    dst = cache + b * a.kv_sb + h * a.kv_sh + row * a.kv_ss;
  }
  if (head >= a.Hq + a.Hkv) {  // v: copy
    dst[t] = src[t];
    dst[t + 64] = src[t + 64];
    return;
  }
  const int64_t p = a.pos[b];
  if (p < 0 || p >= a.cs_rows) {  // no rotation row for this position: unrotated
    dst[t] = src[t];
    dst[t + 64] = src[t + 64];
    return;
  }
  const uint16_t* c = a.cs + p * a.cs_stride;
  if (!a.glm) {
    uint16_t y1, y2;
    skv::rope_half_split(src[t], src[t + 64], c[t], c[t + 64], y1, y2);
    dst[t] = y1;
    dst[t + 64] = y2;
  } else {
    if (t < 32) {
      uint16_t ye, yo;
      skv::rope_half_split(src[2 * t], src[2 * t + 1], c[t], c[t + 32], ye, yo);
      dst[2 * t] = ye;
      dst[2 * t + 1] = yo;
    }
    dst[t + 64] = src[t + 64];
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int skv_rmsnorm(const uint16_t* x, int64_t x_stride, const uint16_t* residual, int64_t residual_stride,
                           uint16_t* residual_out, int64_t residual_out_stride, const uint16_t* weight, uint16_t* out,
                           int64_t out_stride, int rows, int hidden, float eps, void* stream) {
  const char* what = "rmsnorm";
  if (!x || !weight || !out || (residual && !residual_out)) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (rows < 1 || hidden < 8 || hidden % 8 || hidden > 8 * 4 * kThreads) {
    skv_set_error("%s: rows=%d hidden=%d (hidden a multiple of 8 up to %d)", what, rows, hidden, 8 * 4 * kThreads);
    return SKV_EUNSUPPORTED;
  }
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out) || x_stride % 8 || out_stride % 8 ||
      (residual && (!aligned16(residual) || !aligned16(residual_out) || residual_stride % 8 || residual_out_stride % 8))) {
    skv_set_error("%s: rows must be 16-byte aligned", what);
    return SKV_EINVAL;
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (residual)
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(rows), dim3(kThreads), 0, s, x, x_stride, residual, residual_stride,
                       residual_out, residual_out_stride, weight, out, out_stride, hidden, eps);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(rows), dim3(kThreads), 0, s, x, x_stride, residual, residual_stride,
                       residual_out, residual_out_stride, weight, out, out_stride, hidden, eps);
  return skv_check_launch(what);
}

extern "C" int skv_silu_and_mul(const uint16_t* x, int64_t x_stride, uint16_t* out, int64_t out_stride, int rows,
                                int d, void* stream) {
  const char* what = "silu_and_mul";
  if (!x || !out) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (rows < 1 || d < 8 || d % 8) {
    skv_set_error("%s: rows=%d d=%d (d a multiple of 8)", what, rows, d);
    return SKV_EUNSUPPORTED;
  }
  if (!aligned16(x) || !aligned16(out) || x_stride % 8 || out_stride % 8) {
    skv_set_error("%s: rows must be 16-byte aligned", what);
    return SKV_EINVAL;
  }
  const int nvec = d / 8;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((nvec + kThreads - 1) / kThreads, rows), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), x, x_stride, out, out_stride, d, nvec);
  return skv_check_launch(what);
}

extern "C" int skv_rope_qk_append(const uint16_t* qkv, int64_t qkv_stride_b, int batch_size, int q_heads, int kv_heads,
                                  int head_dim, const int64_t* positions, const uint16_t* cos_sin,
                                  int64_t stride_cos_sin, int64_t cos_sin_rows, int rope_mode, uint16_t* q_out,
                                  int64_t q_out_stride_b, uint16_t* k_cache, uint16_t* v_cache, int64_t kv_stride_b,
                                  int64_t kv_stride_h, int64_t kv_stride_s, const int64_t* append_row,
                                  int64_t buf_len, void* stream) {
  const char* what = "rope_qk_append";
  if (!qkv || !positions || !cos_sin || !q_out || !k_cache || !v_cache || !append_row) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (head_dim != kHeadDim || batch_size < 1 || q_heads < 1 || kv_heads < 1 || (rope_mode != 0 && rope_mode != 1)) {
    skv_set_error("%s: batch=%d q_heads=%d kv_heads=%d head_dim=%d rope_mode=%d", what, batch_size, q_heads, kv_heads,
                  head_dim, rope_mode);
    return SKV_EUNSUPPORTED;
  }
  RopeAppendArgs a{};
  a.qkv = qkv;
  a.qkv_sb = qkv_stride_b;
  a.Hq = q_heads;
  a.Hkv = kv_heads;
  a.pos = positions;
  a.cs = cos_sin;
  a.cs_stride = stride_cos_sin;
  a.cs_rows = cos_sin_rows;
  a.glm = rope_mode;
  a.q_out = q_out;
  a.qo_sb = q_out_stride_b;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.kv_sb = kv_stride_b;
  a.kv_sh = kv_stride_h;
  a.kv_ss = kv_stride_s;
  a.row_dev = append_row;
  a.buf_len = buf_len;
  hipLaunchKernelGGL(rope_qk_append_kernel, dim3(q_heads + 2 * kv_heads, batch_size), dim3(64), 0,
                     static_cast<hipStream_t>(stream), a);
  return skv_check_launch(what);
}
