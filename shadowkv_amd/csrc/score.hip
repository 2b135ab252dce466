// a1: query-vs-chunk-landmark scoring with softmax, and the fused GQA max (a2 front).
//
// Semantics follow the reference's CUTLASS pipeline (kernels/batch_gemm_softmax.cu:143-196,
// kernels/batch_gemm_softmax.h:66-242,429-512):
//   D[z,i,j] = bf16(alpha * sum_k A[z,i,k] B[z,j,k])  (fp32 accumulation, one rounding)
//   P[z,i,j] = bf16(exp(D - max_j D) / sum_j exp(D - max_j D))   (fp32 softmax of the bf16 logits)
// and the GQA reduction of models/kvcache/shadow.py:567-568: out[z,j] = max_i P[z,i,j].
//
// The landmark matrix B is the only large operand (n x 128 bf16 per z), so the design is a
// memory-streaming one, not a GEMM tiling:
//   logits_kernel: workgroup = 256 landmarks of one z (grid n/256 x batch); 16 lanes cover one
//     256-byte landmark row with 16-byte loads (a wave reads 4 rows = 1 KB contiguous); the m
//     queries sit in registers; the m partial dots are combined with a 16-lane reduce-scatter;
//     logits are staged in LDS, written out coalesced, and the tile's max and sum(exp) partials
//     go to norm/sum [z][i][tile] (the reference's 256-column partial layout).
//   softmax_kernel: each workgroup merges the partials of its z, then normalises its 256
//     columns for every query row and keeps the running max over rows.
#include "wave_reduce.h"

namespace {

using skv::u32x4;

constexpr int kThreads = 256;
constexpr int kTile = 256;
constexpr int kHeadDim = 128;
constexpr int kMaxM = 16;

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(w[e] << 16);
    f[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
  }
}

template <int M>
__global__ void __launch_bounds__(kThreads) logits_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                                          uint16_t* __restrict__ D, float* __restrict__ norm,
                                                          float* __restrict__ sum, int m, int n, float alpha, int tiles) {
  __shared__ float s_tile[M][kTile];
  const int z = blockIdx.y;
  const int tile = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int grp = lane >> 4;

  float q[M][8];
#pragma unroll
  for (int i = 0; i < M; ++i) {
    if (i < m) {
      u32x4 v = *reinterpret_cast<const u32x4*>(A + (static_cast<int64_t>(z) * m + i) * kHeadDim + li * 8);
      unpack8(v, q[i]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) q[i][e] = 0.f;
    }
  }

  const uint16_t* Bz = B + static_cast<int64_t>(z) * n * kHeadDim;
  const int owner = skv::rs16_owner<M>(li);
  const bool writer = skv::rs16_writer<M>(li) && owner < m;
  // Each wave owns kTile/4 = 64 landmarks, 4 per step (one per 16-lane group): 16 steps.
  constexpr int kSteps = kTile / 16;
  u32x4 rows[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {  // issue all of this lane's row loads up front
    const int jl = wave * (kTile / 4) + s * 4 + grp;
    const int j = tile * kTile + jl;
    rows[s] = u32x4{0u, 0u, 0u, 0u};
    if (j < n) rows[s] = *reinterpret_cast<const u32x4*>(Bz + static_cast<int64_t>(j) * kHeadDim + li * 8);
  }
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int jl = wave * (kTile / 4) + s * 4 + grp;
    const int j = tile * kTile + jl;
    float l[8];
    unpack8(rows[s], l);
    float v[M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf(q[i][e], l[e], acc);
      v[i] = acc;
    }
    const float dot = skv::reduce_scatter16<M>(v, li);
    if (writer) s_tile[owner][jl] = (j < n) ? skv::bf2f(skv::f2bf(alpha * dot)) : -INFINITY;
  }
  __syncthreads();

  for (int i = wave; i < m; i += 4) {
    float x[4];
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      x[u] = s_tile[i][lane * 4 + u];
      mx = fmaxf(mx, x[u]);
    }
    const int j0 = tile * kTile + lane * 4;
    uint16_t* Drow = D + (static_cast<int64_t>(z) * m + i) * n;
    if (j0 + 3 < n && (n & 3) == 0) {
      uint2 packed;
      packed.x = static_cast<uint32_t>(skv::f2bf(x[0])) | (static_cast<uint32_t>(skv::f2bf(x[1])) << 16);
      packed.y = static_cast<uint32_t>(skv::f2bf(x[2])) | (static_cast<uint32_t>(skv::f2bf(x[3])) << 16);
      *reinterpret_cast<uint2*>(Drow + j0) = packed;
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (j0 + u < n) Drow[j0 + u] = skv::f2bf(x[u]);
    }
    mx = skv::wave_max(mx);
    float se = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) se += (x[u] == -INFINITY) ? 0.f : expf(x[u] - mx);
    se = skv::wave_sum(se);
    if (lane == 0) {
      norm[(static_cast<int64_t>(z) * m + i) * tiles + tile] = mx;
      sum[(static_cast<int64_t>(z) * m + i) * tiles + tile] = se;
    }
  }
}

template <bool kWriteSoftmax, bool kWriteMax>
__global__ void __launch_bounds__(kThreads) softmax_kernel(const uint16_t* __restrict__ D, const float* __restrict__ norm,
                                                           const float* __restrict__ sum, uint16_t* __restrict__ P,
                                                           uint16_t* __restrict__ out_max, int m, int n, int tiles) {
  __shared__ float gmax[kMaxM], ginv[kMaxM];
  const int z = blockIdx.y;
  const int tile = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int i = wave; i < m; i += 4) {
    const float* nr = norm + (static_cast<int64_t>(z) * m + i) * tiles;
    const float* sr = sum + (static_cast<int64_t>(z) * m + i) * tiles;
    float mx = -INFINITY;
    for (int t = lane; t < tiles; t += 64) mx = fmaxf(mx, nr[t]);
    mx = skv::wave_max(mx);
    float s = 0.f;
    for (int t = lane; t < tiles; t += 64) s += sr[t] * expf(nr[t] - mx);
    s = skv::wave_sum(s);
    if (lane == 0) {
      gmax[i] = mx;
      ginv[i] = 1.f / s;
    }
  }
  __syncthreads();
  const int j = tile * kTile + threadIdx.x;
  if (j >= n) return;
  float best = -INFINITY;
  for (int i = 0; i < m; ++i) {
    const int64_t o = (static_cast<int64_t>(z) * m + i) * n + j;
    const uint16_t p = skv::f2bf(expf(skv::bf2f(D[o]) - gmax[i]) * ginv[i]);
    if (kWriteSoftmax) P[o] = p;
    best = fmaxf(best, skv::bf2f(p));
  }
  if (kWriteMax) out_max[static_cast<int64_t>(z) * n + j] = skv::f2bf(best);
}

int check_scoring_shape(const char* what, int batch_count, int m, int n, int k) {
  if (k != kHeadDim || m < 1 || m > kMaxM || n < 1 || batch_count < 1) {
    skv_set_error("%s: unsupported shape batch=%d m=%d n=%d k=%d (k must be 128, m in [1,16])", what, batch_count, m, n,
                  k);
    return SKV_EUNSUPPORTED;
  }
  return SKV_OK;
}

int launch_logits(const char* what, const uint16_t* A, const uint16_t* B, uint16_t* D, float* norm, float* sum,
                  int batch_count, int m, int n, int k, float alpha, hipStream_t stream) {
  if (!A || !B || !D || !norm || !sum) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  int rc = check_scoring_shape(what, batch_count, m, n, k);
  if (rc) return rc;
  if ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 15u) {
    skv_set_error("%s: A and B must be 16-byte aligned", what);
    return SKV_EINVAL;
  }
  const int tiles = (n + kTile - 1) / kTile;
  const dim3 grid(tiles, batch_count);
  if (m == 1) hipLaunchKernelGGL(logits_kernel<1>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
  else if (m == 2) hipLaunchKernelGGL(logits_kernel<2>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
  else if (m <= 4) hipLaunchKernelGGL(logits_kernel<4>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
  else if (m <= 8) hipLaunchKernelGGL(logits_kernel<8>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
  else hipLaunchKernelGGL(logits_kernel<16>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
  return skv_check_launch(what);
}

int launch_softmax(const char* what, const uint16_t* D, const float* norm, const float* sum, uint16_t* softmax,
                   uint16_t* out_max, int batch_count, int m, int n, hipStream_t stream) {
  if (!D || !norm || !sum || (!softmax && !out_max)) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  int rc = check_scoring_shape(what, batch_count, m, n, kHeadDim);
  if (rc) return rc;
  const int tiles = (n + kTile - 1) / kTile;
  const dim3 grid(tiles, batch_count);
  if (softmax && out_max)
    hipLaunchKernelGGL((softmax_kernel<true, true>), grid, dim3(kThreads), 0, stream, D, norm, sum, softmax, out_max, m, n, tiles);
  else if (softmax)
    hipLaunchKernelGGL((softmax_kernel<true, false>), grid, dim3(kThreads), 0, stream, D, norm, sum, softmax, out_max, m, n, tiles);
  else
    hipLaunchKernelGGL((softmax_kernel<false, true>), grid, dim3(kThreads), 0, stream, D, norm, sum, softmax, out_max, m, n, tiles);
  return skv_check_launch(what);
}

}  // namespace

extern "C" int skv_score_logits(const uint16_t* A, const uint16_t* B, uint16_t* D, float* norm, float* sum,
                                int batch_count, int m, int n, int k, float alpha, void* stream) {
  return launch_logits("score_logits", A, B, D, norm, sum, batch_count, m, n, k, alpha, static_cast<hipStream_t>(stream));
}

extern "C" int skv_softmax_gqa_max(const uint16_t* D, const float* norm, const float* sum, uint16_t* softmax,
                                   uint16_t* out_max, int batch_count, int m, int n, void* stream) {
  return launch_softmax("softmax_gqa_max", D, norm, sum, softmax, out_max, batch_count, m, n,
                        static_cast<hipStream_t>(stream));
}

extern "C" int skv_batch_gemm_softmax(const uint16_t* A, const uint16_t* B, uint16_t* D, float* norm, float* sum,
                                      uint16_t* softmax, int batch_count, int m, int n, int k, float alpha, float beta,
                                      void* stream) {
  if (beta != 0.f) {
    skv_set_error("batch_gemm_softmax: beta must be 0 (no C operand), got %g", beta);
    return SKV_EUNSUPPORTED;
  }
  if (!softmax) {
    skv_set_error("batch_gemm_softmax: null softmax output");
    return SKV_EINVAL;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = launch_logits("batch_gemm_softmax", A, B, D, norm, sum, batch_count, m, n, k, alpha, s);
  if (rc) return rc;
  return launch_softmax("batch_gemm_softmax", D, norm, sum, softmax, nullptr, batch_count, m, n, s);
}

extern "C" int skv_score_gqa_max(const uint16_t* A, const uint16_t* B, uint16_t* D, float* norm, float* sum,
                                 uint16_t* out, int batch_count, int m, int n, int k, float alpha, void* stream) {
  if (!out) {
    skv_set_error("score_gqa_max: null output");
    return SKV_EINVAL;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = launch_logits("score_gqa_max", A, B, D, norm, sum, batch_count, m, n, k, alpha, s);
  if (rc) return rc;
  return launch_softmax("score_gqa_max", D, norm, sum, nullptr, out, batch_count, m, n, s);
}
