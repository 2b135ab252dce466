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
//   logits_kernel: workgroup = 256 landmarks of one z (grid n/256 x batch), every landmark byte
//     requested at entry; the dots run on v_mfma_f32_16x16x32_bf16 with the (up to 16) queries
//     as the A rows and 16 landmarks as the B columns, so each lane ends up holding finished
//     dots (no cross-lane reduction); logits are staged in LDS, written out coalesced, and the
//     tile's max and sum(exp) partials (DPP wave reductions) go to norm/sum [z][i][tile] (the
//     reference's 256-column partial layout).
//   logits_rows_kernel: the same tile and outputs for up to 4 queries with the dots on the vector
//     ALUs (bf16 dot2), so that every wave load reads 4 whole landmark rows (1 KB contiguous)
//     instead of 64 bytes of 16 rows; the 16 lanes of a row meet by DPP.
//   softmax_kernel: each workgroup merges the partials of its z, then normalises its 256
//     columns for every query row and keeps the running max over rows.
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "softmax_keys.h"
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

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// A finished tile's logits (bf16-rounded, -inf past n) from s_tile[i][0, kTile) to D (coalesced
// bf16 stores) and the tile's (max, sum exp) partials into norm / sum [z][i][tile]. Wave w takes
// query rows w, w + 4, ...
__device__ __forceinline__ void store_tile(const float (*s_tile)[kTile], uint16_t* __restrict__ D, float* __restrict__ norm,
                                           float* __restrict__ sum, int z, int m, int n, int tile, int tiles) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
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
    mx = skv::wave_max_dpp(mx);
    float se = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) se += (x[u] == -INFINITY) ? 0.f : expf(x[u] - mx);
    se = skv::wave_sum_dpp(se);
    if (lane == 0) {
      norm[(static_cast<int64_t>(z) * m + i) * tiles + tile] = mx;
      sum[(static_cast<int64_t>(z) * m + i) * tiles + tile] = se;
    }
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
  constexpr int kGroups = kTile / 4 / 16;  // 16-landmark MFMA groups per wave

  // A operand: lane (li, grp) holds query li (zero rows past m), dims [32*ks + 8*grp, +8).
  u32x4 qf[4];
  const uint16_t* Az = A + (static_cast<int64_t>(z) * m + min(li, m - 1)) * kHeadDim + 8 * grp;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) qf[ks] = skv::load16_or_zero(Az + 32 * ks, li < m);
  // B operand: lane (li, grp) holds landmark wave*64 + 16*kg + li, same dims. All 16 loads are
  // issued before any is waited on.
  const uint16_t* Bz = B + static_cast<int64_t>(z) * n * kHeadDim + 8 * grp;
  u32x4 lf[kGroups][4];
#pragma unroll
  for (int kg = 0; kg < kGroups; ++kg) {
    const int j = tile * kTile + wave * (kTile / 4) + 16 * kg + li;
    const uint16_t* row = Bz + static_cast<int64_t>(min(j, n - 1)) * kHeadDim;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) lf[kg][ks] = skv::load16_or_zero(row + 32 * ks, j < n);
  }
#pragma unroll
  for (int kg = 0; kg < kGroups; ++kg) {
    f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, qf[ks]),
                                                  __builtin_bit_cast(bf16x8_t, lf[kg][ks]), d, 0, 0, 0);
    // D[query 4*grp + v][landmark li]
    const int jl = wave * (kTile / 4) + 16 * kg + li;
    const int j = tile * kTile + jl;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int i = 4 * grp + v;
      if (i < m && i < M) s_tile[i][jl] = (j < n) ? skv::bf2f(skv::f2bf(alpha * d[v])) : -INFINITY;
    }
  }
  __syncthreads();
  store_tile(s_tile, D, norm, sum, z, m, n, tile, tiles);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// acc + a.lo * b.lo + a.hi * b.hi over two bf16 pairs, fp32 accumulation (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc, false);
}

// DPP exchanges within a quad of lanes (quad_perm): the value of lane (l ^ 1), of lane (l ^ 2).
__device__ __forceinline__ float quad_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));
}
__device__ __forceinline__ float quad_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));
}

// Sums v[0, MP) over the 16 lanes of a DPP row (lane c = lane & 15). The exchanges with lane c ^ 1
// and then c ^ 2 each keep half of the values (the lane with the bit set keeps the upper half), so
// lane c is left with R = max(1, MP / 4) partial sums, of indices row_sum_base<MP>(c) + [0, R),
// over the lanes of its class c mod 4; rotations by 4 and 8 within the row add the class's four
// lanes. Every lane ends with its class's R totals in v[0, R).
template <int MP>
__device__ __forceinline__ void row_sums(float* v, int c) {
  if constexpr (MP >= 2) {
    constexpr int H = MP / 2;
    const bool up = (c & 1) != 0;
#pragma unroll
    for (int t = 0; t < H; ++t) {
      const float send = up ? v[t] : v[t + H];
      const float keep = up ? v[t + H] : v[t];
      v[t] = keep + quad_xor1(send);
    }
  } else {
    v[0] += quad_xor1(v[0]);
  }
  if constexpr (MP >= 4) {
    constexpr int H = MP / 4;
    const bool up = (c & 2) != 0;
#pragma unroll
    for (int t = 0; t < H; ++t) {
      const float send = up ? v[t] : v[t + H];
      const float keep = up ? v[t + H] : v[t];
      v[t] = keep + quad_xor2(send);
    }
  } else {
    v[0] += quad_xor2(v[0]);
  }
  constexpr int R = MP >= 4 ? MP / 4 : 1;
#pragma unroll
  for (int t = 0; t < R; ++t) {
    v[t] += skv::row_ror<4>(v[t]);
    v[t] += skv::row_ror<8>(v[t]);
  }
}
template <int MP>
__device__ __forceinline__ int row_sum_base(int c) {
  return (MP >= 2 ? (c & 1) * (MP / 2) : 0) + (MP >= 4 ? ((c >> 1) & 1) * (MP / 4) : 0);
}

// Few queries (m <= MP <= 4): the dots on the vector ALUs, so that every wave load covers whole
// landmark rows (the MFMA operand order splits each row's 256 bytes over four loads of 16 rows,
// which streams 5-10% slower). Workgroup = one 256-landmark tile of one z. Lane (r, c) =
// (lane >> 4, lane & 15) holds dims [8c, 8c + 8) of landmark 4u + r of its wave's 64 in wave load
// u = 0..15 (1 KB of consecutive bytes, non-temporal: the landmarks are read once), all 16 loads
// requested at entry; it sums its 8 products per query (four bf16 dot2 instructions, fp32
// accumulation), and the 16 lanes of a landmark meet in row_sums.
template <int MP>
__global__ void __launch_bounds__(kThreads) logits_rows_kernel(const uint16_t* __restrict__ A,
                                                               const uint16_t* __restrict__ B, uint16_t* __restrict__ D,
                                                               float* __restrict__ norm, float* __restrict__ sum, int m,
                                                               int n, float alpha, int tiles) {
  static_assert(MP == 1 || MP == 2 || MP == 4, "1, 2 or 4 queries per instance");
  constexpr int kWriters = MP;  // lanes c < MP of each landmark hold its MP sums, one each
  __shared__ float s_tile[MP][kTile];
  const int z = blockIdx.y;
  const int tile = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane >> 4;
  const int c = lane & 15;
  // Landmark rows past n (the last tile's) read row n - 1 instead; their logits are replaced by
  // -inf before any use.
  const u32x4* Bz = reinterpret_cast<const u32x4*>(B + static_cast<int64_t>(z) * n * kHeadDim) + c;
  const int jb = tile * kTile + wave * 64 + r;
  u32x4 lf[16];
  if (tile * kTile + kTile <= n) {
    const u32x4* p = Bz + static_cast<int64_t>(jb) * (kHeadDim / 8);
#pragma unroll
    for (int u = 0; u < 16; ++u) lf[u] = skv::load_nt(p + u * 4 * (kHeadDim / 8));
  } else {
#pragma unroll
    for (int u = 0; u < 16; ++u) lf[u] = skv::load_nt(Bz + static_cast<int64_t>(min(jb + 4 * u, n - 1)) * (kHeadDim / 8));
  }
  u32x4 qv[MP];  // dims [8c, 8c + 8) of each query, as bf16 pairs
  const uint16_t* Az = A + static_cast<int64_t>(z) * m * kHeadDim + 8 * c;
#pragma unroll
  for (int i = 0; i < MP; ++i) qv[i] = skv::load16_or_zero(Az + min(i, m - 1) * kHeadDim, i < m);
  const int base = row_sum_base<MP>(c);
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    float acc[MP];
#pragma unroll
    for (int i = 0; i < MP; ++i) {
      acc[i] = dot2(lf[u].x, qv[i].x, 0.f);
      acc[i] = dot2(lf[u].y, qv[i].y, acc[i]);
      acc[i] = dot2(lf[u].z, qv[i].z, acc[i]);
      acc[i] = dot2(lf[u].w, qv[i].w, acc[i]);
    }
    row_sums<MP>(acc, c);
    const int jl = wave * 64 + 4 * u + r;
    const int j = tile * kTile + jl;
    if (c < kWriters && base < m) s_tile[base][jl] = (j < n) ? skv::bf2f(skv::f2bf(alpha * acc[0])) : -INFINITY;
  }
  __syncthreads();
  store_tile(s_tile, D, norm, sum, z, m, n, tile, tiles);
}

template <bool kWriteSoftmax, bool kWriteMax>
__global__ void __launch_bounds__(kThreads) softmax_kernel(const uint16_t* __restrict__ D, const float* __restrict__ norm,
                                                           const float* __restrict__ sum, uint16_t* __restrict__ P,
                                                           uint16_t* __restrict__ out_max, int m, int n, int tiles) {
  __shared__ float gmax[kMaxM], ginv[kMaxM];
  const int z = blockIdx.y;
  const int tile = blockIdx.x;
  skv::merge_softmax_partials<kThreads / 64>(norm, sum, z, m, tiles, gmax, ginv);
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

// The same results for rows of n % 8 == 0 columns, each thread taking kCpt consecutive columns
// (8, 4 or 2: 16-, 8- or 4-byte vectors), chosen so that few rows still spread over many
// workgroups. Every D vector of the thread is requested at entry, before the partials merge, so
// their latencies overlap.
template <int kCpt>
struct ColVec;
template <>
struct ColVec<8> {
  using T = u32x4;
};
template <>
struct ColVec<4> {
  using T = uint32_t __attribute__((ext_vector_type(2)));
};
template <>
struct ColVec<2> {
  using T = uint32_t __attribute__((ext_vector_type(1)));
};

template <bool kWriteSoftmax, bool kWriteMax, int MP, int kCpt>
__global__ void __launch_bounds__(kThreads) softmax_vec_kernel(const uint16_t* __restrict__ D,
                                                               const float* __restrict__ norm,
                                                               const float* __restrict__ sum, uint16_t* __restrict__ P,
                                                               uint16_t* __restrict__ out_max, uint32_t* __restrict__ hist,
                                                               int m, int n, int tiles) {
  using V = typename ColVec<kCpt>::T;
  constexpr int kW = kCpt / 2;  // 32-bit words per vector
  __shared__ float gmax[kMaxM], ginv[kMaxM];
  __shared__ uint32_t lh[256];
  const int z = blockIdx.y;
  const int c0 = (blockIdx.x * kThreads + threadIdx.x) * kCpt;
  if (kWriteMax && hist) lh[threadIdx.x] = 0;  // kThreads == 256 bins; the merge's barrier orders it
  const bool live = c0 < n;  // n % 8 == 0: all kCpt columns live
  V dv[MP];
#pragma unroll
  for (int i = 0; i < MP; ++i) {
    dv[i] = V{};
    if (i < m && live) dv[i] = *reinterpret_cast<const V*>(D + (static_cast<int64_t>(z) * m + i) * n + c0);
  }
  skv::merge_softmax_partials<kThreads / 64>(norm, sum, z, m, tiles, gmax, ginv);
  __syncthreads();
  if (!live && !(kWriteMax && hist)) return;  // (with a histogram every thread reaches its barrier)
  float best[kCpt];
#pragma unroll
  for (int e = 0; e < kCpt; ++e) best[e] = -INFINITY;
#pragma unroll
  for (int i = 0; i < MP; ++i) {
    if (i >= m) continue;  // (not break: the loop must unroll fully so dv stays in registers)
    const float gm = gmax[i], gi = ginv[i];
    V pv;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      uint32_t pw = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint16_t x = static_cast<uint16_t>(h ? (dv[i][w] >> 16) : (dv[i][w] & 0xffffu));
        const uint16_t p = skv::f2bf(expf(skv::bf2f(x) - gm) * gi);
        best[2 * w + h] = fmaxf(best[2 * w + h], skv::bf2f(p));
        pw |= static_cast<uint32_t>(p) << (16 * h);
      }
      pv[w] = pw;
    }
    if (kWriteSoftmax && live) *reinterpret_cast<V*>(P + (static_cast<int64_t>(z) * m + i) * n + c0) = pv;
  }
  if (kWriteMax) {
    V mv;
#pragma unroll
    for (int w = 0; w < kW; ++w)
      mv[w] = static_cast<uint32_t>(skv::f2bf(best[2 * w])) | (static_cast<uint32_t>(skv::f2bf(best[2 * w + 1])) << 16);
    if (live) *reinterpret_cast<V*>(out_max + static_cast<int64_t>(z) * n + c0) = mv;
    if (hist) {
      // this workgroup's keys by high order-key byte; a thread's adjacent columns often share a
      // bin, so equal bins are added together
      if (live) {
        uint32_t run_bin = 0xffffffffu, run = 0;
#pragma unroll
        for (int e = 0; e < kCpt; ++e) {
          const uint32_t bin = skv::bf16_order_key(skv::f2bf(best[e])) >> 8;
          if (bin != run_bin) {
            if (run) atomicAdd(&lh[run_bin], run);
            run_bin = bin;
            run = 0;
          }
          ++run;
        }
        atomicAdd(&lh[run_bin], run);
      }
      __syncthreads();
      hist[(static_cast<int64_t>(z) * gridDim.x + blockIdx.x) * 256 + threadIdx.x] = lh[threadIdx.x];
    }
  }
}

int check_scoring_shape(const char* what, int batch_count, int m, int n, int k) {
  if (k != kHeadDim || m < 1 || m > kMaxM || n < 1 || batch_count < 1) {
    skv_set_error("%s: unsupported shape batch=%d m=%d n=%d k=%d (k must be 128, m in [1,16])", what, batch_count, m, n,
                  k);
    return SKV_EUNSUPPORTED;
  }
  return SKV_OK;
}

// Scoring kernel choice: logits_rows_kernel for m <= 4 queries over at least 1024 tiles in all,
// else logits_kernel (MFMA). Measured on MI355X, cold, rows vs MFMA: 32 x 4 x 15304 (the
// Llama-3-8B lane of 4 sequences) 23.7-24.4 vs 24.9 us, 64 x 4 x 15304 43.6-45.3 vs 48.3 us,
// 8 x 4 x 130680 47.3-50.3 vs 51.6 us; 16 x 4 x 15304 13.9 vs 14.1 us; 8 x 4 x 15304 8.7 vs
// 7.8 us; 8 x 8 x 15304 (twice the dot work per byte, fewer waves) 13.0 vs 8.3 us. Workgroups of
// 2-8 consecutive tiles (the next tile's loads requested before the current tile's dots) measured
// slower at every size. Environment SKV_SCORE_PATH=mfma / rows forces a kernel (rows only for
// m <= 4), read per call.
bool score_rows(int batch_count, int m, int tiles) {
  if (m > 4) return false;
  const char* e = getenv("SKV_SCORE_PATH");
  if (e && strcmp(e, "mfma") == 0) return false;
  if (e && strcmp(e, "rows") == 0) return true;
  return static_cast<int64_t>(tiles) * batch_count >= 1024;
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
  if (score_rows(batch_count, m, tiles)) {
    if (m == 1) hipLaunchKernelGGL(logits_rows_kernel<1>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
    else if (m == 2) hipLaunchKernelGGL(logits_rows_kernel<2>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
    else hipLaunchKernelGGL(logits_rows_kernel<4>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
    return skv_check_launch(what);
  }
  if (m == 1) hipLaunchKernelGGL(logits_kernel<1>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
  else if (m == 2) hipLaunchKernelGGL(logits_kernel<2>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
  else if (m <= 4) hipLaunchKernelGGL(logits_kernel<4>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
  else if (m <= 8) hipLaunchKernelGGL(logits_kernel<8>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
  else hipLaunchKernelGGL(logits_kernel<16>, grid, dim3(kThreads), 0, stream, A, B, D, norm, sum, m, n, alpha, tiles);
  return skv_check_launch(what);
}

// Columns per thread of the vector softmax: the widest vector that still gives >= 512 workgroups
// (2 per CU).
int softmax_cols_per_thread(int batch_count, int n) {
  int cpt = 8;
  while (cpt > 2 && static_cast<int64_t>(batch_count) * ((n + kThreads * cpt - 1) / (kThreads * cpt)) < 512) cpt /= 2;
  return cpt;
}

int launch_softmax(const char* what, const uint16_t* D, const float* norm, const float* sum, uint16_t* softmax,
                   uint16_t* out_max, int batch_count, int m, int n, hipStream_t stream, uint32_t* hist = nullptr) {
  if (!D || !norm || !sum || (!softmax && !out_max)) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  int rc = check_scoring_shape(what, batch_count, m, n, kHeadDim);
  if (rc) return rc;
  const int tiles = (n + kTile - 1) / kTile;
  const bool vec = n % 8 == 0 && ((reinterpret_cast<uintptr_t>(D) | reinterpret_cast<uintptr_t>(softmax) |
                                   reinterpret_cast<uintptr_t>(out_max)) & 15u) == 0;
  if (vec) {
    const int cpt = softmax_cols_per_thread(batch_count, n);
    auto go = [&](auto mp, auto cp) {
      constexpr int MP = decltype(mp)::value;
      constexpr int C = decltype(cp)::value;
      const dim3 vgrid((n + kThreads * C - 1) / (kThreads * C), batch_count);
      if (softmax && out_max)
        hipLaunchKernelGGL((softmax_vec_kernel<true, true, MP, C>), vgrid, dim3(kThreads), 0, stream, D, norm, sum,
                           softmax, out_max, nullptr, m, n, tiles);
      else if (softmax)
        hipLaunchKernelGGL((softmax_vec_kernel<true, false, MP, C>), vgrid, dim3(kThreads), 0, stream, D, norm, sum,
                           softmax, out_max, nullptr, m, n, tiles);
      else
        hipLaunchKernelGGL((softmax_vec_kernel<false, true, MP, C>), vgrid, dim3(kThreads), 0, stream, D, norm, sum,
                           softmax, out_max, hist, m, n, tiles);
    };
    auto by_cols = [&](auto mp) {
      if (cpt == 8) go(mp, std::integral_constant<int, 8>{});
      else if (cpt == 4) go(mp, std::integral_constant<int, 4>{});
      else go(mp, std::integral_constant<int, 2>{});
    };
    if (m <= 4) by_cols(std::integral_constant<int, 4>{});
    else if (m <= 8) by_cols(std::integral_constant<int, 8>{});
    else by_cols(std::integral_constant<int, 16>{});
    return skv_check_launch(what);
  }
  if (hist) {
    skv_set_error("%s: key histograms need n %% 8 == 0 and 16-byte aligned buffers", what);
    return SKV_EINVAL;
  }
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

namespace skv {

int softmax_hist_parts(int rows, int n) {
  if (rows < 1 || n < 8 || n % 8) return 0;
  const int cpt = softmax_cols_per_thread(rows, n);
  return (n + kThreads * cpt - 1) / (kThreads * cpt);
}

int softmax_keys_hist(const uint16_t* D, const float* norm, const float* sum, uint16_t* out_max, uint32_t* hist,
                      int rows, int m, int n, hipStream_t stream) {
  return launch_softmax("softmax_keys_hist", D, norm, sum, nullptr, out_max, rows, m, n, stream, hist);
}

}  // namespace skv
