// Skinny bf16 linear layer of the decode step: y[m, n] = bf16(sum_k x[m, k] * w[n, k]) for the
// few token rows m of one decode step (M <= 16) against a row-major weight [N, K] — the
// decoding model's projections (F.linear on wqkv, wo, gate_up_proj, down_proj and the lm head,
// models/llama.py:192,203,208,214 and the lm head at models/base.py:98).
//
// At M <= 16 the call is bound by reading the weight once from HBM (2*N*K bytes), so the kernel
// is laid out for the load path, not for the matrix cores: every wave load reads 1 KB of ONE
// weight row (64 lanes x 16 B, fully coalesced), and the arithmetic runs on the VALU as bf16 dot2
// with fp32 accumulation (v_dot2c_f32_bf16), which needs no operand shuffles. A workgroup owns R
// weight rows; its waves split K into 512-element blocks (wave w takes blocks w, w+nw, ...) with
// the next block's loads in flight while the current one is multiplied. The per-lane partial
// sums are folded within 16-lane rows by a DPP transpose-reduce (each step halves the values a
// lane holds), then summed across rows and waves in LDS; one rounding to bf16 at the end.
//
// The QKV projection with the new token's RoPE and KV append in its epilogue
// (skv_linear_qkv_rope_append): a workgroup's 8 output rows lie in one head, and with the
// half-split heads' q/k weight rows interleaved (dims d and d + 64 adjacent; GLM's rotation pairs
// are adjacent already) every rotation pair of the workgroup is in it. The workgroup rounds its
// sums to bf16, rotates them with the bf16 per-op rounding of skv_rope_qk_append and writes q to
// q_out and k, v to the append row of the key/value buffers: bit-identical to skv_linear followed
// by skv_rope_qk_append, one launch and the fused row's round trip fewer. The position and
// cos/sin loads are issued before the weight stream starts.
#include "rope_math.h"
#include "skv_common.h"

namespace {

using skv::u32x4;

constexpr int kBlockK = 512;     // k elements per wave load (64 lanes x 8)
constexpr int kMaxWaves = 8;     // workgroup size limit (2 waves per SIMD at 256 VGPRs)
constexpr int kHeadDim = 128;

enum RopeMode { kNoRope = 0, kRopeHalf = 1, kRopeGlm = 2 };

// Epilogue operands: an optional bias added to the fp32 sums before the one bf16 rounding (the
// reference's F.linear(x, w, b), models/glm.py:165), and the RoPE + append epilogue's operands
// (skv_rope_qk_append's, for the fused row of Hq q heads, Hkv k heads and Hkv v heads).
struct RopeEpi {
  const uint16_t* bias;  // [N] or null
  int Hq, Hkv;
  const int64_t* pos;  // [M] positions
  const uint16_t* cs;
  int64_t cs_stride, cs_rows;
  uint16_t* q_out;
  int64_t qo_sb;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t kv_sb, kv_sh, kv_ss;
  const int64_t* row_dev;  // the append row
  int64_t buf_len;
};

// Output dims of rotation pair `p` (rows 2p, 2p + 1 of a workgroup starting at row n0) and whether
// it is rotated: half-split q/k heads hold dims (j/2, 64 + j/2) in row order j (interleaved
// weight), v heads and GLM heads dims (j, j + 1); GLM rotates only dims below 64.
template <int kRope>
__device__ __forceinline__ void rope_pair_dims(const RopeEpi& re, int n1, int& head, int& d1, int& d2, int& kind,
                                               int& ci) {
  head = n1 / kHeadDim;
  const int j = n1 - head * kHeadDim;  // even
  kind = head < re.Hq ? 0 : head < re.Hq + re.Hkv ? 1 : 2;  // q, k, v
  if (kRope == kRopeHalf && kind < 2) {
    d1 = j / 2;
    d2 = 64 + j / 2;
    ci = d1;  // cos at [d1], sin at [d1 + 64]
  } else {
    d1 = j;
    d2 = j + 1;
    ci = (kRope == kRopeGlm && kind < 2 && j < 64) ? j / 2 : -1;  // cos at [j/2], sin at [j/2 + 32]
  }
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// One transpose-reduce step over the lane bit that the DPP pattern CTRL flips: lanes with the
// bit set keep the upper half of their C values, the others the lower half, and each adds the
// partner's copy of the half it keeps.
template <int C, int CTRL>
__device__ __forceinline__ void fold(float* v, bool upper) {
#pragma unroll
  for (int j = 0; j < C / 2; ++j) {
    const float keep = upper ? v[C / 2 + j] : v[j];
    const float send = upper ? v[j] : v[C / 2 + j];
    v[j] = keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), CTRL, 0xf, 0xf, false));
  }
}

// bf16 pair of silu(g) * u from the bf16 pairs g2, u2 (element 0 in the low half), with the
// arithmetic and roundings of the SiLU-and-mul kernel (skv::silu_mul, then one bf16 rounding).
__device__ __forceinline__ uint32_t silu_mul2(uint32_t g2, uint32_t u2) {
  return skv::f2bf2(skv::silu_mul(skv::bf_lo(g2), skv::bf_lo(u2)), skv::silu_mul(skv::bf_hi(g2), skv::bf_hi(u2)));
}

// kGated: x rows hold [gate (K) | up (K)] and the multiplied row is silu(gate) * up, formed from
// the two halves as they are loaded (the down projection reading the gate/up projection's output).
// kAct: the weight rows are (gate, up) pairs, row 2j the gate and row 2j + 1 the up projection of
// output j, and the workgroup writes y[:, j] = bf16(silu(bf16(g)) * bf16(u)) for its R / 2 pairs
// (the gate/up projection with the SiLU-and-mul in its epilogue: no [gate | up] round trip).
// kRope (kRopeHalf / kRopeGlm): the RoPE + append epilogue; y is not written.
template <int R, int MP, bool kGated, bool kAct = false, int kRope = kNoRope>
__global__ void __launch_bounds__(kMaxWaves * 64) linear_kernel(const uint16_t* __restrict__ x, int64_t xs,
                                                               const uint16_t* __restrict__ w, int64_t ws,
                                                               uint16_t* __restrict__ y, int64_t ys, int M, int N,
                                                               int K, RopeEpi re) {
  constexpr int V = R * MP;  // partial sums per lane
  static_assert(V >= 16 && V <= 64 && (V & (V - 1)) == 0, "R * MP must be 16, 32 or 64");
  static_assert(!(kGated && kAct) && (!kAct || R % 2 == 0), "gate/up pairs need an even row count");
  static_assert(kRope == kNoRope || (!kGated && !kAct && R % 2 == 0 && kHeadDim % R == 0),
                "the RoPE epilogue takes whole rotation pairs of one head per workgroup");
  constexpr bool kFin = kAct || kRope != kNoRope;
  __shared__ float red[kMaxWaves * 4 * V];
  __shared__ float fin[kFin ? V : 1];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar loop control
  const int nw = blockDim.x >> 6;
  const int n0 = blockIdx.x * R;
  const int nblk = (K + kBlockK - 1) / kBlockK;

  // Row bases are wave-uniform (scalar registers); the lane's 32-bit byte offset is added per
  // load, so the loads take the scalar-base + vector-offset form.
  const char* wr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wr[r] = reinterpret_cast<const char*>(w + static_cast<int64_t>(min(n0 + r, N - 1)) * ws);
  const char* xr[MP];
#pragma unroll
  for (int m = 0; m < MP; ++m) xr[m] = reinterpret_cast<const char*>(x + static_cast<int64_t>(min(m, M - 1)) * xs);

  float acc[R][MP];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MP; ++m) acc[r][m] = 0.f;

  // Block b's operands: lane k offset b*512 + 8*lane. A lane past K (only in a last, partial
  // block) reads the row's first 16 bytes instead (valid for any K >= 8), and mac() zeroes its x,
  // so it adds 0. The select sits at the use, not at the load, so a prefetch never has to wait
  // for its own data.
  auto load = [&](int b, u32x4* wv, u32x4* xv, u32x4* xu) {
    const int k = b * kBlockK + 8 * lane;
    const uint32_t boff = 2u * static_cast<uint32_t>(k < K ? k : 0);
#pragma unroll
    for (int r = 0; r < R; ++r) wv[r] = skv::load_nt(reinterpret_cast<const u32x4*>(wr[r] + boff));
#pragma unroll
    for (int m = 0; m < MP; ++m) {
      xv[m] = *reinterpret_cast<const u32x4*>(xr[m] + boff);
      if (kGated) xu[m] = *reinterpret_cast<const u32x4*>(xr[m] + boff + 2u * static_cast<uint32_t>(K));
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the multiply that follows
  };
  auto mac = [&](int b, const u32x4* wv, const u32x4* xv, const u32x4* xu) {
    const bool ok = b * kBlockK + 8 * lane < K;
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int m = 0; m < MP; ++m) {
        const uint32_t xe = ok ? (kGated ? silu_mul2(xv[m][e], xu[m][e]) : xv[m][e]) : 0u;
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][m] = dot2(wv[r][e], xe, acc[r][m]);
      }
  };

  // The wave's blocks are b_j = wave + j*nw, j < nb. Two register sets alternate; inside the
  // loop every prefetch is unconditional, so the compiler's wait before each multiply covers only
  // that block's loads (a conditional prefetch would make it wait for both sets).
  const int nb = wave < nblk ? (nblk - 1 - wave) / nw + 1 : 0;  // wave-uniform
  u32x4 wa[R], xa[MP], ua[MP], wb[R], xb[MP], ub[MP];
  // RoPE epilogue thread t < (R/2)*MP takes pair p = t / MP of token row m = t % MP: its position
  // and append row are requested first, its cos/sin after the first weight block (so the wait for
  // the position leaves the weight loads in flight).
  int64_t rp_pos = -1, rp_row = -1;
  uint16_t rp_c = 0, rp_s = 0;
  const int et = threadIdx.x;
  // The bias of the sum this thread finishes (thread t < R*MP: row t / MP), requested up front.
  float bias_v = 0.f;
  if (re.bias && et < V && n0 + et / MP < N) bias_v = skv::bf2f(re.bias[n0 + et / MP]);
  if constexpr (kRope != kNoRope) {
    if (et < (R / 2) * MP && et % MP < M) {
      rp_pos = re.pos[et % MP];
      rp_row = *re.row_dev;
    }
  }
  if (nb > 0) load(wave, wa, xa, ua);
  if constexpr (kRope != kNoRope) {
    if (et < (R / 2) * MP && et % MP < M) {
      int head, d1, d2, kind, ci;
      rope_pair_dims<kRope>(re, n0 + 2 * (et / MP), head, d1, d2, kind, ci);
      if (ci >= 0 && rp_pos >= 0 && rp_pos < re.cs_rows) {
        const uint16_t* c = re.cs + rp_pos * re.cs_stride;
        rp_c = c[ci];
        rp_s = c[ci + (kRope == kRopeHalf ? 64 : 32)];
      }
    }
  }
  if (nb > 0) {
    int b = wave, i = 1;  // set a holds block b = b_{i-1}; b_i is the next block to load
    for (; i + 1 < nb; i += 2, b += 2 * nw) {
      load(b + nw, wb, xb, ub);
      mac(b, wa, xa, ua);
      load(b + 2 * nw, wa, xa, ua);
      mac(b + nw, wb, xb, ub);
    }
    if (i < nb) {
      load(b + nw, wb, xb, ub);
      mac(b, wa, xa, ua);
      mac(b + nw, wb, xb, ub);
    } else {
      mac(b, wa, xa, ua);
    }
  }

  // Fold the R*MP partial sums within each 16-lane row: bit 3 of the lane (row_mirror), bit 2
  // (row_half_mirror), bit 1 (quad_perm 3,2,1,0), bit 0 (quad_perm 1,0,3,2). Lane p of a row then
  // holds values p*V/16 .. p*V/16 + V/16 - 1 of the flattened [R][MP] array, summed over the row.
  float v[V];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MP; ++m) v[r * MP + m] = acc[r][m];
  const int p = lane & 15;
  fold<V, 0x140>(v, p & 8);
  fold<V / 2, 0x141>(v, p & 4);
  fold<V / 4, 0x1B>(v, p & 2);
  fold<V / 8, 0xB1>(v, p & 1);
  constexpr int kPer = V / 16;
  float* dst = red + (wave * 4 + (lane >> 4)) * V + p * kPer;
#pragma unroll
  for (int j = 0; j < kPer; ++j) dst[j] = v[j];
  __syncthreads();
  if (static_cast<int>(threadIdx.x) < V) {
    const int t = threadIdx.x;
    float s = 0.f;
    for (int i = 0; i < nw * 4; ++i) s += red[i * V + t];
    const int r = t / MP, m = t % MP;
    if (re.bias) s += bias_v;  // (uniform: without a bias no add, so -0 sums stay -0)
    if (kFin) fin[t] = s;
    else if (m < M && n0 + r < N) y[static_cast<int64_t>(m) * ys + n0 + r] = skv::f2bf(s);
  }
  if constexpr (kRope != kNoRope) {
    __syncthreads();
    if (et < (R / 2) * MP && et % MP < M) {
      const int p = et / MP, m = et % MP;
      int head, d1, d2, kind, ci;
      rope_pair_dims<kRope>(re, n0 + 2 * p, head, d1, d2, kind, ci);
      const uint16_t x1 = skv::f2bf(fin[(2 * p) * MP + m]), x2 = skv::f2bf(fin[(2 * p + 1) * MP + m]);
      uint16_t y1 = x1, y2 = x2;
      if (ci >= 0 && rp_pos >= 0 && rp_pos < re.cs_rows) skv::rope_half_split(x1, x2, rp_c, rp_s, y1, y2);
      uint16_t* dst = nullptr;
      if (kind == 0) {
        dst = re.q_out + m * re.qo_sb + static_cast<int64_t>(head) * kHeadDim;
      } else if (rp_row >= 0 && rp_row < re.buf_len) {  // beyond the buffer: nothing appended
        const int h = kind == 1 ? head - re.Hq : head - re.Hq - re.Hkv;
        dst = (kind == 1 ? re.k_cache : re.v_cache) + m * re.kv_sb + h * re.kv_sh + rp_row * re.kv_ss;
      }
      if (dst) {
        dst[d1] = y1;
        dst[d2] = y2;
      }
    }
  }
  if (kAct) {
    __syncthreads();
    if (static_cast<int>(threadIdx.x) < V / 2) {
      const int t = threadIdx.x;
      const int r = 2 * (t / MP), m = t % MP;  // gate row r, up row r + 1 of this workgroup
      if (m < M && n0 + r + 1 < N) {
        const float g = skv::bround(fin[r * MP + m]), u = skv::bround(fin[(r + 1) * MP + m]);
        y[static_cast<int64_t>(m) * ys + (n0 + r) / 2] = skv::f2bf(skv::silu_mul(g, u));
      }
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int g_waves_override = -1;  // SKV_LINEAR_WAVES, read once

template <int R, int MP, bool kGated, bool kAct = false, int kRope = kNoRope>
void launch(const uint16_t* x, int64_t xs, const uint16_t* w, int64_t ws, uint16_t* y, int64_t ys, int M, int N, int K,
            hipStream_t s, const RopeEpi& re = RopeEpi{}) {
  const int groups = (N + R - 1) / R;
  const int nblk = (K + kBlockK - 1) / kBlockK;
  // Waves per workgroup, from sweeps of the Llama-3-8B projections and lm head on MI355X with
  // cold weights: at up to 4 rows four waves win on every shape; at 8 rows (twice the
  // registers, half the resident waves) four win on the 4096-row weights, one on wider ones,
  // two on the vocabulary-sized head. At most one wave per k block.
  int nw = MP <= 4 ? 4 : groups <= 512 ? 4 : groups >= 8192 ? 2 : 1;
  if (g_waves_override > 0) nw = g_waves_override;
  while (nw > 1 && nw > nblk) nw /= 2;
  hipLaunchKernelGGL((linear_kernel<R, MP, kGated, kAct, kRope>), dim3(groups), dim3(64 * nw), 0, s, x, xs, w, ws, y,
                     ys, M, N, K, re);
}

template <bool kGated, bool kAct = false>
int linear_impl(const char* what, const uint16_t* x, int64_t x_stride, const uint16_t* weight, int64_t weight_stride,
                uint16_t* y, int64_t y_stride, int m, int n, int k, void* stream, const uint16_t* bias = nullptr) {
  if (!x || !weight || !y) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  // The gated form recomputes the activations of its rows in every workgroup, and its 8- and
  // 16-row variants would hold two more sets of x registers: it is offered up to 4 rows only.
  constexpr int kMaxRows = kGated ? 4 : 16;
  if (m < 1 || m > kMaxRows || n < 1 || k < 8 || k % 8) {
    skv_set_error("%s: m=%d n=%d k=%d (1 <= m <= %d, k a multiple of 8)", what, m, n, k, kMaxRows);
    return SKV_EUNSUPPORTED;
  }
  if (kAct && n % 2) {
    skv_set_error("%s: n=%d weight rows do not form (gate, up) pairs", what, n);
    return SKV_EINVAL;
  }
  const int64_t x_need = kGated ? 2 * static_cast<int64_t>(k) : k;
  if (!aligned16(x) || !aligned16(weight) || x_stride % 8 || weight_stride % 8 || x_stride < x_need ||
      weight_stride < k || y_stride < (kAct ? n / 2 : n)) {
    skv_set_error("%s: x and weight rows must be 16-byte aligned and hold %lld and k elements", what,
                  (long long)x_need);
    return SKV_EINVAL;
  }
  if (g_waves_override < 0) {
    const char* e = getenv("SKV_LINEAR_WAVES");
    const int v = e ? atoi(e) : 0;
    g_waves_override = (v == 1 || v == 2 || v == 4 || v == 8) ? v : 0;
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  RopeEpi re{};
  re.bias = bias;
  if (m == 1)
    launch<16, 1, kGated, kAct>(x, x_stride, weight, weight_stride, y, y_stride, m, n, k, s, re);
  else if (m == 2)
    launch<8, 2, kGated, kAct>(x, x_stride, weight, weight_stride, y, y_stride, m, n, k, s, re);
  else if (m <= 4)
    launch<8, 4, kGated, kAct>(x, x_stride, weight, weight_stride, y, y_stride, m, n, k, s, re);
  else if constexpr (!kGated) {
    if (m <= 8)
      launch<8, 8, false, kAct>(x, x_stride, weight, weight_stride, y, y_stride, m, n, k, s, re);
    else
      launch<2, 16, false, kAct>(x, x_stride, weight, weight_stride, y, y_stride, m, n, k, s, re);
  }
  return skv_check_launch(what);
}

}  // namespace

extern "C" int skv_linear(const uint16_t* x, int64_t x_stride, const uint16_t* weight, int64_t weight_stride,
                          uint16_t* y, int64_t y_stride, int m, int n, int k, void* stream) {
  return linear_impl<false>("linear", x, x_stride, weight, weight_stride, y, y_stride, m, n, k, stream);
}

extern "C" int skv_linear_bias(const uint16_t* x, int64_t x_stride, const uint16_t* weight, int64_t weight_stride,
                               const uint16_t* bias, uint16_t* y, int64_t y_stride, int m, int n, int k,
                               void* stream) {
  if (!bias) {
    skv_set_error("linear_bias: null bias");
    return SKV_EINVAL;
  }
  return linear_impl<false>("linear_bias", x, x_stride, weight, weight_stride, y, y_stride, m, n, k, stream, bias);
}

extern "C" int skv_linear_silu_mul(const uint16_t* x, int64_t x_stride, const uint16_t* weight,
                                   int64_t weight_stride, uint16_t* y, int64_t y_stride, int m, int n, int k,
                                   void* stream) {
  return linear_impl<true>("linear_silu_mul", x, x_stride, weight, weight_stride, y, y_stride, m, n, k, stream);
}

extern "C" int skv_linear_gate_up_silu(const uint16_t* x, int64_t x_stride, const uint16_t* weight,
                                       int64_t weight_stride, uint16_t* y, int64_t y_stride, int m, int n, int k,
                                       void* stream) {
  return linear_impl<false, true>("linear_gate_up_silu", x, x_stride, weight, weight_stride, y, y_stride, m, n, k,
                                  stream);
}

namespace {

template <int kRope>
void launch_qkv_rope(const uint16_t* x, int64_t xs, const uint16_t* w, int64_t ws, int m, int n, int k, hipStream_t s,
                     const RopeEpi& re) {
  if (m == 1) launch<16, 1, false, false, kRope>(x, xs, w, ws, nullptr, 0, m, n, k, s, re);
  else if (m == 2) launch<8, 2, false, false, kRope>(x, xs, w, ws, nullptr, 0, m, n, k, s, re);
  else if (m <= 4) launch<8, 4, false, false, kRope>(x, xs, w, ws, nullptr, 0, m, n, k, s, re);
  else launch<8, 8, false, false, kRope>(x, xs, w, ws, nullptr, 0, m, n, k, s, re);
}

}  // namespace

extern "C" int skv_linear_qkv_rope_append(const uint16_t* x, int64_t x_stride, const uint16_t* weight,
                                          int64_t weight_stride, const uint16_t* bias, int m, int k, int q_heads,
                                          int kv_heads,
                                          const int64_t* positions, const uint16_t* cos_sin, int64_t stride_cos_sin,
                                          int64_t cos_sin_rows, int rope_mode, uint16_t* q_out,
                                          int64_t q_out_stride_b, uint16_t* k_cache, uint16_t* v_cache,
                                          int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_s,
                                          const int64_t* append_row, int64_t buf_len, void* stream) {
  const char* what = "linear_qkv_rope_append";
  if (!x || !weight || !positions || !cos_sin || !q_out || !k_cache || !v_cache || !append_row) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (m < 1 || m > 8 || k < 8 || k % 8 || q_heads < 1 || kv_heads < 1 || (rope_mode != 0 && rope_mode != 1)) {
    skv_set_error("%s: m=%d (1..8) k=%d (a multiple of 8) q_heads=%d kv_heads=%d rope_mode=%d", what, m, k, q_heads,
                  kv_heads, rope_mode);
    return SKV_EUNSUPPORTED;
  }
  if (!aligned16(x) || !aligned16(weight) || x_stride % 8 || weight_stride % 8 || x_stride < k || weight_stride < k) {
    skv_set_error("%s: x and weight rows must be 16-byte aligned and hold k elements", what);
    return SKV_EINVAL;
  }
  if (q_out_stride_b < static_cast<int64_t>(q_heads) * kHeadDim || kv_stride_s < kHeadDim || buf_len < 0) {
    skv_set_error("%s: q_out rows of %lld elements (%d heads of 128 needed), key/value rows of %lld", what,
                  (long long)q_out_stride_b, q_heads, (long long)kv_stride_s);
    return SKV_EINVAL;
  }
  const int n = (q_heads + 2 * kv_heads) * kHeadDim;
  RopeEpi re{bias, q_heads, kv_heads, positions, cos_sin, stride_cos_sin, cos_sin_rows, q_out, q_out_stride_b,
             k_cache, v_cache, kv_stride_b, kv_stride_h, kv_stride_s, append_row, buf_len};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (rope_mode == 0) launch_qkv_rope<kRopeHalf>(x, x_stride, weight, weight_stride, m, n, k, s, re);
  else launch_qkv_rope<kRopeGlm>(x, x_stride, weight, weight_stride, m, n, k, s, re);
  return skv_check_launch(what);
}
