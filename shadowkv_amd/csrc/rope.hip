// a7: rotary position embedding with per-op bf16 rounding, standalone entry points.
//
// The math of every variant is the reference's (kernels/rope_new.cu:49-56, 262-269, 354-371):
//   y1 = bf16(bf16(x1*cos) + bf16(-x2*sin)),  y2 = bf16(bf16(x2*cos) + bf16(x1*sin)),
// which is also torch's `(x*cos) + (rotate_half(x)*sin)` on bf16 tensors
// (models/tensor_op.py:132-156). One thread computes one rotation pair.
#include "rope_math.h"

namespace {

constexpr int kThreads = 256;

// output[b,h,s] = rope(x[b,h,s], cos_sin[position_ids[b,h,s]]); half-split layout.
__global__ void __launch_bounds__(kThreads) rope_plain_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ cs,
                                                              const int64_t* __restrict__ pid, uint16_t* __restrict__ out,
                                                              int heads, int seq_len, int half, int64_t sxb, int64_t sxh,
                                                              int64_t sxs, int64_t sxe, int64_t scs, int64_t spb,
                                                              int64_t sph, int64_t sps, int64_t cs_rows, int64_t total) {
  int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= total) return;
  const int d = static_cast<int>(g % half);
  int64_t row = g / half;
  const int s = static_cast<int>(row % seq_len);
  row /= seq_len;
  const int h = static_cast<int>(row % heads);
  const int b = static_cast<int>(row / heads);
  const int64_t p = pid[b * spb + h * sph + s * sps];
  if (p < 0 || p >= cs_rows) return;  // positions outside the table leave the row unwritten
  const uint16_t* c = cs + p * scs;
  const int64_t xo = b * sxb + h * sxh + s * sxs;
  uint16_t y1, y2;
  skv::rope_half_split(x[xo + d * sxe], x[xo + (d + half) * sxe], c[d], c[d + half], y1, y2);
  out[xo + d * sxe] = y1;
  out[xo + (d + half) * sxe] = y2;
}

// Two-table variant (kernels/rope.cu:26-62): output[b,h,s] from separate cos and sin rows of
// position_ids[b,h,s], the first half rotated with cos[d], sin[d] and the second with
// cos[d + half], sin[d + half] (equal halves in the usual tables, but taken as stored).
__global__ void __launch_bounds__(kThreads) rope_two_table_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ cosp, const uint16_t* __restrict__ sinp,
    const int64_t* __restrict__ pid, uint16_t* __restrict__ out, int heads, int seq_len, int half, int64_t sxb,
    int64_t sxh, int64_t sxs, int64_t sxe, int64_t sc, int64_t ss, int64_t spb, int64_t sph, int64_t sps,
    int64_t rows, int64_t total) {
  int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= total) return;
  const int d = static_cast<int>(g % half);
  int64_t row = g / half;
  const int s = static_cast<int>(row % seq_len);
  row /= seq_len;
  const int h = static_cast<int>(row % heads);
  const int b = static_cast<int>(row / heads);
  const int64_t p = pid[b * spb + h * sph + s * sps];
  if (p < 0 || p >= rows) return;  // positions outside the tables leave the row unwritten
  const uint16_t* c = cosp + p * sc;
  const uint16_t* sn = sinp + p * ss;
  const int64_t xo = b * sxb + h * sxh + s * sxs;
  const uint16_t x1 = x[xo + d * sxe], x2 = x[xo + (d + half) * sxe];
  out[xo + d * sxe] = skv::badd(skv::bmul(x1, c[d]), skv::bmul(skv::bneg(x2), sn[d]));
  out[xo + (d + half) * sxe] = skv::badd(skv::bmul(x2, c[d + half]), skv::bmul(x1, sn[d + half]));
}

// Push variant: rows of hit chunks (s/chunk < cnt) and rows past `end` are skipped; cnts null:
// no hit rows (every row is rotated).
template <bool kGlm>
__global__ void __launch_bounds__(kThreads) rope_push_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ cs,
                                                             const int32_t* __restrict__ pid, uint16_t* __restrict__ out,
                                                             const int32_t* __restrict__ cnts, int heads, int seq_len, int half,
                                                             int64_t sxb, int64_t sxh, int64_t sxs, int64_t scs, int64_t spb,
                                                             int64_t sph, int64_t sps, int64_t sob, int64_t soh, int64_t sos,
                                                             int start, int end, int chunk, int64_t cs_rows, int64_t total) {
  int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= total) return;
  const int d = static_cast<int>(g % half);
  int64_t row = g / half;
  const int s = static_cast<int>(row % seq_len);
  row /= seq_len;
  const int h = static_cast<int>(row % heads);
  const int b = static_cast<int>(row / heads);
  if (cnts && s / chunk < cnts[b * heads + h]) return;
  if (start + s >= end) return;
  const int64_t p = static_cast<int64_t>(pid[b * spb + h * sph + (s / chunk) * sps]) * chunk + s % chunk;
  if (p < 0 || p >= cs_rows) return;  // positions outside the table leave the row unwritten
  const uint16_t* c = cs + p * scs;
  const uint16_t* xr = x + b * sxb + h * sxh + s * sxs;
  uint16_t* o = out + b * sob + h * soh + static_cast<int64_t>(start + s) * sos;
  if (!kGlm) {
    uint16_t y1, y2;
    skv::rope_half_split(xr[d], xr[d + half], c[d], c[d + half], y1, y2);
    o[d] = y1;
    o[d + half] = y2;
  } else {
    // half == 64: threads d < 32 rotate the interleaved pair (2d, 2d+1) with [cos(32)|sin(32)];
    // threads 32..63 copy dims d+32 and d+64, i.e. 64..127 unchanged.
    if (d < 32) {
      uint16_t y1, y2;
      skv::rope_half_split(xr[2 * d], xr[2 * d + 1], c[d], c[d + 32], y1, y2);
      o[2 * d] = y1;
      o[2 * d + 1] = y2;
    } else {
      o[d + 32] = xr[d + 32];
      o[d + 64] = xr[d + 64];
    }
  }
}

int launch_push(bool glm, const uint16_t* x, const uint16_t* cos_sin, const int32_t* position_ids, uint16_t* output,
                const int32_t* cnts, int batch_size, int heads, int seq_len, int embed_dim, int64_t stride_xb,
                int64_t stride_xh, int64_t stride_xs, int64_t stride_xe, int64_t stride_cos_sin, int64_t stride_pid_b,
                int64_t stride_pid_h, int64_t stride_pid_s, int64_t stride_output_b, int64_t stride_output_h,
                int64_t stride_output_s, int start, int end, int half_dim, int chunk_size, int64_t cos_sin_rows,
                void* stream, const char* what = nullptr, bool cnts_optional = false) {
  if (!what) what = glm ? "apply_rotary_pos_emb_push_cache_opt_glm" : "apply_rotary_pos_emb_push_cache_opt";
  if (!x || !cos_sin || !position_ids || !output || (!cnts && !cnts_optional)) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (batch_size <= 0 || heads <= 0 || seq_len <= 0 || chunk_size <= 0 || half_dim <= 0 ||
      embed_dim != 2 * half_dim || stride_xe != 1) {
    skv_set_error("%s: invalid shape (batch=%d heads=%d seq=%d embed=%d half=%d chunk=%d stride_xe=%lld)", what,
                  batch_size, heads, seq_len, embed_dim, half_dim, chunk_size, (long long)stride_xe);
    return SKV_EINVAL;
  }
  if (glm && half_dim != 64) {
    skv_set_error("%s: the GLM layout needs half_dim == 64, got %d", what, half_dim);
    return SKV_EUNSUPPORTED;
  }
  const int64_t total = static_cast<int64_t>(batch_size) * heads * seq_len * half_dim;
  const dim3 grid(static_cast<unsigned>((total + kThreads - 1) / kThreads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (glm)
    hipLaunchKernelGGL(rope_push_kernel<true>, grid, dim3(kThreads), 0, s, x, cos_sin, position_ids, output, cnts, heads,
                       seq_len, half_dim, stride_xb, stride_xh, stride_xs, stride_cos_sin, stride_pid_b, stride_pid_h,
                       stride_pid_s, stride_output_b, stride_output_h, stride_output_s, start, end, chunk_size,
                       cos_sin_rows, total);
  else
    hipLaunchKernelGGL(rope_push_kernel<false>, grid, dim3(kThreads), 0, s, x, cos_sin, position_ids, output, cnts, heads,
                       seq_len, half_dim, stride_xb, stride_xh, stride_xs, stride_cos_sin, stride_pid_b, stride_pid_h,
                       stride_pid_s, stride_output_b, stride_output_h, stride_output_s, start, end, chunk_size,
                       cos_sin_rows, total);
  return skv_check_launch(what);
}

}  // namespace

extern "C" int skv_apply_rotary_pos_emb_new(const uint16_t* x, const uint16_t* cos_sin, const int64_t* position_ids,
                                            uint16_t* output, int batch_size, int heads, int seq_len, int embed_dim,
                                            int64_t stride_xb, int64_t stride_xh, int64_t stride_xs, int64_t stride_xe,
                                            int64_t stride_cos_sin, int64_t stride_pid_b, int64_t stride_pid_h,
                                            int64_t stride_pid_s, int half_dim, int64_t cos_sin_rows, void* stream) {
  const char* what = "apply_rotary_pos_emb_new";
  if (!x || !cos_sin || !position_ids || !output) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (batch_size <= 0 || heads <= 0 || seq_len <= 0 || half_dim <= 0 || embed_dim != 2 * half_dim) {
    skv_set_error("%s: invalid shape (batch=%d heads=%d seq=%d embed=%d half=%d)", what, batch_size, heads, seq_len,
                  embed_dim, half_dim);
    return SKV_EINVAL;
  }
  const int64_t total = static_cast<int64_t>(batch_size) * heads * seq_len * half_dim;
  hipLaunchKernelGGL(rope_plain_kernel, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), x, cos_sin, position_ids, output, heads, seq_len, half_dim,
                     stride_xb, stride_xh, stride_xs, stride_xe, stride_cos_sin, stride_pid_b, stride_pid_h, stride_pid_s,
                     cos_sin_rows, total);
  return skv_check_launch(what);
}

extern "C" int skv_apply_rotary_pos_emb_push_cache_opt(
    const uint16_t* x, const uint16_t* cos_sin, const int32_t* position_ids, uint16_t* output, const int32_t* cnts,
    int batch_size, int heads, int seq_len, int embed_dim, int64_t stride_xb, int64_t stride_xh, int64_t stride_xs,
    int64_t stride_xe, int64_t stride_cos_sin, int64_t stride_pid_b, int64_t stride_pid_h, int64_t stride_pid_s,
    int64_t stride_output_b, int64_t stride_output_h, int64_t stride_output_s, int offset_output_s_start,
    int offset_output_s_end, int half_dim, int chunk_size, int64_t cos_sin_rows, void* stream) {
  return launch_push(false, x, cos_sin, position_ids, output, cnts, batch_size, heads, seq_len, embed_dim, stride_xb,
                     stride_xh, stride_xs, stride_xe, stride_cos_sin, stride_pid_b, stride_pid_h, stride_pid_s,
                     stride_output_b, stride_output_h, stride_output_s, offset_output_s_start, offset_output_s_end,
                     half_dim, chunk_size, cos_sin_rows, stream);
}

extern "C" int skv_apply_rotary_pos_emb_push_cache_opt_glm(
    const uint16_t* x, const uint16_t* cos_sin, const int32_t* position_ids, uint16_t* output, const int32_t* cnts,
    int batch_size, int heads, int seq_len, int embed_dim, int64_t stride_xb, int64_t stride_xh, int64_t stride_xs,
    int64_t stride_xe, int64_t stride_cos_sin, int64_t stride_pid_b, int64_t stride_pid_h, int64_t stride_pid_s,
    int64_t stride_output_b, int64_t stride_output_h, int64_t stride_output_s, int offset_output_s_start,
    int offset_output_s_end, int half_dim, int chunk_size, int64_t cos_sin_rows, void* stream) {
  return launch_push(true, x, cos_sin, position_ids, output, cnts, batch_size, heads, seq_len, embed_dim, stride_xb,
                     stride_xh, stride_xs, stride_xe, stride_cos_sin, stride_pid_b, stride_pid_h, stride_pid_s,
                     stride_output_b, stride_output_h, stride_output_s, offset_output_s_start, offset_output_s_end,
                     half_dim, chunk_size, cos_sin_rows, stream);
}

extern "C" int skv_apply_rotary_pos_emb(const uint16_t* x, const uint16_t* cos, const uint16_t* sin,
                                        const int64_t* position_ids, uint16_t* output, int batch_size, int heads,
                                        int seq_len, int embed_dim, int64_t stride_xb, int64_t stride_xh,
                                        int64_t stride_xs, int64_t stride_xe, int64_t stride_cos, int64_t stride_sin,
                                        int64_t stride_pid_b, int64_t stride_pid_h, int64_t stride_pid_s,
                                        int half_dim, int64_t table_rows, void* stream) {
  const char* what = "apply_rotary_pos_emb";
  if (!x || !cos || !sin || !position_ids || !output) {
    skv_set_error("%s: null pointer", what);
    return SKV_EINVAL;
  }
  if (batch_size <= 0 || heads <= 0 || seq_len <= 0 || half_dim <= 0 || embed_dim != 2 * half_dim) {
    skv_set_error("%s: invalid shape (batch=%d heads=%d seq=%d embed=%d half=%d)", what, batch_size, heads, seq_len,
                  embed_dim, half_dim);
    return SKV_EINVAL;
  }
  const int64_t total = static_cast<int64_t>(batch_size) * heads * seq_len * half_dim;
  hipLaunchKernelGGL(rope_two_table_kernel, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream), x, cos, sin, position_ids, output, heads,
                     seq_len, half_dim, stride_xb, stride_xh, stride_xs, stride_xe, stride_cos, stride_sin,
                     stride_pid_b, stride_pid_h, stride_pid_s, table_rows, total);
  return skv_check_launch(what);
}

extern "C" int skv_apply_rotary_pos_emb_new_v2(const uint16_t* x, const uint16_t* cos_sin, const int32_t* position_ids,
                                               uint16_t* output, int batch_size, int heads, int seq_len, int embed_dim,
                                               int64_t stride_xb, int64_t stride_xh, int64_t stride_xs,
                                               int64_t stride_xe, int64_t stride_cos_sin, int64_t stride_pid_b,
                                               int64_t stride_pid_h, int64_t stride_pid_s, int half_dim,
                                               int chunk_size, int64_t cos_sin_rows, void* stream) {
  // Every row rotated at position position_ids[b,h,s/chunk]*chunk + s%chunk and written where it
  // was read (output addressed with x's strides): the push kernel with no hit rows, start 0.
  return launch_push(false, x, cos_sin, position_ids, output, nullptr, batch_size, heads, seq_len, embed_dim, stride_xb,
                     stride_xh, stride_xs, stride_xe, stride_cos_sin, stride_pid_b, stride_pid_h, stride_pid_s,
                     stride_xb, stride_xh, stride_xs, 0, seq_len, half_dim, chunk_size, cos_sin_rows, stream,
                     "apply_rotary_pos_emb_new_v2", true);
}

extern "C" int skv_apply_rotary_pos_emb_push_cache(
    const uint16_t* x, const uint16_t* cos_sin, const int32_t* position_ids, uint16_t* output, const int32_t* cnts,
    int batch_size, int heads, int seq_len, int embed_dim, int64_t stride_xb, int64_t stride_xh, int64_t stride_xs,
    int64_t stride_xe, int64_t stride_cos_sin, int64_t stride_pid_b, int64_t stride_pid_h, int64_t stride_pid_s,
    int64_t stride_output_b, int64_t stride_output_h, int64_t stride_output_s, int offset_output_s_start,
    int offset_output_s_end, int half_dim, int chunk_size, int64_t cos_sin_rows, void* stream) {
  return launch_push(false, x, cos_sin, position_ids, output, cnts, batch_size, heads, seq_len, embed_dim, stride_xb,
                     stride_xh, stride_xs, stride_xe, stride_cos_sin, stride_pid_b, stride_pid_h, stride_pid_s,
                     stride_output_b, stride_output_h, stride_output_s, offset_output_s_start, offset_output_s_end,
                     half_dim, chunk_size, cos_sin_rows, stream, "apply_rotary_pos_emb_push_cache");
}
