/*
 * shadowkv_amd — C ABI of the MI355X (gfx950) ShadowKV sparse-decode kernels.
 *
 * Every entry point takes raw device pointers (or a device-accessible pinned-host
 * pointer where stated), element strides as int64_t, plain int shapes and a HIP
 * stream passed as `void*` (a hipStream_t; NULL is the legacy default stream).
 * Every entry point is asynchronous on that stream, allocates nothing, and returns
 * SKV_OK (0) or a nonzero status; skv_last_error() then describes the failure.
 *
 * bf16 tensors are passed as uint16_t bit patterns. Citations name the reference
 * interface (WilliamBy/ShadowKV, path:line) each entry point replaces.
 */
#ifndef SHADOWKV_AMD_H
#define SHADOWKV_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SKV_OK 0
#define SKV_EINVAL 1       /* bad pointer, shape, stride or alignment */
#define SKV_EUNSUPPORTED 2 /* shape outside what the kernels implement */
#define SKV_ELAUNCH 3      /* HIP launch or runtime error */

/* Library version string and the message of the last failing call on this host thread. */
const char* skv_version(void);
const char* skv_last_error(void);

/* Translate a pinned host pointer (hipHostMalloc / torch pin_memory) to the device
 * address kernels must use for it. No reference counterpart: the reference relies on
 * CUDA UVA implicitly (kernels/copy.cuh:492 reads the host pointer directly). */
int skv_host_device_pointer(const void* host_ptr, void** device_ptr);

/* ---- a3: cache-hit reorder ------------------------------------------------------
 * Replaces reorder_keys_and_compute_offsets (kernels/functions.h:37-42,
 * kernels/gather_copy.cu:189-235, device kernels/map.cuh:475-516).
 * Per row r < batch_size*heads, with old = cached_pos_ids[r, :map_size] (slot order)
 * and new = cur_pos_ids[r, :map_size] (unique chunk ids, any order):
 *   cached_pos_ids[r] <- [hit ids ordered by ascending old slot] ++ [miss ids ascending]
 *   offsets[r]        <- [old slots of the hits, ascending]     ++ [miss ids ascending]
 *   cnts[r]           <- number of hits
 * map_size may be any value in [1, 2048] (the reference launches only 128/256/512/1024).
 * Old ids must be unique apart from -1 (empty slot, never a hit); new ids unique and >= 0. */
int skv_reorder_keys_and_compute_offsets(int64_t* cached_pos_ids, const int64_t* cur_pos_ids,
                                         int32_t* offsets, int32_t* cnts, int batch_size, int heads,
                                         int map_size, void* stream);

/* ---- a4: value fetch into the GPU chunk cache ---------------------------------------
 * Replaces gather_copy_with_offsets (kernels/functions.h:44-51, kernels/gather_copy.cu:239-324,
 * device kernels/copy.cuh:438-498). For row r, chunk unit = chunk_elems bf16 values:
 *   slot(i) = v_cache_buffer + r*gpu_v_stride + gpu_v_offset + i*chunk_elems
 *   i <  cnts[r]: slot(i) <- slot(offsets[r,i])              (in-place forward compaction)
 *   i >= cnts[r]: slot(i) <- values + r*cpu_v_length + offsets[r,i]*chunk_elems (host store)
 * `values` is the device address of the pinned host store (see skv_host_device_pointer).
 * The reference's `temp` staging buffer and `signals` flags have no equivalent here.
 * gpu_v_length must equal map_size*chunk_elems (the reference's per-row temp length). */
int skv_gather_copy_with_offsets(const void* values, void* v_cache_buffer, const int32_t* offsets,
                                 const int32_t* cnts, int batch_size, int heads, int64_t cpu_v_length,
                                 int64_t gpu_v_length, int64_t gpu_v_offset, int64_t gpu_v_stride,
                                 int map_size, int chunk_elems, void* stream);

/* The i >= cnts[r] half of skv_gather_copy_with_offsets alone: the host-link gather of the
 * misses, no in-buffer hit move. Together with skv_gather_copy_d2d_with_offsets on the value
 * buffer (the hit move, issued first on another stream) it does the same work as
 * skv_gather_copy_with_offsets, split so that the host-link stream carries only host-link
 * transfers (the reference runs both halves inside one gather_copy_with_offsets call,
 * models/kvcache/shadow.py:578-582). */
int skv_gather_copy_misses_with_offsets(const void* values, void* v_cache_buffer, const int32_t* offsets,
                                        const int32_t* cnts, int batch_size, int heads, int64_t cpu_v_length,
                                        int64_t gpu_v_length, int64_t gpu_v_offset, int64_t gpu_v_stride,
                                        int map_size, int chunk_elems, void* stream);

/* ---- a5: key-hit compaction ------------------------------------------------------------
 * Replaces gather_copy_d2d_with_offsets (kernels/functions.h:27-35, kernels/gather_copy.cu:112-185,
 * device kernels/copy.cuh:353-390): the i < cnts[r] part of skv_gather_copy_with_offsets on `keys`. */
int skv_gather_copy_d2d_with_offsets(void* keys, const int32_t* offsets, const int32_t* cnts,
                                     int batch_size, int heads, int64_t gpu_k_length,
                                     int64_t gpu_k_offset, int64_t gpu_k_stride, int map_size,
                                     int chunk_elems, void* stream);

/* Plain chunk gather without cache hits. Replaces gather_copy (kernels/functions.h:23-25,
 * kernels/gather_copy.cu:47-109): dst + r*gpu_v_length + i*chunk_elems <-
 * values + r*cpu_v_length + position_ids[r*map_size+i]*chunk_elems. */
int skv_gather_copy(const void* values, void* v_cache_buffer, const int64_t* position_ids,
                    int batch_size, int heads, int64_t cpu_v_length, int64_t gpu_v_length,
                    int map_size, int chunk_elems, void* stream);

/* ---- a7: RoPE ---------------------------------------------------------------------------
 * Replaces apply_rotary_pos_emb_new (kernels/functions.h:61-67, kernels/rope_new.cu:26-84):
 * output[b,h,s] = rope(x[b,h,s], cos_sin[position_ids[b,h,s]]) with the half-split layout,
 * cos_sin row = [cos(half_dim) | sin(half_dim)], per-op bf16 rounding. Rows whose position is outside
 * [0, cos_sin_rows) are left unwritten (no counterpart argument in the reference). */
int skv_apply_rotary_pos_emb_new(const uint16_t* x, const uint16_t* cos_sin, const int64_t* position_ids,
                                 uint16_t* output, int batch_size, int heads, int seq_len, int embed_dim,
                                 int64_t stride_xb, int64_t stride_xh, int64_t stride_xs, int64_t stride_xe,
                                 int64_t stride_cos_sin, int64_t stride_pid_b, int64_t stride_pid_h,
                                 int64_t stride_pid_s, int half_dim, int64_t cos_sin_rows, void* stream);

/* Replaces apply_rotary_pos_emb (kernels/functions.h:53-59, kernels/rope.cu:26-88): the rotation
 * with separate cos and sin tables (rows of stride_cos / stride_sin, table_rows rows, indexed by
 * position_ids[b,h,s], int64): output[b,h,s,d] = bf16(bf16(x1*cos[d]) + bf16(-x2*sin[d])),
 * output[b,h,s,d+half] = bf16(bf16(x2*cos[d+half]) + bf16(x1*sin[d+half])), output addressed with
 * x's strides; rows whose position is outside [0, table_rows) are left unwritten. Bound by the
 * reference's module but not called by its Python. */
int skv_apply_rotary_pos_emb(const uint16_t* x, const uint16_t* cos, const uint16_t* sin, const int64_t* position_ids,
                             uint16_t* output, int batch_size, int heads, int seq_len, int embed_dim,
                             int64_t stride_xb, int64_t stride_xh, int64_t stride_xs, int64_t stride_xe,
                             int64_t stride_cos, int64_t stride_sin, int64_t stride_pid_b, int64_t stride_pid_h,
                             int64_t stride_pid_s, int half_dim, int64_t table_rows, void* stream);

/* Replaces apply_rotary_pos_emb_new_v2 (kernels/functions.h:69-75, kernels/rope_new.cu:86-144): every
 * row s rotated at table row position_ids[b,h,s/chunk_size]*chunk_size + s%chunk_size (int32 chunk
 * ids) with the half-split [cos|sin] table, written to output at x's strides (stride_xe must be 1).
 * Bound by the reference's module but not called by its Python. */
int skv_apply_rotary_pos_emb_new_v2(const uint16_t* x, const uint16_t* cos_sin, const int32_t* position_ids,
                                    uint16_t* output, int batch_size, int heads, int seq_len, int embed_dim,
                                    int64_t stride_xb, int64_t stride_xh, int64_t stride_xs, int64_t stride_xe,
                                    int64_t stride_cos_sin, int64_t stride_pid_b, int64_t stride_pid_h,
                                    int64_t stride_pid_s, int half_dim, int chunk_size, int64_t cos_sin_rows,
                                    void* stream);

/* Replaces apply_rotary_pos_emb_push_cache (kernels/functions.h:77-86, kernels/rope_new.cu:146-222):
 * the same contract as skv_apply_rotary_pos_emb_push_cache_opt below (the reference's "_opt" form is
 * a faster launch of the same rows). Bound by the reference's module but not called by its Python. */
int skv_apply_rotary_pos_emb_push_cache(
    const uint16_t* x, const uint16_t* cos_sin, const int32_t* position_ids, uint16_t* output,
    const int32_t* cnts, int batch_size, int heads, int seq_len, int embed_dim, int64_t stride_xb,
    int64_t stride_xh, int64_t stride_xs, int64_t stride_xe, int64_t stride_cos_sin, int64_t stride_pid_b,
    int64_t stride_pid_h, int64_t stride_pid_s, int64_t stride_output_b, int64_t stride_output_h,
    int64_t stride_output_s, int offset_output_s_start, int offset_output_s_end, int half_dim,
    int chunk_size, int64_t cos_sin_rows, void* stream);

/* Replaces apply_rotary_pos_emb_push_cache_opt (kernels/functions.h:88-97, kernels/rope_new.cu:224-302):
 * for rows s with s/chunk_size >= cnts[b*heads+h] and start+s < end, writes
 * rope(x[b,h,s], cos_sin[position_ids[b,h,s/chunk]*chunk + s%chunk]) to output[b,h,start+s];
 * rows whose table row falls outside [0, cos_sin_rows) are skipped. */
int skv_apply_rotary_pos_emb_push_cache_opt(
    const uint16_t* x, const uint16_t* cos_sin, const int32_t* position_ids, uint16_t* output,
    const int32_t* cnts, int batch_size, int heads, int seq_len, int embed_dim, int64_t stride_xb,
    int64_t stride_xh, int64_t stride_xs, int64_t stride_xe, int64_t stride_cos_sin, int64_t stride_pid_b,
    int64_t stride_pid_h, int64_t stride_pid_s, int64_t stride_output_b, int64_t stride_output_h,
    int64_t stride_output_s, int offset_output_s_start, int offset_output_s_end, int half_dim,
    int chunk_size, int64_t cos_sin_rows, void* stream);

/* Replaces apply_rotary_pos_emb_push_cache_opt_glm (kernels/functions.h:99-108,
 * kernels/rope_new.cu:305-404): GLM interleaved pairs (2i, 2i+1), i < 32, with
 * cos_sin row = [cos(32) | sin(32)]; dims 64..127 copied unchanged. */
int skv_apply_rotary_pos_emb_push_cache_opt_glm(
    const uint16_t* x, const uint16_t* cos_sin, const int32_t* position_ids, uint16_t* output,
    const int32_t* cnts, int batch_size, int heads, int seq_len, int embed_dim, int64_t stride_xb,
    int64_t stride_xh, int64_t stride_xs, int64_t stride_xe, int64_t stride_cos_sin, int64_t stride_pid_b,
    int64_t stride_pid_h, int64_t stride_pid_s, int64_t stride_output_b, int64_t stride_output_h,
    int64_t stride_output_s, int offset_output_s_start, int offset_output_s_end, int half_dim,
    int chunk_size, int64_t cos_sin_rows, void* stream);

/* ---- a6: low-rank key rebuild ------------------------------------------------------------
 * Replaces batch_gather_gemm (kernels/functions.h:110-116, kernels/batch_gather_gemm.cu:136-213):
 * for bh < batch_size*heads and rows r in [offset_array[bh]*chunk_size, sparse_budget):
 *   output[bh, r, :] = bf16( a[bh/heads, pos(r), :rank] . b[bh, :, :rank]^T ),
 *   pos(r) = position_ids[bh*(sparse_budget/chunk_size) + r/chunk_size]*chunk_size + r%chunk_size.
 * a: [batch, seq_len, rank]; b: [batch*heads, embed_dim, rank]; output [batch*heads, sparse_budget, embed_dim].
 * Hit rows (r < offset_array[bh]*chunk_size) are left untouched. embed_dim must be 128; a, b and
 * output must be 16-byte aligned. */
int skv_batch_gather_gemm(const uint16_t* a, const uint16_t* b, const int32_t* position_ids,
                          uint16_t* output, int batch_size, int heads, int seq_len, int embed_dim,
                          int rank, int sparse_budget, int max_seq_len, int chunk_size,
                          const int32_t* offset_array, void* stream);

/* a6+a7 fused: the rebuild above followed by the RoPE push, in one pass, writing rotated keys
 * of miss rows straight into the key cache. Replaces batch_gather_gemm_rotary_pos_emb_cuda
 * (models/tensor_op.py:206-243 = batch_gather_gemm + apply_rotary_pos_emb_push_cache_opt[_glm]).
 *   u row of (b,h,p):  u + b*u_stride_b + h*u_stride_h + p*u_stride_row      (u_stride_h = 0: head-shared U)
 *   sv of (b,h):       sv + b*sv_stride_b + h*sv_stride_h, [head_dim rows][rank], row stride sv_stride_n
 *   chunk ids:         position_ids[b*pid_stride_b + h*pid_stride_h + c]       (int64)
 *   out row of (b,h,r): cache + b*stride_cache_b + h*stride_cache_h + (sparse_start+r)*stride_cache_s
 * rope_mode 0: half-split with cos_sin row [cos(64)|sin(64)]; 1: GLM interleaved (see above).
 * Rows whose position falls outside [0, u_rows) or [0, cos_sin_rows) are not written.
 * head_dim must be 128, rank a multiple of 8 in [8, 192]; U, SV, cache and cos_sin rows must be
 * 16-byte aligned (base pointers, and strides multiples of 8 elements). */
int skv_rebuild_k_rope(const uint16_t* u, int64_t u_stride_b, int64_t u_stride_h, int64_t u_stride_row,
                       int64_t u_rows, const uint16_t* sv, int64_t sv_stride_b, int64_t sv_stride_h,
                       int64_t sv_stride_n, const int64_t* position_ids, int64_t pid_stride_b, int64_t pid_stride_h,
                       const int32_t* cnts, const uint16_t* cos_sin, int64_t stride_cos_sin, int64_t cos_sin_rows,
                       int rope_mode,
                       uint16_t* cache, int64_t stride_cache_b, int64_t stride_cache_h,
                       int64_t stride_cache_s, int sparse_start, int batch_size, int heads,
                       int num_chunks, int chunk_size, int rank, int head_dim, void* stream);

/* ---- a1: landmark scoring ------------------------------------------------------------------
 * Replaces batch_gemm_softmax (kernels/functions.h:118-121, kernels/batch_gemm_softmax.cu:143-196):
 *   D[z, i, j]       = bf16(alpha * sum_k A[z, i, k] * B[z, j, k])          (A [batch][m][k], B [batch][n][k])
 *   softmax[z, i, :] = bf16(softmax_fp32(D[z, i, :]))
 * norm/sum [batch][m][ceil(n/256)] receive per-256-column partial max and sum of exp(D - max).
 * k must be 128, m in [1, 16], beta must be 0 (the reference passes no C operand). */
int skv_batch_gemm_softmax(const uint16_t* A, const uint16_t* B, uint16_t* D, float* norm, float* sum,
                           uint16_t* softmax, int batch_count, int m, int n, int k, float alpha,
                           float beta, void* stream);

/* a1+a2 fused front: the scoring above, then the GQA max over the m rows of each batch entry,
 * written as out[z, j] = max_i softmax[z, i, j] (bf16). Replaces batch_gemm_softmax + torch.max
 * (models/kvcache/shadow.py:553-568). D/norm/sum are caller-provided scratch as above. */
int skv_score_gqa_max(const uint16_t* A, const uint16_t* B, uint16_t* D, float* norm, float* sum,
                      uint16_t* out, int batch_count, int m, int n, int k, float alpha, void* stream);

/* The two kernels of the scoring above, callable separately: logits + per-tile partials, then
 * the softmax normalisation with the optional per-row probabilities (softmax, [batch][m][n])
 * and/or the GQA max (out_max, [batch][n]); at least one output must be non-null. */
int skv_score_logits(const uint16_t* A, const uint16_t* B, uint16_t* D, float* norm, float* sum, int batch_count,
                     int m, int n, int k, float alpha, void* stream);
int skv_softmax_gqa_max(const uint16_t* D, const float* norm, const float* sum, uint16_t* softmax, uint16_t* out_max,
                        int batch_count, int m, int n, void* stream);

/* ---- a2: chunk top-k and landmark-id gather ---------------------------------------------------
 * Replaces torch.topk(scores, k).indices + k_landmark_idx.gather (models/kvcache/shadow.py:571-573):
 *   out_ids[r, j] = landmark_idx[r*idx_stride + sel_j],
 * where sel_0..sel_{k-1} are the k largest of scores[r*score_stride + 0..n-1] under the total
 * order (value descending, index ascending), emitted in that order. k in [1, 4096], k <= n. */
int skv_topk_gather(const uint16_t* scores, int64_t score_stride, const int64_t* landmark_idx,
                    int64_t idx_stride, int rows, int n, int k, int64_t* out_ids, void* stream);

/* a1 tail + a2 + a3 fused: one launch performs the softmax normalisation of D from its partials,
 * the GQA max over the m rows, the top-k (value desc, index asc), the landmark-id gather and the
 * reorder of the selected ids against position_ids (in place), writing offsets and cnts exactly
 * as skv_softmax_gqa_max + skv_topk_gather + skv_reorder_keys_and_compute_offsets would.
 * Replaces models/kvcache/shadow.py:553-574 after the scoring GEMM. D/norm/sum as produced by
 * skv_score_logits for `rows` batch entries of m query rows; landmark_idx rows of idx_stride;
 * position_ids/offsets [rows][select_sets]; cnts [rows]. Chunk ids (landmark ids and previous
 * slot ids) must lie in [0, num_chunks) (-1 marks an empty previous slot); num_chunks <= 606208
 * at select_sets <= 256 and <= 548864 at 2048 (two chunk bitmaps and the winner list in LDS).
 * out_scores ([rows][n] bf16 GQA-max probabilities) and out_selected ([rows][select_sets] ids in
 * top-k order) are optional, except that out_scores is required as staging when n is too large
 * for LDS. With out_scores given and few rows (rows <= 32, m*n >= 32768) the probabilities are
 * first computed by the many-workgroup softmax kernel (as skv_softmax_gqa_max, a second launch on
 * the same stream) and the selection starts from them; results are identical.
 * position_ids, offsets and cnts all null: selection only (no previous slots, no reorder, no
 * num_chunks limit); out_selected is then required and receives the ids in top-k order, as
 * skv_softmax_gqa_max + skv_topk_gather would (the selection of a device chunk pool).
 * select_sets <= 2048. */
int skv_select_chunks(const uint16_t* D, const float* norm, const float* sum, int rows, int m, int n,
                      const int64_t* landmark_idx, int64_t idx_stride, int select_sets, int num_chunks,
                      int64_t* position_ids, int32_t* offsets, int32_t* cnts, uint16_t* out_scores,
                      int64_t* out_selected, void* stream);

/* Bytes of the workspace skv_select_chunks_ws needs for `rows` rows of n landmarks and
 * select_sets winners (0 for invalid arguments). */
int64_t skv_select_workspace_bytes(int rows, int n, int select_sets);

/* skv_select_chunks with a caller-owned device workspace (skv_select_workspace_bytes; no
 * initialisation needed; calls that overlap on one workspace race). With out_scores given and few
 * rows (rows <= 32, m*n >= 32768) each row's selection is spread over many workgroups: the
 * softmax kernel writes the keys, then per-slice histograms of the high and low key bytes, the
 * per-slice counts above and at the threshold, the winners at their rank positions, and one
 * workgroup per row for the id bitmap and the reorder (six launches on the stream). Otherwise it
 * behaves as skv_select_chunks. Results are identical. Variant of skv_select_chunks (same
 * reference lines: models/kvcache/shadow.py:553-574). */
int skv_select_chunks_ws(const uint16_t* D, const float* norm, const float* sum, int rows, int m, int n,
                         const int64_t* landmark_idx, int64_t idx_stride, int select_sets, int num_chunks,
                         int64_t* position_ids, int32_t* offsets, int32_t* cnts, uint16_t* out_scores,
                         int64_t* out_selected, void* workspace, int64_t workspace_bytes, void* stream);

/* skv_select_chunks_ws (workspace may be null, as for skv_select_chunks) with the hit moves folded
 * into its last launch: after the reorder, the workgroup that owns row r compacts the row's hits
 * in place in each non-null buffer, exactly as skv_gather_copy_d2d_with_offsets would with the
 * offsets and cnts just written: slot(i) <- slot(offsets[r,i]) for i < cnts[r], where
 *   slot(i) = buffer + r*buf_stride + buf_offset + i*chunk_elems   (bf16 elements).
 * Requires position_ids/offsets/cnts (the reorder), chunk_elems a positive multiple of 8,
 * buf_offset and buf_stride multiples of 8, buf_stride >= buf_offset + select_sets*chunk_elems and
 * 16-byte aligned buffers. With it the value buffer needs only the host-link half of the fetch
 * (skv_gather_copy_misses_with_offsets) and the key buffer no compaction before the rebuild.
 * Variant of skv_select_chunks_ws (same reference lines, models/kvcache/shadow.py:553-574, plus
 * the hit moves of gather_copy_with_offsets / gather_copy_d2d_with_offsets,
 * models/kvcache/shadow.py:578-590). */
int skv_select_chunks_compact(const uint16_t* D, const float* norm, const float* sum, int rows, int m, int n,
                              const int64_t* landmark_idx, int64_t idx_stride, int select_sets, int num_chunks,
                              int64_t* position_ids, int32_t* offsets, int32_t* cnts, uint16_t* out_scores,
                              int64_t* out_selected, void* workspace, int64_t workspace_bytes, void* v_buffer,
                              void* k_buffer, int64_t buf_offset, int64_t buf_stride, int chunk_elems,
                              void* stream);

/* ---- a8: sparse decode attention ----------------------------------------------------------------
 * Replaces flash_attn_with_kvcache(q, k_cache, v_cache, causal=True) for one query token
 * (models/attention/shadow.py:48): for b, query head hq, kv head h = hq / (q_heads/kv_heads):
 *   out[b, hq] = softmax(scale * q[b,hq] . K[b,h,:kv_len]^T) . V[b,h,:kv_len]   (fp32 math, bf16 out)
 * q row: q + b*q_stride_b + hq*q_stride_h; K/V row s of (b,h): base + b*kv_stride_b + h*kv_stride_h
 * + s*kv_stride_s; out row: out + b*o_stride_b + hq*o_stride_h. head_dim must be 128.
 * workspace: caller-provided device scratch of skv_sparse_attn_workspace_bytes(...) bytes, 16-byte
 * aligned and zero-filled before its first use: its head holds per-row arrival counters that every
 * call leaves at zero (so a zeroed workspace stays valid across calls, shapes and graph replays);
 * calls that overlap on one workspace race. kv_len at most 262144.
 * kv_len_dev (optional, no reference counterpart): device int32 holding the live length, read
 * when the kernel runs and clamped to [1, kv_len]; kv_len is then the maximum. This keeps the
 * call valid inside a captured HIP graph while the cache grows by one row per replay. */
int64_t skv_sparse_attn_workspace_bytes(int batch_size, int q_heads, int kv_len);
/* Diagnostic of the one-launch merge (no reference counterpart): for the current device, whether
 * the probe confirmed that workgroups sharing blockIdx mod 8 run on one XCD (*state 1; -1 not
 * confirmed, the attention then merges in a second launch; 0 not probed yet), the XCC id seen
 * for each class (4 bits each, *xcc_map), and whether any fused attention workgroup since the
 * library loaded found itself on another XCC (*misplaced nonzero). Synchronous. */
int skv_sparse_attn_xcd_check(int32_t* state, uint32_t* xcc_map, uint32_t* misplaced);
int skv_sparse_attn_decode(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t* k_cache,
                           const uint16_t* v_cache, int64_t kv_stride_b, int64_t kv_stride_h,
                           int64_t kv_stride_s, int batch_size, int q_heads, int kv_heads, int head_dim,
                           int kv_len, const int32_t* kv_len_dev, float scale, void* workspace,
                           int64_t workspace_bytes, uint16_t* out, int64_t o_stride_b, int64_t o_stride_h,
                           void* stream);

/* Allocation-free form of skv_sparse_attn_decode. No reference counterpart: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops). The split
 * partials live in a device array inside the library, one per GPU, of
 * skv_sparse_attn_noalloc_max_bytes() bytes (32 MiB), held until the process ends; calls needing more
 * (skv_sparse_attn_workspace_bytes above it, e.g. batch 8 x 32 query heads beyond 16064 keys) return
 * SKV_EUNSUPPORTED. The call allocates nothing. All calls on one GPU share that array: calls that
 * overlap on one GPU (on different streams, or from several threads) race; `stream` must belong to
 * the current device. Arguments and results as skv_sparse_attn_decode. */
int64_t skv_sparse_attn_noalloc_max_bytes(void);
int skv_sparse_attn_decode_noalloc(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h,
                                   const uint16_t* k_cache, const uint16_t* v_cache, int64_t kv_stride_b,
                                   int64_t kv_stride_h, int64_t kv_stride_s, int batch_size, int q_heads,
                                   int kv_heads, int head_dim, int kv_len, const int32_t* kv_len_dev, float scale,
                                   uint16_t* out, int64_t o_stride_b, int64_t o_stride_h, void* stream);

/* ---- new-token operations around the path (fused) ------------------------------------
 * skv_rmsnorm replaces the residual add + flashinfer rmsnorm pair of the reference model
 * (models/llama.py:191, :204-206, :215 and models/base.py:94, through layer_norm of
 * models/tensor_op.py:39-44): with residual non-null,
 *   residual_out[r] = bf16(x[r] + residual[r])        (the bf16 residual add)
 *   out[r] = bf16(h * rsqrt(mean(h^2) + eps) * weight), h = residual_out[r] in fp32;
 * with residual null, h = x[r]. rows of `hidden` bf16 (a multiple of 8, at most 8192), all rows
 * 16-byte aligned (strides in elements, multiples of 8). */
int skv_rmsnorm(const uint16_t* x, int64_t x_stride, const uint16_t* residual, int64_t residual_stride,
                uint16_t* residual_out, int64_t residual_out_stride, const uint16_t* weight, uint16_t* out,
                int64_t out_stride, int rows, int hidden, float eps, void* stream);

/* Replaces vllm silu_and_mul (models/llama.py:208-214 at :212, models/glm.py:193):
 * out[r, j] = bf16(bf16(silu(x[r, j])) * x[r, d + j]), j < d (a multiple of 8): silu in fp32 rounded
 * to bf16, then the bf16 product, vLLM's two roundings; rows 16-byte aligned. */
int skv_silu_and_mul(const uint16_t* x, int64_t x_stride, uint16_t* out, int64_t out_stride, int rows, int d,
                     void* stream);

/* Replaces F.linear on the decoding model's weights at decode batch sizes (wqkv, wo, gate_up_proj,
 * down_proj: models/llama.py:192,203,208,214; lm_head: models/base.py:98):
 * y[i, j] = bf16(sum_k x[i, k] * weight[j, k]) in fp32, i < m <= 16, j < n, k a multiple of 8.
 * weight is row-major [n, k] (row stride weight_stride); x and weight rows 16-byte aligned. */
int skv_linear(const uint16_t* x, int64_t x_stride, const uint16_t* weight, int64_t weight_stride, uint16_t* y,
               int64_t y_stride, int m, int n, int k, void* stream);

/* skv_linear with a bias: y[i, j] = bf16(sum_k x[i, k] * w[j, k] + bias[j]), the bias added to the
 * fp32 sum before the one rounding (F.linear(x, w, b) with a bias epilogue: GLM's query_key_value
 * projection, models/glm.py:165). bias: n bf16 values. */
int skv_linear_bias(const uint16_t* x, int64_t x_stride, const uint16_t* weight, int64_t weight_stride,
                    const uint16_t* bias, uint16_t* y, int64_t y_stride, int m, int n, int k, void* stream);

/* skv_linear on the SiLU-and-mul of the gate/up projection, formed as the rows are read: x rows
 * hold [gate (k) | up (k)] (x_stride >= 2k) and the multiplied row is bf16(bf16(silu(gate)) * up)
 * as skv_silu_and_mul computes it, so the result equals skv_silu_and_mul followed by skv_linear
 * (models/llama.py:212 then :214, models/glm.py:193-195: the activation and down_proj of the
 * reference's MLP). m <= 4 (SKV_EUNSUPPORTED above: every workgroup recomputes the activations of
 * its rows, which only pays off for a few rows). */
int skv_linear_silu_mul(const uint16_t* x, int64_t x_stride, const uint16_t* weight, int64_t weight_stride,
                        uint16_t* y, int64_t y_stride, int m, int n, int k, void* stream);

/* The gate/up projection with the SiLU-and-mul in its epilogue: weight rows are (gate, up) pairs,
 * row 2j the gate and row 2j + 1 the up projection of output j (the reference's gate_up_proj
 * [gate (n/2 rows) | up (n/2 rows)] with its halves interleaved row by row), and
 *   y[i, j] = bf16(bf16(silu(g)) * u),  g = bf16(x[i] . w[2j]),  u = bf16(x[i] . w[2j + 1]),
 * exactly skv_linear on the reference layout followed by skv_silu_and_mul (models/llama.py:208-212,
 * models/glm.py:190-193), without writing the [gate | up] rows. n even; y rows hold n/2 elements;
 * m <= 16. */
int skv_linear_gate_up_silu(const uint16_t* x, int64_t x_stride, const uint16_t* weight, int64_t weight_stride,
                            uint16_t* y, int64_t y_stride, int m, int n, int k, void* stream);

/* ---- f1: prefill encoder ----------------------------------------------------------------
 * Replace the chunk statistics, outlier selection and landmark compaction of prefill_kv_cache
 * (models/kvcache/shadow.py:486-519). skv_chunk_stats: for each (b, h, chunk i < chunks) of the
 * post-RoPE keys (row s of (b,h) at keys + b*stride_b + h*stride_h + s*stride_s, head_dim 128),
 * candidates[(b*heads + h)*chunks + i] = bf16(mean of rows i*c .. i*c+c-1) (fp32 sum, one
 * rounding) and min_cos[...] = min over those rows of cos(candidate, row), in fp32 with norms
 * clamped to 1e-8 (the reference computes it with bf16 operations). */
int skv_chunk_stats(const uint16_t* keys, int64_t stride_b, int64_t stride_h, int64_t stride_s, int batch_size,
                    int heads, int chunks, int chunk_size, uint16_t* candidates, float* min_cos, void* stream);

/* Per row r < rows of min_cos [rows, chunks]: outlier_idx[r] = the `outliers` chunk ids of smallest
 * min_cos, in ascending (min_cos, id) order (torch.topk(largest=False) at shadow.py:490, ties to the
 * lowest id); landmark_idx[r] = every other chunk id ascending ([rows, chunks - outliers],
 * shadow.py:513-516). chunks <= 131072, outliers <= 512. */
int skv_select_outliers(const float* min_cos, int rows, int chunks, int outliers, int64_t* outlier_idx,
                        int64_t* landmark_idx, void* stream);

/* dst[r][j] = src[r][idx[r][j]] for 128-element bf16 rows: src [rows, src_rows, 128], idx and dst
 * [rows, dst_rows(, 128)] (the landmark gather, shadow.py:517-519); ids outside [0, src_rows) skip. */
int skv_gather_rows(const uint16_t* src, int rows, int src_rows, const int64_t* idx, int dst_rows, uint16_t* dst,
                    void* stream);

/* The value fetch of the misses and the key rebuild in one launch: the work of
 * skv_gather_copy_misses_with_offsets(values, v_cache_buffer, offsets, cnts, batch_size, heads,
 * cpu_v_length, num_chunks*chunk_size*head_dim, gpu_v_offset, gpu_v_stride, num_chunks,
 * chunk_size*head_dim) and of skv_rebuild_k_rope(u, ..., cache, ...) with the same cnts, whose
 * workgroups run side by side (the first ones gather from the host link, the rest rebuild keys).
 * Both buffers' hits must already be in place (the selection's folded hit moves,
 * skv_select_chunks_compact with both buffers). No reference counterpart as one call: it replaces
 * the pair at models/kvcache/shadow.py:578-593 (value fetch on copy_stream, key rebuild on the
 * current stream) for callers that run the step on one stream, saving the two cross-stream waits
 * around the fetch. Results are those of the two calls. fetch_workgroups: the fetch workgroups to
 * aim for, counted in 4-wave workgroups (0: the library default, 64, or SKV_FUSED_FETCH_WGS).
 * rebuild_workgroups: 0 gives every rebuild tile a workgroup of its own; a positive cap (rounded
 * up to a multiple of 8) makes that many workgroups loop over the tiles, so the rebuild spreads over
 * the fetch instead of filling the GPU at its start (taken by the half-split RoPE instances of rank
 * <= 160 with 128-row tiles, the tiles of a 4-sequence decode lane; the others ignore it). */
int skv_fetch_misses_rebuild_k_rope(const void* values, void* v_cache_buffer, const int32_t* offsets,
                                    int64_t cpu_v_length, int64_t gpu_v_offset, int64_t gpu_v_stride,
                                    const uint16_t* u, int64_t u_stride_b, int64_t u_stride_h, int64_t u_stride_row,
                                    int64_t u_rows, const uint16_t* sv, int64_t sv_stride_b, int64_t sv_stride_h,
                                    int64_t sv_stride_n, const int64_t* position_ids, int64_t pid_stride_b,
                                    int64_t pid_stride_h, const int32_t* cnts, const uint16_t* cos_sin,
                                    int64_t stride_cos_sin, int64_t cos_sin_rows, int rope_mode, uint16_t* cache,
                                    int64_t stride_cache_b, int64_t stride_cache_h, int64_t stride_cache_s,
                                    int sparse_start, int batch_size, int heads, int num_chunks, int chunk_size,
                                    int rank, int head_dim, int fetch_workgroups, int rebuild_workgroups,
                                    void* stream);

/* ---- f3: device chunk pool (a GPU cache of P >= S chunk slots per (b, h) and layer) ------
 * No reference counterpart: extends the slot reuse of reorder_keys_and_compute_offsets
 * (kernels/map.cuh:475-516, models/kvcache/shadow.py:574-593) to a cache larger than the
 * selection. skv_pool_assign, per row r < rows: selected[r] [select_sets] chunk ids (int64) are
 * looked up in slot_of[r] [num_chunks] (slot or -1); hits keep their slot; the misses take the
 * least recently used slots holding no selected chunk (empty first, then ascending slot_used,
 * ties to the lowest slot), the k-th miss in selection order the k-th such slot in ascending slot
 * order; slot_of, slot_chunk[r] [pool_slots] (chunk or -1) and slot_used[r] [pool_slots] (step of
 * last use, -1 = never) are updated, clock[r] advanced by one. Outputs: slot_list[r] [select_sets]
 * (slot of each selected chunk), cnts[r] = select_sets - misses, and for i in [cnts[r],
 * select_sets): miss_ids[r][i] / miss_slot[r][i] (int32). select_sets <= 2048, select_sets <=
 * pool_slots <= 16384. */
int skv_pool_assign(const int64_t* selected, int rows, int select_sets, int num_chunks, int pool_slots,
                    int32_t* slot_of, int32_t* slot_chunk, int32_t* slot_used, int32_t* clock, int32_t* slot_list,
                    int32_t* miss_ids, int32_t* miss_slot, int32_t* cnts, void* stream);

/* The miss gather of a chunk pool: for r < batch_size*heads and i in [cnts[r], map_size), chunk
 * miss_ids[r*map_size + i] of host row r (values + r*cpu_v_length) is copied to pool slot
 * miss_slot[r*map_size + i] at v_cache_buffer + r*gpu_v_stride + pool_offset + slot*chunk_elems. */
int skv_gather_copy_misses_to_slots(const void* values, void* v_cache_buffer, const int32_t* miss_ids,
                                    const int32_t* cnts, const int32_t* miss_slot, int batch_size, int heads,
                                    int64_t cpu_v_length, int64_t pool_offset, int64_t gpu_v_stride, int map_size,
                                    int pool_slots, int chunk_elems, void* stream);

/* skv_rebuild_k_rope for a chunk pool: the rows of entries i in [cnts[r], num_chunks) (chunk
 * miss_ids[r][i], int32) are written to cache rows pool_start + miss_slot[r][i]*chunk_size + j. */
int skv_rebuild_k_rope_slots(const uint16_t* u, int64_t u_stride_b, int64_t u_stride_h, int64_t u_stride_row,
                             int64_t u_rows, const uint16_t* sv, int64_t sv_stride_b, int64_t sv_stride_h,
                             int64_t sv_stride_n, const int32_t* miss_ids, const int32_t* miss_slot,
                             const int32_t* cnts, const uint16_t* cos_sin, int64_t stride_cos_sin,
                             int64_t cos_sin_rows, int rope_mode, uint16_t* cache, int64_t stride_cache_b,
                             int64_t stride_cache_h, int64_t stride_cache_s, int pool_start, int pool_slots,
                             int batch_size, int heads, int num_chunks, int chunk_size, int rank, int head_dim,
                             void* stream);

/* The chunk pool's miss gather (skv_gather_copy_misses_to_slots with pool_offset = gpu_v_offset,
 * map_size = num_chunks) and key rebuild (skv_rebuild_k_rope_slots) in one launch, their
 * workgroups side by side, as skv_fetch_misses_rebuild_k_rope does for the reference layout (the
 * pool's hits keep their slots, so nothing moves first). No reference counterpart: the chunk pool
 * extends the cache past the reference's select_sets slots (models/kvcache/shadow.py:574-593);
 * for callers that run the pooled step on one stream. Results are those of the two calls. */
int skv_fetch_misses_rebuild_k_rope_slots(const void* values, void* v_cache_buffer, int64_t cpu_v_length,
                                          int64_t gpu_v_offset, int64_t gpu_v_stride, const uint16_t* u,
                                          int64_t u_stride_b, int64_t u_stride_h, int64_t u_stride_row,
                                          int64_t u_rows, const uint16_t* sv, int64_t sv_stride_b,
                                          int64_t sv_stride_h, int64_t sv_stride_n, const int32_t* miss_ids,
                                          const int32_t* miss_slot, const int32_t* cnts, const uint16_t* cos_sin,
                                          int64_t stride_cos_sin, int64_t cos_sin_rows, int rope_mode,
                                          uint16_t* cache, int64_t stride_cache_b, int64_t stride_cache_h,
                                          int64_t stride_cache_s, int pool_start, int pool_slots, int batch_size,
                                          int heads, int num_chunks, int chunk_size, int rank, int head_dim,
                                          int fetch_workgroups, int rebuild_workgroups, void* stream);

/* skv_sparse_attn_decode over a chunk pool: virtual keys [0, kv_len) = rows [0, sparse_start) ++
 * the select_sets chunks of slot_list[(b*kv_heads + h)*select_sets + j] (rows sparse_start +
 * slot*chunk_size + ...) ++ rows from sparse_start + pool_slots*chunk_size on (the generated
 * tokens). The buffers must hold kv_len + (pool_slots - select_sets)*chunk_size rows. */
int skv_sparse_attn_decode_paged(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t* k_cache,
                                 const uint16_t* v_cache, int64_t kv_stride_b, int64_t kv_stride_h,
                                 int64_t kv_stride_s, int batch_size, int q_heads, int kv_heads, int head_dim,
                                 int kv_len, const int32_t* kv_len_dev, float scale, void* workspace,
                                 int64_t workspace_bytes, uint16_t* out, int64_t o_stride_b, int64_t o_stride_h,
                                 const int32_t* slot_list, int sparse_start, int select_sets, int chunk_size,
                                 int pool_slots, void* stream);

/* skv_sparse_attn_decode with the selected region's values read in place from the value store. No
 * reference counterpart: it is for a value store kept in device memory (HBM), where gathering the
 * selected chunks into v_cache first would only copy them. Keys [0, kv_len) and the values outside
 * [sparse_start, sparse_start + select_sets*chunk_size) come from k_cache / v_cache as in
 * skv_sparse_attn_decode; value row sparse_start + j*chunk_size + r is row c*chunk_size + r of
 * (b, h) in v_store, c = position_ids[(b*kv_heads + h)*select_sets + j] (clamped to
 * [0, store_chunks)), rows of head_dim elements, (b, h) at vs_stride_b / vs_stride_h elements.
 * The same arithmetic as skv_sparse_attn_decode over a v_cache holding those rows: the results are
 * bit-identical. */
int skv_sparse_attn_decode_vstore(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t* k_cache,
                                  const uint16_t* v_cache, int64_t kv_stride_b, int64_t kv_stride_h,
                                  int64_t kv_stride_s, int batch_size, int q_heads, int kv_heads, int head_dim,
                                  int kv_len, const int32_t* kv_len_dev, float scale, void* workspace,
                                  int64_t workspace_bytes, uint16_t* out, int64_t o_stride_b, int64_t o_stride_h,
                                  const uint16_t* v_store, int64_t vs_stride_b, int64_t vs_stride_h,
                                  int64_t store_chunks, const int64_t* position_ids, int sparse_start,
                                  int select_sets, int chunk_size, void* stream);

/* Replaces the new token's rotary embedding (vllm rotary_embedding, models/llama.py:149-150,
 * models/glm.py:200-201) and the
 * KV append of update_kv_cache (models/kvcache/shadow.py:621-633) in one launch. qkv row of batch b:
 * [q_heads*128 | kv_heads*128 (k) | kv_heads*128 (v)] at qkv + b*qkv_stride_b. q and k are rotated
 * at positions[b] with the bf16 per-op rounding of the reference (rope_mode 0: half-split with
 * cos_sin rows [cos(64)|sin(64)]; 1: GLM interleaved pairs on dims 0..63, cos_sin [cos(32)|sin(32)]);
 * positions outside [0, cos_sin_rows) leave q/k unrotated. Rotated q goes to q_out[b, h, :]
 * (row stride q_out_stride_b, head stride 128); rotated k and raw v go to row *append_row (a
 * device int64, read when the kernel runs) of the key/value buffers
 * (cache + b*kv_stride_b + h*kv_stride_h + row*kv_stride_s); a row outside [0, buf_len) is not
 * written. The qkv buffer itself is not modified. */
int skv_rope_qk_append(const uint16_t* qkv, int64_t qkv_stride_b, int batch_size, int q_heads, int kv_heads,
                       int head_dim, const int64_t* positions, const uint16_t* cos_sin, int64_t stride_cos_sin,
                       int64_t cos_sin_rows, int rope_mode, uint16_t* q_out, int64_t q_out_stride_b,
                       uint16_t* k_cache, uint16_t* v_cache, int64_t kv_stride_b, int64_t kv_stride_h,
                       int64_t kv_stride_s, const int64_t* append_row, int64_t buf_len, void* stream);

/* The fused QKV projection (models/llama.py:192, models/glm.py:165 with its bias) with
 * skv_rope_qk_append in its epilogue: the [q | k | v] row of each of the m (<= 8) token rows x[b]
 * (k elements) is formed against the weight (plus bias, when not NULL, in the same row order) and
 * rounded to bf16, then rotated and appended exactly as skv_rope_qk_append does it (same arguments
 * and results; the fused row itself is not written). For rope_mode 0 the weight (and bias) is the
 * projection's with each q and k head's rows interleaved as (0, 64, 1, 65, ..., 63, 127), so that
 * both rows of a rotation pair fall in one workgroup (v rows unchanged); for rope_mode 1 (GLM:
 * pairs (2i, 2i+1)) it is the projection's weight as is. Weight rows: (q_heads + 2*kv_heads) * 128.
 * Bit-identical to skv_linear (skv_linear_bias) followed by skv_rope_qk_append. */
int skv_linear_qkv_rope_append(const uint16_t* x, int64_t x_stride, const uint16_t* weight, int64_t weight_stride,
                               const uint16_t* bias, int m, int k, int q_heads, int kv_heads, const int64_t* positions,
                               const uint16_t* cos_sin, int64_t stride_cos_sin, int64_t cos_sin_rows, int rope_mode,
                               uint16_t* q_out, int64_t q_out_stride_b, uint16_t* k_cache, uint16_t* v_cache,
                               int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_s,
                               const int64_t* append_row, int64_t buf_len, void* stream);

/* ---- measurement -------------------------------------------------------------------------
 * HBM read envelope probe. No reference counterpart: it measures what a read-only launch of a
 * given size reaches, the ceiling the streaming kernels are read against. Reads `tiles` tiles of
 * 64 KB from src, tiles_per_workgroup (1..64) consecutive tiles per workgroup of 256 threads, each
 * tile's 16 loads per thread in flight together, in one of two orders: pattern 0, every wave
 * instruction reads 1 KB of consecutive bytes; pattern 1, the tile as 256 rows of 256 bytes read
 * 64 bytes from each of 16 rows per instruction (the order of the scoring and attention kernels'
 * MFMA operand loads); pattern + 2, the same with non-temporal loads (global_load ... nt).
 * Thread t of workgroup g writes the XOR of the 16-byte vectors it read to
 * sink[g*256 + t] (16 bytes each; sink_bytes >= ceil(tiles / tiles_per_workgroup) * 4096). */
int skv_hbm_read_probe(const void* src, int64_t tiles, int tiles_per_workgroup, int pattern, void* sink,
                       int64_t sink_bytes, void* stream);

/* MFMA peak probe. No reference counterpart: it measures the bf16 matrix rate the rebuild's MFMA
 * utilisation is read against. Every wave of `workgroups` workgroups of 256 threads issues
 * iters x 4 independent v_mfma_f32_32x32x16_bf16 on register operands (no memory traffic) and
 * thread t of workgroup g writes one float to sink[g*256 + t] (sink_bytes >= workgroups * 1024).
 * skv_mfma_peak_probe_flops gives the flops of one call (0 for bad arguments). */
int skv_mfma_peak_probe(int workgroups, int iters, float* sink, int64_t sink_bytes, void* stream);
int64_t skv_mfma_peak_probe_flops(int workgroups, int iters);

#ifdef __cplusplus
}
#endif

#endif /* SHADOWKV_AMD_H */
