"""Drop-in for the reference's native module `kernels.shadowkv` (kernels/main.cu:24-36).

Every function keeps the reference's name, argument order and in-place output contract
(kernels/functions.h:23-121) and runs a hand-written gfx950 HIP kernel from
libshadowkv_amd.so on torch's current HIP stream. Differences from the reference, all of
them loud instead of silent:
  * unsupported sizes raise ValueError (the reference launches nothing for a map_size
    outside {128, 256, 512, 1024}, kernels/gather_copy.cu:132-323);
  * the host value store is addressed with the stride of the tensor actually passed
    (`values.stride(1)` of the [B, H, chunks, chunk*D] layer view) — the reference's
    `cpu_v_length` argument is checked against it but not used to address memory;
  * `temp` and `signals` are accepted for signature compatibility and ignored: the kernels
    need neither a staging buffer nor inter-workgroup flags.
Functions without a reference counterpart (score_gqa_max, topk_gather, rebuild_k_rope,
sparse_attn_decode) expose the fused kernels used by the decode path.
"""
from __future__ import annotations

import ctypes
import math

import torch

from .. import _lib

__all__ = [
    "gather_copy", "gather_copy_d2d_with_offsets", "reorder_keys_and_compute_offsets", "gather_copy_with_offsets",
    "apply_rotary_pos_emb_new", "apply_rotary_pos_emb_push_cache_opt", "apply_rotary_pos_emb_push_cache_opt_glm",
    "batch_gather_gemm", "batch_gemm_softmax", "score_gqa_max", "score_logits", "softmax_gqa_max", "select_chunks", "topk_gather", "rebuild_k_rope",
    "sparse_attn_workspace_bytes", "sparse_attn_workspace", "sparse_attn_decode", "sparse_attn_xcd_check",
    "device_address", "select_workspace_bytes",
]


def _stream() -> int:
    return int(torch.cuda.current_stream().cuda_stream)


def _dev(t: torch.Tensor, name: str, dtype: torch.dtype | None = None) -> int:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    return t.data_ptr()


def _span(t: torch.Tensor) -> int:
    """Elements addressable from t.data_ptr() to the end of its storage."""
    return t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()


def _need(t: torch.Tensor, elems: int, name: str) -> None:
    if _span(t) < elems:
        raise ValueError(f"{name} holds {_span(t)} elements from its start, {elems} are addressed")


_host_base_cache: dict[int, int] = {}


def device_address(t: torch.Tensor) -> int:
    """Device address of a device tensor, or of a pinned host tensor (zero-copy access)."""
    if t.is_cuda:
        return t.data_ptr()
    if not t.is_pinned():
        raise ValueError("host tensors passed to the kernels must be pinned (pin_memory=True)")
    base = t.untyped_storage().data_ptr()
    dev = _host_base_cache.get(base)
    if dev is None:
        dev = _lib.host_device_pointer(base)
        _host_base_cache[base] = dev
    return dev + (t.data_ptr() - base)


def max_offset(sizes, strides) -> int:
    """Largest element offset addressed by an index space of `sizes` with `strides` (>= 0)."""
    if any(sz <= 0 for sz in sizes):
        return -1
    if any(st < 0 for st in strides):
        raise ValueError("negative strides are not supported")
    return sum((sz - 1) * st for sz, st in zip(sizes, strides))


def _need_offsets(t: torch.Tensor, sizes, strides, name: str) -> None:
    """Every offset of the index space must fall inside t's storage (from t.data_ptr())."""
    _need(t, max_offset(sizes, strides) + 1, name)


def _check_map(map_size: int) -> None:
    if not 1 <= map_size <= 2048:
        raise ValueError(f"map_size (select_sets) must be in [1, 2048], got {map_size}")


# ---------------------------------------------------------------------------------------------
# a3: reorder (kernels/gather_copy.cu:189-235)

def reorder_keys_and_compute_offsets(cached_pos_ids, cur_pos_ids, offsets, cnts, batch_size, heads, map_size=256):
    _check_map(map_size)
    rows = batch_size * heads
    for t, n, dt in ((cached_pos_ids, "cached_pos_ids", torch.int64), (cur_pos_ids, "cur_pos_ids", torch.int64),
                     (offsets, "offsets", torch.int32), (cnts, "cnts", torch.int32)):
        _dev(t, n, dt)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    for t, n, e in ((cached_pos_ids, "cached_pos_ids", rows * map_size), (cur_pos_ids, "cur_pos_ids", rows * map_size),
                    (offsets, "offsets", rows * map_size), (cnts, "cnts", rows)):
        _need(t, e, n)
    _lib.call("skv_reorder_keys_and_compute_offsets", cached_pos_ids.data_ptr(), cur_pos_ids.data_ptr(),
              offsets.data_ptr(), cnts.data_ptr(), batch_size, heads, map_size, _stream())


# ---------------------------------------------------------------------------------------------
# a4/a5: chunk copies (kernels/gather_copy.cu:47-185, 239-324)

def _host_row_stride(values: torch.Tensor, rows: int, cpu_v_length: int) -> int:
    """Per-(b,h) element stride of the host store [B, H, chunks, chunk*D] (or a flat buffer)."""
    if values.dim() == 4:
        if values.stride(0) != values.shape[1] * values.stride(1) or values.stride(3) != 1 or \
                values.stride(2) != values.shape[3]:
            raise ValueError("host value store must be contiguous per layer: [B, H, chunks, chunk*D]")
        stride = values.stride(1)
        if cpu_v_length > stride:
            raise ValueError(f"cpu_v_length={cpu_v_length} exceeds the host row stride {stride}")
        return stride
    if not values.is_contiguous():
        raise ValueError("host value store must be contiguous")
    return cpu_v_length


def gather_copy_with_offsets(values, v_cache_buffer, temp, offsets, cnts, signals, batch_size, heads, cpu_v_length,
                             gpu_v_length, gpu_v_offset, gpu_v_stride, map_size=256, *, misses_only=False):
    """Value fetch: hit rows moved within v_cache_buffer to their new slots, then miss chunks
    gathered from pinned host `values`. misses_only: the gather alone (the hit move issued
    beforehand by gather_copy_d2d_with_offsets on the value buffer, e.g. on another stream)."""
    del temp, signals  # no staging buffer or flags are needed
    _check_map(map_size)
    if gpu_v_length % map_size:
        raise ValueError(f"gpu_v_length={gpu_v_length} is not map_size*chunk_elems")
    chunk_elems = gpu_v_length // map_size
    rows = batch_size * heads
    row_stride = _host_row_stride(values, rows, cpu_v_length)
    _need(values, (rows - 1) * row_stride + row_stride, "values")
    _dev(v_cache_buffer, "v_cache_buffer", torch.bfloat16)
    _need(v_cache_buffer, (rows - 1) * gpu_v_stride + gpu_v_offset + gpu_v_length, "v_cache_buffer")
    _dev(offsets, "offsets", torch.int32)
    _dev(cnts, "cnts", torch.int32)
    _need(offsets, rows * map_size, "offsets")
    _need(cnts, rows, "cnts")
    if values.dtype != torch.bfloat16:
        raise ValueError("values must be bf16")
    _lib.call("skv_gather_copy_misses_with_offsets" if misses_only else "skv_gather_copy_with_offsets",
              device_address(values), v_cache_buffer.data_ptr(), offsets.data_ptr(), cnts.data_ptr(), batch_size,
              heads, row_stride, gpu_v_length, gpu_v_offset, gpu_v_stride, map_size, chunk_elems, _stream())


def gather_copy_d2d_with_offsets(keys, offsets, cnts, batch_size, heads, gpu_v_length, gpu_v_offset, gpu_v_stride,
                                 map_size=256):
    _check_map(map_size)
    if gpu_v_length % map_size:
        raise ValueError(f"gpu_v_length={gpu_v_length} is not map_size*chunk_elems")
    rows = batch_size * heads
    _dev(keys, "keys", torch.bfloat16)
    _need(keys, (rows - 1) * gpu_v_stride + gpu_v_offset + gpu_v_length, "keys")
    _dev(offsets, "offsets", torch.int32)
    _dev(cnts, "cnts", torch.int32)
    _need(offsets, rows * map_size, "offsets")
    _need(cnts, rows, "cnts")
    _lib.call("skv_gather_copy_d2d_with_offsets", keys.data_ptr(), offsets.data_ptr(), cnts.data_ptr(), batch_size,
              heads, gpu_v_length, gpu_v_offset, gpu_v_stride, map_size, gpu_v_length // map_size, _stream())


def gather_copy(values, v_cache_buffer, position_ids, batch_size, heads, cpu_v_length, gpu_v_length, map_size=256):
    _check_map(map_size)
    if gpu_v_length % map_size:
        raise ValueError(f"gpu_v_length={gpu_v_length} is not map_size*chunk_elems")
    rows = batch_size * heads
    row_stride = _host_row_stride(values, rows, cpu_v_length)
    _need(values, rows * row_stride, "values")
    _dev(v_cache_buffer, "v_cache_buffer", torch.bfloat16)
    _need(v_cache_buffer, rows * gpu_v_length, "v_cache_buffer")
    _dev(position_ids, "position_ids", torch.int64)
    _need(position_ids, rows * map_size, "position_ids")
    _lib.call("skv_gather_copy", device_address(values), v_cache_buffer.data_ptr(), position_ids.data_ptr(),
              batch_size, heads, row_stride, gpu_v_length, map_size, gpu_v_length // map_size, _stream())


# ---------------------------------------------------------------------------------------------
# a7: RoPE (kernels/rope_new.cu)

def apply_rotary_pos_emb_new(x, cos_sin, position_ids, output, batch_size, heads, seq_len, embed_dim, stride_xb,
                             stride_xh, stride_xs, stride_xe, stride_cos_sin, stride_pid_b, stride_pid_h, stride_pid_s,
                             half_dim):
    _dev(x, "x", torch.bfloat16)
    _dev(cos_sin, "cos_sin", torch.bfloat16)
    _dev(position_ids, "position_ids", torch.int64)
    _dev(output, "output", torch.bfloat16)
    # x and output are both addressed with x's strides (reference rope_new.cu:45-47)
    xs = (batch_size, heads, seq_len, embed_dim)
    xst = (stride_xb, stride_xh, stride_xs, stride_xe)
    _need_offsets(x, xs, xst, "x")
    _need_offsets(output, xs, xst, "output")
    _need_offsets(position_ids, (batch_size, heads, seq_len), (stride_pid_b, stride_pid_h, stride_pid_s), "position_ids")
    _lib.call("skv_apply_rotary_pos_emb_new", x.data_ptr(), cos_sin.data_ptr(), position_ids.data_ptr(),
              output.data_ptr(), batch_size, heads, seq_len, embed_dim, stride_xb, stride_xh, stride_xs, stride_xe,
              stride_cos_sin, stride_pid_b, stride_pid_h, stride_pid_s, half_dim, cos_sin.shape[0], _stream())


def apply_rotary_pos_emb(x, cos, sin, position_ids, output, batch_size, heads, seq_len, embed_dim, stride_xb,
                         stride_xh, stride_xs, stride_xe, stride_cos, stride_sin, stride_pid_b, stride_pid_h,
                         stride_pid_s, half_dim):
    """RoPE with separate cos and sin tables (kernels/functions.h:53-59): output at x's strides."""
    _dev(x, "x", torch.bfloat16)
    _dev(cos, "cos", torch.bfloat16)
    _dev(sin, "sin", torch.bfloat16)
    _dev(position_ids, "position_ids", torch.int64)
    _dev(output, "output", torch.bfloat16)
    xs = (batch_size, heads, seq_len, embed_dim)
    xst = (stride_xb, stride_xh, stride_xs, stride_xe)
    _need_offsets(x, xs, xst, "x")
    _need_offsets(output, xs, xst, "output")
    _need_offsets(position_ids, (batch_size, heads, seq_len), (stride_pid_b, stride_pid_h, stride_pid_s), "position_ids")
    rows = min(cos.numel() // max(1, stride_cos), sin.numel() // max(1, stride_sin))
    if rows < 1 or cos.shape[-1] < embed_dim or sin.shape[-1] < embed_dim:
        raise ValueError("apply_rotary_pos_emb: cos/sin tables need rows of embed_dim entries")
    _lib.call("skv_apply_rotary_pos_emb", x.data_ptr(), cos.data_ptr(), sin.data_ptr(), position_ids.data_ptr(),
              output.data_ptr(), batch_size, heads, seq_len, embed_dim, stride_xb, stride_xh, stride_xs, stride_xe,
              stride_cos, stride_sin, stride_pid_b, stride_pid_h, stride_pid_s, half_dim, rows, _stream())


def apply_rotary_pos_emb_new_v2(x, cos_sin, position_ids, output, batch_size, heads, seq_len, embed_dim, stride_xb,
                                stride_xh, stride_xs, stride_xe, stride_cos_sin, stride_pid_b, stride_pid_h,
                                stride_pid_s, half_dim, chunk_size):
    """RoPE of every row at the position of its chunk id (kernels/functions.h:69-75): row s of (b, h)
    at table row position_ids[b, h, s // chunk_size] * chunk_size + s % chunk_size (int32 ids)."""
    _dev(x, "x", torch.bfloat16)
    _dev(cos_sin, "cos_sin", torch.bfloat16)
    _dev(position_ids, "position_ids", torch.int32)
    _dev(output, "output", torch.bfloat16)
    xs = (batch_size, heads, seq_len, embed_dim)
    xst = (stride_xb, stride_xh, stride_xs, stride_xe)
    _need_offsets(x, xs, xst, "x")
    _need_offsets(output, xs, xst, "output")
    _need_offsets(position_ids, (batch_size, heads, (seq_len + chunk_size - 1) // chunk_size),
                  (stride_pid_b, stride_pid_h, stride_pid_s), "position_ids")
    _lib.call("skv_apply_rotary_pos_emb_new_v2", x.data_ptr(), cos_sin.data_ptr(), position_ids.data_ptr(),
              output.data_ptr(), batch_size, heads, seq_len, embed_dim, stride_xb, stride_xh, stride_xs, stride_xe,
              stride_cos_sin, stride_pid_b, stride_pid_h, stride_pid_s, half_dim, chunk_size, cos_sin.shape[0],
              _stream())


def apply_rotary_pos_emb_push_cache(x, cos_sin, position_ids, output, cnts, batch_size, heads, seq_len, embed_dim,
                                    stride_xb, stride_xh, stride_xs, stride_xe, stride_cos_sin, stride_pid_b,
                                    stride_pid_h, stride_pid_s, stride_output_b, stride_output_h, stride_output_s,
                                    offset_output_s_start, offset_output_s_end, half_dim, chunk_size):
    """kernels/functions.h:77-86: the contract of apply_rotary_pos_emb_push_cache_opt."""
    _push("skv_apply_rotary_pos_emb_push_cache", x, cos_sin, position_ids, output, cnts, batch_size, heads,
          seq_len, embed_dim, stride_xb, stride_xh, stride_xs, stride_xe, stride_cos_sin, stride_pid_b, stride_pid_h,
          stride_pid_s, stride_output_b, stride_output_h, stride_output_s, offset_output_s_start, offset_output_s_end,
          half_dim, chunk_size)


def _push(name, x, cos_sin, position_ids, output, cnts, *ints):
    _dev(x, "x", torch.bfloat16)
    _dev(cos_sin, "cos_sin", torch.bfloat16)
    _dev(position_ids, "position_ids", torch.int32)
    _dev(output, "output", torch.bfloat16)
    _dev(cnts, "cnts", torch.int32)
    (b, h, s, d, sxb, sxh, sxs, sxe, _scs, spb, sph, sps, sob, soh, sos, start, end, _half, chunk) = ints
    _need_offsets(x, (b, h, s, d), (sxb, sxh, sxs, sxe), "x")
    _need_offsets(position_ids, (b, h, (s + chunk - 1) // chunk), (spb, sph, sps), "position_ids")
    rows = max(0, min(s, end - start))
    _need(output, max_offset((b, h, rows, d), (sob, soh, sos, 1)) + 1 + start * sos, "output")
    _need(cnts, b * h, "cnts")
    _lib.call(name, x.data_ptr(), cos_sin.data_ptr(), position_ids.data_ptr(), output.data_ptr(), cnts.data_ptr(),
              *ints, cos_sin.shape[0], _stream())


def apply_rotary_pos_emb_push_cache_opt(x, cos_sin, position_ids, output, cnts, batch_size, heads, seq_len, embed_dim,
                                        stride_xb, stride_xh, stride_xs, stride_xe, stride_cos_sin, stride_pid_b,
                                        stride_pid_h, stride_pid_s, stride_output_b, stride_output_h, stride_output_s,
                                        offset_output_s_start, offset_output_s_end, half_dim, chunk_size):
    _push("skv_apply_rotary_pos_emb_push_cache_opt", x, cos_sin, position_ids, output, cnts, batch_size, heads,
          seq_len, embed_dim, stride_xb, stride_xh, stride_xs, stride_xe, stride_cos_sin, stride_pid_b, stride_pid_h,
          stride_pid_s, stride_output_b, stride_output_h, stride_output_s, offset_output_s_start, offset_output_s_end,
          half_dim, chunk_size)


def apply_rotary_pos_emb_push_cache_opt_glm(x, cos_sin, position_ids, output, cnts, batch_size, heads, seq_len,
                                            embed_dim, stride_xb, stride_xh, stride_xs, stride_xe, stride_cos_sin,
                                            stride_pid_b, stride_pid_h, stride_pid_s, stride_output_b, stride_output_h,
                                            stride_output_s, offset_output_s_start, offset_output_s_end, half_dim,
                                            chunk_size):
    _push("skv_apply_rotary_pos_emb_push_cache_opt_glm", x, cos_sin, position_ids, output, cnts, batch_size, heads,
          seq_len, embed_dim, stride_xb, stride_xh, stride_xs, stride_xe, stride_cos_sin, stride_pid_b, stride_pid_h,
          stride_pid_s, stride_output_b, stride_output_h, stride_output_s, offset_output_s_start, offset_output_s_end,
          half_dim, chunk_size)


# ---------------------------------------------------------------------------------------------
# a6: gathered low-rank GEMM (kernels/batch_gather_gemm.cu:136-213)

def batch_gather_gemm(a, b, cos, sin, position_ids, output, batch_size, heads, seq_len, embed_dim, rank,
                      sparse_budget, max_seq_len, chunk_size, offset_array):
    del cos, sin  # the reference's RoPE epilogue is disabled; rebuild_k_rope fuses it instead
    for t, n in ((a, "a"), (b, "b"), (output, "output")):
        _dev(t, n, torch.bfloat16)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    _dev(position_ids, "position_ids", torch.int32)
    _dev(offset_array, "offset_array", torch.int32)
    _need(a, batch_size * seq_len * rank, "a")
    _need(b, batch_size * heads * embed_dim * rank, "b")
    _need(output, batch_size * heads * sparse_budget * embed_dim, "output")
    _need(position_ids, batch_size * heads * (sparse_budget // chunk_size), "position_ids")
    _lib.call("skv_batch_gather_gemm", a.data_ptr(), b.data_ptr(), position_ids.data_ptr(), output.data_ptr(),
              batch_size, heads, seq_len, embed_dim, rank, sparse_budget, max_seq_len, chunk_size,
              offset_array.data_ptr(), _stream())


def rebuild_k_rope(u, sv, position_ids, cnts, cos_sin, cache, sparse_start, chunk_size, miss_slot=None,
                   pool_slots=None):
    """Fused a6+a7: rebuild the miss rows of every (b, h) and push them, rotated, into `cache`.

    u: [B, ctx, R] (head-shared, the reference layout) or [B, H, ctx, R] (per-head);
    sv: [B, H, 128, R] (reference layout) or [H, 128, R] (shared across the batch);
    position_ids: [B, H, S] int64 chunk ids; cnts: [B*H] int32 hit counts;
    cos_sin: [rows, 128] ([cos|sin], half-split RoPE) or [rows, 64] (GLM interleaved);
    cache: [B, H, buf_len, 128] key buffer; rows sparse_start + r are written.
    Chunk pool: position_ids are the int32 miss ids [B, H, S] of pool_assign and miss_slot
    [B, H, S] int32 their slots; entry i goes to rows sparse_start + miss_slot[i]*chunk_size + j.
    """
    B, H, S = position_ids.shape
    _dev(position_ids, "position_ids", torch.int32 if miss_slot is not None else torch.int64)
    slots = S if miss_slot is None else pool_slots
    geo = _rebuild_geometry(u, sv, position_ids, cnts, cos_sin, cache, sparse_start, chunk_size, slots)
    (u_sb, u_sh, u_sr, u_rows, sv_sb, sv_sh, sv_sn, mode, rank) = geo
    if miss_slot is not None:
        _dev(miss_slot, "miss_slot", torch.int32)
        if not (position_ids.is_contiguous() and miss_slot.is_contiguous()) or miss_slot.numel() != B * H * S:
            raise ValueError("pool miss lists must be contiguous [B, H, S]")
        _lib.call("skv_rebuild_k_rope_slots", u.data_ptr(), u_sb, u_sh, u_sr, u_rows, sv.data_ptr(), sv_sb, sv_sh,
                  sv_sn, position_ids.data_ptr(), miss_slot.data_ptr(), cnts.data_ptr(), cos_sin.data_ptr(),
                  cos_sin.stride(0), cos_sin.shape[0], mode, cache.data_ptr(), cache.stride(0), cache.stride(1),
                  cache.stride(2), sparse_start, pool_slots, B, H, S, chunk_size, rank, 128, _stream())
        return
    _lib.call("skv_rebuild_k_rope", u.data_ptr(), u_sb, u_sh, u_sr, u_rows, sv.data_ptr(), sv_sb, sv_sh, sv_sn,
              position_ids.data_ptr(), position_ids.stride(0), position_ids.stride(1), cnts.data_ptr(),
              cos_sin.data_ptr(), cos_sin.stride(0), cos_sin.shape[0], mode, cache.data_ptr(), cache.stride(0),
              cache.stride(1), cache.stride(2), sparse_start, B, H, S, chunk_size, rank, 128, _stream())


def _rebuild_geometry(u, sv, position_ids, cnts, cos_sin, cache, sparse_start, chunk_size, slots):
    """Checks of the rebuild operands and their strides: (u_sb, u_sh, u_sr, u_rows, sv_sb, sv_sh,
    sv_sn, rope mode, rank)."""
    B, H, S = position_ids.shape
    _dev(u, "u", torch.bfloat16)
    _dev(sv, "sv", torch.bfloat16)
    _dev(cnts, "cnts", torch.int32)
    _dev(cos_sin, "cos_sin", torch.bfloat16)
    _dev(cache, "cache", torch.bfloat16)
    if u.dim() == 3:
        u_sb, u_sh, u_sr, u_rows = u.stride(0), 0, u.stride(1), u.shape[1]
        if u.shape[0] != B:
            raise ValueError("u batch mismatch")
    elif u.dim() == 4:
        u_sb, u_sh, u_sr, u_rows = u.stride(0), u.stride(1), u.stride(2), u.shape[2]
        if u.shape[0] != B or u.shape[1] != H:
            raise ValueError("u batch/head mismatch")
    else:
        raise ValueError("u must be [B, ctx, R] or [B, H, ctx, R]")
    rank = u.shape[-1]
    if u.stride(-1) != 1:
        raise ValueError("u rows must be contiguous")
    if sv.dim() == 4:
        sv_sb, sv_sh, sv_sn = sv.stride(0), sv.stride(1), sv.stride(2)
    elif sv.dim() == 3:
        sv_sb, sv_sh, sv_sn = 0, sv.stride(0), sv.stride(1)
    else:
        raise ValueError("sv must be [B, H, 128, R] or [H, 128, R]")
    if sv.shape[-1] != rank or sv.shape[-2] != 128 or sv.stride(-1) != 1:
        raise ValueError("sv must end in a contiguous [128, rank] block")
    if cos_sin.shape[-1] == 128:
        mode = 0
    elif cos_sin.shape[-1] == 64:
        mode = 1
    else:
        raise ValueError(f"Invalid cos_sin shape {tuple(cos_sin.shape)}")
    if cache.dim() != 4 or cache.shape[-1] != 128 or cache.stride(-1) != 1:
        raise ValueError("cache must be [B, H, buf_len, 128]")
    if sparse_start + slots * chunk_size > cache.shape[2]:
        raise ValueError("sparse region exceeds the cache buffer")
    if position_ids.stride(2) != 1:
        raise ValueError("position_ids must be contiguous along the chunk axis")
    _need(cnts, B * H, "cnts")
    return u_sb, u_sh, u_sr, u_rows, sv_sb, sv_sh, sv_sn, mode, rank


def fetch_misses_rebuild_k_rope(values, v_cache_buffer, offsets, cnts, cpu_v_length, gpu_v_offset, gpu_v_stride,
                                u, sv, position_ids, cos_sin, cache, sparse_start, chunk_size, fetch_workgroups=0,
                                rebuild_workgroups=0):
    """The value fetch of the misses (gather_copy_with_offsets(..., misses_only=True)) and the key
    rebuild (rebuild_k_rope) in one launch on the current stream, their workgroups side by side.
    Both buffers' hits must already be in place (select_chunks with move=(v_buffer, k_buffer, ...)).
    Same arguments and results as the two calls; the value chunk is chunk_size * 128 elements.
    fetch_workgroups: the fetch workgroups to aim for, in 4-wave workgroups (0: the library's
    default). rebuild_workgroups: 0 gives every rebuild tile its own workgroup; a positive cap makes
    that many workgroups loop over the tiles (where the kernel instance supports it), spreading the
    rebuild over the fetch."""
    B, H, S = position_ids.shape
    _dev(position_ids, "position_ids", torch.int64)
    u_sb, u_sh, u_sr, u_rows, sv_sb, sv_sh, sv_sn, mode, rank = _rebuild_geometry(
        u, sv, position_ids, cnts, cos_sin, cache, sparse_start, chunk_size, S)
    rows = B * H
    chunk_elems = chunk_size * 128
    row_stride = _host_row_stride(values, rows, cpu_v_length)
    _need(values, (rows - 1) * row_stride + row_stride, "values")
    if values.dtype != torch.bfloat16:
        raise ValueError("values must be bf16")
    _dev(v_cache_buffer, "v_cache_buffer", torch.bfloat16)
    _need(v_cache_buffer, (rows - 1) * gpu_v_stride + gpu_v_offset + S * chunk_elems, "v_cache_buffer")
    _dev(offsets, "offsets", torch.int32)
    _need(offsets, rows * S, "offsets")
    _lib.call("skv_fetch_misses_rebuild_k_rope", device_address(values), v_cache_buffer.data_ptr(), offsets.data_ptr(),
              row_stride, gpu_v_offset, gpu_v_stride, u.data_ptr(), u_sb, u_sh, u_sr, u_rows, sv.data_ptr(), sv_sb,
              sv_sh, sv_sn, position_ids.data_ptr(), position_ids.stride(0), position_ids.stride(1), cnts.data_ptr(),
              cos_sin.data_ptr(), cos_sin.stride(0), cos_sin.shape[0], mode, cache.data_ptr(), cache.stride(0),
              cache.stride(1), cache.stride(2), sparse_start, B, H, S, chunk_size, rank, 128, int(fetch_workgroups),
              int(rebuild_workgroups), _stream())


def fetch_misses_rebuild_k_rope_slots(values, v_cache_buffer, miss_ids, cnts, miss_slot, cpu_v_length, pool_offset,
                                      gpu_v_stride, u, sv, cos_sin, cache, sparse_start, chunk_size, pool_slots,
                                      fetch_workgroups=0, rebuild_workgroups=0):
    """A chunk pool's miss gather (gather_copy_misses_to_slots) and key rebuild (rebuild_k_rope with
    miss_slot) in one launch on the current stream, their workgroups side by side: entries i >=
    cnts[r] of pool_assign's miss list, chunk miss_ids[b, h, i] (int32 [B, H, S]) into slot
    miss_slot[b, h, i] of both buffers. Same arguments and results as the two calls (pool_offset =
    sparse_start * 128); fetch_workgroups / rebuild_workgroups as for fetch_misses_rebuild_k_rope."""
    B, H, S = miss_ids.shape
    _dev(miss_ids, "miss_ids", torch.int32)
    _dev(miss_slot, "miss_slot", torch.int32)
    if not (miss_ids.is_contiguous() and miss_slot.is_contiguous()) or miss_slot.numel() != B * H * S:
        raise ValueError("miss_ids and miss_slot must be contiguous [B, H, S]")
    if pool_slots < S:
        raise ValueError(f"pool_slots={pool_slots} holds fewer than the {S} selected chunks")
    u_sb, u_sh, u_sr, u_rows, sv_sb, sv_sh, sv_sn, mode, rank = _rebuild_geometry(
        u, sv, miss_ids, cnts, cos_sin, cache, sparse_start, chunk_size, pool_slots)
    rows = B * H
    chunk_elems = chunk_size * 128
    row_stride = _host_row_stride(values, rows, cpu_v_length)
    _need(values, (rows - 1) * row_stride + row_stride, "values")
    if values.dtype != torch.bfloat16:
        raise ValueError("values must be bf16")
    _dev(v_cache_buffer, "v_cache_buffer", torch.bfloat16)
    _need(v_cache_buffer, (rows - 1) * gpu_v_stride + pool_offset + pool_slots * chunk_elems, "v_cache_buffer")
    _lib.call("skv_fetch_misses_rebuild_k_rope_slots", device_address(values), v_cache_buffer.data_ptr(), row_stride,
              pool_offset, gpu_v_stride, u.data_ptr(), u_sb, u_sh, u_sr, u_rows, sv.data_ptr(), sv_sb, sv_sh, sv_sn,
              miss_ids.data_ptr(), miss_slot.data_ptr(), cnts.data_ptr(), cos_sin.data_ptr(), cos_sin.stride(0),
              cos_sin.shape[0], mode, cache.data_ptr(), cache.stride(0), cache.stride(1), cache.stride(2),
              sparse_start, pool_slots, B, H, S, chunk_size, rank, 128, int(fetch_workgroups),
              int(rebuild_workgroups), _stream())


# ---------------------------------------------------------------------------------------------
# a1/a2: scoring, GQA max, top-k

def _check_scoring(A, B, D, Norm, Sum, batch_count, m, n, k):
    for t, nm in ((A, "A"), (B, "B"), (D, "D")):
        _dev(t, nm, torch.bfloat16)
        if not t.is_contiguous():
            raise ValueError(f"{nm} must be contiguous")
    _dev(Norm, "Norm", torch.float32)
    _dev(Sum, "Sum", torch.float32)
    tiles = (n + 255) // 256
    _need(A, batch_count * m * k, "A")
    _need(B, batch_count * n * k, "B")
    _need(D, batch_count * m * n, "D")
    _need(Norm, batch_count * m * tiles, "Norm")
    _need(Sum, batch_count * m * tiles, "Sum")


def batch_gemm_softmax(A, B, D, Norm, Sum, Softmax, batch_count, m, n, k, alpha=1.0, beta=0.0):
    _check_scoring(A, B, D, Norm, Sum, batch_count, m, n, k)
    _dev(Softmax, "Softmax", torch.bfloat16)
    _need(Softmax, batch_count * m * n, "Softmax")
    _lib.call("skv_batch_gemm_softmax", A.data_ptr(), B.data_ptr(), D.data_ptr(), Norm.data_ptr(), Sum.data_ptr(),
              Softmax.data_ptr(), batch_count, m, n, k, float(alpha), float(beta), _stream())


def score_gqa_max(A, B, D, Norm, Sum, out, batch_count, m, n, k, alpha=1.0 / math.sqrt(128)):
    """out[z, j] = max_i softmax(alpha * A[z] . B[z]^T)[i, j] in bf16; D/Norm/Sum are scratch."""
    _check_scoring(A, B, D, Norm, Sum, batch_count, m, n, k)
    _dev(out, "out", torch.bfloat16)
    _need(out, batch_count * n, "out")
    _lib.call("skv_score_gqa_max", A.data_ptr(), B.data_ptr(), D.data_ptr(), Norm.data_ptr(), Sum.data_ptr(),
              out.data_ptr(), batch_count, m, n, k, float(alpha), _stream())


def score_logits(A, B, D, Norm, Sum, batch_count, m, n, k, alpha=1.0 / math.sqrt(128)):
    """First scoring kernel: D = bf16(alpha A.B^T) and per-256-column max / sum(exp) partials."""
    _check_scoring(A, B, D, Norm, Sum, batch_count, m, n, k)
    _lib.call("skv_score_logits", A.data_ptr(), B.data_ptr(), D.data_ptr(), Norm.data_ptr(), Sum.data_ptr(),
              batch_count, m, n, k, float(alpha), _stream())


def softmax_gqa_max(D, Norm, Sum, out, batch_count, m, n, softmax=None):
    """Second scoring kernel: softmax over n from the partials, max over the m rows into out [batch, n]."""
    for t, nm in ((D, "D"), (out, "out")):
        _dev(t, nm, torch.bfloat16)
    _dev(Norm, "Norm", torch.float32)
    _dev(Sum, "Sum", torch.float32)
    tiles = (n + 255) // 256
    _need(D, batch_count * m * n, "D")
    _need(Norm, batch_count * m * tiles, "Norm")
    _need(Sum, batch_count * m * tiles, "Sum")
    _need(out, batch_count * n, "out")
    sm = 0
    if softmax is not None:
        _dev(softmax, "softmax", torch.bfloat16)
        _need(softmax, batch_count * m * n, "softmax")
        sm = softmax.data_ptr()
    _lib.call("skv_softmax_gqa_max", D.data_ptr(), Norm.data_ptr(), Sum.data_ptr(), sm or None, out.data_ptr(),
              batch_count, m, n, _stream())


def select_workspace_bytes(rows: int, n: int, select_sets: int) -> int:
    return int(_lib.lib().skv_select_workspace_bytes(rows, n, select_sets))


def select_chunks(D, Norm, Sum, rows, m, n, landmark_idx, select_sets, num_chunks, position_ids, offsets, cnts,
                  out_scores=None, out_selected=None, workspace=None, move=None):
    """Fused softmax + GQA max + top-k + id gather + reorder (one workgroup per row; for few rows
    the softmax + GQA max runs first on many workgroups into out_scores, a second launch).

    D/Norm/Sum: outputs of score_logits for `rows` entries of m query rows; landmark_idx: [rows, n]
    view with contiguous rows, chunk ids in [0, num_chunks); position_ids: [rows, select_sets] int64
    (in: previous slots, -1 = empty; out: reordered); offsets: [rows * select_sets] int32; cnts:
    [rows] int32; out_scores: optional [rows, n] bf16 GQA-max probabilities; out_selected: optional
    [rows, select_sets] ids in top-k order (the reference's selected_chunks; costs a sort);
    workspace: optional device buffer of select_workspace_bytes(rows, n, select_sets) bytes, with
    which few rows (<= 32) are each selected by many workgroups. position_ids, offsets and cnts
    None: selection only (no previous slots, no reorder), the ids in top-k order into the then
    required out_selected (what a chunk pool selects before its own hit lookup).
    move: optional (v_buffer, k_buffer, buf_offset, buf_stride, chunk_elems): the hit moves folded
    into the selection's last launch, i.e. gather_copy_d2d_with_offsets(buffer, offsets, cnts, ...)
    on each buffer given (either may be None; buffer rows of buf_stride elements, the selected
    region at buf_offset, chunks of chunk_elems) done by the selection itself."""
    _dev(D, "D", torch.bfloat16)
    _dev(Norm, "Norm", torch.float32)
    _dev(Sum, "Sum", torch.float32)
    _dev(landmark_idx, "landmark_idx", torch.int64)
    reorder = position_ids is not None
    if reorder:
        _dev(position_ids, "position_ids", torch.int64)
        _dev(offsets, "offsets", torch.int32)
        _dev(cnts, "cnts", torch.int32)
    elif offsets is not None or cnts is not None or out_selected is None:
        raise ValueError("without position_ids, offsets and cnts must be None and out_selected given")
    if landmark_idx.dim() != 2 or landmark_idx.shape[1] != n or landmark_idx.stride(1) != 1:
        raise ValueError("landmark_idx must be [rows, n] with contiguous rows")
    if not (1 <= select_sets <= min(n, 2048)):
        raise ValueError(f"select_sets={select_sets} must be in [1, min(n={n}, 2048)]")
    tiles = (n + 255) // 256
    _need(D, rows * m * n, "D")
    _need(Norm, rows * m * tiles, "Norm")
    _need(Sum, rows * m * tiles, "Sum")
    _need(landmark_idx, (rows - 1) * landmark_idx.stride(0) + n, "landmark_idx")
    if reorder:
        for t, nm, e in ((position_ids, "position_ids", rows * select_sets), (offsets, "offsets", rows * select_sets),
                         (cnts, "cnts", rows)):
            if not t.is_contiguous():
                raise ValueError(f"{nm} must be contiguous")
            _need(t, e, nm)
    sp = None
    if out_scores is not None:
        _dev(out_scores, "out_scores", torch.bfloat16)
        _need(out_scores, rows * n, "out_scores")
        sp = out_scores.data_ptr()
    op = None
    if out_selected is not None:
        _dev(out_selected, "out_selected", torch.int64)
        if not out_selected.is_contiguous():
            raise ValueError("out_selected must be contiguous")
        _need(out_selected, rows * select_sets, "out_selected")
        op = out_selected.data_ptr()
    args = (D.data_ptr(), Norm.data_ptr(), Sum.data_ptr(), rows, m, n, landmark_idx.data_ptr(),
            landmark_idx.stride(0), select_sets, num_chunks, position_ids.data_ptr() if reorder else None,
            offsets.data_ptr() if reorder else None, cnts.data_ptr() if reorder else None, sp, op)
    wp, nbytes = None, 0
    if workspace is not None:
        _dev(workspace, "workspace")
        nbytes = workspace.numel() * workspace.element_size()
        if nbytes < select_workspace_bytes(rows, n, select_sets):
            raise ValueError(f"workspace of {nbytes} bytes, {select_workspace_bytes(rows, n, select_sets)} needed")
        wp = workspace.data_ptr()
    if move is not None:
        if not reorder:
            raise ValueError("the folded hit moves need position_ids, offsets and cnts")
        v_buf, k_buf, buf_offset, buf_stride, chunk_elems = move
        if v_buf is None and k_buf is None:
            raise ValueError("move names no buffer")
        ptrs = []
        for t, nm in ((v_buf, "v_buffer"), (k_buf, "k_buffer")):
            if t is None:
                ptrs.append(None)
                continue
            _dev(t, nm, torch.bfloat16)
            if not t.is_contiguous():
                raise ValueError(f"{nm} must be contiguous")
            _need(t, (rows - 1) * buf_stride + buf_offset + select_sets * chunk_elems, nm)
            ptrs.append(t.data_ptr())
        _lib.call("skv_select_chunks_compact", *args, wp, nbytes, ptrs[0], ptrs[1], int(buf_offset), int(buf_stride),
                  int(chunk_elems), _stream())
    elif workspace is None:
        _lib.call("skv_select_chunks", *args, _stream())
    else:
        _lib.call("skv_select_chunks_ws", *args, wp, nbytes, _stream())


def topk_gather(scores, landmark_idx, k, out_ids):
    """out_ids[r] = landmark_idx[r, top-k of scores[r] by (value desc, index asc)]; 2-D row views."""
    _dev(scores, "scores", torch.bfloat16)
    _dev(landmark_idx, "landmark_idx", torch.int64)
    _dev(out_ids, "out_ids", torch.int64)
    if scores.dim() != 2 or landmark_idx.shape != scores.shape or scores.stride(1) != 1 or landmark_idx.stride(1) != 1:
        raise ValueError("scores and landmark_idx must be [rows, n] with contiguous rows")
    rows, n = scores.shape
    if not 1 <= k <= min(n, 4096):
        raise ValueError(f"k={k} must be in [1, min(n={n}, 4096)]")
    if not out_ids.is_contiguous():
        raise ValueError("out_ids must be contiguous")
    _need(out_ids, rows * k, "out_ids")
    _lib.call("skv_topk_gather", scores.data_ptr(), scores.stride(0), landmark_idx.data_ptr(), landmark_idx.stride(0),
              rows, n, k, out_ids.data_ptr(), _stream())


# ---------------------------------------------------------------------------------------------
# a8: sparse decode attention

def sparse_attn_workspace_bytes(batch_size: int, q_heads: int, kv_len: int) -> int:
    return int(_lib.lib().skv_sparse_attn_workspace_bytes(batch_size, q_heads, kv_len))


def sparse_attn_workspace(batch_size: int, q_heads: int, kv_len: int, device) -> torch.Tensor:
    """A zero-filled attention workspace for calls of up to these sizes."""
    return torch.zeros(sparse_attn_workspace_bytes(batch_size, q_heads, kv_len), dtype=torch.uint8, device=device)


def sparse_attn_xcd_check() -> dict:
    """The one-launch merge's XCD mapping on the current device: state (1 confirmed, -1 not, 0 not
    probed), the XCC id per blockIdx class mod 8, and whether any fused workgroup ran elsewhere."""
    st, mp, mis = ctypes.c_int32(0), ctypes.c_uint32(0), ctypes.c_uint32(0)
    _lib.call("skv_sparse_attn_xcd_check", ctypes.byref(st), ctypes.byref(mp), ctypes.byref(mis))
    return dict(state=st.value, xcc=[(mp.value >> (4 * x)) & 15 for x in range(8)], misplaced=mis.value)


def sparse_attn_decode(q, k_cache, v_cache, kv_len, out, workspace, scale=None, kv_len_dev=None, pool=None,
                       vstore=None):
    """out[b, hq] = softmax(scale q[b,hq] K[b,h,:L]^T) V[b,h,:L], h = hq // (Hq/Hkv).

    q: [B, Hq, 128] view; k_cache/v_cache: [B, Hkv, >=kv_len, 128] views; out: [B, Hq, 128];
    workspace: uint8 device tensor of sparse_attn_workspace_bytes(B, Hq, kv_len) bytes, zero-filled
    before its first use (sparse_attn_workspace allocates one); every call leaves its arrival
    counters at zero again.
    L = kv_len, or, with kv_len_dev (device int32 [1]), the value it holds when the kernel runs,
    clamped to [1, kv_len].
    pool: optional (slot_list [B, Hkv, S] int32, sparse_start, S, chunk, pool_slots): the keys
    [sparse_start, sparse_start + S*chunk) are read through the slot list (a chunk pool), the
    later keys (pool_slots - S)*chunk rows further down.
    vstore: optional (store [B, Hkv, chunks, chunk*128] device tensor, position_ids [B, Hkv, S] int64,
    sparse_start, S, chunk): the values of [sparse_start, sparse_start + S*chunk) read in place
    from the store (slot j holds chunk position_ids[b, h, j]) instead of from v_cache; results are
    bit-identical to v_cache holding those rows.
    """
    _dev(q, "q", torch.bfloat16)
    _dev(k_cache, "k_cache", torch.bfloat16)
    _dev(v_cache, "v_cache", torch.bfloat16)
    _dev(out, "out", torch.bfloat16)
    _dev(workspace, "workspace")
    B, Hq, D = q.shape
    if k_cache.shape[:2] != v_cache.shape[:2] or k_cache.stride() != v_cache.stride() or k_cache.shape[0] != B:
        raise ValueError("k_cache and v_cache must be [B, Hkv, L, 128] with identical strides")
    delta = 0
    if pool is not None:
        slot_list, sp0, S, chunk, pslots = pool
        _dev(slot_list, "slot_list", torch.int32)
        if not slot_list.is_contiguous() or slot_list.numel() != B * k_cache.shape[1] * S or pslots < S:
            raise ValueError("slot_list must be contiguous [B, Hkv, S] with S <= pool_slots")
        delta = (pslots - S) * chunk
    if kv_len + delta > k_cache.shape[2] or kv_len < 1:
        raise ValueError(f"kv_len={kv_len} outside the cache length {k_cache.shape[2]}")
    if q.stride(2) != 1 or k_cache.stride(3) != 1 or out.stride(2) != 1:
        raise ValueError("the head dimension must be contiguous")
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    ldev = None
    if kv_len_dev is not None:
        _dev(kv_len_dev, "kv_len_dev", torch.int32)
        ldev = kv_len_dev.data_ptr()
    _need_offsets(q, (B, Hq, D), q.stride(), "q")
    _need_offsets(out, (B, Hq, D), out.stride(), "out")
    if vstore is not None:
        if pool is not None:
            raise ValueError("pool and vstore are exclusive")
        store, pids, sp0, S, chunk = vstore
        _dev(store, "store", torch.bfloat16)
        _dev(pids, "position_ids", torch.int64)
        Hk = k_cache.shape[1]
        if store.dim() != 4 or store.shape[:2] != (B, Hk) or store.shape[3] != chunk * D or \
                store.stride(3) != 1 or store.stride(2) != chunk * D:
            raise ValueError("store must be [B, Hkv, chunks, chunk*128] with contiguous chunks")
        if not pids.is_contiguous() or pids.numel() != B * Hk * S:
            raise ValueError("position_ids must be contiguous [B, Hkv, S]")
        if not 0 <= sp0 <= sp0 + S * chunk <= k_cache.shape[2]:
            raise ValueError("the selected region lies outside the buffers")
        _lib.call("skv_sparse_attn_decode_vstore", q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(),
                  v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), B, Hq, Hk, D, kv_len,
                  ldev, float(scale), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                  out.data_ptr(), out.stride(0), out.stride(1), store.data_ptr(), store.stride(0), store.stride(1),
                  store.shape[2], pids.data_ptr(), sp0, S, chunk, _stream())
        return
    if pool is not None:
        _lib.call("skv_sparse_attn_decode_paged", q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(),
                  v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), B, Hq, k_cache.shape[1],
                  D, kv_len, ldev, float(scale), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                  out.data_ptr(), out.stride(0), out.stride(1), slot_list.data_ptr(), sp0, S, chunk, pslots,
                  _stream())
        return
    _lib.call("skv_sparse_attn_decode", q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
              k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), B, Hq, k_cache.shape[1], D, kv_len, ldev,
              float(scale), workspace.data_ptr(), workspace.numel() * workspace.element_size(), out.data_ptr(),
              out.stride(0), out.stride(1), _stream())


# ---------------------------------------------------------------------------------------------
# new-token operations around the path (fused)

def _rows2d(t, name):
    if t.dim() < 2 or t.stride(-1) != 1:
        raise ValueError(f"{name} must have contiguous rows")
    if t.dim() > 2:
        for d in range(t.dim() - 2):
            if t.stride(d) != t.stride(d + 1) * t.shape[d + 1]:
                raise ValueError(f"{name} must flatten to rows")
    return t.numel() // t.shape[-1], t.stride(-2)


def rmsnorm(x, weight, eps, out, residual=None, residual_out=None):
    """out = bf16(h * rsqrt(mean(h^2) + eps) * weight) per row, h = x, or with `residual`
    h = residual_out = bf16(x + residual) (the residual add fused in front). Rows of x / out /
    residual / residual_out: [..., hidden] with contiguous rows."""
    _dev(x, "x", torch.bfloat16)
    _dev(out, "out", torch.bfloat16)
    _dev(weight, "weight", torch.bfloat16)
    rows, xs = _rows2d(x, "x")
    hidden = x.shape[-1]
    orows, os_ = _rows2d(out, "out")
    if orows != rows or out.shape[-1] != hidden or weight.numel() != hidden:
        raise ValueError("rmsnorm: shape mismatch")
    rp, rs, rop, ros = None, 0, None, 0
    if residual is not None:
        if residual_out is None:
            raise ValueError("rmsnorm: residual needs residual_out")
        _dev(residual, "residual", torch.bfloat16)
        _dev(residual_out, "residual_out", torch.bfloat16)
        rr, rs = _rows2d(residual, "residual")
        ro, ros = _rows2d(residual_out, "residual_out")
        if rr != rows or ro != rows or residual.shape[-1] != hidden or residual_out.shape[-1] != hidden:
            raise ValueError("rmsnorm: residual shape mismatch")
        rp, rop = residual.data_ptr(), residual_out.data_ptr()
    _lib.call("skv_rmsnorm", x.data_ptr(), xs, rp, rs, rop, ros, weight.data_ptr(), out.data_ptr(), os_, rows, hidden,
              float(eps), _stream())


def silu_and_mul(x, out):
    """out[..., j] = bf16(bf16(silu(x[..., j])) * x[..., d + j]), d = out.shape[-1] = x.shape[-1] / 2
    (vLLM silu_and_mul's two roundings)."""
    _dev(x, "x", torch.bfloat16)
    _dev(out, "out", torch.bfloat16)
    rows, xs = _rows2d(x, "x")
    orows, os_ = _rows2d(out, "out")
    d = out.shape[-1]
    if orows != rows or x.shape[-1] != 2 * d:
        raise ValueError("silu_and_mul: shape mismatch")
    _lib.call("skv_silu_and_mul", x.data_ptr(), xs, out.data_ptr(), os_, rows, d, _stream())


LINEAR_MAX_ROWS = 16


def linear(x, weight, out, bias=None):
    """out = bf16(x @ weight.T [+ bias]) in fp32 (one rounding) for decode-sized x (at most 16 rows of
    [..., k]); weight [n, k] with contiguous rows, bias [n]. The HBM-bound skinny form of F.linear
    (weights read once)."""
    _dev(x, "x", torch.bfloat16)
    _dev(weight, "weight", torch.bfloat16)
    _dev(out, "out", torch.bfloat16)
    rows, xs = _rows2d(x, "x")
    orows, os_ = _rows2d(out, "out")
    if weight.dim() != 2 or weight.stride(-1) != 1:
        raise ValueError("linear: weight must be [n, k] with contiguous rows")
    n, k = weight.shape
    if x.shape[-1] != k or out.shape[-1] != n or orows != rows:
        raise ValueError(f"linear: shape mismatch x {tuple(x.shape)} weight {tuple(weight.shape)} out {tuple(out.shape)}")
    if bias is None:
        _lib.call("skv_linear", x.data_ptr(), xs, weight.data_ptr(), weight.stride(0), out.data_ptr(), os_, rows, n, k,
                  _stream())
        return
    _dev(bias, "bias", torch.bfloat16)
    if bias.numel() != n or not bias.is_contiguous():
        raise ValueError(f"linear: bias must be a contiguous [{n}]")
    _lib.call("skv_linear_bias", x.data_ptr(), xs, weight.data_ptr(), weight.stride(0), bias.data_ptr(), out.data_ptr(),
              os_, rows, n, k, _stream())


LINEAR_SILU_MUL_MAX_ROWS = 4


def linear_silu_mul(gate_up, weight, out):
    """out = bf16(act @ weight.T), act = bf16(bf16(silu(g)) * u), for gate_up rows [g (k) | u (k)]:
    the SiLU-and-mul of the gate/up projection formed while the down projection reads it
    (bit-identical to silu_and_mul followed by linear). At most 4 rows (every workgroup recomputes
    its rows' activations); weight [n, k] with contiguous rows."""
    _dev(gate_up, "gate_up", torch.bfloat16)
    _dev(weight, "weight", torch.bfloat16)
    _dev(out, "out", torch.bfloat16)
    rows, xs = _rows2d(gate_up, "gate_up")
    orows, os_ = _rows2d(out, "out")
    if weight.dim() != 2 or weight.stride(-1) != 1:
        raise ValueError("linear_silu_mul: weight must be [n, k] with contiguous rows")
    n, k = weight.shape
    if gate_up.shape[-1] != 2 * k or out.shape[-1] != n or orows != rows:
        raise ValueError(f"linear_silu_mul: shape mismatch gate_up {tuple(gate_up.shape)} weight "
                         f"{tuple(weight.shape)} out {tuple(out.shape)}")
    if rows > LINEAR_SILU_MUL_MAX_ROWS:
        raise ValueError(f"linear_silu_mul: {rows} rows (at most {LINEAR_SILU_MUL_MAX_ROWS})")
    _lib.call("skv_linear_silu_mul", gate_up.data_ptr(), xs, weight.data_ptr(), weight.stride(0), out.data_ptr(), os_,
              rows, n, k, _stream())


def interleave_gate_up(weight):
    """The reference's gate_up_proj weight [gate (f rows) | up (f rows)] with its halves interleaved
    row by row (row 2j = gate row j, row 2j + 1 = up row j), the layout linear_gate_up_silu reads."""
    f = weight.shape[0] // 2
    return weight.view(2, f, weight.shape[1]).transpose(0, 1).reshape(2 * f, weight.shape[1]).contiguous()


def linear_gate_up_silu(x, weight_il, out):
    """out = bf16(bf16(silu(g)) * u) with g, u the bf16 gate and up projections of x, from the
    interleaved gate/up weight (interleave_gate_up): silu_and_mul(linear(x, gate_up)) in one
    launch, bit-identical. x [..., k] (at most 16 rows), weight_il [2f, k], out [..., f]."""
    _dev(x, "x", torch.bfloat16)
    _dev(weight_il, "weight", torch.bfloat16)
    _dev(out, "out", torch.bfloat16)
    rows, xs = _rows2d(x, "x")
    orows, os_ = _rows2d(out, "out")
    if weight_il.dim() != 2 or weight_il.stride(-1) != 1:
        raise ValueError("linear_gate_up_silu: weight must be [n, k] with contiguous rows")
    n, k = weight_il.shape
    if n % 2 or x.shape[-1] != k or out.shape[-1] != n // 2 or orows != rows:
        raise ValueError(f"linear_gate_up_silu: shape mismatch x {tuple(x.shape)} weight {tuple(weight_il.shape)} "
                         f"out {tuple(out.shape)}")
    _lib.call("skv_linear_gate_up_silu", x.data_ptr(), xs, weight_il.data_ptr(), weight_il.stride(0), out.data_ptr(),
              os_, rows, n, k, _stream())


def rope_qk_append(qkv, q_heads, kv_heads, positions, cos_sin, q_out, k_cache, v_cache, append_row):
    """The new token's q and k rotated at positions[b] (bf16 per-op rounding; half-split for a
    [rows, 128] cos_sin, GLM-interleaved for [rows, 64]) and the KV append in one launch:
    q_out[b] <- rotated q; row *append_row of k_cache/v_cache [B, Hkv, buf_len, 128] <- rotated k,
    raw v. qkv: [B, (Hq + 2 Hkv) * 128] rows (views of the fused projection are fine)."""
    B = qkv.shape[0]
    D = 128
    _dev(qkv, "qkv", torch.bfloat16)
    _dev(q_out, "q_out", torch.bfloat16)
    _dev(positions, "positions", torch.int64)
    _dev(cos_sin, "cos_sin", torch.bfloat16)
    _dev(append_row, "append_row", torch.int64)
    for t, nm in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        _dev(t, nm, torch.bfloat16)
        if t.dim() != 4 or t.shape[0] != B or t.shape[1] != kv_heads or t.shape[3] != D or t.stride(3) != 1:
            raise ValueError(f"{nm} must be [B, Hkv, buf_len, 128]")
    if k_cache.stride() != v_cache.stride() or k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must share a layout")
    width = (q_heads + 2 * kv_heads) * D
    if qkv.shape[-1] != width or qkv.stride(-1) != 1 or qkv.numel() != B * width:
        raise ValueError(f"qkv must be [B, {width}]")
    qkv_sb = qkv.stride(0)
    if q_out.numel() != B * q_heads * D or not q_out.is_contiguous():
        raise ValueError("q_out must be a contiguous [B, Hq, 128]")
    if positions.numel() < B:
        raise ValueError("positions too short")
    mode = 0 if cos_sin.shape[-1] == 128 else 1 if cos_sin.shape[-1] == 64 else -1
    if mode < 0:
        raise ValueError(f"Invalid cos_sin shape {tuple(cos_sin.shape)}")
    _need_offsets(qkv, (B, width), (qkv_sb, 1), "qkv")
    _lib.call("skv_rope_qk_append", qkv.data_ptr(), qkv_sb, B, q_heads, kv_heads, D, positions.data_ptr(),
              cos_sin.data_ptr(), cos_sin.stride(0), cos_sin.shape[0], mode, q_out.data_ptr(), q_heads * D,
              k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
              append_row.data_ptr(), k_cache.shape[2], _stream())


def qkv_rope_weight(weight, q_heads, kv_heads, glm):
    """The fused QKV weight [(Hq + 2 Hkv) * 128, k] (or its bias [(Hq + 2 Hkv) * 128]) in the row
    order linear_qkv_rope_append reads: for the half-split rotation each q and k head's rows
    interleaved as (0, 64, 1, 65, ..., 63, 127) (v rows unchanged); for GLM's interleaved pairs the
    weight as is."""
    D = 128
    if weight.shape[0] != (q_heads + 2 * kv_heads) * D:
        raise ValueError(f"qkv_rope_weight: {weight.shape[0]} rows for {q_heads} + 2 x {kv_heads} heads")
    if glm:
        return weight.contiguous()
    qk = (q_heads + kv_heads) * D
    order = torch.arange(D, device=weight.device).view(2, D // 2).t().reshape(-1)  # 0, 64, 1, 65, ...
    idx = (torch.arange(q_heads + kv_heads, device=weight.device)[:, None] * D + order).reshape(-1)
    idx = torch.cat([idx, torch.arange(qk, weight.shape[0], device=weight.device)])
    return weight.index_select(0, idx).contiguous()


QKV_ROPE_MAX_ROWS = 8


def linear_qkv_rope_append(x, weight_rope, q_heads, kv_heads, positions, cos_sin, q_out, k_cache, v_cache,
                           append_row, bias_rope=None):
    """linear(x, wqkv[, bias]) followed by rope_qk_append(...) in one launch, bit-identical, on the
    weight (and bias) in qkv_rope_weight's row order (half-split for a [rows, 128] cos_sin, GLM for
    [rows, 64]). x: [..., k] token rows (at most 8); the other arguments as rope_qk_append's."""
    D = 128
    _dev(x, "x", torch.bfloat16)
    _dev(weight_rope, "weight", torch.bfloat16)
    _dev(q_out, "q_out", torch.bfloat16)
    _dev(positions, "positions", torch.int64)
    _dev(cos_sin, "cos_sin", torch.bfloat16)
    _dev(append_row, "append_row", torch.int64)
    B, xs = _rows2d(x, "x")
    if weight_rope.dim() != 2 or weight_rope.stride(-1) != 1:
        raise ValueError("linear_qkv_rope_append: weight must be [n, k] with contiguous rows")
    n, k = weight_rope.shape
    if n != (q_heads + 2 * kv_heads) * D or x.shape[-1] != k:
        raise ValueError(f"linear_qkv_rope_append: shape mismatch x {tuple(x.shape)} weight {tuple(weight_rope.shape)}"
                         f" for {q_heads} + 2 x {kv_heads} heads")
    if B > QKV_ROPE_MAX_ROWS:
        raise ValueError(f"linear_qkv_rope_append: {B} rows (at most {QKV_ROPE_MAX_ROWS})")
    for t, nm in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        _dev(t, nm, torch.bfloat16)
        if t.dim() != 4 or t.shape[0] != B or t.shape[1] != kv_heads or t.shape[3] != D or t.stride(3) != 1:
            raise ValueError(f"{nm} must be [B, Hkv, buf_len, 128]")
    if k_cache.stride() != v_cache.stride() or k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must share a layout")
    if q_out.numel() != B * q_heads * D or not q_out.is_contiguous():
        raise ValueError("q_out must be a contiguous [B, Hq, 128]")
    if positions.numel() < B:
        raise ValueError("positions too short")
    mode = 0 if cos_sin.shape[-1] == 128 else 1 if cos_sin.shape[-1] == 64 else -1
    if mode < 0:
        raise ValueError(f"Invalid cos_sin shape {tuple(cos_sin.shape)}")
    bp = None
    if bias_rope is not None:
        _dev(bias_rope, "bias", torch.bfloat16)
        if bias_rope.numel() != n or not bias_rope.is_contiguous():
            raise ValueError(f"linear_qkv_rope_append: bias must be a contiguous [{n}]")
        bp = bias_rope.data_ptr()
    _lib.call("skv_linear_qkv_rope_append", x.data_ptr(), xs, weight_rope.data_ptr(), weight_rope.stride(0), bp, B, k,
              q_heads, kv_heads, positions.data_ptr(), cos_sin.data_ptr(), cos_sin.stride(0), cos_sin.shape[0], mode,
              q_out.data_ptr(), q_heads * D, k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
              k_cache.stride(1), k_cache.stride(2), append_row.data_ptr(), k_cache.shape[2], _stream())

# ---------------------------------------------------------------------------------------------
# f1: prefill encoder (chunk statistics, outlier selection, landmark gather)

def chunk_stats(keys, chunks, chunk_size, candidates, min_cos):
    """keys [B, H, >= chunks*chunk_size, 128] bf16 (rows contiguous) -> candidates [B, H, chunks, 128]
    bf16 chunk means and min_cos [B, H, chunks] fp32 (minimum row-to-mean cosine per chunk)."""
    _dev(keys, "keys", torch.bfloat16)
    _dev(candidates, "candidates", torch.bfloat16)
    _dev(min_cos, "min_cos", torch.float32)
    if keys.dim() != 4 or keys.shape[-1] != 128 or keys.stride(-1) != 1:
        raise ValueError("keys must be [B, H, rows, 128] with contiguous rows")
    B, H, rows, _ = keys.shape
    if chunks * chunk_size > rows:
        raise ValueError(f"{chunks} chunks of {chunk_size} rows exceed the {rows} key rows")
    if not candidates.is_contiguous() or candidates.numel() < B * H * chunks * 128:
        raise ValueError("candidates must be contiguous [B, H, chunks, 128]")
    if not min_cos.is_contiguous() or min_cos.numel() < B * H * chunks:
        raise ValueError("min_cos must be contiguous [B, H, chunks]")
    _lib.call("skv_chunk_stats", keys.data_ptr(), keys.stride(0), keys.stride(1), keys.stride(2), B, H, chunks,
              chunk_size, candidates.data_ptr(), min_cos.data_ptr(), _stream())


def select_outliers(min_cos, outliers, outlier_idx, landmark_idx):
    """min_cos [rows, chunks] fp32 -> outlier_idx [rows, outliers] (ascending min_cos, ties to the
    lowest id) and landmark_idx [rows, chunks - outliers] (the other ids ascending), int64."""
    _dev(min_cos, "min_cos", torch.float32)
    _dev(outlier_idx, "outlier_idx", torch.int64)
    _dev(landmark_idx, "landmark_idx", torch.int64)
    if min_cos.dim() != 2 or not min_cos.is_contiguous():
        raise ValueError("min_cos must be contiguous [rows, chunks]")
    rows, chunks = min_cos.shape
    if tuple(outlier_idx.shape) != (rows, outliers) or not outlier_idx.is_contiguous():
        raise ValueError("outlier_idx must be contiguous [rows, outliers]")
    if tuple(landmark_idx.shape) != (rows, chunks - outliers) or not landmark_idx.is_contiguous():
        raise ValueError("landmark_idx must be contiguous [rows, chunks - outliers]")
    _lib.call("skv_select_outliers", min_cos.data_ptr(), rows, chunks, outliers, outlier_idx.data_ptr(),
              landmark_idx.data_ptr(), _stream())


def gather_rows(src, idx, dst):
    """dst[r, j] = src[r, idx[r, j]] for 128-element bf16 rows; src [rows, n_src, 128], idx [rows, n]
    int64, dst [rows, n, 128], all contiguous."""
    _dev(src, "src", torch.bfloat16)
    _dev(idx, "idx", torch.int64)
    _dev(dst, "dst", torch.bfloat16)
    for t, nm in ((src, "src"), (idx, "idx"), (dst, "dst")):
        if not t.is_contiguous():
            raise ValueError(f"{nm} must be contiguous")
    if src.dim() != 3 or src.shape[-1] != 128 or idx.dim() != 2 or tuple(dst.shape) != (*idx.shape, 128) or \
            src.shape[0] != idx.shape[0]:
        raise ValueError("gather_rows: src [rows, n_src, 128], idx [rows, n], dst [rows, n, 128]")
    _lib.call("skv_gather_rows", src.data_ptr(), src.shape[0], src.shape[1], idx.data_ptr(), idx.shape[1],
              dst.data_ptr(), _stream())


# ---------------------------------------------------------------------------------------------
# f3: device chunk pool

def pool_assign(selected, num_chunks, slot_of, slot_chunk, slot_used, clock, slot_list, miss_ids, miss_slot, cnts):
    """Map the selection onto a chunk pool (one row per (b, h)): selected [rows, S] int64; tables
    slot_of [rows, num_chunks], slot_chunk / slot_used [rows, P], clock [rows] (int32, updated);
    outputs slot_list [rows, S], miss_ids / miss_slot [rows, S] (misses at [cnts[r], S)), cnts [rows]."""
    _dev(selected, "selected", torch.int64)
    for t, nm in ((slot_of, "slot_of"), (slot_chunk, "slot_chunk"), (slot_used, "slot_used"), (clock, "clock"),
                  (slot_list, "slot_list"), (miss_ids, "miss_ids"), (miss_slot, "miss_slot"), (cnts, "cnts")):
        _dev(t, nm, torch.int32)
        if not t.is_contiguous():
            raise ValueError(f"{nm} must be contiguous")
    if not selected.is_contiguous() or selected.dim() != 2:
        raise ValueError("selected must be contiguous [rows, S]")
    rows, S = selected.shape
    P = slot_chunk.numel() // rows
    if slot_of.numel() != rows * num_chunks or slot_chunk.numel() != rows * P or slot_used.numel() != rows * P or \
            clock.numel() != rows or cnts.numel() < rows:
        raise ValueError("pool tables do not match the selection's rows")
    for t, nm in ((slot_list, "slot_list"), (miss_ids, "miss_ids"), (miss_slot, "miss_slot")):
        _need(t, rows * S, nm)
    _lib.call("skv_pool_assign", selected.data_ptr(), rows, S, num_chunks, P, slot_of.data_ptr(),
              slot_chunk.data_ptr(), slot_used.data_ptr(), clock.data_ptr(), slot_list.data_ptr(), miss_ids.data_ptr(),
              miss_slot.data_ptr(), cnts.data_ptr(), _stream())


def gather_copy_misses_to_slots(values, v_cache_buffer, miss_ids, cnts, miss_slot, batch_size, heads, cpu_v_length,
                                pool_offset, gpu_v_stride, map_size, pool_slots, chunk_elems):
    """The miss gather of a chunk pool: entries i >= cnts[r] (chunk miss_ids, slot miss_slot) of every
    row r from the pinned host store into v_cache_buffer + r*gpu_v_stride + pool_offset + slot*chunk."""
    rows = batch_size * heads
    row_stride = _host_row_stride(values, rows, cpu_v_length)
    _need(values, (rows - 1) * row_stride + row_stride, "values")
    _dev(v_cache_buffer, "v_cache_buffer", torch.bfloat16)
    _need(v_cache_buffer, (rows - 1) * gpu_v_stride + pool_offset + pool_slots * chunk_elems, "v_cache_buffer")
    for t, nm in ((miss_ids, "miss_ids"), (miss_slot, "miss_slot")):
        _dev(t, nm, torch.int32)
        _need(t, rows * map_size, nm)
    _dev(cnts, "cnts", torch.int32)
    _need(cnts, rows, "cnts")
    _lib.call("skv_gather_copy_misses_to_slots", device_address(values), v_cache_buffer.data_ptr(), miss_ids.data_ptr(),
              cnts.data_ptr(), miss_slot.data_ptr(), batch_size, heads, row_stride, pool_offset, gpu_v_stride,
              map_size, pool_slots, chunk_elems, _stream())


HBM_PROBE_TILE_BYTES = 65536
HBM_PROBE_PATTERNS = {"contiguous": 0, "operand": 1}


def hbm_read_probe(src, tiles_per_workgroup, pattern, sink, nontemporal=False):
    """Read-only HBM envelope probe (no reference counterpart): reads src (a multiple of 64 KB) in
    64 KB tiles, tiles_per_workgroup per workgroup of 256 threads, in the "contiguous" order (1 KB
    of consecutive bytes per wave instruction) or the "operand" order (64 bytes from each of 16
    rows of 256 bytes per instruction, as the scoring and attention kernels load MFMA operands),
    with plain or non-temporal loads. Thread t of workgroup g writes the XOR of the 16-byte vectors
    it read to sink[g*256 + t]."""
    _dev(src, "src")
    _dev(sink, "sink")
    if not src.is_contiguous() or not sink.is_contiguous():
        raise ValueError("hbm_read_probe: src and sink must be contiguous")
    nbytes = src.numel() * src.element_size()
    if nbytes % HBM_PROBE_TILE_BYTES:
        raise ValueError(f"hbm_read_probe: src holds {nbytes} bytes, not a multiple of {HBM_PROBE_TILE_BYTES}")
    if pattern not in HBM_PROBE_PATTERNS:
        raise ValueError(f"hbm_read_probe: pattern must be one of {sorted(HBM_PROBE_PATTERNS)}")
    _lib.call("skv_hbm_read_probe", src.data_ptr(), nbytes // HBM_PROBE_TILE_BYTES, tiles_per_workgroup,
              HBM_PROBE_PATTERNS[pattern] + (2 if nontemporal else 0), sink.data_ptr(),
              sink.numel() * sink.element_size(), _stream())


def mfma_peak_probe(workgroups, iters, sink):
    """MFMA peak probe (no reference counterpart): every wave of `workgroups` 256-thread workgroups
    issues iters x 4 independent bf16 32x32x16 MFMAs on register operands; one float per thread is
    written to sink (float32, at least workgroups * 256). Returns the flops of the call."""
    _dev(sink, "sink", torch.float32)
    _need(sink, workgroups * 256, "sink")
    _lib.call("skv_mfma_peak_probe", workgroups, iters, sink.data_ptr(), sink.numel() * 4, _stream())
    return int(_lib.lib().skv_mfma_peak_probe_flops(workgroups, iters))
