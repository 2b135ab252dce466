"""Tensor helpers of the sparse-decode path (reference: models/tensor_op.py:125-243).

The torch-level helpers (repeat_kv, rotate_half, apply_rotary_pos_emb[_single]) restate the
reference's math; the `*_cuda` helpers route to the gfx950 kernels in
shadowkv_amd.kernels.shadowkv with the reference's argument lists. RoPE tables are built as
in models/llama.py:138-142 ([cos(64) | sin(64)] rows) and models/glm.py:132-133
([cos(32) | sin(32)] rows, interleaved pairs).
"""
from __future__ import annotations

import torch

from ..kernels import shadowkv


def repeat_kv(hidden_states: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[B, H, L, D] -> [B, H*n_rep, L, D], each kv head repeated for its query-head group."""
    if n_rep == 1:
        return hidden_states
    b, h, l, d = hidden_states.shape
    return hidden_states.unsqueeze(2).expand(b, h, n_rep, l, d).reshape(b, h * n_rep, l, d)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary_pos_emb(q, k, cos, sin, position_ids):
    cos = cos[position_ids].unsqueeze(1)
    sin = sin[position_ids].unsqueeze(1)
    return (q * cos) + (rotate_half(q) * sin), (k * cos) + (rotate_half(k) * sin)


def apply_rotary_pos_emb_single(q, cos, sin, position_ids, unsqueeze_dim=1):
    if position_ids.dim() == 3:
        position_ids = position_ids.reshape(-1, position_ids.shape[-1])
        c, s = cos[position_ids], sin[position_ids]
    else:
        c, s = cos[position_ids].unsqueeze(unsqueeze_dim), sin[position_ids].unsqueeze(unsqueeze_dim)
    return (q * c) + (rotate_half(q) * s)


def build_cos_sin_cache(max_length: int, theta: float, head_dim: int = 128, device="cpu",
                        dtype=torch.bfloat16) -> torch.Tensor:
    """Half-split RoPE table [max_length + 1024, head_dim] = [cos(head_dim/2) | sin(head_dim/2)]."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    t = torch.arange(max_length + 1024, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = emb.cos().to(dtype), emb.sin().to(dtype)
    half = head_dim // 2
    return torch.cat((cos[:, :half], sin[:, :half]), dim=-1).to(device)


def build_glm_cos_sin_cache(max_length: int, base: float, device="cpu", dtype=torch.bfloat16) -> torch.Tensor:
    """GLM partial-rotary table [max_length + 1024, 64] = [cos(32) | sin(32)] over 64 rotated dims."""
    theta = 1.0 / (base ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
    idx_theta = torch.outer(torch.arange(max_length + 1024, dtype=torch.float32), theta)
    return torch.cat((idx_theta.cos(), idx_theta.sin()), dim=-1).to(dtype).to(device)


def apply_rotary_pos_emb_glm_single(x: torch.Tensor, cos_sin: torch.Tensor, position_ids: torch.Tensor) -> torch.Tensor:
    """GLM interleaved RoPE on the first 64 dims (models/glm.py:208-230); x [B, H, L, 128]."""
    if position_ids.dim() == 1:
        position_ids = position_ids.view(1, 1, -1).expand(x.shape[0], x.shape[1], -1)
    elif position_ids.dim() == 2:
        position_ids = position_ids.unsqueeze(1).expand(-1, x.shape[1], -1)
    cache = cos_sin[position_ids]
    xr, xp = x[..., :64], x[..., 64:]
    c, s = cache[..., :32], cache[..., 32:]
    out = torch.stack((xr[..., 0::2] * c - xr[..., 1::2] * s, xr[..., 1::2] * c + xr[..., 0::2] * s), -1).flatten(3)
    return torch.cat((out, xp), dim=-1)


def apply_rotary_pos_emb_cuda(x, cos_sin, position_ids):
    """RoPE by token position on the device (reference: models/tensor_op.py:159-174)."""
    b, h, s, d = x.shape
    out = torch.empty_like(x)
    shadowkv.apply_rotary_pos_emb_new(x, cos_sin, position_ids, out, b, h, s, d, x.stride(0), x.stride(1), x.stride(2),
                                      x.stride(3), cos_sin.stride(0), position_ids.stride(0), position_ids.stride(1),
                                      position_ids.stride(2), d // 2)
    return out


def apply_rotary_pos_emb_cuda_push_cache(x, cos_sin, position_ids, chunk_size, cache, sparse_start, sparse_end, cnts):
    """Rotate rebuilt miss rows into the key cache (reference: models/tensor_op.py:176-204)."""
    b, h, s, d = x.shape
    args = (x, cos_sin, position_ids, cache, cnts, b, h, s, d, x.stride(0), x.stride(1), x.stride(2), x.stride(3),
            cos_sin.stride(0), position_ids.stride(0), position_ids.stride(1), position_ids.stride(2),
            cache.stride(0), cache.stride(1), cache.stride(2), sparse_start, sparse_end, d // 2, chunk_size)
    if cos_sin.shape[-1] == 128:
        shadowkv.apply_rotary_pos_emb_push_cache_opt(*args)
    elif cos_sin.shape[-1] == 64:
        shadowkv.apply_rotary_pos_emb_push_cache_opt_glm(*args)
    else:
        raise ValueError(f"Invalid cos_sin shape {cos_sin.shape}")
    return cache


def batch_gather_gemm_rotary_pos_emb_cuda(a, b, cos_sin, position_ids, output, chunk_size, cache, sparse_start,
                                          sparse_end, cnts):
    """K rebuild for the miss chunks + RoPE push into `cache` (reference: models/tensor_op.py:206-243).

    One fused kernel replaces the reference's GEMM + RoPE pair; `output` (the reference's
    pre-RoPE scratch) is not needed and is ignored. position_ids: [B, H, S] chunk ids.
    """
    del output
    if position_ids.shape[-1] * chunk_size != sparse_end - sparse_start:
        raise ValueError("sparse region length does not match the selected chunks")
    if position_ids.dtype != torch.int64:
        position_ids = position_ids.to(torch.int64)
    shadowkv.rebuild_k_rope(a, b, position_ids, cnts, cos_sin, cache, sparse_start, chunk_size)
    return cache
