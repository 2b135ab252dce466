"""Pins the per-head split of the low-rank key factors (models/kvcache/shadow.py:437-442).

The reference factors the pre-RoPE keys of all heads at once, K [ctx, H*D] = U diag(s) Vh, and
splits diag(s) Vh [R, H*D] into per-head SV [H, D, R] (`view(bsz, -1, H, D).transpose(1, 2)
.transpose(-1, -2)`). What fixes the split independently of that line: head h's keys must come
back as U @ SV[h]^T. The make_golden cases build K = A.Bm + sigma N with A.Bm of exact rank R, so a
correct rank-R split leaves only the noise outside the signal's row and column spaces:
relative error ~ sigma sqrt((1 - R/(H D)) (1 - R/ctx)) / rms(K_h). A split that takes the dims of
a head from the wrong places (heads and dims transposed, heads permuted) reconstructs another
head's or mixed dims' keys, an error of order sqrt(2).
"""
from __future__ import annotations

import math

import torch

NOISE = 0.05  # sigma of the cases' additive noise (make_golden.decode_small_case, single_layer_case)


def head_errors(k_pre: torch.Tensor, U: torch.Tensor, SV: torch.Tensor) -> torch.Tensor:
    """Relative Frobenius error of U[b] @ SV[b, h]^T against k_pre[b, h], shape [B, H].
    k_pre [B, H, ctx, D]; U [B, ctx, R]; SV [B, H, D, R]."""
    k = k_pre.double()
    rec = torch.einsum("bcr,bhdr->bhcd", U.double(), SV.double())
    return (k - rec).flatten(2).norm(dim=-1) / k.flatten(2).norm(dim=-1)


def noise_floor(k_pre: torch.Tensor, rank: int) -> torch.Tensor:
    """Expected relative error of an exact rank-R split, per (b, h): the noise left outside the
    signal's R-dimensional row and column spaces over the head's RMS."""
    B, H, ctx, D = k_pre.shape
    keep = math.sqrt((1 - rank / (H * D)) * (1 - rank / ctx))
    rms = k_pre.double().flatten(2).pow(2).mean(-1).sqrt()
    return NOISE * keep / rms


def bound(k_pre: torch.Tensor, rank: int) -> torch.Tensor:
    """Acceptance bound: 3% over the noise floor plus 0.005 for the bf16 rounding of U and SV (the
    measured errors of both cases sit within 0.3% of the floor)."""
    return 1.03 * noise_floor(k_pre, rank) + 0.005


def transposed_split(SV: torch.Tensor) -> torch.Tensor:
    """The plausible mistake: the same [R, H*D] rows split as [R, D, H] (dims outer, heads inner)."""
    B, H, D, R = SV.shape
    flat = SV.permute(0, 3, 1, 2).reshape(B, R, H * D)  # back to diag(s) Vh rows
    return flat.view(B, R, D, H).permute(0, 3, 2, 1).contiguous()
