"""CPU restatement of the ShadowKV sparse decode step (TEST INFRASTRUCTURE ONLY).

Index and copy semantics are numpy; bf16/fp32 arithmetic uses torch on the CPU, which is
what the reference's own torch code does (bf16 ops widen to fp32 and round to nearest even).
Pins for every function are listed in its docstring; the tests that apply them live in
tests/test_oracle_*.py.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

__all__ = [
    "reorder", "cached_gather_copy", "compact_hits", "gather_copy_plain", "rope_half_split", "rope_push",
    "rope_push_glm", "rope_two_tables", "rebuild_k", "rebuild_k_rope", "score_logits_softmax", "score_gqa_max", "topk_total_order",
    "topk_gather", "sparse_attention", "build_cos_sin_cache", "build_glm_cos_sin_cache", "encode_layer",
    "decode_layer_step", "LayerState", "prefill_geometry", "pool_assign", "pool_from_layer", "decode_layer_step_pooled",
]


# --------------------------------------------------------------------------------------------
# a3: reorder — kernels/map.cuh:342-403 (ballot compaction: hits first, then misses, both in
# selection order) followed by block_sort2 (map.cuh:229-259, enabled by SORT_OFFSET at
# map.cuh:503-506): hits re-sorted by old slot, misses by chunk id. Old ids of -1 never hit
# (EMPTY_KEY, map.cuh:26,140-144).
# Pinned by: the reference's known-answer procedure (kernels/test_cached_gather_copy.cu:70-156,
# restated independently in tests/golden/make_golden.py) on its own seeded inputs, and by
# brute force on tiny rows with unsorted old ids (tests/test_oracle_index.py).

def reorder(old: np.ndarray, new: np.ndarray):
    """old, new: [rows, S] int64. Returns (new_slot_ids [rows,S] int64, offsets [rows,S] int32, cnts [rows] int32)."""
    old = np.asarray(old, dtype=np.int64)
    new = np.asarray(new, dtype=np.int64)
    rows, S = old.shape
    ids = np.empty((rows, S), dtype=np.int64)
    offs = np.empty((rows, S), dtype=np.int32)
    cnts = np.empty(rows, dtype=np.int32)
    for r in range(rows):
        slot_of = {int(k): j for j, k in enumerate(old[r]) if k != -1}
        hit_slots = sorted(slot_of[int(k)] for k in new[r] if int(k) in slot_of)
        misses = sorted(int(k) for k in new[r] if int(k) not in slot_of)
        c = len(hit_slots)
        ids[r, :c] = [old[r, j] for j in hit_slots]
        offs[r, :c] = hit_slots
        ids[r, c:] = misses
        offs[r, c:] = misses
        cnts[r] = c
    return ids, offs, cnts


# --------------------------------------------------------------------------------------------
# a4/a5: chunk copies — kernels/copy.cuh:122-180 (gather), 353-390 (d2d compaction),
# 438-498 (cached copy); closed form of kernels/test_cached_gather_copy.cu:158-216.
# Pinned by: the closed form itself (pure index copy) evaluated on pattern-coded chunks whose
# contents name their origin (tests/test_oracle_index.py).

def cached_gather_copy(host: np.ndarray, dev: np.ndarray, offsets: np.ndarray, cnts: np.ndarray) -> np.ndarray:
    """host [rows, chunks, E], dev [rows, S, E] (slot order). Returns the refreshed dev buffer:
    slot i <- old dev slot offsets[i] for i < cnt, host chunk offsets[i] otherwise."""
    out = dev.copy()
    for r in range(dev.shape[0]):
        c = int(cnts[r])
        out[r, :c] = dev[r, offsets[r, :c]]
        out[r, c:] = host[r, offsets[r, c:]]
    return out


def compact_hits(dev: np.ndarray, offsets: np.ndarray, cnts: np.ndarray) -> np.ndarray:
    """The i < cnt part of cached_gather_copy (copy.cuh:353-390); miss slots keep their content."""
    out = dev.copy()
    for r in range(dev.shape[0]):
        c = int(cnts[r])
        out[r, :c] = dev[r, offsets[r, :c]]
    return out


def gather_copy_plain(host: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """dst slot i <- host chunk ids[i] (kernels/copy.cuh:248-274, gather_copy.cu:47-109)."""
    return np.stack([host[r, ids[r]] for r in range(host.shape[0])])


# --------------------------------------------------------------------------------------------
# a7: RoPE — kernels/rope_new.cu:262-269 (push, half-split) and :354-371 (GLM); identical to
# torch's (x*cos) + (rotate_half(x)*sin) in bf16 (models/tensor_op.py:132-156).
# Pinned by: an independent numpy float32 implementation with explicit round-to-nearest-even
# (tests/test_oracle_float.py, bit-exact), position 0 = identity, and agreement with exact
# complex rotation within bf16 rounding.

def rope_half_split(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [..., D] bf16, cos/sin [..., D/2] bf16 -> rotated bf16 with per-op rounding."""
    h = x.shape[-1] // 2
    c = torch.cat((cos, cos), dim=-1)
    s = torch.cat((sin, sin), dim=-1)
    rot = torch.cat((-x[..., h:], x[..., :h]), dim=-1)
    return (x * c) + (rot * s)


def rope_two_tables(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Reference apply_rotary_pos_emb (kernels/rope.cu:26-62): x [..., D] bf16 with full-width cos
    and sin rows [..., D] bf16; the first half rotated with cos[:D/2], sin[:D/2], the second with
    cos[D/2:], sin[D/2:], every product and sum rounded to bf16.
    Pinned by: numpy float32 with explicit round-to-nearest-even (tests/test_oracle_float.py) and,
    for tables with equal halves, equality with rope_half_split."""
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    return torch.cat(((x1 * cos[..., :h]) + ((-x2) * sin[..., :h]), (x2 * cos[..., h:]) + (x1 * sin[..., h:])), dim=-1)


def rope_push(x: torch.Tensor, cos_sin: torch.Tensor, chunk_ids: torch.Tensor, cnts: torch.Tensor, chunk: int,
              cache: torch.Tensor, start: int, end: int) -> torch.Tensor:
    """Reference apply_rotary_pos_emb_push_cache_opt (rope_new.cu:224-302) on CPU tensors.

    x [B, H, S*chunk, D] bf16, cos_sin [rows, D] = [cos|sin], chunk_ids [B, H, S], cnts [B*H];
    cache [B, H, buf, D] is updated in place and returned."""
    B, H, R, D = x.shape
    half = D // 2
    for b in range(B):
        for h in range(H):
            c = int(cnts[b * H + h])
            rows = torch.arange(c * chunk, R)
            rows = rows[start + rows < end]
            if rows.numel() == 0:
                continue
            pos = chunk_ids[b, h, rows // chunk].long() * chunk + rows % chunk
            cs = cos_sin[pos]
            cache[b, h, start + rows] = rope_half_split(x[b, h, rows], cs[:, :half], cs[:, half:])
    return cache


def rope_push_glm(x, cos_sin, chunk_ids, cnts, chunk, cache, start, end):
    """Reference apply_rotary_pos_emb_push_cache_opt_glm (rope_new.cu:305-404): interleaved
    pairs (2i, 2i+1) of dims 0..63 with [cos(32)|sin(32)] rows; dims 64..127 copied."""
    B, H, R, D = x.shape
    for b in range(B):
        for h in range(H):
            c = int(cnts[b * H + h])
            rows = torch.arange(c * chunk, R)
            rows = rows[start + rows < end]
            if rows.numel() == 0:
                continue
            pos = chunk_ids[b, h, rows // chunk].long() * chunk + rows % chunk
            cs = cos_sin[pos]
            xr = x[b, h, rows]
            xe, xo = xr[:, 0:64:2], xr[:, 1:64:2]
            co, si = cs[:, :32], cs[:, 32:]
            ye = (xe * co) + ((-xo) * si)
            yo = (xo * co) + (xe * si)
            y = xr.clone()
            y[:, 0:64:2] = ye
            y[:, 1:64:2] = yo
            cache[b, h, start + rows] = y
    return cache


# --------------------------------------------------------------------------------------------
# a6: low-rank key rebuild — math of models/kvcache/shadow.py:245-250 (gathered U rows times
# SV) with the offload-class layouts (U [B, ctx, R] head-shared, SV [B, H, D, R]) and the row
# map of kernels/special_batch_gather_predicated_tile_iterator.h:294; fp32 accumulation, one
# rounding to bf16 (CUTLASS epilogue, kernels/batch_gather_gemm.cu:145-147 alpha=1 beta=0).
# Pinned by: basis-vector U rows (K rows equal SV columns exactly), a float64 numpy product
# (tests/test_oracle_float.py).

def rebuild_k(U: torch.Tensor, SV: torch.Tensor, chunk_ids: torch.Tensor, chunk: int) -> torch.Tensor:
    """U [B, ctx, R] (or [B, H, ctx, R]), SV [B, H, D, R], chunk_ids [B, H, S] -> [B, H, S*chunk, D] bf16."""
    B, H, S = chunk_ids.shape
    pos = (chunk_ids.long().unsqueeze(-1) * chunk + torch.arange(chunk)).reshape(B, H, S * chunk)
    if U.dim() == 3:
        rows = torch.stack([torch.stack([U[b, pos[b, h]] for h in range(H)]) for b in range(B)])
    else:
        rows = torch.stack([torch.stack([U[b, h, pos[b, h]] for h in range(H)]) for b in range(B)])
    out = torch.matmul(rows.float(), SV.float().transpose(-1, -2))
    return out.to(torch.bfloat16)


def rebuild_k_rope(U, SV, chunk_ids, cnts, cos_sin, chunk, cache, start, glm: bool = False):
    """Fused a6+a7: rebuild then push (models/tensor_op.py:206-243). Updates cache in place."""
    k = rebuild_k(U, SV, chunk_ids, chunk)
    end = start + chunk_ids.shape[-1] * chunk
    if glm:
        return rope_push_glm(k, cos_sin, chunk_ids, cnts, chunk, cache, start, end)
    return rope_push(k, cos_sin, chunk_ids, cnts, chunk, cache, start, end)


# --------------------------------------------------------------------------------------------
# a1: scoring — kernels/batch_gemm_softmax.cu:143-196 semantics: D = bf16(alpha * q.L^T) with
# fp32 accumulation, softmax in fp32 over the bf16 logits, bf16 probabilities; GQA max over
# the query rows of a kv head (models/kvcache/shadow.py:567-568).
# Pinned by: identical landmarks (softmax = 1/n exactly before rounding), n = 1 (1.0), a
# float64 numpy softmax (tests/test_oracle_float.py).

def score_logits_softmax(q: torch.Tensor, landmarks: torch.Tensor, alpha: float):
    """q [Z, m, D] bf16, landmarks [Z, n, D] bf16 -> (D [Z, m, n] bf16, P [Z, m, n] bf16)."""
    logits = (torch.matmul(q.float(), landmarks.float().transpose(-1, -2)) * alpha).to(torch.bfloat16)
    probs = torch.softmax(logits.float(), dim=-1).to(torch.bfloat16)
    return logits, probs


def score_gqa_max(q: torch.Tensor, landmarks: torch.Tensor, alpha: float) -> torch.Tensor:
    """-> [Z, n] bf16 = max over the m query rows of the softmax probabilities."""
    return score_logits_softmax(q, landmarks, alpha)[1].max(dim=1).values


# --------------------------------------------------------------------------------------------
# a2: top-k — models/kvcache/shadow.py:571-573 under the total order (value desc, index asc).
# Pinned by: tie-aware agreement with torch.topk (same set above the k-th value, same count at
# it) and brute force on tiny rows (tests/test_oracle_index.py).

def topk_total_order(scores: torch.Tensor, k: int) -> torch.Tensor:
    """scores [rows, n] -> indices [rows, k] ordered by (value desc, index asc)."""
    return torch.sort(scores.float(), dim=-1, descending=True, stable=True).indices[:, :k]


def topk_gather(scores: torch.Tensor, landmark_idx: torch.Tensor, k: int) -> torch.Tensor:
    return landmark_idx.gather(-1, topk_total_order(scores, k))


# --------------------------------------------------------------------------------------------
# a8: sparse attention — replaces flash_attn_with_kvcache (models/attention/shadow.py:48) for
# one query token: repeat_kv (models/tensor_op.py:125-130) + fp32 softmax, as the reference's
# torch fallback does (models/attention/sparq.py:45-51), in fp32 throughout.
# Pinned by: L = 1 (output = V row), identical keys (output = mean of V), float64 numpy.

def sparse_attention(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, L: int, scale: float | None = None):
    """q [B, Hq, D], K/V [B, Hkv, >=L, D] -> [B, Hq, D] bf16."""
    B, Hq, D = q.shape
    G = Hq // K.shape[1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    k = K[:, :, :L].float().repeat_interleave(G, dim=1)
    v = V[:, :, :L].float().repeat_interleave(G, dim=1)
    s = torch.einsum("bhd,bhld->bhl", q.float(), k) * scale
    p = torch.softmax(s, dim=-1)
    return torch.einsum("bhl,bhld->bhd", p, v).to(torch.bfloat16)


# --------------------------------------------------------------------------------------------
# RoPE tables — models/llama.py:138-142,162-167 and models/glm.py:132-133.

def build_cos_sin_cache(max_length: int, theta: float, head_dim: int = 128) -> torch.Tensor:
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = torch.outer(torch.arange(max_length + 1024, dtype=torch.float32), inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    half = head_dim // 2
    return torch.cat((emb.cos().to(torch.bfloat16)[:, :half], emb.sin().to(torch.bfloat16)[:, :half]), dim=-1)


def build_glm_cos_sin_cache(max_length: int, base: float) -> torch.Tensor:
    theta = 1.0 / (base ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))
    idx = torch.outer(torch.arange(max_length + 1024, dtype=torch.float32), theta)
    return torch.cat((idx.cos(), idx.sin()), dim=-1).to(torch.bfloat16)


# --------------------------------------------------------------------------------------------
# Encoder (prefill) and one decode step of one layer, composed from the functions above.
# encode_layer follows models/kvcache/shadow.py:411-544 (get_svd, prefill_kv_cache) and
# models/attention/shadow.py:8-13 (SVD of pre-RoPE K, then RoPE).

def prefill_geometry(ctx: int, budget: int, chunk: int) -> dict:
    """Prompt geometry of the offload cache: outlier chunks (budget/1024)*24 (shadow.py:329), 4 local
    chunks and the aligned chunk count, a multiple of 8 (:477-482), the local rows left over, the
    sparse region after the outliers (:500-501), the reference's buffer length (:346), the landmark
    count n = aligned chunks - outliers and S = budget/chunk.
    Pinned by: the derived-size table of the hot-path survey (tests/test_geometry_tables.py)."""
    local_chunk, outlier_chunk = 4, (budget // 1024) * 24
    chunks = ctx // chunk - local_chunk
    chunks -= chunks % 8
    prefill_local = ctx - chunks * chunk
    sparse_start = prefill_local + outlier_chunk * chunk
    return dict(S=budget // chunk, outlier_chunk=outlier_chunk, chunks=chunks, prefill_local=prefill_local,
                n=chunks - outlier_chunk, sparse_start=sparse_start, sparse_end=sparse_start + budget,
                buf_len=budget + 128 + (outlier_chunk + local_chunk) * chunk)


class LayerState:
    """Decode state of one layer as the offload cache holds it (CPU tensors)."""

    def __init__(self, **kw):
        self.__dict__.update(kw)


def _rope_tokens(x: torch.Tensor, cos_sin: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
    """x [B, H, L, D] RoPE by token position pos [L]: half-split with a [cos|sin] table of width D
    (models/llama.py:149-154), or, with a width-64 table, GLM's interleaved pairs (2i, 2i+1) of
    dims 0..63 and dims 64.. passed through (models/glm.py:212-235)."""
    cs = cos_sin[pos]
    if cos_sin.shape[-1] == 64:
        co, si = cs[:, :32], cs[:, 32:]
        xe, xo = x[..., 0:64:2], x[..., 1:64:2]
        y = x.clone()
        y[..., 0:64:2] = (xe * co) - (xo * si)
        y[..., 1:64:2] = (xo * co) + (xe * si)
        return y
    half = x.shape[-1] // 2
    return rope_half_split(x, cs[:, :half], cs[:, half:])


def encode_layer(k_pre: torch.Tensor, v: torch.Tensor, q_pre_last: torch.Tensor, cos_sin: torch.Tensor, *,
                 rank: int, chunk: int, budget: int, buf_len: int | None = None,
                 outliers: torch.Tensor | None = None, init_scores: torch.Tensor | None = None) -> LayerState:
    """k_pre/v [B, H, ctx, D] bf16 (pre-RoPE keys), q_pre_last [B, Hq, 1, D] (pre-RoPE last query).

    outliers: optional outlier chunk ids [B, H, outlier_chunk] (in outlier-slot order) to use instead
    of the bf16 min-cosine top-k; init_scores: optional GQA-max scores [B, H, n] for the initial
    selection, taken with topk_gather's order (value desc, index asc) instead of torch.topk. Both let
    a device encoder be checked from identical decisions (the reference leaves ties to torch)."""
    B, H, ctx, D = k_pre.shape
    Hq = q_pre_last.shape[1]
    G = Hq // H
    outlier_chunk = (budget // 1024) * 24
    S = budget // chunk
    # get_svd (shadow.py:411-444): SVD of [B, ctx, H*D] in fp32, keep rank R.
    kflat = k_pre.transpose(1, 2).reshape(B, ctx, H * D)
    u, s, vh = torch.linalg.svd(kflat.float(), full_matrices=False)
    U = u[:, :, :rank].to(torch.bfloat16)
    SV = (s[:, :rank].unsqueeze(-1) * vh[:, :rank]).to(torch.bfloat16).view(B, rank, H, D).permute(0, 2, 3, 1)
    SV = SV.contiguous()
    pos = torch.arange(ctx)
    k = _rope_tokens(k_pre, cos_sin, pos)
    q_last = _rope_tokens(q_pre_last, cos_sin, torch.tensor([ctx - 1]))
    # prefill_kv_cache (shadow.py:463-544)
    max_ctx_chunks = ctx // chunk
    host_v = v[:, :, :max_ctx_chunks * chunk].reshape(B, H, max_ctx_chunks, chunk * D).clone()
    geo = prefill_geometry(ctx, budget, chunk)
    chunks, prefill_local = geo["chunks"], geo["prefill_local"]
    sparse_start, sparse_end = geo["sparse_start"], geo["sparse_end"]
    buf_len = buf_len or geo["buf_len"]
    kbuf = torch.zeros(B, H, buf_len, D, dtype=torch.bfloat16)
    vbuf = torch.zeros(B, H, buf_len, D, dtype=torch.bfloat16)
    kbuf[:, :, :prefill_local] = k[:, :, -prefill_local:]
    vbuf[:, :, :prefill_local] = v[:, :, -prefill_local:]
    kctx = k[:, :, :chunks * chunk].reshape(B, H, chunks, chunk, D)
    cand = kctx.mean(dim=-2)
    cos = F.cosine_similarity(cand.unsqueeze(3).expand(-1, -1, -1, chunk, -1), kctx, dim=-1)
    if outliers is None:
        out_idx = cos.min(dim=-1).values.topk(outlier_chunk, largest=False).indices
    else:
        out_idx = outliers.to(torch.int64)
    gidx = out_idx.view(B, H, -1, 1, 1).expand(-1, -1, -1, chunk, D)
    kbuf[:, :, prefill_local:sparse_start] = kctx.gather(2, gidx).reshape(B, H, -1, D)
    vctx = v[:, :, :chunks * chunk].reshape(B, H, chunks, chunk, D)
    vbuf[:, :, prefill_local:sparse_start] = vctx.gather(2, gidx).reshape(B, H, -1, D)
    keep = torch.ones(B, H, chunks, dtype=torch.bool)
    keep.scatter_(-1, out_idx, False)
    rest = torch.arange(chunks).expand(B, H, -1).masked_select(keep).view(B, H, -1)
    landmarks = cand.gather(2, rest.unsqueeze(-1).expand(-1, -1, -1, D)).contiguous()
    if init_scores is None:
        sc = torch.einsum("bhgd,bhcd->bhgc", q_last.reshape(B, H, G, D), landmarks) / math.sqrt(128)
        sc = F.softmax(sc, dim=-1, dtype=torch.float32).to(torch.bfloat16).max(dim=-2).values
        sel = rest.gather(-1, sc.topk(S, dim=-1).indices)
    else:
        n = rest.shape[-1]
        sel = topk_gather(init_scores.reshape(B * H, n).to(torch.bfloat16), rest.reshape(B * H, n), S).view(B, H, S)
    tok = (sel.unsqueeze(-1) * chunk + torch.arange(chunk)).view(B, H, -1).unsqueeze(-1).expand(-1, -1, -1, D)
    vbuf[:, :, sparse_start:sparse_end] = v.gather(2, tok)
    kbuf[:, :, sparse_start:sparse_end] = k.gather(2, tok)
    return LayerState(U=U, SV=SV, landmarks=landmarks, landmark_idx=rest.contiguous(), host_v=host_v, kbuf=kbuf,
                      vbuf=vbuf, position_ids=sel.contiguous(), prefill_local=prefill_local,
                      sparse_start=sparse_start, sparse_end=sparse_end, chunk=chunk, budget=budget, ctx=ctx,
                      chunks=chunks, buf_len=buf_len)


def decode_layer_step(st: LayerState, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                      cos_sin: torch.Tensor, gen_offset: int = 0, scores: torch.Tensor | None = None) -> dict:
    """One decode step of one layer (models/attention/shadow.py:22-50 with the offload class).

    q [B, Hq, D] post-RoPE query, k_new/v_new [B, H, D] post-RoPE key and value of the new token.
    scores: optional GQA-max chunk scores [B, H, n] to select from instead of computing them (so a
    device implementation's selection can be checked bit for bit from identical scores).
    Mutates st (buffers, position_ids) like the cache does and returns the intermediates."""
    B, H, n, D = st.landmarks.shape
    Hq = q.shape[1]
    G = Hq // H
    S = st.budget // st.chunk
    L = st.sparse_end + gen_offset + 1
    st.kbuf[:, :, L - 1] = k_new
    st.vbuf[:, :, L - 1] = v_new
    if scores is None:
        scores = score_gqa_max(q.reshape(B * H, G, D), st.landmarks.reshape(B * H, n, D), 1.0 / math.sqrt(128))
    else:
        scores = scores.reshape(B * H, n).to(torch.bfloat16)
    selected = topk_gather(scores, st.landmark_idx.reshape(B * H, n), S)
    ids, offs, cnts = reorder(st.position_ids.reshape(B * H, S).numpy(), selected.numpy())
    E = st.chunk * D
    vreg = st.vbuf[:, :, st.sparse_start:st.sparse_end].reshape(B * H, S, E)
    kreg = st.kbuf[:, :, st.sparse_start:st.sparse_end].reshape(B * H, S, E)
    vnew = cached_gather_copy(st.host_v.reshape(B * H, -1, E).view(torch.int16).numpy(),
                              vreg.view(torch.int16).numpy(), offs, cnts)
    st.vbuf[:, :, st.sparse_start:st.sparse_end] = torch.from_numpy(vnew).view(torch.bfloat16).reshape(
        B, H, S * st.chunk, D)
    kcomp = compact_hits(kreg.view(torch.int16).numpy(), offs, cnts)
    st.kbuf[:, :, st.sparse_start:st.sparse_end] = torch.from_numpy(kcomp).view(torch.bfloat16).reshape(
        B, H, S * st.chunk, D)
    st.position_ids = torch.from_numpy(ids).view(B, H, S)
    # RoPE flavour by table width, as the reference's dispatch (models/tensor_op.py:176-204)
    rebuild_k_rope(st.U, st.SV, st.position_ids, torch.from_numpy(cnts), cos_sin, st.chunk, st.kbuf,
                   st.sparse_start, glm=cos_sin.shape[-1] == 64)
    out = sparse_attention(q, st.kbuf, st.vbuf, L)
    return dict(scores=scores.view(B, H, n), selected=selected.view(B, H, S), cnts=cnts, offsets=offs, out=out, L=L)


# --------------------------------------------------------------------------------------------
# f3: chunk pool — no reference counterpart; it extends the slot reuse of the reorder
# (kernels/map.cuh:475-516) to a device cache of P >= S chunk slots per (b, h). The policy is this
# build's own: a selected chunk found in the pool keeps its slot; the misses take the least
# recently used slots holding no selected chunk (empty slots first, then ascending step of last
# use, ties to the lowest slot), the k-th miss in selection order the k-th such slot in ascending
# slot order. Pinned by: brute-force simulation of that rule on small random and adversarial
# streams and by the invariants checked in tests/test_oracle_pool.py (every selected chunk
# resident after a step, table consistency, hits = |selection ∩ pool|, P == S reduces to the
# reference's set of buffered chunks).

def pool_assign(selected, slot_of, slot_chunk, slot_used, clock):
    """selected [rows, S] int64; tables (numpy int32, updated in place): slot_of [rows, chunks]
    (slot or -1), slot_chunk / slot_used [rows, P] (chunk or -1; step of last use or -1), clock
    [rows]. Returns slot_list [rows, S], miss_ids / miss_slot [rows, S] (misses at [cnts, S)) and
    cnts [rows] (the hit counts), all int32."""
    selected = np.asarray(selected, dtype=np.int64)
    rows, S = selected.shape
    P = slot_chunk.shape[1]
    slot_list = np.zeros((rows, S), np.int32)
    miss_ids = np.zeros((rows, S), np.int32)
    miss_slot = np.zeros((rows, S), np.int32)
    cnts = np.zeros(rows, np.int32)
    for r in range(rows):
        t = int(clock[r]) + 1
        hit = np.zeros(P, dtype=bool)
        misses = []
        for j, c in enumerate(selected[r]):
            sl = int(slot_of[r, c])
            if sl >= 0:
                slot_list[r, j] = sl
                slot_used[r, sl] = t
                hit[sl] = True
            else:
                misses.append(j)
        m = len(misses)
        free = [v for v in range(P) if not hit[v]]
        free.sort(key=lambda v: (int(slot_used[r, v]), v))
        victims = sorted(free[:m])
        base = S - m
        for k, j in enumerate(misses):
            v, c = victims[k], int(selected[r, j])
            old = int(slot_chunk[r, v])
            if old >= 0:
                slot_of[r, old] = -1
            slot_of[r, c] = v
            slot_chunk[r, v] = c
            slot_used[r, v] = t
            slot_list[r, j] = v
            miss_ids[r, base + k] = c
            miss_slot[r, base + k] = v
        cnts[r] = base
        clock[r] = t
    return slot_list, miss_ids, miss_slot, cnts


def pool_from_layer(st: LayerState, P: int) -> dict:
    """A chunk pool of P slots holding the layer's initial selection in slots 0..S-1: buffers with
    (P - S)*chunk more rows between the selected region and the generated tokens, and the tables."""
    B, H, buf, D = st.kbuf.shape
    S, c = st.budget // st.chunk, st.chunk
    delta = (P - S) * c
    rows = B * H
    kbuf = torch.zeros(B, H, buf + delta, D, dtype=st.kbuf.dtype)
    vbuf = torch.zeros_like(kbuf)
    kbuf[:, :, :st.sparse_end] = st.kbuf[:, :, :st.sparse_end]
    vbuf[:, :, :st.sparse_end] = st.vbuf[:, :, :st.sparse_end]
    sel = st.position_ids.reshape(rows, S).numpy()
    slot_of = np.full((rows, st.chunks), -1, np.int32)
    slot_chunk = np.full((rows, P), -1, np.int32)
    slot_used = np.full((rows, P), -1, np.int32)
    for r in range(rows):
        slot_of[r, sel[r]] = np.arange(S)
        slot_chunk[r, :S] = sel[r]
        slot_used[r, :S] = 0
    return dict(P=P, delta=delta, kbuf=kbuf, vbuf=vbuf, slot_of=slot_of, slot_chunk=slot_chunk, slot_used=slot_used,
                clock=np.zeros(rows, np.int32))


def decode_layer_step_pooled(st: LayerState, pool: dict, q, k_new, v_new, cos_sin, gen_offset: int = 0,
                             scores=None) -> dict:
    """decode_layer_step with a chunk pool: the selection (top-k of the GQA-max scores, or of the
    given scores) is mapped onto the pool by pool_assign, the misses' values copied from the host
    store and their keys rebuilt into their slots, and attention taken over [local | outliers |
    the selected chunks through the slot list | generated]. Mutates pool; returns the intermediates."""
    B, H, n, D = st.landmarks.shape
    G = q.shape[1] // H
    S, c = st.budget // st.chunk, st.chunk
    sp0, delta, rows = st.sparse_start, pool["delta"], B * H
    L = st.sparse_end + gen_offset + 1  # virtual length (the new token included)
    kbuf, vbuf = pool["kbuf"], pool["vbuf"]
    kbuf[:, :, L - 1 + delta] = k_new
    vbuf[:, :, L - 1 + delta] = v_new
    if scores is None:
        scores = score_gqa_max(q.reshape(rows, G, D), st.landmarks.reshape(rows, n, D), 1.0 / math.sqrt(128))
    else:
        scores = scores.reshape(rows, n).to(torch.bfloat16)
    selected = topk_gather(scores, st.landmark_idx.reshape(rows, n), S)
    slot_list, miss_ids, miss_slot, cnts = pool_assign(selected.numpy(), pool["slot_of"], pool["slot_chunk"],
                                                       pool["slot_used"], pool["clock"])
    # keys of the misses: rebuilt + rotated into a scratch [B, H, S*c, D] (rows of entries i >= cnts),
    # then moved to their slots; values from the host store
    scratch = torch.zeros(B, H, S * c, D, dtype=kbuf.dtype)
    ids = torch.from_numpy(miss_ids.astype(np.int64)).view(B, H, S)
    rebuild_k_rope(st.U, st.SV, ids, torch.from_numpy(cnts), cos_sin, c, scratch, 0, glm=cos_sin.shape[-1] == 64)
    for r in range(rows):
        b, h = divmod(r, H)
        for i in range(int(cnts[r]), S):
            v, cid = int(miss_slot[r, i]), int(miss_ids[r, i])
            kbuf[b, h, sp0 + v * c:sp0 + (v + 1) * c] = scratch[b, h, i * c:(i + 1) * c]
            vbuf[b, h, sp0 + v * c:sp0 + (v + 1) * c] = st.host_v[b, h, cid].view(c, D)
    # the virtual sequence the attention reads
    sel_rows = (torch.from_numpy(slot_list.astype(np.int64)).view(B, H, S, 1) * c + sp0 +
                torch.arange(c).view(1, 1, 1, c)).reshape(B, H, S * c)
    def virtual(buf):
        mid = buf.gather(2, sel_rows.unsqueeze(-1).expand(-1, -1, -1, D))
        tail = buf[:, :, st.sparse_end + delta:L + delta]
        return torch.cat([buf[:, :, :sp0], mid, tail], dim=2)
    out = sparse_attention(q, virtual(kbuf), virtual(vbuf), L)
    return dict(scores=scores.view(B, H, n), selected=selected.view(B, H, S), slot_list=slot_list, cnts=cnts,
                miss_ids=miss_ids, miss_slot=miss_slot, out=out, L=L)
