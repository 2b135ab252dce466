"""ShadowKV offload cache on MI355X: drop-in for ShadowKVCache_CPU (models/kvcache/shadow.py:301-651).

State per layer l (B = batch, H = kv heads, G = query heads per kv head, D = 128, c = chunk):
  * U[l] [B, ctx, R] and SV[l] [B, H, D, R] (bf16): low-rank factors of the pre-RoPE keys,
    shared across heads as in the reference (get_svd, shadow.py:411-444);
  * k_landmark[l] [B, H, n, D] / k_landmark_idx[l] [B, H, n]: chunk means of the post-RoPE keys
    that are not outliers, and their chunk ids (shadow.py:486-519);
  * v_cache_cpu[l] [B, H, max_length/c, c*D] in pinned host memory: every value chunk;
  * k/v_cache_buffer[l] [B, H, buf_len, D] on the device: [local | outliers | S selected chunks
    | generated tokens], the selected region at sparse_start..sparse_end in slot order;
  * position_ids[l] [B, H, S] (int64): chunk id held by each slot.

A decode step (driven by ShadowAttention.decode) scores the query against the landmarks,
selects S = sparse_budget/c chunks, reorders them against the previous slots, refills the
value slots from host memory (misses only) and rebuilds the key slots of the misses from
U.SV with RoPE — every one of these is a gfx950 kernel of libshadowkv_amd.so.

Deliberate differences from the reference, each an explicit error instead of a silent one:
  * `max_decode_len` sizes the buffers for the requested number of generated tokens; the
    reference's fixed 128-slot tail holds only 160 - prefill_local tokens and later writes are
    dropped (shadow.py:346, 628-629). update_kv_cache raises when the tail is full;
  * the host value store is addressed with its allocated row stride, so max_length may exceed
    the prompt length (the reference passes a prompt-derived stride, shadow.py:580);
  * G == 1 is supported (the reference's max-over-groups is skipped there and fails, :567-571);
  * top-k ties are broken by the lowest landmark index (torch leaves the choice open).
"""
from __future__ import annotations

import gc
import math

import torch
import torch.nn.functional as F

from ...kernels import shadowkv
from ..tensor_op import batch_gather_gemm_rotary_pos_emb_cuda
from .base import KVCacheBase


class ShadowKVCache_CPU(KVCacheBase):
    """ShadowKV with values offloaded to pinned host memory and low-rank keys rebuilt on the GPU."""

    def __init__(self, config, batch_size: int = 1, max_length: int = 32 * 1024, device: str = "cuda:0",
                 dtype=torch.bfloat16, sparse_budget: int = 2048, chunk_size: int = 8, rank: int = 160,
                 max_decode_len: int | None = None, zero_host_store: bool = True) -> None:
        self.config = config
        self.batch_size = batch_size
        self.max_length = max_length
        self.device = device
        self.dtype = dtype
        self.num_key_value_groups = config.num_attention_heads // config.num_key_value_heads
        self.head_dim = config.hidden_size // config.num_attention_heads
        self.num_attention_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        self.num_layers = config.num_hidden_layers

        self.sparse_budget = int(sparse_budget)
        self.chunk_size = chunk_size
        self.rank = rank
        self.local_chunk = 4
        self.outlier_chunk = int((self.sparse_budget // 1024) * 24)
        self.select_sets = self.sparse_budget // self.chunk_size
        if self.select_sets * self.chunk_size != self.sparse_budget:
            raise ValueError(f"sparse_budget {self.sparse_budget} is not a multiple of chunk_size {chunk_size}")

        L, B, H, D = self.num_layers, batch_size, self.num_key_value_heads, self.head_dim
        # One pinned host buffer per layer, [B, H, max_length/c, c*D] each (indexable like the reference's
        # [L, ...] tensor): torch's pinned allocator rounds each request up to a power of two, which a
        # single 64 GB allocation (Llama-3-8B, batch 8, 122K) would double.
        alloc = torch.zeros if zero_host_store else torch.empty
        self.v_cache_cpu = [alloc(B, H, max_length // chunk_size, D * chunk_size, dtype=dtype, pin_memory=True)
                            for _ in range(L)]
        # Sparse region ends at most at (local 4 chunks + 7 alignment chunks + 7 tokens) + outliers + budget.
        ref_len = self.sparse_budget + 128 + (self.outlier_chunk + self.local_chunk) * chunk_size
        if max_decode_len is None:
            self.buf_len = ref_len
        else:
            worst_sparse_end = (self.local_chunk + 8) * chunk_size - 1 + self.outlier_chunk * chunk_size \
                + self.sparse_budget
            self.buf_len = max(ref_len, worst_sparse_end + int(max_decode_len))
        self.k_cache_buffer = torch.zeros(L, B, H, self.buf_len, D, device=device, dtype=dtype)
        self.v_cache_buffer = torch.zeros(L, B, H, self.buf_len, D, device=device, dtype=dtype)

        self.kv_offset = 0
        self.prefill = 0
        self.gen_offset = 0
        self.prefilled_batch = 0
        self.incoming_q_len = 1

        self.k_landmark = None
        self.k_landmark_idx = None
        self.U = None
        self.SV = None

        # The reference's staging buffer and copy flags are not needed by the kernels.
        self.temp = None
        self.signals = None
        self.output = None

        rows = B * H
        self.block_num = rows
        self.offsets = torch.zeros(rows * self.select_sets, device=device, dtype=torch.int32)
        self.cnts = torch.zeros(rows, device=device, dtype=torch.int32)
        self.position_ids = torch.full((L, B, H, self.select_sets), -1, device=device, dtype=torch.int64)
        self.selected_chunks = torch.zeros(B, H, self.select_sets, device=device, dtype=torch.int64)
        self.keep_selected = False  # also emit the selected ids in top-k order into selected_chunks

        self.copy_stream = torch.cuda.Stream(device=device)
        self.key_stream = None  # optional: run the key rebuild on this stream (joined before attention)
        self.attn_workspace = None
        self.attn_out = None
        # Device-resident append row / attention length (use_device_lengths); None = host integers.
        self.append_row_dev = None
        self.kv_len_dev = None

    def print_stats(self):
        print(f"ShadowKV_CPU | sparse budget {self.sparse_budget} | chunk size {self.chunk_size} |rank {self.rank} "
              f"| cached {self.kv_offset} | local_chunk {self.local_chunk} | outlier_chunk {self.outlier_chunk}")

    # ------------------------------------------------------------------ encoding (prefill)
    def get_svd(self, new_k_cache: torch.Tensor, layer_idx: int):
        """Rank-R factors of the pre-RoPE keys [b, ctx, H*D] (or [b, H, ctx, D]) (shadow.py:411-444)."""
        if new_k_cache.shape[1] <= 32:
            k = new_k_cache.transpose(1, 2).reshape(new_k_cache.shape[0], -1, self.num_key_value_heads * self.head_dim)
        else:
            k = new_k_cache
        bsz = k.shape[0]
        if layer_idx == 0 and self.prefilled_batch == 0:
            self.U = torch.zeros(self.num_layers, self.batch_size, k.shape[1], self.rank, dtype=self.dtype)
            self.SV = torch.zeros(self.num_layers, self.batch_size, self.num_key_value_heads, self.head_dim, self.rank,
                                  dtype=self.dtype)
        u, s, vh = torch.linalg.svd(k.float(), full_matrices=False)
        pb = self.prefilled_batch
        self.U[layer_idx][pb:pb + bsz].copy_(u[:, :, :self.rank].to(self.dtype))
        sv = (s[:, :self.rank].unsqueeze(-1) * vh[:, :self.rank]).to(self.dtype)  # [b, R, H*D] = diag(s) V^T
        sv = sv.view(bsz, self.rank, self.num_key_value_heads, self.head_dim).permute(0, 2, 3, 1)  # [b, H, D, R]
        self.SV[layer_idx][pb:pb + bsz].copy_(sv)
        del u, s, vh

    def register_k_landmark(self, k_landmark: torch.Tensor, k_landmark_idx: torch.Tensor, layer_idx: int):
        n = k_landmark.shape[-2]
        bsz = k_landmark.shape[0]
        B, H, G = self.batch_size, self.num_key_value_heads, self.num_key_value_groups
        if layer_idx == 0 and self.prefilled_batch == 0:
            self.k_landmark = torch.zeros(self.num_layers, B, H, n, self.head_dim, dtype=self.dtype)
            self.k_landmark_idx = torch.zeros(self.num_layers, B, H, n, dtype=torch.long)
            tiles = (n + 255) // 256
            self.gemm_o = torch.zeros(B, H, G, n, dtype=torch.bfloat16)
            self.chunk_attn = torch.zeros(B, H, n, dtype=torch.bfloat16)
            self.norm = torch.zeros(B * H, G, tiles, dtype=torch.float32)
            self.sum = torch.zeros(B * H, G, tiles, dtype=torch.float32)
        pb = self.prefilled_batch
        self.k_landmark[layer_idx][pb:pb + bsz].copy_(k_landmark)
        self.k_landmark_idx[layer_idx][pb:pb + bsz].copy_(k_landmark_idx)

    def prefill_kv_cache(self, new_v_cache: torch.Tensor, layer_idx: int, key_states_roped: torch.Tensor,
                         last_query_states: torch.Tensor = None):
        """Build one layer's decode state from the prefill K/V (shadow.py:463-544)."""
        bsz, H, incoming, D = new_v_cache.shape
        c, pb, l = self.chunk_size, self.prefilled_batch, layer_idx
        self.prefill = incoming
        max_ctx_chunks = incoming // c
        self.max_ctx_chunks_len = max_ctx_chunks * c
        if max_ctx_chunks > self.v_cache_cpu[l].shape[2]:
            raise ValueError(f"prompt of {incoming} tokens exceeds max_length {self.max_length}")
        self.v_cache_cpu[l][pb:pb + bsz, :, :max_ctx_chunks].copy_(
            new_v_cache[:, :, :self.max_ctx_chunks_len].reshape(bsz, H, max_ctx_chunks, c * D))

        chunks = incoming // c - self.local_chunk
        self.chunks = chunks - chunks % 8
        self.prefill_local = incoming - self.chunks * c
        self.k_cache_buffer[l][pb:pb + bsz, :, :self.prefill_local].copy_(key_states_roped[:, :, -self.prefill_local:])
        self.v_cache_buffer[l][pb:pb + bsz, :, :self.prefill_local].copy_(new_v_cache[:, :, -self.prefill_local:])

        ctx = key_states_roped[:, :, :self.chunks * c].reshape(bsz, H, self.chunks, c, D)
        cand = ctx.mean(dim=-2)
        cos = F.cosine_similarity(cand.unsqueeze(3).expand(-1, -1, -1, c, -1), ctx, dim=-1)
        outlier_idx = cos.min(dim=-1).values.topk(self.outlier_chunk, largest=False).indices
        gidx = outlier_idx.view(bsz, H, -1, 1, 1).expand(-1, -1, -1, c, D)
        outlier_k = ctx.gather(2, gidx).reshape(bsz, H, self.outlier_chunk * c, D)
        vctx = new_v_cache[:, :, :self.chunks * c].reshape(bsz, H, self.chunks, c, D)
        outlier_v = vctx.gather(2, gidx).reshape(bsz, H, self.outlier_chunk * c, D)

        self.sparse_start = self.prefill_local + self.outlier_chunk * c
        self.sparse_end = self.sparse_start + self.sparse_budget
        if self.sparse_end > self.buf_len:
            raise ValueError("sparse region does not fit the device buffers")
        self.kernel_offset = self.sparse_start * D
        self.kernel_stride = self.buf_len * D
        self.k_cache_buffer[l][pb:pb + bsz, :, self.prefill_local:self.sparse_start].copy_(outlier_k)
        self.v_cache_buffer[l][pb:pb + bsz, :, self.prefill_local:self.sparse_start].copy_(outlier_v)

        keep = torch.ones(bsz, H, self.chunks, dtype=torch.bool, device=key_states_roped.device)
        keep.scatter_(-1, outlier_idx, False)
        rest_idx = torch.arange(self.chunks, device=key_states_roped.device).expand(bsz, H, -1)
        rest_idx = rest_idx.masked_select(keep).view(bsz, H, -1)
        landmarks = cand.gather(2, rest_idx.unsqueeze(-1).expand(-1, -1, -1, D))
        self.register_k_landmark(landmarks, rest_idx, l)

        # Initial selection from the last prompt query (shadow.py:522-534).
        G = self.num_key_value_groups
        lm = self.k_landmark[l][pb:pb + bsz].to(last_query_states.device)
        scores = torch.einsum("bhgd,bhcd->bhgc", last_query_states.reshape(-1, H, G, D), lm) / math.sqrt(128)
        scores = F.softmax(scores, dim=-1, dtype=torch.float32).to(self.dtype).max(dim=-2).values
        top = scores.topk(self.select_sets, dim=-1).indices
        selected = self.k_landmark_idx[l][pb:pb + bsz].to(last_query_states.device).gather(-1, top)
        self.position_ids[l][pb:pb + bsz].copy_(selected)
        if int(selected.max()) >= self.chunks or int(selected.min()) < 0:
            raise AssertionError("initial selection outside the chunk range")
        tok = (selected.unsqueeze(-1) * c + torch.arange(c, device=selected.device)).view(bsz, H, -1)
        tok = tok.unsqueeze(-1).expand(-1, -1, -1, D)
        self.v_cache_buffer[l][pb:pb + bsz, :, self.sparse_start:self.sparse_end].copy_(new_v_cache.gather(-2, tok))
        self.k_cache_buffer[l][pb:pb + bsz, :, self.sparse_start:self.sparse_end].copy_(key_states_roped.gather(-2, tok))

        if layer_idx == self.num_layers - 1:
            if not self.sparse_budget < incoming:
                raise AssertionError("sparse budget must be smaller than the prompt")
            self.prefilled_batch += bsz
            if self.prefilled_batch == self.batch_size:
                self.kv_offset += incoming
                if bool((self.position_ids == -1).any()):
                    raise AssertionError("the offload cache was not built for every layer and sequence")

    # ------------------------------------------------------------------ decoding
    def get_retrieval_position_ids(self, layer_idx: int, query_states: torch.Tensor) -> torch.Tensor:
        """Select S chunks for the current query and reorder them against the previous slots."""
        B, H, G, D = self.batch_size, self.num_key_value_heads, self.num_key_value_groups, self.head_dim
        self.incoming_q_len = query_states.shape[-2]
        if self.incoming_q_len != 1:
            raise ValueError("decode scoring takes one query token per step")
        n = self.k_landmark.shape[-2]
        q = query_states if query_states.is_contiguous() else query_states.contiguous()
        shadowkv.score_logits(q, self.k_landmark[layer_idx], self.gemm_o, self.norm, self.sum, B * H, G, n, D,
                              1.0 / math.sqrt(128))
        # softmax + GQA max + top-k + landmark-id gather + reorder in one launch. The GQA-max scores are kept in
        # chunk_attn; the selected ids in top-k order (selected_chunks) only when keep_selected is set.
        shadowkv.select_chunks(self.gemm_o, self.norm, self.sum, B * H, G, n, self.k_landmark_idx[layer_idx].view(B * H, n),
                               self.select_sets, self.chunks, self.position_ids[layer_idx].view(B * H, -1), self.offsets,
                               self.cnts, out_scores=self.chunk_attn,
                               out_selected=self.selected_chunks if self.keep_selected else None)
        return self.position_ids[layer_idx]

    def _gen_len(self, layer_idx: int) -> int:
        return self.gen_offset if layer_idx == self.num_layers - 1 else self.gen_offset + self.incoming_q_len

    def _live_view(self, buf: torch.Tensor, layer_idx: int) -> torch.Tensor:
        if self.kv_len_dev is not None:
            return buf[:, :, :self.buf_len]  # length read on the device (kv_len_dev)
        return buf[:, :, :self.sparse_end + self._gen_len(layer_idx)]

    def get_value_cache(self, layer_idx: int, position_ids: torch.Tensor, hits_moved: bool = False) -> torch.Tensor:
        """The layer's value buffer with the selected chunks in place: cache hits moved to their
        new slots (unless move_value_hits already did, hits_moved) and misses gathered from host."""
        shadowkv.gather_copy_with_offsets(self.v_cache_cpu[layer_idx], self.v_cache_buffer[layer_idx], self.temp,
                                          self.offsets, self.cnts, self.signals, self.batch_size,
                                          self.num_key_value_heads, int(self.max_ctx_chunks_len * self.head_dim),
                                          int(self.sparse_budget * self.head_dim), self.kernel_offset,
                                          self.kernel_stride, self.select_sets, misses_only=hits_moved)
        return self._live_view(self.v_cache_buffer[layer_idx], layer_idx)

    def move_value_hits(self, layer_idx: int):
        """The in-buffer half of the value fetch alone (hit rows to their new slots), so that a
        later get_value_cache(..., hits_moved=True) on the copy stream is host-link work only."""
        shadowkv.gather_copy_d2d_with_offsets(self.v_cache_buffer[layer_idx], self.offsets, self.cnts, self.batch_size,
                                              self.num_key_value_heads, int(self.sparse_budget * self.head_dim),
                                              self.kernel_offset, self.kernel_stride, self.select_sets)

    def get_key_cache(self, layer_idx: int, position_ids: torch.Tensor, rope_func, cos_sin_cache) -> torch.Tensor:
        shadowkv.gather_copy_d2d_with_offsets(self.k_cache_buffer[layer_idx], self.offsets, self.cnts, self.batch_size,
                                              self.num_key_value_heads, int(self.sparse_budget * self.head_dim),
                                              self.kernel_offset, self.kernel_stride, self.select_sets)
        batch_gather_gemm_rotary_pos_emb_cuda(self.U[layer_idx], self.SV[layer_idx], cos_sin_cache, position_ids,
                                              self.output, self.chunk_size, self.k_cache_buffer[layer_idx],
                                              self.sparse_start, self.sparse_end, self.cnts)
        return self._live_view(self.k_cache_buffer[layer_idx], layer_idx)

    def H2D(self):
        gc.collect()
        torch.cuda.synchronize()
        self.SV = self.SV.to(self.device)
        self.U = self.U.to(self.device)
        self.k_landmark = self.k_landmark.to(self.device)
        self.k_landmark_idx = self.k_landmark_idx.to(self.device)
        self.gemm_o = self.gemm_o.to(self.device)
        self.chunk_attn = self.chunk_attn.to(self.device)
        self.norm = self.norm.to(self.device)
        self.sum = self.sum.to(self.device)
        self._alloc_attention()
        torch.cuda.synchronize()

    def _alloc_attention(self):
        B, Hq = self.batch_size, self.num_attention_heads
        nbytes = shadowkv.sparse_attn_workspace_bytes(B, Hq, self.buf_len)
        self.attn_workspace = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        self.attn_out = torch.empty(B, Hq, self.head_dim, dtype=self.dtype, device=self.device)

    def check_capacity(self, incoming: int = 1):
        if self.sparse_end + self.gen_offset + incoming > self.buf_len:
            raise RuntimeError(f"decode capacity exhausted: {self.gen_offset} tokens generated, buffer holds "
                               f"{self.buf_len - self.sparse_end}; construct the cache with a larger max_decode_len")

    def advance(self, incoming: int = 1):
        """Host bookkeeping of one decode step (the device scalars advance inside the step)."""
        self.kv_offset += incoming
        self.gen_offset += incoming

    def use_device_lengths(self):
        """Keep the append row and the attention length in device scalars that the decode step
        advances itself (at layer 0), so a whole step can be captured in a HIP graph and replayed.
        The host counters stay authoritative for the capacity check."""
        row = self.sparse_end + self.gen_offset - 1  # advanced before the step's first append
        self.append_row_dev = torch.full((1,), row, dtype=torch.int64, device=self.device)
        self.kv_len_dev = torch.full((1,), row + 1, dtype=torch.int32, device=self.device)

    def rope_and_append(self, qkv: torch.Tensor, position_ids: torch.Tensor, cos_sin: torch.Tensor, layer_idx: int,
                        q_out: torch.Tensor) -> torch.Tensor:
        """Fused new-token step (device-resident lengths only): q and k of the fused projection
        rows qkv [B, (Hq + 2 Hkv) * 128] rotated at position_ids [B], rotated q written to q_out
        [B, Hq, 128], rotated k and v appended at the device append row, in one launch (the work
        of the rotary embedding plus update_kv_cache). Returns q_out viewed [B, Hq, 1, 128]."""
        if self.append_row_dev is None:
            raise RuntimeError("rope_and_append needs use_device_lengths()")
        self.check_capacity(1)
        if layer_idx == 0:
            self.append_row_dev.add_(1)
            self.kv_len_dev.add_(1)
        shadowkv.rope_qk_append(qkv, self.num_attention_heads, self.num_key_value_heads, position_ids, cos_sin, q_out,
                                self.k_cache_buffer[layer_idx], self.v_cache_buffer[layer_idx], self.append_row_dev)
        if layer_idx == self.num_layers - 1:
            self.advance(1)
        return q_out.view(q_out.shape[0], self.num_attention_heads, 1, self.head_dim)

    def update_kv_cache(self, new_k_cache: torch.Tensor, new_v_cache: torch.Tensor, layer_idx: int):
        incoming = new_k_cache.shape[-2]
        self.check_capacity(incoming)
        if self.append_row_dev is not None:
            if incoming != 1:
                raise ValueError("device-resident lengths advance one token per decode step")
            if layer_idx == 0:
                self.append_row_dev.add_(1)
                self.kv_len_dev.add_(1)
            self.v_cache_buffer[layer_idx].index_copy_(2, self.append_row_dev, new_v_cache)
            self.k_cache_buffer[layer_idx].index_copy_(2, self.append_row_dev, new_k_cache)
        else:
            start = self.sparse_end + self.gen_offset
            self.v_cache_buffer[layer_idx][:, :, start:start + incoming].copy_(new_v_cache, non_blocking=True)
            self.k_cache_buffer[layer_idx][:, :, start:start + incoming].copy_(new_k_cache, non_blocking=True)
        if layer_idx == self.num_layers - 1:
            self.advance(incoming)

    def clear(self):
        self.k_cache_buffer.zero_()
        self.v_cache_buffer.zero_()
        self.position_ids.fill_(-1)
        self.k_landmark = None
        self.k_landmark_idx = None
        self.U = None
        self.SV = None
        self.kv_offset = 0
        self.prefill = 0
        self.gen_offset = 0
        self.prefill_local = 0
        self.prefilled_batch = 0
        self.append_row_dev = None
        self.kv_len_dev = None

    def get_kv_len(self):
        return self.kv_offset
