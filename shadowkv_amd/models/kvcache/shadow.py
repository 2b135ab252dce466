"""ShadowKV offload cache on MI355X: drop-in for ShadowKVCache_CPU (models/kvcache/shadow.py:301-651).

State per layer l (B = batch, H = kv heads, G = query heads per kv head, D = 128, c = chunk):
  * U[l] [B, ctx, R] and SV[l] [B, H, D, R] (bf16): low-rank factors of the pre-RoPE keys,
    shared across heads as in the reference (get_svd, shadow.py:411-444);
  * k_landmark[l] [B, H, n, D] / k_landmark_idx[l] [B, H, n]: chunk means of the post-RoPE keys
    that are not outliers, and their chunk ids (shadow.py:486-519);
  * v_cache_cpu[l] [B, H, max_length/c, c*D] in pinned host memory (or, with
    value_store="device", in device memory): every value chunk;
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

from ...kernels import shadowkv
from ...streams import side_stream
from ..tensor_op import batch_gather_gemm_rotary_pos_emb_cuda
from .base import KVCacheBase


def low_rank_factors(k: torch.Tensor, rank: int):
    """Leading rank-R factors of k [b, rows, cols] (rows >= cols): u [b, rows, R] and svt = diag(s) V^T
    [b, R, cols] in fp32, with k ~ u @ svt. The reference's full SVD (shadow.py:411-444) is replaced by
    the top R eigenpairs of the fp32 Gram matrix k^T k (k = U diag(s) V^T gives k^T k V = V diag(s^2)
    and U = k V / s): one hipBLASLt GEMM, one rocSOLVER symmetric eigendecomposition of [cols, cols]
    and one GEMM. The product u @ svt does not depend on the sign of each factor pair. MI355X,
    [122880, 1024]: 22 ms vs 2.1 s for the full SVD; rank-160 reconstructions agree to 5e-4."""
    kf = k.float()
    gram = torch.matmul(kf.transpose(1, 2), kf)
    w, v = torch.linalg.eigh(gram)  # ascending eigenvalues
    w, v = w.flip(-1)[..., :rank], v.flip(-1)[..., :rank]
    s = w.clamp_min(0).sqrt()
    u = torch.matmul(kf, v) / s.clamp_min(1e-30).unsqueeze(1)
    return u, s.unsqueeze(-1) * v.transpose(1, 2)


def outlier_chunks(sparse_budget: int) -> int:
    """Outlier chunks kept exactly per (b, h): 24 per 1024 tokens of budget (shadow.py:329)."""
    return int((int(sparse_budget) // 1024) * 24)


class ShadowKVCache_CPU(KVCacheBase):
    """ShadowKV with values offloaded to pinned host memory and low-rank keys rebuilt on the GPU."""

    def __init__(self, config, batch_size: int = 1, max_length: int = 32 * 1024, device: str = "cuda:0",
                 dtype=torch.bfloat16, sparse_budget: int = 2048, chunk_size: int = 8, rank: int = 160,
                 max_decode_len: int | None = None, zero_host_store: bool = True,
                 chunk_cache: int | None = None, copy_stream: torch.cuda.Stream | None = None,
                 host_stores: int | None = None, value_store: str = "host") -> None:
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
        self.outlier_chunk = outlier_chunks(self.sparse_budget)
        self.select_sets = self.sparse_budget // self.chunk_size
        if self.select_sets * self.chunk_size != self.sparse_budget:
            raise ValueError(f"sparse_budget {self.sparse_budget} is not a multiple of chunk_size {chunk_size}")

        # Chunk pool (chunk_cache = P >= S slots per (b, h) and layer): the selected region becomes a
        # pool of P chunk slots that keeps chunks across steps (least recently used replaced); the
        # attention reads the selection through a slot list. None: the reference's slot reuse.
        self.pooled = chunk_cache is not None
        self.pool_slots = self.select_sets if chunk_cache is None else int(chunk_cache)
        if self.pool_slots < self.select_sets:
            raise ValueError(f"chunk_cache={chunk_cache} holds fewer than the {self.select_sets} selected chunks")
        self.pool_delta = (self.pool_slots - self.select_sets) * chunk_size  # rows between selection end and tail

        L, B, H, D = self.num_layers, batch_size, self.num_key_value_heads, self.head_dim
        # One pinned host buffer per layer, [B, H, max_length/c, c*D] each (indexable like the reference's
        # [L, ...] tensor): torch's pinned allocator rounds each request up to a power of two, which a
        # single 64 GB allocation (Llama-3-8B, batch 8, 122K) would double.
        # host_stores (None: one per layer): k distinct stores, layer l using store l % k. Layers
        # then share the host copy of their values (what the last layer to write a store wrote),
        # for callers that need the decode shapes but not distinct contents per layer (the
        # full-size tests: one process may pin only about 65 GiB on the MI355X hosts).
        # value_store="device" keeps the value store in device memory instead (the whole store of the
        # Llama-3.1-8B batch-8 ctx-122880 workload, 64 GB, fits MI355X's 288 GB of HBM): the same
        # kernels then gather the missed chunks from HBM, and nothing crosses the host link.
        if value_store not in ("host", "device"):
            raise ValueError(f"value_store must be 'host' or 'device', not {value_store!r}")
        self.value_store = value_store
        # With the store in device memory (and no chunk pool) the selected values are not gathered
        # into v_cache_buffer at all: the attention reads them in place from the store
        # (skv_sparse_attn_decode_vstore; bit-identical to the gathered buffer), and only the key
        # buffer's hits move. False: gather from the device store as from a host one.
        self.values_in_place = value_store == "device" and chunk_cache is None
        alloc = torch.zeros if zero_host_store else torch.empty
        stores = L if host_stores is None else max(1, min(L, int(host_stores)))
        where = dict(pin_memory=True) if value_store == "host" else dict(device=device)
        own = [alloc(B, H, max_length // chunk_size, D * chunk_size, dtype=dtype, **where) for _ in range(stores)]
        self.v_cache_cpu = [own[l % stores] for l in range(L)]
        # Sparse region ends at most at (local 4 chunks + 7 alignment chunks + 7 tokens) + outliers + budget.
        ref_len = self.sparse_budget + 128 + (self.outlier_chunk + self.local_chunk) * chunk_size
        if max_decode_len is None:
            self.buf_len = ref_len
        else:
            worst_sparse_end = (self.local_chunk + 8) * chunk_size - 1 + self.outlier_chunk * chunk_size \
                + self.sparse_budget
            self.buf_len = max(ref_len, worst_sparse_end + int(max_decode_len))
        self.buf_len += self.pool_delta
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
        # Optional (off by default, as the reference's get_retrieval_position_ids only computes ids,
        # offsets and counts): fold the value buffer's hit moves into the selection's last launch,
        # so that the value fetch follows the selection directly (the key buffer's moves stay a
        # launch of the key path, which overlaps the fetch). With it on, get_retrieval_position_ids
        # also moves buffer contents: callers must then fetch through get_value_cache /
        # get_key_cache / fetch_and_rebuild, which skip the moves already done (_folded[l] names the
        # buffers whose hits the last selection of layer l moved); a second compaction through the
        # shadowkv module's gather_copy_with_offsets would move the hits twice.
        self.fold_hit_moves = False
        self._folded = [set() for _ in range(L)]
        # One-stream fetch (callers that run the whole step on one stream): the selection moves
        # both buffers' hits, and fetch_and_rebuild() issues the value fetch and the key rebuild
        # as one launch on the current stream (no copy-stream hop before or after the fetch).
        self.one_stream_fetch = False

        # value-fetch stream: the given one, else the process's shared fetch side stream
        self.copy_stream = copy_stream if copy_stream is not None else side_stream(device, "fetch")
        self.key_stream = None  # optional: run the key rebuild on this stream (joined before attention)
        # optional: run the one-launch value fetch + key rebuild (one_stream_active) on this stream
        # instead of the current one (joined before attention), with this many fetch workgroups
        # (4-wave workgroups; 0: the library default) and at most this many rebuild workgroups
        # looping over the tiles (0: one per tile)
        self.lane_stream = None
        self.fused_fetch_workgroups = 0
        self.fused_rebuild_workgroups = 0
        self.attn_workspace = None
        self.attn_out = None
        self.select_workspace = None  # allocated with the landmarks
        # Device-resident append row / attention length (use_device_lengths); None = host integers.
        self.append_row_dev = None
        self.kv_len_dev = None
        # Chunk pool tables (allocated with the prompt geometry) and per-step scratch.
        self.slot_of = self.slot_chunk = self.slot_used = self.pool_clock = None
        if self.pooled:
            S = self.select_sets
            self.slot_list = torch.zeros(rows, S, device=device, dtype=torch.int32)
            self.miss_ids = torch.zeros(rows, S, device=device, dtype=torch.int32)
            self.miss_slot = torch.zeros(rows, S, device=device, dtype=torch.int32)

    def print_stats(self):
        print(f"ShadowKV_CPU | sparse budget {self.sparse_budget} | chunk size {self.chunk_size} |rank {self.rank} "
              f"| cached {self.kv_offset} | local_chunk {self.local_chunk} | outlier_chunk {self.outlier_chunk}")

    # ------------------------------------------------------------------ encoding (prefill)
    @staticmethod
    def _require_device(*tensors):
        for t in tensors:
            if t is not None and not t.is_cuda:
                raise ValueError("the prefill encoder runs on the device: pass the prompt tensors as device tensors "
                                 "(load_layer_state installs a state encoded elsewhere)")

    def get_svd(self, new_k_cache: torch.Tensor, layer_idx: int):
        """Rank-R factors of the pre-RoPE keys [b, ctx, H*D] (or [b, H, ctx, D]) (shadow.py:411-444),
        on the device. The reference takes a full fp32 SVD of [ctx, H*D]; the leading R factors are
        the top R eigenpairs of the fp32 Gram matrix instead (low_rank_factors)."""
        self._require_device(new_k_cache)
        H, D, R = self.num_key_value_heads, self.head_dim, self.rank
        if new_k_cache.shape[1] <= 32:
            k = new_k_cache.transpose(1, 2).reshape(new_k_cache.shape[0], -1, H * D)
        else:
            k = new_k_cache
        bsz, ctx = k.shape[0], k.shape[1]
        if layer_idx == 0 and self.prefilled_batch == 0:
            self.U = torch.zeros(self.num_layers, self.batch_size, ctx, R, dtype=self.dtype, device=self.device)
            self.SV = torch.zeros(self.num_layers, self.batch_size, H, D, R, dtype=self.dtype, device=self.device)
        u, svt = low_rank_factors(k, R)
        pb = self.prefilled_batch
        self.U[layer_idx][pb:pb + bsz].copy_(u.to(self.dtype))
        self.SV[layer_idx][pb:pb + bsz].copy_(svt.to(self.dtype).view(bsz, R, H, D).permute(0, 2, 3, 1))  # [b,H,D,R]
        del u, svt

    def _alloc_landmarks(self, n: int):
        B, H, G = self.batch_size, self.num_key_value_heads, self.num_key_value_groups
        tiles = (n + 255) // 256
        dev = self.device
        self.k_landmark = torch.zeros(self.num_layers, B, H, n, self.head_dim, dtype=self.dtype, device=dev)
        self.k_landmark_idx = torch.zeros(self.num_layers, B, H, n, dtype=torch.long, device=dev)
        self.gemm_o = torch.zeros(B, H, G, n, dtype=torch.bfloat16, device=dev)
        self.chunk_attn = torch.zeros(B, H, n, dtype=torch.bfloat16, device=dev)
        self.norm = torch.zeros(B * H, G, tiles, dtype=torch.float32, device=dev)
        self.sum = torch.zeros(B * H, G, tiles, dtype=torch.float32, device=dev)
        # scratch of the selection, which spreads each row over many workgroups when rows are few
        nbytes = shadowkv.select_workspace_bytes(B * H, n, self.select_sets)
        self.select_workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)

    def register_k_landmark(self, k_landmark: torch.Tensor, k_landmark_idx: torch.Tensor, layer_idx: int):
        n = k_landmark.shape[-2]
        bsz = k_landmark.shape[0]
        if layer_idx == 0 and self.prefilled_batch == 0:
            self._alloc_landmarks(n)
        pb = self.prefilled_batch
        self.k_landmark[layer_idx][pb:pb + bsz].copy_(k_landmark)
        self.k_landmark_idx[layer_idx][pb:pb + bsz].copy_(k_landmark_idx)

    def _set_geometry(self, incoming: int):
        c = self.chunk_size
        self.prefill = incoming
        self.max_ctx_chunks_len = (incoming // c) * c
        chunks = incoming // c - self.local_chunk
        self.chunks = chunks - chunks % 8
        self.prefill_local = incoming - self.chunks * c
        self.sparse_start = self.prefill_local + self.outlier_chunk * c
        self.sparse_end = self.sparse_start + self.sparse_budget
        if self.sparse_end > self.buf_len:
            raise ValueError("sparse region does not fit the device buffers")
        self.kernel_offset = self.sparse_start * self.head_dim
        self.kernel_stride = self.buf_len * self.head_dim

    def _copy_chunks(self, src: torch.Tensor, dst: torch.Tensor, ids: torch.Tensor, start_row: int):
        """dst[b, h, start_row + i*c + j] = src[b, h, ids[b*H+h, i]*c + j] for the chunk-gather kernel:
        src [b, H, rows, D] device rows, dst a [b, H, buf_len, D] slice of a device buffer."""
        bsz, H, rows, D = src.shape
        c = self.chunk_size
        m = ids.shape[-1]
        nch = rows // c
        src_chunks = src[:, :, :nch * c].reshape(bsz, H, nch, c * D)
        offs = ids.reshape(-1).to(torch.int32)
        cnts = torch.zeros(bsz * H, dtype=torch.int32, device=src.device)
        shadowkv.gather_copy_with_offsets(src_chunks, dst, None, offs, cnts, None, bsz, H, nch * c * D, m * c * D,
                                          start_row * D, self.buf_len * D, m, misses_only=True)

    def prefill_kv_cache(self, new_v_cache: torch.Tensor, layer_idx: int, key_states_roped: torch.Tensor,
                         last_query_states: torch.Tensor = None):
        """Build one layer's decode state from the prefill K/V (shadow.py:463-544), on the device:
        value chunks to the pinned host store; local rows; chunk means and minimum row cosines
        (skv_chunk_stats); the outlier chunks and the landmark ids (skv_select_outliers); the
        landmarks (skv_gather_rows); outlier and initially selected K/V chunks copied by the
        chunk-gather kernel; the initial selection by the decode path's scoring, GQA max and top-k."""
        self._require_device(new_v_cache, key_states_roped, last_query_states)
        bsz, H, incoming, D = new_v_cache.shape
        c, pb, l, G = self.chunk_size, self.prefilled_batch, layer_idx, self.num_key_value_groups
        max_ctx_chunks = incoming // c
        if max_ctx_chunks > self.v_cache_cpu[l].shape[2]:
            raise ValueError(f"prompt of {incoming} tokens exceeds max_length {self.max_length}")
        self._set_geometry(incoming)
        v = new_v_cache if new_v_cache.stride(-1) == 1 and new_v_cache.stride(-2) == D else new_v_cache.contiguous()
        k = key_states_roped if key_states_roped.stride(-1) == 1 and key_states_roped.stride(-2) == D \
            else key_states_roped.contiguous()
        self.v_cache_cpu[l][pb:pb + bsz, :, :max_ctx_chunks].copy_(
            v[:, :, :self.max_ctx_chunks_len].reshape(bsz, H, max_ctx_chunks, c * D))
        kbuf = self.k_cache_buffer[l][pb:pb + bsz]
        vbuf = self.v_cache_buffer[l][pb:pb + bsz]
        kbuf[:, :, :self.prefill_local].copy_(k[:, :, -self.prefill_local:])
        vbuf[:, :, :self.prefill_local].copy_(v[:, :, -self.prefill_local:])

        rows, chunks, n = bsz * H, self.chunks, self.chunks - self.outlier_chunk
        dev = k.device
        cand = torch.empty(bsz, H, chunks, D, dtype=self.dtype, device=dev)
        min_cos = torch.empty(bsz, H, chunks, dtype=torch.float32, device=dev)
        shadowkv.chunk_stats(k, chunks, c, cand, min_cos)
        outlier_idx = torch.empty(rows, self.outlier_chunk, dtype=torch.int64, device=dev)
        landmark_idx = torch.empty(rows, n, dtype=torch.int64, device=dev)
        shadowkv.select_outliers(min_cos.view(rows, chunks), self.outlier_chunk, outlier_idx, landmark_idx)
        landmarks = torch.empty(rows, n, D, dtype=self.dtype, device=dev)
        shadowkv.gather_rows(cand.view(rows, chunks, D), landmark_idx, landmarks)
        self._copy_chunks(k, kbuf, outlier_idx, self.prefill_local)
        self._copy_chunks(v, vbuf, outlier_idx, self.prefill_local)
        self.register_k_landmark(landmarks.view(bsz, H, n, D), landmark_idx.view(bsz, H, n), l)

        # Initial selection from the last prompt query (shadow.py:522-534): the decode path's
        # scoring + softmax/GQA max + top-k, ids in top-k order; the selected chunks' exact K/V.
        q = last_query_states.reshape(rows, G, D).contiguous()
        tiles = (n + 255) // 256
        logits = torch.empty(rows, G, n, dtype=torch.bfloat16, device=dev)
        part_max = torch.empty(rows, G, tiles, dtype=torch.float32, device=dev)
        part_sum = torch.empty(rows, G, tiles, dtype=torch.float32, device=dev)
        shadowkv.score_logits(q, landmarks, logits, part_max, part_sum, rows, G, n, D, 1.0 / math.sqrt(128))
        scores = torch.empty(rows, n, dtype=torch.bfloat16, device=dev)
        shadowkv.softmax_gqa_max(logits, part_max, part_sum, scores, rows, G, n)
        self.chunk_attn[pb:pb + bsz].copy_(scores.view(bsz, H, n))  # as after a decode step: the last layer's
        selected = torch.empty(rows, self.select_sets, dtype=torch.int64, device=dev)
        shadowkv.topk_gather(scores, landmark_idx, self.select_sets, selected)
        self.position_ids[l][pb:pb + bsz].copy_(selected.view(bsz, H, -1))
        self._copy_chunks(v, vbuf, selected, self.sparse_start)
        self._copy_chunks(k, kbuf, selected, self.sparse_start)
        self.init_pool(l, pb, bsz)
        self._finish_layer(l, bsz, incoming)

    def init_pool(self, layer_idx: int, pb: int = 0, bsz: int | None = None):
        """Pool tables of one layer from its initial selection: slot j holds position_ids[j]
        (the layout of the selected region), the other slots are empty."""
        if not self.pooled:
            return
        bsz = self.batch_size if bsz is None else bsz
        H, S, P, L = self.num_key_value_heads, self.select_sets, self.pool_slots, self.num_layers
        rows = self.batch_size * H
        if self.slot_of is None or self.slot_of.shape[-1] != self.chunks:
            dev = self.device
            self.slot_of = torch.full((L, rows, self.chunks), -1, dtype=torch.int32, device=dev)
            self.slot_chunk = torch.full((L, rows, P), -1, dtype=torch.int32, device=dev)
            self.slot_used = torch.full((L, rows, P), -1, dtype=torch.int32, device=dev)
            self.pool_clock = torch.zeros(L, rows, dtype=torch.int32, device=dev)
        r0, r1 = pb * H, (pb + bsz) * H
        sel = self.position_ids[layer_idx][pb:pb + bsz].reshape(bsz * H, S)
        slots = torch.arange(S, dtype=torch.int32, device=sel.device).expand(bsz * H, S)
        self.slot_of[layer_idx, r0:r1].fill_(-1)
        self.slot_of[layer_idx, r0:r1].scatter_(1, sel, slots)
        self.slot_chunk[layer_idx, r0:r1].fill_(-1)
        self.slot_chunk[layer_idx, r0:r1, :S].copy_(sel)
        self.slot_used[layer_idx, r0:r1].fill_(-1)
        self.slot_used[layer_idx, r0:r1, :S].fill_(0)
        self.pool_clock[layer_idx, r0:r1].fill_(0)

    def _finish_layer(self, layer_idx: int, bsz: int, incoming: int):
        if layer_idx == self.num_layers - 1:
            if not self.sparse_budget < incoming:
                raise AssertionError("sparse budget must be smaller than the prompt")
            self.prefilled_batch += bsz
            if self.prefilled_batch == self.batch_size:
                self.kv_offset += incoming
                if bool((self.position_ids == -1).any()):
                    raise AssertionError("the offload cache was not built for every layer and sequence")

    def load_layer_state(self, layer_idx: int, *, U, SV, landmarks, landmark_idx, host_v, k_buffer, v_buffer,
                         position_ids, ctx: int):
        """Install one layer's encoded prompt state for the whole batch, produced elsewhere (a saved
        encoding, or the CPU restatement of the reference's encoder): U [B, ctx, R], SV [B, H, D, R],
        landmarks [B, H, n, D], landmark_idx [B, H, n], host_v [B, H, ctx/c, c*D], k/v_buffer
        [B, H, <= buf_len, D] laid out [local | outliers | selected], position_ids [B, H, S]."""
        B, H = self.batch_size, self.num_key_value_heads
        if U.shape[0] != B or self.prefilled_batch not in (0, B) or (layer_idx > 0 and self.U is None):
            raise ValueError("load_layer_state installs whole-batch states, layer 0 first")
        self._set_geometry(ctx)
        if landmarks.shape[-2] != self.chunks - self.outlier_chunk:
            raise ValueError("landmark count does not match the prompt geometry")
        if layer_idx == 0:
            self.U = torch.zeros(self.num_layers, B, U.shape[1], self.rank, dtype=self.dtype, device=self.device)
            self.SV = torch.zeros(self.num_layers, B, H, self.head_dim, self.rank, dtype=self.dtype, device=self.device)
            self._alloc_landmarks(landmarks.shape[-2])
        self.U[layer_idx].copy_(U)
        self.SV[layer_idx].copy_(SV)
        self.k_landmark[layer_idx].copy_(landmarks)
        self.k_landmark_idx[layer_idx].copy_(landmark_idx)
        self.v_cache_cpu[layer_idx][:, :, :host_v.shape[2]].copy_(host_v)
        n = k_buffer.shape[2]
        self.k_cache_buffer[layer_idx][:, :, :n].copy_(k_buffer)
        self.v_cache_buffer[layer_idx][:, :, :n].copy_(v_buffer)
        self.position_ids[layer_idx].copy_(position_ids)
        self.init_pool(layer_idx)
        if layer_idx == self.num_layers - 1:
            self.prefilled_batch = B
            self.kv_offset = ctx

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
        if self.pooled:
            # GQA-max scores, the selection in top-k order (kept in position_ids), then the pool's
            # hits, victims and miss list (cnts = hits; misses at [cnts, S) of miss_ids / miss_slot).
            rows, S = B * H, self.select_sets
            sel = self.position_ids[layer_idx].view(rows, S)
            shadowkv.select_chunks(self.gemm_o, self.norm, self.sum, rows, G, n,
                                   self.k_landmark_idx[layer_idx].view(rows, n), S, self.chunks, None, None, None,
                                   out_scores=self.chunk_attn, out_selected=sel, workspace=self.select_workspace)
            shadowkv.pool_assign(sel, self.chunks, self.slot_of[layer_idx], self.slot_chunk[layer_idx],
                                 self.slot_used[layer_idx], self.pool_clock[layer_idx], self.slot_list,
                                 self.miss_ids, self.miss_slot, self.cnts)
            if self.keep_selected:
                self.selected_chunks.copy_(self.position_ids[layer_idx])
            return self.position_ids[layer_idx]
        # softmax + GQA max + top-k + landmark-id gather + reorder in one launch. The GQA-max scores are kept in
        # chunk_attn; the selected ids in top-k order (selected_chunks) only when keep_selected is set. With
        # fold_hit_moves the same launch also moves the value buffer's hits to their new slots.
        move = None
        if self.fold_hit_moves and self.values_in_place:
            # (no value buffer to update: the key buffer's hits, where the key rebuild follows at once)
            if self.one_stream_active():
                move = (self.k_cache_buffer[layer_idx], None, self.kernel_offset, self.kernel_stride,
                        self.chunk_size * D)
        elif self.fold_hit_moves:
            move = (self.v_cache_buffer[layer_idx], self.k_cache_buffer[layer_idx] if self.one_stream_active() else None,
                    self.kernel_offset, self.kernel_stride, self.chunk_size * D)
        shadowkv.select_chunks(self.gemm_o, self.norm, self.sum, B * H, G, n, self.k_landmark_idx[layer_idx].view(B * H, n),
                               self.select_sets, self.chunks, self.position_ids[layer_idx].view(B * H, -1), self.offsets,
                               self.cnts, out_scores=self.chunk_attn,
                               out_selected=self.selected_chunks if self.keep_selected else None,
                               workspace=self.select_workspace, move=move)
        if move is None:
            self._folded[layer_idx] = set()
        elif self.values_in_place:
            self._folded[layer_idx] = {"k"}
        else:
            self._folded[layer_idx] = {"v", "k"} if move[1] is not None else {"v"}
        return self.position_ids[layer_idx]

    def _gen_len(self, layer_idx: int) -> int:
        return self.gen_offset if layer_idx == self.num_layers - 1 else self.gen_offset + self.incoming_q_len

    def _live_view(self, buf: torch.Tensor, layer_idx: int) -> torch.Tensor:
        if self.kv_len_dev is not None:
            return buf[:, :, :self.buf_len]  # length read on the device (kv_len_dev)
        return buf[:, :, :self.sparse_end + self._gen_len(layer_idx) + self.pool_delta]

    def attention_args(self, view_len: int):
        """(kv_len, pool) for the sparse attention over a _live_view of view_len rows: the virtual
        length (rows minus the pool's extra slots) and, with a chunk pool, its slot list geometry."""
        if not self.pooled:
            return view_len, None
        B, H = self.batch_size, self.num_key_value_heads
        return view_len - self.pool_delta, (self.slot_list.view(B, H, -1), self.sparse_start, self.select_sets,
                                            self.chunk_size, self.pool_slots)

    def value_store_args(self, layer_idx: int):
        """The attention's vstore argument (store, position_ids, sparse_start, S, chunk) when the
        selected values are read in place from a device store, else None."""
        if not self.values_in_place:
            return None
        return (self.v_cache_cpu[layer_idx], self.position_ids[layer_idx], self.sparse_start, self.select_sets,
                self.chunk_size)

    def get_value_cache(self, layer_idx: int, position_ids: torch.Tensor, hits_moved: bool = False) -> torch.Tensor:
        """The layer's value buffer with the selected chunks in place: cache hits moved to their
        new slots (unless move_value_hits already did, hits_moved) and misses gathered from host.
        With a chunk pool the hits stay where they are and the misses go to their assigned slots."""
        if self.pooled:
            B, H, D = self.batch_size, self.num_key_value_heads, self.head_dim
            shadowkv.gather_copy_misses_to_slots(self.v_cache_cpu[layer_idx], self.v_cache_buffer[layer_idx],
                                                 self.miss_ids, self.cnts, self.miss_slot, B, H,
                                                 int(self.max_ctx_chunks_len * D), self.sparse_start * D,
                                                 self.buf_len * D, self.select_sets, self.pool_slots,
                                                 self.chunk_size * D)
            return self._live_view(self.v_cache_buffer[layer_idx], layer_idx)
        if self.values_in_place:  # the attention reads the selected values from the store
            return self._live_view(self.v_cache_buffer[layer_idx], layer_idx)
        if "v" in self._folded[layer_idx]:  # the selection moved the hits
            self._folded[layer_idx].discard("v")
            hits_moved = True
        shadowkv.gather_copy_with_offsets(self.v_cache_cpu[layer_idx], self.v_cache_buffer[layer_idx], self.temp,
                                          self.offsets, self.cnts, self.signals, self.batch_size,
                                          self.num_key_value_heads, int(self.max_ctx_chunks_len * self.head_dim),
                                          int(self.sparse_budget * self.head_dim), self.kernel_offset,
                                          self.kernel_stride, self.select_sets, misses_only=hits_moved)
        return self._live_view(self.v_cache_buffer[layer_idx], layer_idx)

    def move_value_hits(self, layer_idx: int):
        """The in-buffer half of the value fetch alone (hit rows to their new slots), so that a
        later get_value_cache(..., hits_moved=True) on the copy stream is host-link work only.
        Nothing to move with a chunk pool, nor when the selection already moved them."""
        if self.pooled or self.values_in_place or "v" in self._folded[layer_idx]:
            return
        shadowkv.gather_copy_d2d_with_offsets(self.v_cache_buffer[layer_idx], self.offsets, self.cnts, self.batch_size,
                                              self.num_key_value_heads, int(self.sparse_budget * self.head_dim),
                                              self.kernel_offset, self.kernel_stride, self.select_sets)

    def get_key_cache(self, layer_idx: int, position_ids: torch.Tensor, rope_func, cos_sin_cache) -> torch.Tensor:
        if self.pooled:  # the misses' keys rebuilt into their slots; hits stay in place
            B, H, S = self.batch_size, self.num_key_value_heads, self.select_sets
            shadowkv.rebuild_k_rope(self.U[layer_idx], self.SV[layer_idx], self.miss_ids.view(B, H, S), self.cnts,
                                    cos_sin_cache, self.k_cache_buffer[layer_idx], self.sparse_start, self.chunk_size,
                                    miss_slot=self.miss_slot.view(B, H, S), pool_slots=self.pool_slots)
            return self._live_view(self.k_cache_buffer[layer_idx], layer_idx)
        if "k" in self._folded[layer_idx]:  # the selection moved the hits
            self._folded[layer_idx].discard("k")
        else:
            shadowkv.gather_copy_d2d_with_offsets(self.k_cache_buffer[layer_idx], self.offsets, self.cnts,
                                                  self.batch_size, self.num_key_value_heads,
                                                  int(self.sparse_budget * self.head_dim), self.kernel_offset,
                                                  self.kernel_stride, self.select_sets)
        batch_gather_gemm_rotary_pos_emb_cuda(self.U[layer_idx], self.SV[layer_idx], cos_sin_cache, position_ids,
                                              self.output, self.chunk_size, self.k_cache_buffer[layer_idx],
                                              self.sparse_start, self.sparse_end, self.cnts)
        return self._live_view(self.k_cache_buffer[layer_idx], layer_idx)

    def one_stream_active(self) -> bool:
        """The decode step's value fetch and key rebuild run as one launch on the current stream
        (one_stream_fetch, with the selection moving both buffers' hits, or with a chunk pool, whose
        hits stay in their slots)."""
        return self.one_stream_fetch and (self.pooled or self.fold_hit_moves)

    def fetch_and_rebuild(self, layer_idx: int, position_ids: torch.Tensor, cos_sin_cache: torch.Tensor):
        """get_value_cache and get_key_cache as one launch on the current stream: the misses'
        value chunks gathered from the host store beside the misses' key rebuild + RoPE, after a
        selection that moved both buffers' hits (one_stream_fetch). Returns (keys, values), the
        live views of the two buffers. With a chunk pool: the miss list of pool_assign, each miss
        fetched and rebuilt into its slot of both buffers."""
        if self.pooled:
            B, H, S, D = self.batch_size, self.num_key_value_heads, self.select_sets, self.head_dim
            shadowkv.fetch_misses_rebuild_k_rope_slots(
                self.v_cache_cpu[layer_idx], self.v_cache_buffer[layer_idx], self.miss_ids.view(B, H, S), self.cnts,
                self.miss_slot.view(B, H, S), int(self.max_ctx_chunks_len * D), self.sparse_start * D,
                self.buf_len * D, self.U[layer_idx], self.SV[layer_idx], cos_sin_cache, self.k_cache_buffer[layer_idx],
                self.sparse_start, self.chunk_size, self.pool_slots, fetch_workgroups=self.fused_fetch_workgroups,
                rebuild_workgroups=self.fused_rebuild_workgroups)
            return (self._live_view(self.k_cache_buffer[layer_idx], layer_idx),
                    self._live_view(self.v_cache_buffer[layer_idx], layer_idx))
        if self._folded[layer_idx] != ({"k"} if self.values_in_place else {"v", "k"}):
            raise RuntimeError("fetch_and_rebuild needs a selection that moved both buffers' hits "
                               "(the key buffer's with the values read in place; one_stream_fetch)")
        self._folded[layer_idx].clear()
        if position_ids.dtype != torch.int64:
            position_ids = position_ids.to(torch.int64)
        if self.values_in_place:  # nothing to fetch: the key rebuild alone
            batch_gather_gemm_rotary_pos_emb_cuda(self.U[layer_idx], self.SV[layer_idx], cos_sin_cache, position_ids,
                                                  self.output, self.chunk_size, self.k_cache_buffer[layer_idx],
                                                  self.sparse_start, self.sparse_end, self.cnts)
            return (self._live_view(self.k_cache_buffer[layer_idx], layer_idx),
                    self._live_view(self.v_cache_buffer[layer_idx], layer_idx))
        shadowkv.fetch_misses_rebuild_k_rope(self.v_cache_cpu[layer_idx], self.v_cache_buffer[layer_idx], self.offsets,
                                             self.cnts, int(self.max_ctx_chunks_len * self.head_dim),
                                             self.kernel_offset, self.kernel_stride, self.U[layer_idx],
                                             self.SV[layer_idx], position_ids, cos_sin_cache,
                                             self.k_cache_buffer[layer_idx], self.sparse_start, self.chunk_size,
                                             fetch_workgroups=self.fused_fetch_workgroups,
                                             rebuild_workgroups=self.fused_rebuild_workgroups)
        return (self._live_view(self.k_cache_buffer[layer_idx], layer_idx),
                self._live_view(self.v_cache_buffer[layer_idx], layer_idx))

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
        self.attn_workspace = shadowkv.sparse_attn_workspace(B, Hq, self.buf_len, self.device)  # zero-filled
        self.attn_out = torch.empty(B, Hq, self.head_dim, dtype=self.dtype, device=self.device)

    def check_capacity(self, incoming: int = 1):
        if self.sparse_end + self.gen_offset + incoming + self.pool_delta > self.buf_len:
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
        # physical append row (after the pool's extra slots); the attention length stays virtual
        self.append_row_dev = torch.full((1,), row + self.pool_delta, dtype=torch.int64, device=self.device)
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

    def qkv_rope_and_append(self, x: torch.Tensor, wqkv_rope: torch.Tensor, position_ids: torch.Tensor,
                            cos_sin: torch.Tensor, layer_idx: int, q_out: torch.Tensor,
                            bias_rope: torch.Tensor | None = None) -> torch.Tensor:
        """rope_and_append() with the QKV projection of the token rows x [B, hidden] (and its bias) in
        the same launch (shadowkv.linear_qkv_rope_append, weight and bias in qkv_rope_weight's row
        order): the fused projection row is never written. Returns q_out viewed [B, Hq, 1, 128]."""
        if self.append_row_dev is None:
            raise RuntimeError("qkv_rope_and_append needs use_device_lengths()")
        self.check_capacity(1)
        if layer_idx == 0:
            self.append_row_dev.add_(1)
            self.kv_len_dev.add_(1)
        shadowkv.linear_qkv_rope_append(x, wqkv_rope, self.num_attention_heads, self.num_key_value_heads,
                                        position_ids, cos_sin, q_out, self.k_cache_buffer[layer_idx],
                                        self.v_cache_buffer[layer_idx], self.append_row_dev, bias_rope)
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
            start = self.sparse_end + self.gen_offset + self.pool_delta
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
        self.slot_of = self.slot_chunk = self.slot_used = self.pool_clock = None

    def get_kv_len(self):
        return self.kv_offset
