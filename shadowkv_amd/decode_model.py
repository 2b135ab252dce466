"""Random-init decoder that drives the sparse decode path end to end (throughput measurement).

It reproduces the decode loop of the reference's model wrappers (models/base.py:85-176,
models/llama.py:183-218): per layer RMSNorm -> fused QKV projection -> RoPE ->
ShadowAttention.decode -> o_proj + residual -> RMSNorm -> gate/up -> SiLU*up -> down +
residual; final norm, lm_head, greedy argmax. Weights are random (no checkpoint is
available), dense products go to torch (hipBLASLt), RoPE and everything inside the attention
handler run the gfx950 kernels of libshadowkv_amd.so.

`synthesize_state` fills a ShadowKVCache_CPU with the decode-time state a long prefill would
produce — low-rank factors, landmarks, landmark ids, the pinned host value store, the
selected/local/outlier regions — from seeded random tensors of the right shapes, without
running the prefill (a 122K-token SVD per layer and sequence). The sparse value region is
filled from the host store by the chunk-gather kernel and the sparse key region by the
rebuild kernel, so the cache starts consistent.
"""
from __future__ import annotations

import math
import types
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .kernels import shadowkv
from .models.attention import ShadowAttention
from .models.kvcache import ShadowKVCache_CPU
from .models.tensor_op import (apply_rotary_pos_emb_cuda, apply_rotary_pos_emb_glm_single, build_cos_sin_cache,
                               build_glm_cos_sin_cache)
from .streams import capture_graph, side_stream


@dataclass(frozen=True)
class ModelShape:
    name: str
    layers: int
    hidden: int
    ffn: int
    heads: int
    kv_heads: int
    vocab: int
    rope_theta: float
    head_dim: int = 128
    eps: float = 1e-5
    rope: str = "half"  # "half": Llama half-split; "glm": interleaved pairs on the first 64 dims
    qkv_bias: bool = False  # GLM's query_key_value projection has a bias (models/glm.py:165)


LLAMA31_8B = ModelShape("Llama-3.1-8B", 32, 4096, 14336, 32, 8, 128256, 500000.0)
LLAMA3_8B_1M = ModelShape("Llama-3-8B-1M", 32, 4096, 14336, 32, 8, 128256, 3580000.0)
GLM4_9B = ModelShape("GLM-4-9B", 40, 4096, 13696, 32, 2, 151552, 10000.0, rope="glm", qkv_bias=True)



# Fetch workgroups (4-wave) of each lane's one-launch fetch + rebuild with two lanes on their own
# side streams (the two launches overlap on the host link), and the cap on its rebuild workgroups,
# which then loop over the key tiles: the rebuild spreads over the ~300 us fetch instead of
# filling the GPU at its start, where it slowed the other lane's attention and projections.
# Measured on MI355X, Llama-3.1-8B batch 8 ctx 122880, tokens/s: with 56 fetch workgroups, rebuild
# cap 32 / 40 / 48 / 56 / 64: 400.6 / 402.3 / 405.2 / 399.6 / 396.4, against 395.0 with one
# workgroup per tile; with the cap at 48, fetch workgroups 48 / 56 / 64 / 80 / 96: 396.8 / 404.4 /
# 408.1 / 364.5 / 351.4 (two lanes' 80 or more host-read workgroups at once slow the link).
LANE_FETCH_WORKGROUPS = 64
LANE_REBUILD_WORKGROUPS = 48


# Token rows up to which the decoder's projections use the library's skinny linear kernel; above
# it, torch's GEMM (hipBLASLt). Measured on MI355X with cold Llama-3-8B weights, µs per launch,
# skinny vs hipBLASLt: 8 rows qkv 13.1 / 14.4, o_proj 10.8 / 15.8, gate_up 50.6 / 58.9, down
# 26.6 / 26.7; 12 rows 29.0 / 14.3, 21.0 / 15.8, 125.3 / 59.5, 63.3 / 25.8; 16 rows 30.9 / 14.3,
# 21.6 / 15.7, 132.6 / 59.5, 64.8 / 26.6 (the kernel's 9-16-row form streams two weight rows per
# workgroup).
SKINNY_LINEAR_ROWS = 8


def pool_miss_fraction(pool_slots: int | None, landmarks: int) -> float:
    """Expected fraction of a step's selected chunks that a chunk pool of pool_slots slots per
    (b, h) misses once it is full, for selections independent from step to step (the synthetic
    decode): 1 - pool_slots / landmarks (measured, Llama-3.1-8B ctx 122880, 15304 landmarks: hit
    rates 16.7 / 32.6 / 61.8% with 2048 / 4096 / 8192 slots); 1 without a pool."""
    return 1.0 if pool_slots is None else 1.0 - min(1.0, pool_slots / landmarks)


def lane_fetch_workgroups(miss_fraction: float = 1.0) -> int:
    """Fetch workgroups of a decode lane's one-launch fetch + rebuild: LANE_FETCH_WORKGROUPS for
    the full miss traffic, fewer as a chunk pool takes misses away (host reads in flight slow the
    other lane's kernels; the fetch then still ends within that lane's compute). Measured on
    MI355X, Llama-3.1-8B batch 8 ctx 122880, two lanes, tokens/s by fetch workgroups: 2048 slots
    48 / 64: 430.4 / 399.3; 4096 slots 32 / 64: 487.1 / 421.5; 8192 slots 16 / 32: 510.8 /
    506.9. The rule: the square of the miss fraction times LANE_FETCH_WORKGROUPS, to the nearest
    multiple of 8, at least 16."""
    return max(16, 8 * round(LANE_FETCH_WORKGROUPS * miss_fraction * miss_fraction / 8))


def auto_lanes(shape: ModelShape, batch: int, sparse_budget: int, value_store: str = "host",
               miss_fraction: float = 1.0) -> int:
    """Batch lanes for the decode step: 2 when a layer's value fetch over the host link outlasts
    three passes over the layer's dense weights, else 1. Each lane streams the dense weights once
    per layer, so a second lane only pays off where the fetch it hides is long: measured on one
    MI355X (tokens/s, 1 vs 2 lanes): Llama-3.1-8B ctx 122880 batch 2 197 / 160 (fetch / weights
    2.2), batch 4 262 / 271 (4.4), batch 8 271 / 383 (8.9); GLM-4-9B ctx 262144 batch 4 393 / 261
    (1.2). Rates: 52 GB/s host link, 6 TB/s weight stream. With the value store in device memory
    there is no host-link fetch to hide: one lane (Llama-3.1-8B batch 8: 740.6 vs 640.6 tokens/s
    for two lanes). A chunk pool takes the fraction 1 - miss_fraction of the fetch away (12288
    slots, 80% hits: 608.5 tokens/s with one lane vs 526.3 with two)."""
    if batch % 2 or value_store == "device":
        return 1
    d = shape.head_dim
    weights = 2 * shape.hidden * ((shape.heads + 2 * shape.kv_heads) * d + shape.heads * d + 3 * shape.ffn)
    fetch = batch * shape.kv_heads * sparse_budget * d * 2 * miss_fraction
    return 2 if fetch / 52e9 > 3 * weights / 6e12 else 1

def synthesize_state(cache: ShadowKVCache_CPU, ctx: int, seed: int = 0, cos_sin: torch.Tensor | None = None) -> None:
    """Give `cache` the post-prefill state of a ctx-token prompt (random contents, exact shapes)."""
    dev = torch.device(cache.device)
    g = torch.Generator(device=dev).manual_seed(seed)
    L, B, H, D, c, R = cache.num_layers, cache.batch_size, cache.num_key_value_heads, cache.head_dim, \
        cache.chunk_size, cache.rank
    S = cache.select_sets
    cache._set_geometry(ctx)
    n = cache.chunks - cache.outlier_chunk
    G = cache.num_key_value_groups
    tiles = (n + 255) // 256

    cache.U = torch.empty(L, B, ctx, R, dtype=cache.dtype, device=dev)
    cache.SV = torch.empty(L, B, H, D, R, dtype=cache.dtype, device=dev)
    cache.k_landmark = torch.empty(L, B, H, n, D, dtype=cache.dtype, device=dev)
    cache.k_landmark_idx = torch.empty(L, B, H, n, dtype=torch.int64, device=dev)
    cache.gemm_o = torch.zeros(B, H, G, n, dtype=torch.bfloat16, device=dev)
    cache.chunk_attn = torch.zeros(B, H, n, dtype=torch.bfloat16, device=dev)
    cache.norm = torch.zeros(B * H, G, tiles, dtype=torch.float32, device=dev)
    cache.sum = torch.zeros(B * H, G, tiles, dtype=torch.float32, device=dev)
    cache.select_workspace = torch.empty(shadowkv.select_workspace_bytes(B * H, n, cache.select_sets),
                                         dtype=torch.uint8, device=dev)
    if cos_sin is None:
        cos_sin = build_cos_sin_cache(ctx + 4096, 500000.0, D, device=dev)
    zero_cnts = torch.zeros(B * H, dtype=torch.int32, device=dev)
    host_stage = torch.empty(B, H, cache.v_cache_cpu[0].shape[2], c * D, dtype=cache.dtype, device=dev)
    for layer in range(L):
        # U rows ~ N(0, 1/R) and SV ~ N(0, 1): rebuilt keys are O(1), like real post-SVD factors.
        cache.U[layer].copy_(torch.randn(B, ctx, R, generator=g, device=dev) / math.sqrt(R))
        cache.SV[layer].copy_(torch.randn(B, H, D, R, generator=g, device=dev))
        cache.k_landmark[layer].copy_(torch.randn(B, H, n, D, generator=g, device=dev))
        # landmark ids: every aligned chunk except `outlier_chunk` random ones, ascending (shadow.py:513-516)
        order = torch.rand(B * H, cache.chunks, generator=g, device=dev).argsort(dim=-1)
        keep = torch.ones(B * H, cache.chunks, dtype=torch.bool, device=dev)
        keep.scatter_(1, order[:, :cache.outlier_chunk], False)
        rest = torch.arange(cache.chunks, device=dev).expand(B * H, -1).masked_select(keep).view(B, H, n)
        cache.k_landmark_idx[layer].copy_(rest)
        pick = torch.rand(B * H, n, generator=g, device=dev).argsort(dim=-1)[:, :S].view(B, H, S)
        cache.position_ids[layer].copy_(rest.gather(-1, pick))
        # host value store of this layer
        host_stage.normal_(generator=g)
        cache.v_cache_cpu[layer].copy_(host_stage, non_blocking=False)
        # local + outlier regions: random rows; selected region: the selected chunks themselves
        cache.k_cache_buffer[layer].normal_(generator=g)
        cache.v_cache_buffer[layer].normal_(generator=g)
        _fill_selected_values(cache, layer, host_stage)
        shadowkv.rebuild_k_rope(cache.U[layer], cache.SV[layer], cache.position_ids[layer], zero_cnts, cos_sin,
                                cache.k_cache_buffer[layer], cache.sparse_start, c)
        cache.init_pool(layer)
    torch.cuda.synchronize()
    cache.kv_offset = ctx
    cache.prefilled_batch = B
    cache._alloc_attention()


def encode_state(cache: ShadowKVCache_CPU, ctx: int, seed: int = 0, cos_sin: torch.Tensor | None = None,
                 rope: str = "half") -> None:
    """Give `cache` the post-prefill state of a ctx-token prompt built by the device encoder, one
    sequence at a time through every layer (shadow.py:411-544 as the reference's prefill drives it,
    models/base.py:292-340): pre-RoPE keys K = A.B + 0.05 N(0, 1) with A [ctx, R] and B [R, H*D]
    of variance 1/sqrt(R) (a rank-R signal of unit variance plus noise, R = the cache's rank),
    values and the last prompt query ~ N(0, 1), bf16, all seeded; then get_svd, RoPE by token
    position (`rope`: "half" or "glm" with the matching table), and prefill_kv_cache (chunk
    statistics, outliers, landmarks, value offload to the pinned host store, initial selection
    from the last query)."""
    dev = torch.device(cache.device)
    g = torch.Generator(device=dev).manual_seed(seed)
    L, B, H, D, R = cache.num_layers, cache.batch_size, cache.num_key_value_heads, cache.head_dim, cache.rank
    Hq = cache.num_attention_heads
    if cos_sin is None:
        cos_sin = build_cos_sin_cache(ctx + 4096, 500000.0, D, device=dev)
    pos = torch.arange(ctx, device=dev)

    def rotate(x: torch.Tensor, p: torch.Tensor) -> torch.Tensor:  # x [1, h, s, D] by token positions p [s]
        if rope == "glm":
            return apply_rotary_pos_emb_glm_single(x, cos_sin, p)
        return apply_rotary_pos_emb_cuda(x, cos_sin, p.view(1, 1, -1).expand(x.shape[0], x.shape[1], -1))

    for _ in range(B):
        for layer in range(L):
            a = torch.randn(ctx, R, generator=g, device=dev) / R ** 0.25
            b = torch.randn(R, H * D, generator=g, device=dev) / R ** 0.25
            k = torch.addmm(torch.randn(ctx, H * D, generator=g, device=dev), a, b, beta=0.05).to(cache.dtype)
            del a, b
            cache.get_svd(k.view(1, ctx, H * D), layer)
            k_rot = rotate(k.view(1, ctx, H, D).transpose(1, 2).contiguous(), pos)
            del k
            v = torch.randn(1, H, ctx, D, generator=g, device=dev).to(cache.dtype)
            q = torch.randn(1, Hq, 1, D, generator=g, device=dev).to(cache.dtype)
            cache.prefill_kv_cache(v, layer, k_rot, rotate(q, pos[ctx - 1:]))
            del k_rot, v, q
    torch.cuda.synchronize()
    cache._alloc_attention()


def _fill_selected_values(cache: ShadowKVCache_CPU, layer: int, values: torch.Tensor) -> None:
    """Selected value region <- the chunks named by position_ids, through the cached-copy kernel
    with zero hits (every slot is a miss)."""
    B, H, S = cache.batch_size, cache.num_key_value_heads, cache.select_sets
    D, c = cache.head_dim, cache.chunk_size
    cnts = torch.zeros(B * H, dtype=torch.int32, device=cache.device)
    offsets = cache.position_ids[layer].to(torch.int32).reshape(-1).contiguous()
    shadowkv.gather_copy_with_offsets(values, cache.v_cache_buffer[layer], None, offsets, cnts, None, B, H,
                                      values.shape[2] * c * D, cache.sparse_budget * D, cache.kernel_offset,
                                      cache.kernel_stride, S)


class _Lane:
    """One slice of the batch with its own ShadowKV cache (and value-fetch stream) and attention handler."""

    def __init__(self, rows: slice, cache: ShadowKVCache_CPU):
        self.rows, self.cache = rows, cache
        self.attn = None


class SyntheticDecoder:
    """Random-init decoder-only model (Llama layout) decoding with the ShadowKV offload cache.

    With lanes > 1 the batch is split into that many independent slices, each with its own
    cache and value-fetch stream, and the layers are software-pipelined on the one compute
    stream: while lane 0's value chunks for layer i stream in over the host link, the compute
    stream finishes lane 1's layer i-1 and starts lane 1's layer i (and so on round the lanes).
    """

    def __init__(self, shape: ModelShape, batch: int, ctx: int, *, sparse_budget: int = 2048, rank: int = 160,
                 chunk_size: int = 8, decode_len: int = 128, device: str = "cuda:0", seed: int = 0,
                 dtype=torch.bfloat16, lanes: int = 1, fused: bool = True, chunk_cache: int | None = None,
                 one_stream_fetch: bool | None = None, state: str = "synthetic", host_stores: int | None = None,
                 lane_streams: bool | None = None, value_store: str = "host"):
        self.shape, self.batch, self.ctx, self.device, self.dtype = shape, batch, ctx, device, dtype
        # fused: residual add + RMSNorm, SiLU-and-mul and RoPE + KV append as single kernels and
        # the projections on the skinny linear kernel (libshadowkv_amd), instead of torch operations
        self.fused = fused
        s = shape
        D = s.head_dim
        if lanes < 1 or batch % lanes:
            raise ValueError(f"batch {batch} is not divisible into {lanes} lanes")
        g = torch.Generator(device=device).manual_seed(seed)

        def w(*size, scale=0.02):
            return (torch.randn(*size, generator=g, device=device) * scale).to(dtype)

        self.embed = w(s.vocab, s.hidden, scale=1.0)
        self.lm_head = w(s.vocab, s.hidden)
        self.norm_w = torch.ones(s.hidden, dtype=dtype, device=device)
        self.layers = []
        for _ in range(s.layers):
            self.layers.append(types.SimpleNamespace(
                wqkv=w((s.heads + 2 * s.kv_heads) * D, s.hidden), wo=w(s.hidden, s.heads * D),
                bqkv=w((s.heads + 2 * s.kv_heads) * D, scale=0.1) if s.qkv_bias else None,
                gate_up=w(2 * s.ffn, s.hidden), down=w(s.hidden, s.ffn),
                in_norm=torch.ones(s.hidden, dtype=dtype, device=device),
                post_norm=torch.ones(s.hidden, dtype=dtype, device=device)))
        if s.rope == "glm":  # [rows, 64] table: the kernels take GLM's interleaved rotation from its width
            if not fused:
                raise ValueError("the GLM rotary embedding runs in the fused new-token kernel (fused=True)")
            self.cos_sin = build_glm_cos_sin_cache(ctx + decode_len, s.rope_theta, device=device)
        else:
            self.cos_sin = build_cos_sin_cache(ctx + decode_len, s.rope_theta, D, device=device)
        cfg = types.SimpleNamespace(num_attention_heads=s.heads, num_key_value_heads=s.kv_heads,
                                    hidden_size=s.heads * D, num_hidden_layers=s.layers)
        lb = batch // lanes
        # Two lanes: each lane's one-launch fetch + rebuild on its own side stream (default), else
        # the shared fetch and rebuild streams.
        self.lane_streams = (lanes == 2 and one_stream_fetch is not False) if lane_streams is None \
            else bool(lane_streams)
        if self.lane_streams and lanes != 2:
            raise ValueError("lane_streams takes two lanes")
        self.lanes = []
        for i in range(lanes):
            cache = ShadowKVCache_CPU(cfg, batch_size=lb, max_length=ctx, device=device, sparse_budget=sparse_budget,
                                      chunk_size=chunk_size, rank=rank, max_decode_len=decode_len,
                                      zero_host_store=False, chunk_cache=chunk_cache, host_stores=host_stores,
                                      value_store=value_store)
            # The prompt's state: random contents of the exact shapes, or built by the device encoder
            # from low-rank keys (encode_state).
            if state == "encoded":
                encode_state(cache, ctx, seed=seed + 1 + i, cos_sin=self.cos_sin, rope=shape.rope)
            elif state == "synthetic":
                synthesize_state(cache, ctx, seed=seed + 1 + i, cos_sin=self.cos_sin)
            else:
                raise ValueError(f"state must be 'synthetic' or 'encoded', not {state!r}")
            lane = _Lane(slice(i * lb, (i + 1) * lb), cache)
            lane.attn = ShadowAttention(cache, s.heads // s.kv_heads, D, s.hidden, self._rope_for(lane), None,
                                        self.cos_sin)
            cache.use_device_lengths()
            # The selection launch also moves the value buffer's hits (both buffers' with one lane),
            # so the value fetch follows it directly; this decoder fetches only through the cache.
            cache.fold_hit_moves = True
            # One lane: the step runs on the compute stream alone, the value fetch and key rebuild
            # as one launch after a selection that moved both buffers' hits (with a chunk pool:
            # after the pool's assignment, the hits staying in their slots) (no cross-stream wait
            # before or after the fetch; MI355X tokens/s vs the two-stream step: GLM-4-9B batch 4
            # 429.8 vs 418.4, Llama-3-8B-1M 38.42 vs 37.81).
            cache.one_stream_fetch = (lanes == 1) if one_stream_fetch is None else bool(one_stream_fetch)
            if self.lane_streams:
                # Each lane's value fetch and key rebuild as one launch on a side stream of its own
                # (lane 0 on the fetch stream, lane 1 on the rebuild stream), after a selection that
                # moved both buffers' hits. A lane's fetch can then start while the other lane's is
                # still running: with one shared fetch stream each fetch followed the previous one
                # only ~10 us after it ended (the cross-stream dependency on its selection, resolved
                # long before, still costs that in a graph replay), idling the host link for 5% of
                # the step (Llama-3.1-8B batch 8 ctx 122880 on MI355X: 402 vs 386 tokens/s with 56
                # fetch workgroups and one rebuild workgroup per tile; the workgroup counts above).
                cache.one_stream_fetch = True
                cache.lane_stream = side_stream(device, ("fetch", "rebuild")[i])
                if value_store == "host":  # (a store in HBM takes the library's wide fetch)
                    cache.fused_fetch_workgroups = lane_fetch_workgroups(
                        pool_miss_fraction(chunk_cache, cache.k_landmark.shape[-2]))
                    cache.fused_rebuild_workgroups = LANE_REBUILD_WORKGROUPS
            elif lanes > 1:
                # All lanes share one value-fetch stream and one key-rebuild stream (their fetches
                # follow one another on the host link anyway); taking the key rebuild off the
                # compute stream keeps it out of the stretch between two lanes' fetches.
                # Three streams in all (compute, fetch, rebuild): within the 4 hardware queues of a
                # process, so no two of them share a queue.
                cache.key_stream = side_stream(device, "rebuild")
            self.lanes.append(lane)
        self.cache = self.lanes[0].cache  # lane 0's cache (shapes are identical across lanes)
        # The down projection forming SiLU-and-mul from the gate/up rows (one launch instead of two).
        # Alone it is slower, every workgroup recomputing the activations (4 rows: 32.5 vs 23.4 µs
        # for the two kernels; 8 rows: 126 vs 27.7 µs), but where two lanes keep the host link busy
        # the step gains from the launch it saves (Llama-3.1-8B batch 8: 384.9 vs 381.7 tokens/s);
        # the one-lane compute chain loses (GLM-4-9B batch 4: 385.4 vs 396.5 tokens/s).
        self.gated_down = lanes > 1 and lb <= 4
        # The gate/up projection with the SiLU-and-mul in its epilogue (interleaved gate/up weight
        # rows; bit-identical to the two kernels, one launch and no [gate | up] round trip). Taken
        # on one-lane chains, where the saved launch is on the critical path (GLM-4-9B batch 4:
        # 418.5 vs 413.5 tokens/s; Llama-3-8B-1M 37.8 vs 37.7); two lanes keep the gated down
        # projection above (Llama-3.1-8B batch 8: 383.5 vs 380.3 tokens/s, with a 2048-slot chunk
        # pool 423.9 vs 415.7: the epilogue's extra barrier in each of the 3584 gate/up workgroups).
        self.act_epilogue = fused and lanes == 1
        # The QKV projection with the new token's RoPE and KV append in its epilogue (q/k weight rows
        # of half-split heads interleaved; bit-identical to the projection followed by the RoPE +
        # append kernel, one launch fewer per layer): lanes of at most 8 rows.
        self.qkv_rope_epilogue = fused and lb <= shadowkv.QKV_ROPE_MAX_ROWS
        if fused:
            for lw in self.layers:
                lw.gate_up_il = shadowkv.interleave_gate_up(lw.gate_up)
                lw.wqkv_rope = shadowkv.qkv_rope_weight(lw.wqkv, s.heads, s.kv_heads, s.rope == "glm")
                lw.bqkv_rope = None if lw.bqkv is None else \
                    shadowkv.qkv_rope_weight(lw.bqkv, s.heads, s.kv_heads, s.rope == "glm")
        # RoPE position of the token being decoded, per sequence; advanced on the device by each step.
        self.pos = torch.full((batch,), ctx, dtype=torch.int64, device=device)
        self.graph = None
        self.graph_steps = 1
        self.static_tokens = None

    def _rope_for(self, lane: _Lane):
        s, D = self.shape, self.shape.head_dim

        def rope(q: torch.Tensor, k: torch.Tensor, position_ids: torch.Tensor):
            """RoPE of the new token's q [b, 1, Hq*D] and k [b, 1, Hkv*D] (views into the fused QKV
            output) at position_ids [b], in place like the reference's rotary_embedding
            (models/llama.py:149-154); each rotation pair is read and written by one thread."""
            b = q.shape[0]
            views = []
            for x, h in ((q, s.heads), (k, s.kv_heads)):
                xv = x.view(b, h, 1, D)
                shadowkv.apply_rotary_pos_emb_new(xv, self.cos_sin, position_ids, xv, b, h, 1, D, xv.stride(0),
                                                  xv.stride(1), xv.stride(2), xv.stride(3), self.cos_sin.stride(0),
                                                  position_ids.stride(0), 0, 0, D // 2)
                views.append(x.view(b, 1, h, D).transpose(1, 2))
            return views[0], views[1]
        return rope

    def _norm(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        return F.rms_norm(x, (x.shape[-1],), w, self.shape.eps)

    def _linear(self, x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None = None) -> torch.Tensor:
        """x @ w.T (+ b); fused: the library's skinny linear (weights streamed once) up to
        SKINNY_LINEAR_ROWS token rows."""
        rows = x.numel() // x.shape[-1]
        if not self.fused or rows > SKINNY_LINEAR_ROWS:
            return F.linear(x, w, b)
        out = torch.empty(*x.shape[:-1], w.shape[0], dtype=self.dtype, device=self.device)
        shadowkv.linear(x, w, out, bias=b)
        return out

    def _layer_begin(self, idx: int, state, lane: _Lane):
        """Norm, fused QKV and the first half of the attention handler (value fetch in flight).
        state: the residual stream h, or (h, x) with x = this layer's normalised input (fused)."""
        s, D = self.shape, self.shape.head_dim
        lw = self.layers[idx]
        if self.fused:
            h, x = state
            b = h.shape[0]
            q_out = torch.empty(b, s.heads, D, dtype=self.dtype, device=self.device)
            if self.qkv_rope_epilogue and b <= shadowkv.QKV_ROPE_MAX_ROWS:
                q = lane.cache.qkv_rope_and_append(x.view(b, -1), lw.wqkv_rope, self.pos[lane.rows], self.cos_sin,
                                                   idx, q_out, bias_rope=lw.bqkv_rope)
            else:
                qkv = self._linear(x, lw.wqkv, lw.bqkv)
                q = lane.cache.rope_and_append(qkv.view(b, -1), self.pos[lane.rows], self.cos_sin, idx, q_out)
            return lane.attn.decode_begin_appended(q, idx)
        h = state
        b = h.shape[0]
        x = self._norm(h, lw.in_norm)
        qkv = F.linear(x, lw.wqkv, lw.bqkv)
        q, k, v = qkv.split([s.heads * D, s.kv_heads * D, s.kv_heads * D], dim=-1)
        v = v.view(b, 1, s.kv_heads, D).transpose(1, 2)
        return lane.attn.decode_begin(q, k, v, self.pos[lane.rows], idx)

    def _layer_end(self, idx: int, state, lane: _Lane, pending):
        """Attention over the assembled buffers, o_proj + residual, norm, SwiGLU MLP + residual
        (fused: the residual add travels with the following norm, the next layer's input norm or,
        after the last layer, the final norm)."""
        s = self.shape
        lw = self.layers[idx]
        a = lane.attn.decode_end(pending)
        if self.fused:
            h, _ = state
            b = h.shape[0]
            o = self._linear(a.reshape(b, 1, s.heads * s.head_dim), lw.wo)
            h2, x2 = torch.empty_like(h), torch.empty_like(h)
            shadowkv.rmsnorm(o, lw.post_norm, s.eps, x2, residual=h, residual_out=h2)
            if self.act_epilogue and b <= SKINNY_LINEAR_ROWS:  # SiLU-and-mul in the gate/up epilogue
                act = torch.empty(b, 1, s.ffn, dtype=self.dtype, device=self.device)
                shadowkv.linear_gate_up_silu(x2, lw.gate_up_il, act)
                down = self._linear(act, lw.down)
            else:
                gate_up = self._linear(x2, lw.gate_up)
                if self.gated_down and b <= shadowkv.LINEAR_SILU_MUL_MAX_ROWS:  # SiLU-and-mul formed by the down projection
                    down = torch.empty(b, 1, s.hidden, dtype=self.dtype, device=self.device)
                    shadowkv.linear_silu_mul(gate_up, lw.down, down)
                else:
                    act = torch.empty(b, 1, s.ffn, dtype=self.dtype, device=self.device)
                    shadowkv.silu_and_mul(gate_up, act)
                    down = self._linear(act, lw.down)
            w_next = self.layers[idx + 1].in_norm if idx + 1 < s.layers else self.norm_w
            h3, x3 = torch.empty_like(h), torch.empty_like(h)
            shadowkv.rmsnorm(down, w_next, s.eps, x3, residual=h2, residual_out=h3)
            return h3, x3
        h = state
        b = h.shape[0]
        h = h + F.linear(a.reshape(b, 1, s.heads * s.head_dim), lw.wo)
        x = self._norm(h, lw.post_norm)
        gate, up = F.linear(x, lw.gate_up).chunk(2, dim=-1)
        return h + F.linear(F.silu(gate) * up, lw.down)

    @staticmethod
    def _greedy(logits: torch.Tensor) -> torch.Tensor:
        """argmax over the vocabulary as two short reductions (blocks of 256, then the block maxima),
        so no reduction spans several workgroups; first maximal index wins, as in torch.argmax."""
        B, V = logits.shape
        blk = 256
        pad = -V % blk
        if pad:
            logits = F.pad(logits, (0, pad), value=float("-inf"))
        vals, idx = logits.view(B, -1, blk).max(dim=-1)  # [B, V/256]
        best = vals.argmax(dim=-1, keepdim=True)  # [B, 1]
        return best * blk + idx.gather(1, best)

    def _head(self, state, lane: _Lane) -> torch.Tensor:
        """Final norm, lm_head, greedy token; advances the lane's RoPE positions."""
        x = state[1] if self.fused else self._norm(state, self.norm_w)  # fused: normalised already
        logits = self._linear(x[:, -1], self.lm_head).float()  # [b, vocab]
        self.pos[lane.rows].add_(1)
        return self._greedy(logits)  # [b, 1]

    def _embed(self, tokens: torch.Tensor):
        """Token embedding; fused: (residual, normalised input of layer 0)."""
        h = F.embedding(tokens, self.embed)
        if not self.fused:
            return h
        x = torch.empty_like(h)
        shadowkv.rmsnorm(h, self.layers[0].in_norm, self.shape.eps, x)
        return h, x

    @torch.inference_mode()
    def decode_step(self, tokens: torch.Tensor) -> torch.Tensor:
        """One greedy decode step for the whole batch: tokens [B, 1] -> next tokens [B, 1]."""
        return self.decode_steps(tokens, 1)

    @torch.inference_mode()
    def decode_steps(self, tokens: torch.Tensor, steps: int) -> torch.Tensor:
        """`steps` greedy decode steps for the whole batch: tokens [B, 1] -> the last step's tokens.

        Every step-dependent integer (RoPE position, cache append row, attention length) lives
        on the device and is advanced by the step itself, so steps can be captured. The lanes are
        one software pipeline over (step, layer) units: issue order for two lanes is begin0(0)
        begin1(0) end0(0) begin0(1) end1(0) begin1(1) ..., so each lane's value fetch overlaps the
        other lanes' work between its begin and its end. A lane's step boundary is a unit like any
        other (end of its last layer, lm head, embedding of the new token, begin of layer 0), so
        across steps the first lane's next fetch is issued while the second lane finishes its
        last layer and lm head, instead of after both."""
        if steps < 1:
            raise ValueError(f"steps must be >= 1, got {steps}")
        lanes = self.lanes
        L = self.shape.layers
        cur = [tokens[lane.rows] for lane in lanes]
        hs = [None] * len(lanes)
        pending = [None] * len(lanes)
        for u in range(steps * L + 1):
            idx = u % L
            for i, lane in enumerate(lanes):
                if pending[i] is not None:
                    hs[i] = self._layer_end((u - 1) % L, hs[i], lane, pending[i])
                    pending[i] = None
                    if idx == 0:  # the lane's step is complete
                        cur[i] = self._head(hs[i], lane)
                if u < steps * L:
                    if idx == 0:
                        hs[i] = self._embed(cur[i])
                    pending[i] = self._layer_begin(idx, hs[i], lane)
        return torch.cat(cur) if len(cur) > 1 else cur[0]

    def _caches(self):
        return [lane.cache for lane in self.lanes]

    def capture(self, tokens: torch.Tensor, steps: int = 1) -> None:
        """Capture `steps` decode steps (one continuous lane pipeline), reading and then
        overwriting a static token buffer, in a HIP graph, captured on the process's "capture" side
        stream. The graph's only other streams are the lanes' value-fetch and key-rebuild streams,
        each forked from the capture stream and joined back to it. Nothing runs during capture; host counters touched by the traced Python are
        restored."""
        self.static_tokens = tokens.clone()
        saved = [(c.gen_offset, c.kv_offset) for c in self._caches()]
        for c in self._caches():
            c.check_capacity(steps)
        g = torch.cuda.CUDAGraph()
        # On the process's capture side stream, so the capture adds no stream beyond the fixed set;
        # no garbage collection (and so no destructor of a dead decoder) runs inside it.
        with capture_graph(g, self.device):
            self.static_tokens.copy_(self.decode_steps(self.static_tokens, steps))
        for c, (gen, kv) in zip(self._caches(), saved):
            c.gen_offset, c.kv_offset = gen, kv
        self.graph = g
        self.graph_steps = steps

    def replay(self) -> torch.Tensor:
        """The captured decode steps; returns the static token buffer (the last step's tokens [B, 1])."""
        if self.graph is None:
            raise RuntimeError("capture() a decode step first")
        for c in self._caches():
            c.check_capacity(self.graph_steps)
        self.graph.replay()
        for c in self._caches():
            c.advance(self.graph_steps)
        return self.static_tokens
