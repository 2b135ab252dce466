"""ShadowKV attention handler (reference: models/attention/shadow.py:6-50).

decode() keeps the reference's order of operations and its two-stream overlap:
RoPE -> append the new token -> select chunks (score, top-k, reorder) -> [copy stream: value
fetch from host] || [current stream: key compaction + low-rank rebuild + RoPE] -> join ->
sparse attention. The attention is the gfx950 split-L decode kernel in place of
flash_attn_with_kvcache; prefill attention (not on the decode path) is plain fp32 torch.
"""
import math

import torch

from ...kernels import shadowkv
from ..tensor_op import repeat_kv
from .base import AttentionBase


def causal_attention_fp32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block: int = 1024) -> torch.Tensor:
    """Causal GQA attention in fp32, query-blocked; q [B, Hq, L, D], k/v [B, Hkv, L, D] -> [B, L, Hq, D]."""
    B, Hq, L, D = q.shape
    k = repeat_kv(k, Hq // k.shape[1]).float()
    v = repeat_kv(v, Hq // v.shape[1]).float()
    kt = k.transpose(-1, -2).contiguous()
    out = torch.empty(B, L, Hq, D, dtype=q.dtype, device=q.device)
    for s in range(0, L, block):
        e = min(L, s + block)
        scores = torch.matmul(q[:, :, s:e].float(), kt[..., :e]) / math.sqrt(D)
        mask = torch.arange(e, device=q.device)[None, :] > torch.arange(s, e, device=q.device)[:, None]
        scores.masked_fill_(mask, float("-inf"))
        p = torch.softmax(scores, dim=-1)
        out[:, s:e] = torch.matmul(p, v[:, :, :e]).transpose(1, 2).to(q.dtype)
    return out


class ShadowAttention(AttentionBase):

    def prefill(self, query_states, key_states, value_states, position_ids, layer_idx):
        kv_cache = self.kv_cache
        kv_cache.get_svd(key_states, layer_idx=layer_idx)
        query_states, key_states = self.apply_rotary_pos_emb(query_states, key_states, position_ids)
        kv_cache.prefill_kv_cache(value_states, layer_idx, key_states, query_states[:, :, -1:])
        return causal_attention_fp32(query_states, key_states, value_states)

    def decode(self, query_states, key_states, value_states, position_ids, layer_idx):
        return self.decode_end(self.decode_begin(query_states, key_states, value_states, position_ids, layer_idx))

    def decode_begin(self, query_states, key_states, value_states, position_ids, layer_idx):
        """First half of decode(): RoPE, append, chunk selection, the value fetch launched on the
        cache's copy stream and the key rebuild on the current stream (or on the cache's
        key_stream, when it has one). Returns what decode_end() needs; work issued on the current
        stream in between overlaps the value fetch."""
        kv_cache = self.kv_cache
        query_states, key_states = self.apply_rotary_pos_emb(query_states, key_states, position_ids)
        kv_cache.update_kv_cache(key_states, value_states, layer_idx)
        return self.decode_begin_appended(query_states, layer_idx)

    def decode_begin_appended(self, query_states, layer_idx):
        """decode_begin() for a token already rotated and appended (ShadowKVCache_CPU.rope_and_append):
        query_states [B, Hq, 1, 128] post-RoPE."""
        kv_cache = self.kv_cache
        position_ids = kv_cache.get_retrieval_position_ids(layer_idx=layer_idx, query_states=query_states)

        curr_stream = torch.cuda.current_stream()
        if kv_cache.one_stream_active():
            # the value fetch and the key rebuild as one launch (hits moved by the selection), on this
            # stream or on the cache's lane_stream, joined in decode_end
            lane_stream = getattr(kv_cache, "lane_stream", None)
            if lane_stream is None:
                key_states, value_states = kv_cache.fetch_and_rebuild(layer_idx, position_ids, self.cos_sin_cache)
                return query_states, key_states, value_states, [], layer_idx
            with torch.cuda.stream(lane_stream):
                lane_stream.wait_stream(curr_stream)
                key_states, value_states = kv_cache.fetch_and_rebuild(layer_idx, position_ids, self.cos_sin_cache)
                done = [lane_stream.record_event()]
            return query_states, key_states, value_states, done, layer_idx
        copy_stream = kv_cache.copy_stream
        # The value hits move within the GPU buffer here, so the copy stream (whose transfers
        # follow one another on the host link) carries the host-link gather alone.
        kv_cache.move_value_hits(layer_idx)
        with torch.cuda.stream(copy_stream):
            copy_stream.wait_stream(curr_stream)
            value_states = kv_cache.get_value_cache(layer_idx, position_ids, hits_moved=True)
            done = [copy_stream.record_event()]  # this fetch only, even if the stream is shared
        key_stream = getattr(kv_cache, "key_stream", None)
        if key_stream is None:
            key_states = self._key_path(layer_idx, position_ids)
        else:  # the key rebuild on its own stream too, joined in decode_end
            with torch.cuda.stream(key_stream):
                key_stream.wait_stream(curr_stream)
                key_states = self._key_path(layer_idx, position_ids)
                done.append(key_stream.record_event())
        return query_states, key_states, value_states, done, layer_idx

    def _key_path(self, layer_idx, position_ids):
        return self.kv_cache.get_key_cache(layer_idx=layer_idx, position_ids=position_ids,
                                           rope_func=self.apply_rotary_pos_emb_single,
                                           cos_sin_cache=self.cos_sin_cache)

    def decode_end(self, pending):
        """Second half of decode(), on the stream decode_begin() ran on: wait for the value fetch,
        then sparse attention of the new token over the assembled buffers -> [B, 1, Hq, D] (with
        a value store in device memory read in place, the selected values from the store).
        `pending` is decode_begin()'s result."""
        query_states, key_states, value_states, done, layer_idx = pending
        kv_cache = self.kv_cache
        for event in done:
            torch.cuda.current_stream().wait_event(event)
        if kv_cache.attn_workspace is None:
            kv_cache._alloc_attention()
        B, Hq = query_states.shape[0], query_states.shape[1]
        q = query_states.reshape(B, Hq, -1) if query_states.shape[2] == 1 else None
        if q is None:
            raise ValueError("decode attention takes one query token per step")
        out = torch.empty(B, Hq, query_states.shape[-1], dtype=query_states.dtype, device=query_states.device)
        kv_len, pool = kv_cache.attention_args(key_states.shape[2])
        shadowkv.sparse_attn_decode(q, key_states, value_states, kv_len, out, kv_cache.attn_workspace,
                                    kv_len_dev=kv_cache.kv_len_dev, pool=pool,
                                    vstore=kv_cache.value_store_args(layer_idx))
        return out.view(B, 1, Hq, -1)
