"""Runs one decode step of one layer through the product classes (ShadowKVCache_CPU +
ShadowAttention) on a GPU, starting from the prompt tensors of a make_golden case."""
from __future__ import annotations

import types

import torch

from shadowkv_amd.models.attention import ShadowAttention
from shadowkv_amd.models.kvcache import ShadowKVCache_CPU


def rope_tokens_cpu(x, cos_sin, pos):
    half = x.shape[-1] // 2
    cs = cos_sin[pos]
    c = torch.cat((cs[:, :half], cs[:, :half]), dim=-1)
    s = torch.cat((cs[:, half:], cs[:, half:]), dim=-1)
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return (x * c) + (rot * s)


def build_cache(case, device, max_decode_len=None, num_layers=1, chunk_cache=None):
    d = case["dims"]
    B, H, G, D, ctx = d["B"], d["H"], d["G"], d["D"], d["ctx"]
    cfg = types.SimpleNamespace(num_attention_heads=H * G, num_key_value_heads=H, hidden_size=H * G * D,
                                num_hidden_layers=num_layers)
    cache = ShadowKVCache_CPU(cfg, batch_size=B, max_length=ctx, device=str(device), sparse_budget=d["budget"],
                              chunk_size=d["chunk"], rank=d["rank"], max_decode_len=max_decode_len,
                              chunk_cache=chunk_cache)
    # Every layer starts from the oracle's encoded state of the prompt (the decode path is compared
    # with the oracle's decode from exactly that state; the device encoder has its own tests).
    si = case["state_in"]
    for layer in range(num_layers):
        cache.load_layer_state(layer, U=si["U"], SV=si["SV"], landmarks=si["landmarks"],
                               landmark_idx=si["landmark_idx"], host_v=si["host_v"], k_buffer=si["kbuf"],
                               v_buffer=si["vbuf"], position_ids=si["position_ids"], ctx=ctx)
    cache.H2D()
    cache.keep_selected = True
    return cache


def identity_rope(B, Hq, H, D):
    """Stands in for the model's RoPE: inputs are already rotated; only the reference's view/transpose."""
    def f(q, k, position_ids):
        return q.view(B, -1, Hq, D).transpose(1, 2), k.view(B, -1, H, D).transpose(1, 2)
    return f


def run_decode_step_gpu(case, device, cache=None):
    d = case["dims"]
    B, H, G, D = d["B"], d["H"], d["G"], d["D"]
    cache = cache or build_cache(case, device)
    cos_sin = case["cos_sin"].to(device)
    attn = ShadowAttention(cache, G, D, H * G * D, identity_rope(B, H * G, H, D), None, cos_sin)
    q = case["q"].to(device).reshape(B, 1, H * G * D)
    k = case["k_new"].to(device).reshape(B, 1, H * D)
    v = case["v_new"].to(device).reshape(B, H, 1, D)
    out = attn.decode(q, k, v, None, 0)
    torch.cuda.synchronize()
    L = cache.sparse_end + cache.gen_offset
    return dict(out=out.view(B, H * G, D).cpu(), cnts=cache.cnts.cpu().numpy(),
                offsets=cache.offsets.view(B * H, -1).cpu().numpy(), position_ids=cache.position_ids[0].cpu().numpy(),
                kbuf=cache.k_cache_buffer[0, :, :, :L].cpu(), vbuf=cache.v_cache_buffer[0, :, :, :L].cpu(),
                scores=cache.chunk_attn.cpu(), selected=cache.selected_chunks.cpu(), cache=cache)


def assert_bf16_close(got: torch.Tensor, want: torch.Tensor, floor: float = 1e-5, what: str = ""):
    """fp32 sums taken in another order then rounded to bf16: at most one bf16 ulp of the larger
    magnitude apart, plus an absolute floor for values produced by cancellation."""
    g, w = got.float(), want.float()
    m = torch.maximum(g.abs(), w.abs()).clamp_min(2.0 ** -126)
    ulp = torch.exp2(torch.floor(torch.log2(m)) - 7)
    bad = (g - w).abs() > ulp + floor
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond one rounding step, max diff {(g - w).abs().max():.3e}"


def check_scoring(cache, q, landmarks):
    """The scoring stage of one decode step against the oracle: the bf16 logits (gemm_o) within one
    rounding step of the oracle's, and the GQA-max probabilities (chunk_attn) within one rounding
    step of the oracle's softmax taken over the device's own logits (a logit one bf16 ulp away
    moves its exp by up to a few percent, so probabilities are compared from identical logits).
    q [B, Hq, D] and landmarks [B, H, n, D] on the CPU."""
    import oracle
    B, H, n, D = landmarks.shape
    G = q.shape[1] // H
    logits_dev = cache.gemm_o.cpu().view(B * H, G, n)
    logits_ref, _ = oracle.score_logits_softmax(q.reshape(B * H, G, D), landmarks.reshape(B * H, n, D),
                                                1.0 / 128 ** 0.5)
    assert_bf16_close(logits_dev, logits_ref, what="logits")
    probs = torch.softmax(logits_dev.float(), dim=-1).to(torch.bfloat16).max(dim=1).values
    assert_bf16_close(cache.chunk_attn.cpu().view(B * H, n), probs, what="gqa-max probabilities")


def fresh_oracle_state(case):
    """An oracle LayerState holding the fixture's post-prefill state (a copy)."""
    import oracle
    d, st = case["dims"], case["st"]
    kw = {k: v.clone() for k, v in case["state_in"].items()}
    return oracle.LayerState(**kw, prefill_local=st.prefill_local, sparse_start=st.sparse_start,
                             sparse_end=st.sparse_end, chunk=d["chunk"], budget=d["budget"], ctx=d["ctx"],
                             buf_len=st.buf_len, chunks=st.chunks)


class LayerProbe:
    """Records, for chosen layers of every lane of a SyntheticDecoder, what one eager decode step
    did to the layer: the cache state just before the layer's selection (after the new token's
    RoPE and append), the selection's outputs, and the buffers and attention output after the
    layer. It wraps the lanes' ShadowAttention.decode_begin_appended / decode_end and
    synchronises the device around the recorded calls (the step's results do not change)."""

    def __init__(self, dec, layers):
        self.records = {}
        self._open = {}
        for i, lane in enumerate(dec.lanes):
            self._wrap(i, lane, set(layers))

    def _wrap(self, i, lane, layers):
        begin, end = lane.attn.decode_begin_appended, lane.attn.decode_end
        c = lane.cache

        def probe_begin(q, idx):
            if idx not in layers:
                return begin(q, idx)
            torch.cuda.synchronize()
            rec = dict(q=q.reshape(q.shape[0], q.shape[1], -1).cpu(), kbuf=c.k_cache_buffer[idx].cpu(),
                       vbuf=c.v_cache_buffer[idx].cpu(), pos_before=c.position_ids[idx].cpu(),
                       kv_len=int(c.kv_len_dev.item()))
            if c.pooled:  # the pool's tables before the step
                rec.update(tables=[t[idx].cpu().numpy().copy() for t in (c.slot_of, c.slot_chunk, c.slot_used,
                                                                         c.pool_clock)])
            pending = begin(q, idx)
            torch.cuda.synchronize()
            rows = c.batch_size * c.num_key_value_heads
            rec.update(gemm_o=c.gemm_o.cpu(), scores=c.chunk_attn.cpu(), offsets=c.offsets.view(rows, -1).cpu(),
                       cnts=c.cnts.cpu(), pos_after=c.position_ids[idx].cpu())
            if c.pooled:
                rec.update(slot_list=c.slot_list.view(rows, -1).cpu().numpy().copy(),
                           tables_after=[t[idx].cpu().numpy().copy() for t in (c.slot_of, c.slot_chunk, c.slot_used,
                                                                               c.pool_clock)])
            self.records[(i, idx)] = rec
            self._open[id(pending)] = (i, idx)
            return pending

        def probe_end(pending):
            key = self._open.pop(id(pending), None)
            out = end(pending)
            if key is not None:
                torch.cuda.synchronize()
                rec = self.records[key]
                L = rec["kv_len"]
                end_row = L + (c.pool_delta if c.pooled else 0)
                rec.update(out=out.reshape(out.shape[0], out.shape[2], -1).cpu(),
                           kbuf_after=c.k_cache_buffer[key[1]][:, :, :end_row].cpu(),
                           vbuf_after=c.v_cache_buffer[key[1]][:, :, :end_row].cpu())
            return out

        lane.attn.decode_begin_appended = probe_begin
        lane.attn.decode_end = probe_end


def _virtual_vbuf(vbuf, store, pos, sp0, S, c):
    """The value buffer as the gathering path would hold it: with the values read in place from a
    device store the selected region of the device buffer is never filled, so it is taken from the
    store through the slot ids (slot j of (b, h) holds chunk pos[b, h, j])."""
    B, H, nch, _ = store.shape
    out = vbuf.clone()
    rows = store.reshape(B, H, nch * c, -1)
    sel = (pos[..., None] * c + torch.arange(c)).reshape(B, H, S * c)
    out[:, :, sp0:sp0 + S * c] = torch.gather(rows, 2, sel[..., None].expand(-1, -1, -1, rows.shape[-1]))
    return out


def check_layer_record(rec, cache, layer, cos_sin_cpu, what=""):
    """One recorded layer step of one lane against the oracle: the scoring within one bf16
    rounding step; from the device's own GQA-max scores, the selection, offsets, hit counts, slot
    ids and the value buffer bit-exact, hit and untouched key rows bit-exact, rebuilt key rows
    and the attention output within rtol 2e-2 / atol 2e-2."""
    import oracle
    B, H = cache.batch_size, cache.num_key_value_heads
    S, c, sp0, sp1 = cache.select_sets, cache.chunk_size, cache.sparse_start, cache.sparse_end
    landmarks = cache.k_landmark[layer].cpu()
    n, D = landmarks.shape[-2], landmarks.shape[-1]
    q = rec["q"]
    G = q.shape[1] // H
    # scoring: logits within one rounding step; probabilities from the device's own logits
    logits_dev = rec["gemm_o"].view(B * H, G, n)
    logits_ref, _ = oracle.score_logits_softmax(q.reshape(B * H, G, D), landmarks.reshape(B * H, n, D),
                                                1.0 / 128 ** 0.5)
    assert_bf16_close(logits_dev, logits_ref, what=f"{what} logits")
    probs = torch.softmax(logits_dev.float(), dim=-1).to(torch.bfloat16).max(dim=1).values
    assert_bf16_close(rec["scores"].view(B * H, n), probs, what=f"{what} gqa-max probabilities")
    host_v = cache.v_cache_cpu[layer].cpu()
    in_place = getattr(cache, "values_in_place", False)
    vbuf0 = _virtual_vbuf(rec["vbuf"], host_v, rec["pos_before"], sp0, S, c) if in_place else rec["vbuf"].clone()
    st = oracle.LayerState(U=cache.U[layer].cpu(), SV=cache.SV[layer].cpu(), landmarks=landmarks,
                           landmark_idx=cache.k_landmark_idx[layer].cpu(), host_v=host_v,
                           kbuf=rec["kbuf"].clone(), vbuf=vbuf0, position_ids=rec["pos_before"].clone(),
                           prefill_local=cache.prefill_local, sparse_start=sp0, sparse_end=sp1, chunk=c,
                           budget=cache.sparse_budget, ctx=cache.prefill, buf_len=cache.buf_len, chunks=cache.chunks)
    L = rec["kv_len"]
    k_new, v_new = rec["kbuf"][:, :, L - 1], rec["vbuf"][:, :, L - 1]
    res = oracle.decode_layer_step(st, q, k_new, v_new, cos_sin_cpu, gen_offset=L - 1 - sp1, scores=rec["scores"])
    assert res["L"] == L
    assert torch.equal(rec["cnts"], torch.from_numpy(res["cnts"])), f"{what}: hit counts"
    assert torch.equal(rec["offsets"], torch.from_numpy(res["offsets"])), f"{what}: offsets"
    assert torch.equal(rec["pos_after"], st.position_ids), f"{what}: slot ids"
    vbuf_after = _virtual_vbuf(rec["vbuf_after"], host_v, rec["pos_after"], sp0, S, c) if in_place \
        else rec["vbuf_after"]
    assert torch.equal(vbuf_after, st.vbuf[:, :, :L]), f"{what}: value buffer"
    kdev, kref = rec["kbuf_after"], st.kbuf[:, :, :L]
    for r in range(B * H):
        b, h = divmod(r, H)
        miss = sp0 + int(res["cnts"][r]) * c
        assert torch.equal(kdev[b, h, :miss], kref[b, h, :miss]), f"{what}: key rows before the misses, row {r}"
        assert torch.equal(kdev[b, h, sp1:], kref[b, h, sp1:]), f"{what}: generated key rows, row {r}"
    torch.testing.assert_close(kdev.float(), kref.float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(rec["out"].float(), res["out"].float(), rtol=2e-2, atol=2e-2)
    return res


def check_pooled_layer_record(rec, cache, layer, cos_sin_cpu, what=""):
    """One recorded layer step of one lane of a cache with a chunk pool against the oracle's pooled
    step, from the device's own GQA-max scores and the pool's recorded tables: the hit counts, slot
    list, misses and tables bit-exact; the value buffer (pool slots, local and generated rows)
    bit-exact; key rows outside the misses' slots bit-exact, rebuilt ones and the attention output
    within rtol 2e-2 / atol 2e-2."""
    import numpy as np

    import oracle
    B, H = cache.batch_size, cache.num_key_value_heads
    S, c, sp0, sp1 = cache.select_sets, cache.chunk_size, cache.sparse_start, cache.sparse_end
    P, delta = cache.pool_slots, cache.pool_delta
    landmarks = cache.k_landmark[layer].cpu()
    n, D = landmarks.shape[-2], landmarks.shape[-1]
    q = rec["q"]
    G = q.shape[1] // H
    logits_dev = rec["gemm_o"].view(B * H, G, n)
    logits_ref, _ = oracle.score_logits_softmax(q.reshape(B * H, G, D), landmarks.reshape(B * H, n, D),
                                                1.0 / 128 ** 0.5)
    assert_bf16_close(logits_dev, logits_ref, what=f"{what} logits")
    host_v = cache.v_cache_cpu[layer].cpu()
    st = oracle.LayerState(U=cache.U[layer].cpu(), SV=cache.SV[layer].cpu(), landmarks=landmarks,
                           landmark_idx=cache.k_landmark_idx[layer].cpu(), host_v=host_v,
                           kbuf=rec["kbuf"].clone(), vbuf=rec["vbuf"].clone(), position_ids=rec["pos_before"].clone(),
                           prefill_local=cache.prefill_local, sparse_start=sp0, sparse_end=sp1, chunk=c,
                           budget=cache.sparse_budget, ctx=cache.prefill, buf_len=cache.buf_len - delta,
                           chunks=cache.chunks)
    slot_of, slot_chunk, slot_used, clock = (t.copy() for t in rec["tables"])
    pool = dict(P=P, delta=delta, kbuf=rec["kbuf"].clone(), vbuf=rec["vbuf"].clone(), slot_of=slot_of,
                slot_chunk=slot_chunk, slot_used=slot_used, clock=clock)
    L = rec["kv_len"]
    k_new, v_new = rec["kbuf"][:, :, L - 1 + delta], rec["vbuf"][:, :, L - 1 + delta]
    res = oracle.decode_layer_step_pooled(st, pool, q, k_new, v_new, cos_sin_cpu, gen_offset=L - 1 - sp1,
                                          scores=rec["scores"])
    assert res["L"] == L
    assert np.array_equal(rec["cnts"].numpy(), res["cnts"]), f"{what}: hit counts"
    assert np.array_equal(rec["slot_list"], res["slot_list"]), f"{what}: slot list"
    for got, want, name in zip(rec["tables_after"], (pool["slot_of"], pool["slot_chunk"], pool["slot_used"],
                                                     pool["clock"]), ("slot_of", "slot_chunk", "slot_used", "clock")):
        assert np.array_equal(got, want), f"{what}: {name}"
    end_row = L + delta
    assert torch.equal(rec["vbuf_after"], pool["vbuf"][:, :, :end_row]), f"{what}: value buffer"
    kdev, kref = rec["kbuf_after"], pool["kbuf"][:, :, :end_row]
    rebuilt = torch.zeros(B, H, end_row, dtype=torch.bool)
    for r in range(B * H):
        b, h = divmod(r, H)
        for i in range(int(res["cnts"][r]), S):
            v = int(res["miss_slot"][r, i])
            rebuilt[b, h, sp0 + v * c:sp0 + (v + 1) * c] = True
    assert torch.equal(kdev[~rebuilt], kref[~rebuilt]), f"{what}: key rows outside the misses' slots"
    torch.testing.assert_close(kdev.float(), kref.float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(rec["out"].float(), res["out"].float(), rtol=2e-2, atol=2e-2)
    return res
