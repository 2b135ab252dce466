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
