"""The device prefill encoder (chunk statistics, outlier selection, landmark gather, low-rank factors,
and a whole ShadowKVCache_CPU.prefill_kv_cache) against fp32/fp64 torch references and the oracle's
encode_layer (models/kvcache/shadow.py:411-544)."""
import types

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle.shadowkv_oracle import _rope_tokens
from shadowkv_amd.kernels import shadowkv
from shadowkv_amd.models.kvcache import ShadowKVCache_CPU
from shadowkv_amd.models.kvcache.shadow import low_rank_factors
from tests.decode_harness import assert_bf16_close
from tests.golden import make_golden

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _stats_ref(k, chunks, c):
    """bf16(fp32 chunk mean) and the minimum row-to-mean cosine in float64."""
    B, H, _, D = k.shape
    x = k[:, :, :chunks * c].float().reshape(B, H, chunks, c, D)
    cand = (x.sum(-2) / c).to(torch.bfloat16)
    xd, cd = x.double(), cand.double().unsqueeze(-2)
    cos = (xd * cd).sum(-1) / (xd.norm(dim=-1).clamp_min(1e-8) * cd.norm(dim=-1).clamp_min(1e-8))
    return cand, cos.min(-1).values


@pytest.mark.parametrize("B,H,ctx,c", [(2, 8, 2048, 8), (1, 2, 1000, 4), (1, 4, 4096, 16), (2, 2, 96, 3),
                                     (1, 2, 2048, 32), (1, 1, 640, 20)])
def test_chunk_stats(gpu, B, H, ctx, c):
    _say(f"chunk_stats B={B} H={H} ctx={ctx} c={c}")
    g = torch.Generator().manual_seed(ctx + c)
    k = (torch.randn(B, H, ctx, 128, generator=g) + 0.5 * torch.randn(B, H, 1, 128, generator=g)).to(torch.bfloat16)
    k[0, 0, :c] = 0  # a zero chunk: norms clamp, cosine 0
    chunks = ctx // c - 2
    cand = torch.empty(B, H, chunks, 128, dtype=torch.bfloat16, device=gpu)
    mc = torch.empty(B, H, chunks, dtype=torch.float32, device=gpu)
    shadowkv.chunk_stats(k.to(gpu), chunks, c, cand, mc)
    torch.cuda.synchronize()
    want_cand, want_mc = _stats_ref(k, chunks, c)
    assert_bf16_close(cand.cpu(), want_cand, floor=0.0, what="chunk means")
    assert (mc.cpu().double() - want_mc).abs().max() < 2e-6
    assert mc[0, 0, 0].item() == 0.0


@pytest.mark.parametrize("rows,chunks,k,ties", [(16, 248, 24, False), (16, 248, 24, True), (8, 15352, 48, True),
                                                (2, 130728, 48, False), (4, 2000, 512, True), (3, 600, 1, True)])
def test_select_outliers(gpu, rows, chunks, k, ties):
    _say(f"select_outliers rows={rows} chunks={chunks} k={k} ties={ties}")
    g = torch.Generator().manual_seed(chunks + k)
    x = torch.rand(rows, chunks, generator=g) * 2 - 1
    if ties:
        x = (x * 8).round() / 8  # 17 distinct values: the k-th value is shared by many chunks
    x[0, 5] = -0.0
    order = torch.sort(x, dim=-1, stable=True).indices  # ascending value, ties by ascending id
    want_out, want_rest = order[:, :k], torch.sort(order[:, k:], dim=-1).values
    out = torch.empty(rows, k, dtype=torch.int64, device=gpu)
    rest = torch.empty(rows, chunks - k, dtype=torch.int64, device=gpu)
    shadowkv.select_outliers(x.to(gpu), k, out, rest)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), want_out)
    assert torch.equal(rest.cpu(), want_rest)


def test_gather_rows(gpu):
    g = torch.Generator().manual_seed(9)
    src = torch.randn(3, 50, 128, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, 50, (3, 20), generator=g)
    dst = torch.empty(3, 20, 128, dtype=torch.bfloat16, device=gpu)
    shadowkv.gather_rows(src.to(gpu), idx.to(gpu), dst)
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), src.gather(1, idx.unsqueeze(-1).expand(-1, -1, 128)))


def test_low_rank_factors(gpu):
    """u @ svt against the float64 SVD's rank-R reconstruction; the singular values too."""
    _say("low_rank_factors")
    g = torch.Generator().manual_seed(4)
    B, rows, cols, R = 2, 6000, 512, 48
    a = torch.randn(B, rows, 64, generator=g) @ torch.randn(B, 64, cols, generator=g) / 8
    k = (a + 0.2 * torch.randn(B, rows, cols, generator=g)).to(torch.bfloat16)
    u, svt = low_rank_factors(k.to(gpu), R)
    torch.cuda.synchronize()
    uu, s, vh = torch.linalg.svd(k.double(), full_matrices=False)
    want = (uu[..., :R] * s[..., None, :R]) @ vh[..., :R, :]
    got = u.cpu().double() @ svt.cpu().double()
    assert ((got - want).norm() / want.norm()).item() < 1e-3
    assert ((svt.cpu().double().norm(dim=-1) - s[..., :R]).abs() / s[..., :R]).max().item() < 1e-3


def test_get_svd_head_split(gpu):
    """ShadowKVCache_CPU.get_svd's per-head SV (shadow.py:437-442): U @ SV[h]^T gives back head h's
    pre-RoPE keys down to the closed-form noise floor of the rank-R truncation, on both fixtures;
    the transposed split of the same factors does not."""
    from tests import svd_pins

    for case in (make_golden.decode_small_case(), make_golden.single_layer_case()):
        k_pre, d = case["k_pre"], case["dims"]
        _say(f"get_svd head split H={d['H']} ctx={d['ctx']} rank={d['rank']}")
        B, H, ctx, D = k_pre.shape
        cfg = types.SimpleNamespace(num_attention_heads=H * d["G"], num_key_value_heads=H, hidden_size=H * d["G"] * D,
                                    num_hidden_layers=1)
        cache = ShadowKVCache_CPU(cfg, batch_size=B, max_length=ctx, device=str(gpu), sparse_budget=d["budget"],
                                  chunk_size=d["chunk"], rank=d["rank"])
        cache.get_svd(k_pre.to(gpu), 0)
        torch.cuda.synchronize()
        U, SV = cache.U[0].cpu(), cache.SV[0].cpu()
        err = svd_pins.head_errors(k_pre, U, SV)
        lim = svd_pins.bound(k_pre, d["rank"])
        assert (err <= lim).all(), (err, lim)
        assert (svd_pins.head_errors(k_pre, U, svd_pins.transposed_split(SV)) > 2 * lim).all()


def _prefill_on_gpu(gpu, k_pre, v, q_pre_last, cos_sin, chunk, budget, rank):
    B, H, ctx, D = k_pre.shape
    Hq = q_pre_last.shape[1]
    cfg = types.SimpleNamespace(num_attention_heads=Hq, num_key_value_heads=H, hidden_size=Hq * D,
                                num_hidden_layers=1)
    cache = ShadowKVCache_CPU(cfg, batch_size=B, max_length=ctx, device=str(gpu), sparse_budget=budget,
                              chunk_size=chunk, rank=rank)
    k = _rope_tokens(k_pre, cos_sin, torch.arange(ctx))
    q = _rope_tokens(q_pre_last, cos_sin, torch.tensor([ctx - 1]))
    cache.get_svd(k_pre.to(gpu), 0)
    cache.prefill_kv_cache(v.to(gpu), 0, k.to(gpu), q.to(gpu))
    torch.cuda.synchronize()
    return cache, k


def _check_prefill(gpu, k_pre, v, q_pre_last, cos_sin, chunk, budget, rank):
    B, H, ctx, D = k_pre.shape
    cache, k = _prefill_on_gpu(gpu, k_pre, v, q_pre_last, cos_sin, chunk, budget, rank)
    n = cache.k_landmark.shape[-2]
    chunks, n_out = cache.chunks, cache.outlier_chunk
    lidx = cache.k_landmark_idx[0].cpu()
    outlier_set = [sorted(set(range(chunks)) - set(lidx[b, h].tolist())) for b in range(B) for h in range(H)]
    # The outlier sets: the k smallest of the fp32 statistic exactly (up to 1e-6 near-ties), and of the
    # reference's bf16 cosine up to a few bf16 steps.
    kc = k[:, :, :chunks * chunk].reshape(B, H, chunks, chunk, D)
    cand = kc.mean(dim=-2)
    bf = F.cosine_similarity(cand.unsqueeze(3).expand(-1, -1, -1, chunk, -1), kc, dim=-1).min(-1).values.float()
    _, f64 = _stats_ref(k, chunks, chunk)
    for r, outs in enumerate(outlier_set):
        b, h = divmod(r, H)
        assert len(outs) == n_out
        inside = torch.zeros(chunks, dtype=torch.bool)
        inside[outs] = True
        for vals, tol in ((f64[b, h].float(), 1e-6), (bf[b, h], 2e-2)):
            kth = torch.sort(vals).values[n_out - 1]
            assert bool((vals[inside] <= kth + tol).all()) and bool((vals[~inside] >= kth - tol).all()), (r, tol)
    # Everything downstream from the device's own decisions: the oracle with the same outliers (in
    # the device's slot order) and the same initial GQA-max scores.
    mc = torch.empty(B, H, chunks, dtype=torch.float32, device=gpu)
    cands = torch.empty(B, H, chunks, D, dtype=torch.bfloat16, device=gpu)
    shadowkv.chunk_stats(k.to(gpu), chunks, chunk, cands, mc)
    out_idx = torch.empty(B * H, n_out, dtype=torch.int64, device=gpu)
    rest = torch.empty(B * H, chunks - n_out, dtype=torch.int64, device=gpu)
    shadowkv.select_outliers(mc.view(B * H, chunks), n_out, out_idx, rest)
    torch.cuda.synchronize()
    st = oracle.encode_layer(k_pre, v, q_pre_last, cos_sin, rank=rank, chunk=chunk, budget=budget,
                             buf_len=cache.buf_len, outliers=out_idx.cpu().view(B, H, n_out),
                             init_scores=cache.chunk_attn.cpu())
    assert (cache.prefill_local, cache.sparse_start, cache.sparse_end) == (st.prefill_local, st.sparse_start,
                                                                            st.sparse_end)
    assert torch.equal(lidx, st.landmark_idx)
    assert_bf16_close(cache.k_landmark[0].cpu(), st.landmarks, floor=0.0, what="landmarks")
    assert torch.equal(cache.position_ids[0].cpu(), st.position_ids)
    end = st.sparse_end
    assert torch.equal(cache.v_cache_buffer[0, :, :, :end].cpu().view(torch.int16), st.vbuf[:, :, :end].view(torch.int16))
    assert torch.equal(cache.k_cache_buffer[0, :, :, :end].cpu().view(torch.int16), st.kbuf[:, :, :end].view(torch.int16))
    assert torch.equal(cache.v_cache_cpu[0][:, :, :ctx // chunk].view(torch.int16), st.host_v.view(torch.int16))
    # Initial scores: the oracle's softmax/GQA max over the same landmarks.
    q = _rope_tokens(q_pre_last, cos_sin, torch.tensor([ctx - 1]))
    want = oracle.score_gqa_max(q.reshape(B * H, -1, D), st.landmarks.reshape(B * H, n, D), 1.0 / 128 ** 0.5)
    torch.testing.assert_close(cache.chunk_attn.cpu().view(B * H, n).float(), want.float(), rtol=3e-2, atol=1e-5)
    # Low-rank factors: the rebuilt pre-RoPE keys U.SV^T per head against the oracle's (full SVD).
    got = torch.einsum("bcr,bhdr->bhcd", cache.U[0].cpu().float(), cache.SV[0].cpu().float())
    ref = torch.einsum("bcr,bhdr->bhcd", st.U.float(), st.SV.float())
    assert ((got - ref).norm() / ref.norm()).item() < 1e-2
    return cache


@pytest.mark.parametrize("chunk", [8, 4, 16])
def test_prefill_small_case(gpu, chunk):
    _say(f"prefill, small decode case, chunk {chunk}")
    case = make_golden.decode_small_case(chunk)
    d = case["dims"]
    _check_prefill(gpu, case["k_pre"], case["v"], case["q_last"], case["cos_sin"], chunk, d["budget"], d["rank"])


def test_prefill_batch2_llama_heads(gpu):
    """Batch 2, 8 kv heads x 4 query heads, rank 160, ctx 8192, budget 1024."""
    _say("prefill batch 2, 8 heads, ctx 8192")
    g = torch.Generator().manual_seed(2024)
    B, H, G, D, ctx, R = 2, 8, 4, 128, 8192, 160
    a = torch.randn(B, ctx, 128, generator=g) @ torch.randn(B, 128, H * D, generator=g) / 12
    k_pre = (a + 0.1 * torch.randn(B, ctx, H * D, generator=g)).view(B, ctx, H, D).transpose(1, 2)
    k_pre = k_pre.to(torch.bfloat16).contiguous()
    v = torch.randn(B, H, ctx, D, generator=g).to(torch.bfloat16)
    q_last = torch.randn(B, H * G, 1, D, generator=g).to(torch.bfloat16)
    cos_sin = oracle.build_cos_sin_cache(ctx + 64, 500000.0)
    _check_prefill(gpu, k_pre, v, q_last, cos_sin, 8, 1024, R)


def test_prefill_random_configurations(gpu):
    """The device prefill on 5 seeded random configurations (batch 1-2, 1-8 kv heads of 1-16 query
    heads, ranks 16-160, chunks of 4/8/16 rows, budgets 1024/2048, contexts 2-4x the budget)
    against the oracle's encode_layer, checked as in the fixed cases."""
    rng = np.random.default_rng(84)
    for i in range(5):
        B, H, G = int(rng.integers(1, 3)), int(rng.choice([1, 2, 4, 8])), int(rng.choice([1, 4, 16]))
        chunk, budget, R = int(rng.choice([4, 8, 16])), int(rng.choice([1024, 2048])), int(rng.choice([16, 32, 64, 160]))
        ctx = 64 * int(rng.integers(budget * 2 // 64, budget * 4 // 64 + 1))
        _say(f"prefill random configuration {i}: B={B} H={H} G={G} chunk={chunk} budget={budget} rank={R} ctx={ctx}")
        g = torch.Generator().manual_seed(800 + i)
        D = 128
        a = torch.randn(B, ctx, R, generator=g) @ torch.randn(B, R, H * D, generator=g) / R ** 0.5
        k_pre = (a + 0.1 * torch.randn(B, ctx, H * D, generator=g)).view(B, ctx, H, D).transpose(1, 2)
        k_pre = k_pre.to(torch.bfloat16).contiguous()
        v = torch.randn(B, H, ctx, D, generator=g).to(torch.bfloat16)
        q_last = torch.randn(B, H * G, 1, D, generator=g).to(torch.bfloat16)
        cos_sin = oracle.build_cos_sin_cache(ctx + 64, 500000.0)
        _check_prefill(gpu, k_pre, v, q_last, cos_sin, chunk, budget, R)


def test_prefill_rejects_host_tensors(gpu):
    cfg = types.SimpleNamespace(num_attention_heads=8, num_key_value_heads=2, hidden_size=1024, num_hidden_layers=1)
    cache = ShadowKVCache_CPU(cfg, batch_size=1, max_length=2048, device=str(gpu), sparse_budget=1024, chunk_size=8,
                              rank=32)
    with pytest.raises(ValueError):
        cache.get_svd(torch.zeros(1, 2, 2048, 128, dtype=torch.bfloat16), 0)


def test_attention_prefill_builds_the_same_state(gpu):
    """ShadowAttention.prefill (get_svd, RoPE, prefill_kv_cache, causal fp32 attention) leaves the
    same cache state as the direct calls, and returns causal attention of the rotated prompt."""
    from shadowkv_amd.models.attention import ShadowAttention
    _say("ShadowAttention.prefill")
    case = make_golden.decode_small_case(8)
    d = case["dims"]
    B, H, G, D, ctx = d["B"], d["H"], d["G"], d["D"], d["ctx"]
    cs = case["cos_sin"].to(gpu)
    g = torch.Generator().manual_seed(31)
    q_pre = torch.randn(B, H * G, ctx, D, generator=g).to(torch.bfloat16)
    q_pre[:, :, -1:] = case["q_last"]

    def rope(q, k, pos):
        return _rope_tokens(q, cs, pos), _rope_tokens(k, cs, pos)

    cfg = types.SimpleNamespace(num_attention_heads=H * G, num_key_value_heads=H, hidden_size=H * G * D,
                                num_hidden_layers=1)
    cache = ShadowKVCache_CPU(cfg, batch_size=B, max_length=ctx, device=str(gpu), sparse_budget=d["budget"],
                              chunk_size=8, rank=d["rank"])
    attn = ShadowAttention(cache, G, D, H * G * D, rope, None, cs)
    out = attn.prefill(q_pre.to(gpu), case["k_pre"].to(gpu), case["v"].to(gpu), torch.arange(ctx, device=gpu), 0)
    torch.cuda.synchronize()
    direct, _ = _prefill_on_gpu(gpu, case["k_pre"], case["v"], case["q_last"], case["cos_sin"], 8, d["budget"],
                                d["rank"])
    for name in ("U", "SV", "k_landmark", "k_landmark_idx", "position_ids", "k_cache_buffer", "v_cache_buffer"):
        a, b = getattr(cache, name), getattr(direct, name)
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b), name
    # causal attention of the last 16 prompt queries against the fp32 CPU restatement
    q = _rope_tokens(q_pre, case["cos_sin"], torch.arange(ctx))
    k = _rope_tokens(case["k_pre"], case["cos_sin"], torch.arange(ctx))
    rows = torch.arange(ctx - 16, ctx)
    qq = q[:, :, rows].float()
    kk = k.float().repeat_interleave(G, dim=1)
    vv = case["v"].float().repeat_interleave(G, dim=1)
    sc = qq @ kk.transpose(-1, -2) / D ** 0.5
    sc = sc.masked_fill(torch.arange(ctx)[None, :] > rows[:, None], float("-inf"))
    want = (torch.softmax(sc, dim=-1) @ vv).transpose(1, 2)
    torch.testing.assert_close(out[:, -16:].cpu().float(), want, rtol=2e-2, atol=2e-2)
