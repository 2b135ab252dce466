"""GPU parity of the floating-point kernels against the CPU oracle.

RoPE alone is bit-exact (same bf16 rounding sequence). The rebuild, scoring and attention
accumulate in fp32 in a different order than the CPU, so they are checked to the bf16
tolerance of the contract (rtol 2e-2, atol 2e-2) plus tighter, scale-aware bounds where
atol would be vacuous (softmax probabilities are ~1/n).
"""
import math

import numpy as np
import pytest
import torch

import oracle
from shadowkv_amd.kernels import shadowkv
from shadowkv_amd.models import tensor_op

pytestmark = pytest.mark.gpu

RTOL = 2e-2
ATOL = 2e-2


def _say(msg):
    print(msg, flush=True)


def _assert_rounding_close(got: torch.Tensor, want: torch.Tensor, floor: float = 1e-5):
    """fp32 sums taken in another order then rounded to bf16: at most one bf16 ulp of the larger
    magnitude apart, plus an absolute floor for values produced by cancellation."""
    g, w = got.float(), want.float()
    m = torch.maximum(g.abs(), w.abs()).clamp_min(2.0 ** -126)
    ulp = torch.exp2(torch.floor(torch.log2(m)) - 7)
    bad = (g - w).abs() > ulp + floor
    assert not bad.any(), f"{int(bad.sum())} elements beyond one rounding step, max diff {(g - w).abs().max():.3e}"


@pytest.mark.parametrize("glm", [False, True])
def test_rope_push_bit_exact(gpu, glm):
    B, H, S, c, D = 2, 8, 32, 8, 128
    _say(f"rope push glm={glm}")
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, H, S * c, D, generator=g).to(torch.bfloat16)
    cs = oracle.build_glm_cos_sin_cache(4096, 5e6) if glm else oracle.build_cos_sin_cache(4096, 5e5)
    ids = torch.stack([torch.stack([torch.randperm(500, generator=g)[:S].sort().values for _ in range(H)])
                       for _ in range(B)]).to(torch.int32)
    cnts = torch.randint(0, S + 1, (B * H,), generator=g, dtype=torch.int32)
    start, buf = 100, 100 + S * c + 20
    cache = torch.randn(B, H, buf, D, generator=g).to(torch.bfloat16)
    want = (oracle.rope_push_glm if glm else oracle.rope_push)(x, cs, ids, cnts, c, cache.clone(), start,
                                                               start + S * c - 5)
    cg = cache.to(gpu)
    tensor_op.apply_rotary_pos_emb_cuda_push_cache(x.to(gpu), cs.to(gpu), ids.to(gpu), c, cg, start,
                                                   start + S * c - 5, cnts.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(cg.cpu(), want)


def test_rope_plain_bit_exact(gpu):
    B, H, L, D = 2, 4, 50, 128
    cs = oracle.build_cos_sin_cache(1000, 5e5)
    x = torch.randn(B, H, L, D).to(torch.bfloat16)
    pos = torch.randint(0, 1000, (B, H, L))
    out = tensor_op.apply_rotary_pos_emb_cuda(x.to(gpu), cs.to(gpu), pos.to(gpu))
    torch.cuda.synchronize()
    c = cs[pos]
    want = oracle.rope_half_split(x, c[..., :64], c[..., 64:])
    assert torch.equal(out.cpu(), want)


def _rebuild_case(B, H, ctx, R, S, c, seed, per_head_u=False, shared_sv=False):
    g = torch.Generator().manual_seed(seed)
    U = torch.randn(B, H, ctx, R, generator=g) if per_head_u else torch.randn(B, ctx, R, generator=g)
    U = (U / math.sqrt(R)).to(torch.bfloat16)
    SV = torch.randn(H, 128, R, generator=g) if shared_sv else torch.randn(B, H, 128, R, generator=g)
    SV = SV.to(torch.bfloat16)
    ids = torch.stack([torch.stack([torch.randperm(ctx // c, generator=g)[:S].sort().values for _ in range(H)])
                       for _ in range(B)])
    cnts = torch.randint(0, S + 1, (B * H,), generator=g, dtype=torch.int32)
    return U, SV, ids, cnts


def test_batch_gather_gemm_plain(gpu):
    B, H, ctx, R, S, c = 2, 8, 4096, 160, 256, 8
    _say("batch_gather_gemm plain")
    U, SV, ids, cnts = _rebuild_case(B, H, ctx, R, S, c, 1)
    want = oracle.rebuild_k(U, SV, ids, c)
    out = torch.zeros(B * H, S * c, 128, dtype=torch.bfloat16, device=gpu)
    shadowkv.batch_gather_gemm(U.to(gpu), SV.to(gpu), None, None, ids.to(torch.int32).to(gpu), out, B, H, ctx, 128, R,
                               S * c, ctx, c, cnts.to(gpu))
    torch.cuda.synchronize()
    got = out.cpu().view(B, H, S * c, 128)
    for bh in range(B * H):
        b, h = divmod(bh, H)
        miss = int(cnts[bh]) * c
        assert (got[b, h, :miss] == 0).all()  # hit rows untouched
        torch.testing.assert_close(got[b, h, miss:].float(), want[b, h, miss:].float(), rtol=RTOL, atol=ATOL)
        _assert_rounding_close(got[b, h, miss:], want[b, h, miss:])


@pytest.mark.parametrize("glm,per_head_u,shared_sv,R,S,c", [
    (False, False, False, 160, 256, 8), (True, False, False, 160, 256, 8), (False, True, True, 160, 256, 8),
    (False, False, False, 96, 256, 8), (False, False, False, 168, 256, 8), (False, False, False, 8, 256, 8),
    (True, True, True, 40, 256, 8), (False, False, False, 192, 256, 8), (True, False, False, 192, 256, 8),
    (False, False, False, 160, 100, 4), (True, False, True, 104, 100, 4)])
def test_rebuild_k_rope_fused(gpu, glm, per_head_u, shared_sv, R, S, c):
    B, H, ctx = 2, 8, 4096
    _say(f"rebuild_k_rope glm={glm} per_head_u={per_head_u} shared_sv={shared_sv} R={R} S={S} c={c}")
    U, SV, ids, cnts = _rebuild_case(B, H, ctx, R, S, c, 2, per_head_u, shared_sv)
    cs = oracle.build_glm_cos_sin_cache(ctx, 5e6) if glm else oracle.build_cos_sin_cache(ctx, 5e5)
    start, buf = 448, 448 + S * c + 96
    cache = torch.randn(B, H, buf, 128).to(torch.bfloat16)
    SVf = SV.unsqueeze(0).expand(B, -1, -1, -1) if shared_sv else SV
    want = oracle.rebuild_k_rope(U, SVf, ids, cnts, cs, c, cache.clone(), start, glm=glm)
    cg = cache.to(gpu)
    shadowkv.rebuild_k_rope(U.to(gpu), SV.to(gpu), ids.to(gpu), cnts.to(gpu), cs.to(gpu), cg, start, c)
    torch.cuda.synchronize()
    got = cg.cpu()
    assert torch.equal(got[:, :, :start], cache[:, :, :start])
    assert torch.equal(got[:, :, start + S * c:], cache[:, :, start + S * c:])
    for bh in range(B * H):
        b, h = divmod(bh, H)
        miss = start + int(cnts[bh]) * c
        assert torch.equal(got[b, h, start:miss], cache[b, h, start:miss])  # hit rows untouched
        torch.testing.assert_close(got[b, h, miss:start + S * c].float(), want[b, h, miss:start + S * c].float(),
                                   rtol=RTOL, atol=ATOL)


def test_rebuild_k_rope_long_selection(gpu):
    """The 1M-context selection size: 2048 chunks per head (16384 rows) at positions up to 2^18,
    RoPE theta 3.58e6, part of every head already in place (random hit counts)."""
    B, H, ctx, R, S, c = 1, 8, 262144, 160, 2048, 8
    _say("rebuild_k_rope long selection S=2048 ctx=262144")
    U, SV, ids, cnts = _rebuild_case(B, H, ctx, R, S, c, 5)
    cs = oracle.build_cos_sin_cache(ctx, 3.58e6)
    start = 3136
    cache = torch.randn(B, H, start + S * c + 64, 128).to(torch.bfloat16)
    want = oracle.rebuild_k_rope(U, SV, ids, cnts, cs, c, cache.clone(), start)
    cg = cache.to(gpu)
    shadowkv.rebuild_k_rope(U.to(gpu), SV.to(gpu), ids.to(gpu), cnts.to(gpu), cs.to(gpu), cg, start, c)
    torch.cuda.synchronize()
    got = cg.cpu()
    assert torch.equal(got[:, :, :start], cache[:, :, :start])
    assert torch.equal(got[:, :, start + S * c:], cache[:, :, start + S * c:])
    for h in range(H):
        miss = start + int(cnts[h]) * c
        assert torch.equal(got[0, h, start:miss], cache[0, h, start:miss])  # hit rows untouched
        torch.testing.assert_close(got[0, h, miss:start + S * c].float(), want[0, h, miss:start + S * c].float(),
                                   rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("glm", [False, True])
def test_rebuild_k_rope_extreme_hit_counts(gpu, glm):
    """Rows with every chunk a hit (nothing rebuilt), no hit, one hit and one miss."""
    B, H, ctx, R, S, c = 1, 4, 4096, 160, 256, 8
    _say(f"rebuild extreme hit counts glm={glm}")
    U, SV, ids, _ = _rebuild_case(B, H, ctx, R, S, c, 7)
    cnts = torch.tensor([S, 0, 1, S - 1], dtype=torch.int32)
    cs = oracle.build_glm_cos_sin_cache(ctx, 5e6) if glm else oracle.build_cos_sin_cache(ctx, 5e5)
    start = 64
    cache = torch.randn(B, H, start + S * c + 16, 128).to(torch.bfloat16)
    want = oracle.rebuild_k_rope(U, SV, ids, cnts, cs, c, cache.clone(), start, glm=glm)
    cg = cache.to(gpu)
    shadowkv.rebuild_k_rope(U.to(gpu), SV.to(gpu), ids.to(gpu), cnts.to(gpu), cs.to(gpu), cg, start, c)
    torch.cuda.synchronize()
    got = cg.cpu()
    assert torch.equal(got[0, 0], cache[0, 0])  # all hits: the row is untouched
    for h in range(1, H):
        miss = start + int(cnts[h]) * c
        assert torch.equal(got[0, h, :miss], cache[0, h, :miss])
        assert torch.equal(got[0, h, start + S * c:], cache[0, h, start + S * c:])
        torch.testing.assert_close(got[0, h, miss:start + S * c].float(), want[0, h, miss:start + S * c].float(),
                                   rtol=RTOL, atol=ATOL)


def test_rebuild_basis_rows_exact(gpu):
    # U rows that are basis vectors make every K row an SV column: exact through MFMA and RoPE.
    B, H, ctx, R, S, c = 1, 8, 1024, 160, 64, 8
    SV = torch.randn(B, H, 128, R).to(torch.bfloat16)
    U = torch.zeros(B, ctx, R, dtype=torch.bfloat16)
    U[0, torch.arange(ctx), torch.arange(ctx) % R] = 1.0
    g = torch.Generator().manual_seed(9)
    ids = torch.stack([torch.randperm(ctx // c, generator=g)[:S].sort().values for _ in range(H)]).unsqueeze(0)
    cnts = torch.zeros(H, dtype=torch.int32)
    cs = oracle.build_cos_sin_cache(ctx, 5e5)
    cache = torch.zeros(B, H, S * c, 128, dtype=torch.bfloat16)
    want = oracle.rebuild_k_rope(U, SV, ids, cnts, cs, c, cache.clone(), 0)
    cg = cache.to(gpu)
    shadowkv.rebuild_k_rope(U.to(gpu), SV.to(gpu), ids.to(gpu), cnts.to(gpu), cs.to(gpu), cg, 0, c)
    torch.cuda.synchronize()
    assert torch.equal(cg.cpu(), want)


@pytest.mark.parametrize("Z,m,n", [(8, 4, 968), (64, 4, 15304), (8, 16, 32712), (4, 1, 300), (2, 8, 257)])
def test_scoring(gpu, Z, m, n):
    _scoring_case(gpu, Z, m, n, n)


def test_scoring_random_shapes(gpu):
    """Scoring + softmax + GQA max on 10 seeded random shapes (1-40 rows, 1-16 queries, 1-40000
    landmarks, including counts below one 256-column tile)."""
    rng = np.random.default_rng(80)
    for case in range(10):
        Z, m = int(rng.integers(1, 41)), int(rng.integers(1, 17))
        n = int(rng.integers(1, 300)) if case < 3 else int(rng.integers(300, 40001))
        _scoring_case(gpu, Z, m, n, 3000 + case)


def _scoring_case(gpu, Z, m, n, seed):
    _say(f"scoring Z={Z} m={m} n={n}")
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Z, m, 128, generator=g).to(torch.bfloat16)
    L = torch.randn(Z, n, 128, generator=g).to(torch.bfloat16)
    alpha = 1.0 / math.sqrt(128)
    Dw, Pw = oracle.score_logits_softmax(q, L, alpha)
    tiles = (n + 255) // 256
    Dg = torch.empty(Z, m, n, dtype=torch.bfloat16, device=gpu)
    Pg = torch.empty_like(Dg)
    norm = torch.empty(Z, m, tiles, device=gpu)
    ssum = torch.empty_like(norm)
    qg, Lg = q.to(gpu), L.to(gpu)
    shadowkv.batch_gemm_softmax(qg, Lg, Dg, norm, ssum, Pg, Z, m, n, 128, alpha, 0.0)
    out = torch.empty(Z, n, dtype=torch.bfloat16, device=gpu)
    shadowkv.score_gqa_max(qg, Lg, Dg, norm, ssum, out, Z, m, n, 128, alpha)
    torch.cuda.synchronize()
    _assert_rounding_close(Dg.cpu(), Dw)
    Pc = Pg.cpu().float()
    rel = ((Pc - Pw.float()).abs() / Pw.float().clamp_min(1e-30)).max().item()
    assert rel <= 2e-2, rel
    torch.testing.assert_close(Pc, Pw.float(), rtol=RTOL, atol=ATOL)
    assert torch.equal(out.cpu(), Pg.cpu().max(dim=1).values)  # GQA max of the kernel's own probabilities


@pytest.mark.parametrize("Z,m,n", [(32, 4, 15304), (5, 3, 1000), (3, 2, 777), (9, 1, 4100), (2, 4, 100)])
def test_scoring_kernels_agree(gpu, Z, m, n, monkeypatch):
    """The two scoring kernels for m <= 4 queries, the row-contiguous one (vector-ALU dots) and the
    MFMA one, each forced: logits within one rounding step of the oracle's and of each other,
    the tile partials within rounding of each other (sums taken in another order)."""
    _say(f"scoring kernels Z={Z} m={m} n={n}")
    g = torch.Generator().manual_seed(Z * n + m)
    q = torch.randn(Z, m, 128, generator=g).to(torch.bfloat16)
    L = torch.randn(Z, n, 128, generator=g).to(torch.bfloat16)
    alpha = 1.0 / math.sqrt(128)
    Dw, _ = oracle.score_logits_softmax(q, L, alpha)
    qg, Lg = q.to(gpu), L.to(gpu)
    tiles = (n + 255) // 256
    runs = {}
    for path in ("mfma", "rows"):
        monkeypatch.setenv("SKV_SCORE_PATH", path)
        D = torch.full((Z, m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
        norm = torch.full((Z, m, tiles), float("nan"), device=gpu)
        ssum = torch.full_like(norm, float("nan"))
        shadowkv.score_logits(qg, Lg, D, norm, ssum, Z, m, n, 128, alpha)
        torch.cuda.synchronize()
        _assert_rounding_close(D.cpu(), Dw)
        runs[path] = (D.cpu(), norm.cpu(), ssum.cpu())
    (D, norm, ssum), ref = runs["mfma"], runs["rows"]
    _assert_rounding_close(D, ref[0])
    _assert_rounding_close(norm, ref[1])  # tile maxima of logits at most one step apart
    # sum exp(x - max) * exp(max): the tile's sum of exp(x), whichever maximum it was taken against
    torch.testing.assert_close(ssum * norm.exp(), ref[2] * ref[1].exp(), rtol=1e-2, atol=0)


@pytest.mark.parametrize("Z,m,n", [(8, 16, 32712), (32, 4, 15304), (2, 4, 140000), (3, 8, 2048), (1, 1, 8),
                                   (256, 4, 4096), (128, 16, 4096)])
def test_softmax_vector_and_scalar_paths_agree(gpu, Z, m, n):
    """The softmax + GQA-max kernel's vector path (rows of n % 8 == 0 columns, aligned buffers;
    8, 4 or 2 columns per thread, by the workgroup count: 8 for 256 x 4096, 4 for 128 x 4096, 2
    for the few-row shapes) and its one-column-per-thread path (taken here by handing it outputs 2 bytes off alignment)
    give bit-identical probabilities and maxima, also past 512 partial tiles per row (140000
    columns), where the partials merge no longer holds a row's partials in registers; the
    probabilities agree with the oracle's softmax of the same logits within one rounding step."""
    _say(f"softmax paths Z={Z} m={m} n={n}")
    g = torch.Generator().manual_seed(n + m)
    q = torch.randn(Z, m, 128, generator=g).to(torch.bfloat16).to(gpu)
    L = torch.randn(Z, n, 128, generator=g).to(torch.bfloat16).to(gpu)
    tiles = (n + 255) // 256
    D = torch.empty(Z, m, n, dtype=torch.bfloat16, device=gpu)
    norm = torch.empty(Z, m, tiles, device=gpu)
    ssum = torch.empty_like(norm)
    shadowkv.score_logits(q, L, D, norm, ssum, Z, m, n, 128, 1.0 / math.sqrt(128))
    outs = {}
    for name, off in (("vector", 0), ("scalar", 1)):
        sm_buf = torch.empty(Z * m * n + 8, dtype=torch.bfloat16, device=gpu)
        mx_buf = torch.empty(Z * n + 8, dtype=torch.bfloat16, device=gpu)
        sm, mx = sm_buf[off:off + Z * m * n], mx_buf[off:off + Z * n]
        shadowkv.softmax_gqa_max(D, norm, ssum, mx, Z, m, n, softmax=sm)
        torch.cuda.synchronize()
        outs[name] = (sm.view(Z, m, n).cpu(), mx.view(Z, n).cpu())
    assert torch.equal(outs["vector"][0], outs["scalar"][0])
    assert torch.equal(outs["vector"][1], outs["scalar"][1])
    assert torch.equal(outs["vector"][1], outs["vector"][0].max(dim=1).values)
    logits = D.cpu().float()
    _assert_rounding_close(outs["vector"][0], torch.softmax(logits, dim=-1).to(torch.bfloat16), floor=1e-9)


@pytest.mark.parametrize("B,Hq,Hk,L,strided", [(1, 32, 8, 2497, True), (8, 32, 8, 2600, True), (2, 32, 2, 2497, True),
                                               (1, 8, 8, 1, False), (3, 16, 4, 300, False), (1, 32, 8, 19521, True),
                                               (1, 32, 8, 8193, False), (2, 24, 2, 700, True), (1, 16, 1, 129, False),
                                               (1, 32, 2, 1, False), (2, 32, 2, 128, True), (1, 32, 4, 4097, False)])
def test_sparse_attention(gpu, B, Hq, Hk, L, strided):
    _say(f"attention B={B} Hq={Hq} Hk={Hk} L={L}")
    g = torch.Generator().manual_seed(L)
    buf = L + 37 if strided else L
    K = torch.randn(B, Hk, buf, 128, generator=g).to(torch.bfloat16)
    V = torch.randn(B, Hk, buf, 128, generator=g).to(torch.bfloat16)
    q = torch.randn(B, Hq, 128, generator=g).to(torch.bfloat16)
    want = oracle.sparse_attention(q, K, V, L)
    ws = shadowkv.sparse_attn_workspace(B, Hq, L, gpu)
    out = torch.empty(B, Hq, 128, dtype=torch.bfloat16, device=gpu)
    shadowkv.sparse_attn_decode(q.to(gpu), K.to(gpu), V.to(gpu), L, out, ws)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().float(), want.float(), rtol=RTOL, atol=ATOL)
    if L == 1:
        for hq in range(Hq):
            assert torch.equal(out.cpu()[:, hq], V[:, hq // (Hq // Hk), 0])


@pytest.mark.parametrize("B,Hq,Hk,sp0,S,chunk,gen", [(2, 32, 8, 448, 256, 8, 7), (4, 32, 2, 448, 256, 8, 1),
                                                     (1, 8, 8, 40, 13, 4, 0), (3, 12, 4, 64, 20, 16, 5)])
def test_attention_values_in_place_from_store(gpu, B, Hq, Hk, sp0, S, chunk, gen):
    """skv_sparse_attn_decode_vstore (the selected values read in place from a value store in
    device memory, slot j holding chunk position_ids[b, h, j]) equals skv_sparse_attn_decode over a
    value buffer holding those rows, bit for bit (also with a device-resident length), and the
    oracle on the gathered values."""
    _say(f"attention values in place B={B} Hq={Hq} Hk={Hk} S={S} chunk={chunk}")
    g = torch.Generator().manual_seed(S + chunk + B)
    L = sp0 + S * chunk + gen
    buf = L + 9
    nchunks = 3 * S + 5
    K = torch.randn(B, Hk, buf, 128, generator=g).to(torch.bfloat16)
    V = torch.randn(B, Hk, buf, 128, generator=g).to(torch.bfloat16)
    q = torch.randn(B, Hq, 128, generator=g).to(torch.bfloat16)
    store = torch.randn(B, Hk, nchunks, chunk * 128, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(nchunks, generator=g)[:S] for _ in range(B * Hk)]).view(B, Hk, S)
    Vg = V.clone()  # the gathered form: the selected rows copied into the value buffer
    rows = store.view(B, Hk, nchunks * chunk, 128)
    sel = (ids[..., None] * chunk + torch.arange(chunk)).reshape(B, Hk, S * chunk)
    Vg[:, :, sp0:sp0 + S * chunk] = torch.gather(rows, 2, sel[..., None].expand(-1, -1, -1, 128))
    want = oracle.sparse_attention(q, K, Vg, L)
    Kd, Vd, Vgd, qd, sd, idd = K.to(gpu), V.to(gpu), Vg.to(gpu), q.to(gpu), store.to(gpu), ids.to(gpu)
    ws = shadowkv.sparse_attn_workspace(B, Hq, buf, gpu)
    ldev = torch.full((1,), L, dtype=torch.int32, device=gpu)
    outs = []
    for kw in (dict(), dict(kv_len_dev=ldev)):
        ref = torch.empty(B, Hq, 128, dtype=torch.bfloat16, device=gpu)
        got = torch.empty_like(ref)
        n = buf if kw else L
        shadowkv.sparse_attn_decode(qd, Kd, Vgd, n, ref, ws, **kw)
        shadowkv.sparse_attn_decode(qd, Kd, Vd, n, got, ws, vstore=(sd, idd, sp0, S, chunk), **kw)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), ref.cpu()), kw
        torch.testing.assert_close(got.cpu().float(), want.float(), rtol=RTOL, atol=ATOL)
        outs.append(got.cpu())
    assert torch.equal(outs[0], outs[1])


def test_attention_identical_keys_is_mean_of_values(gpu):
    B, Hq, Hk, L = 2, 32, 8, 777
    K = torch.randn(B, Hk, 1, 128).to(torch.bfloat16).expand(-1, -1, L, -1).contiguous()
    V = torch.randn(B, Hk, L, 128).to(torch.bfloat16)
    q = torch.randn(B, Hq, 128).to(torch.bfloat16)
    ws = shadowkv.sparse_attn_workspace(B, Hq, L, gpu)
    out = torch.empty(B, Hq, 128, dtype=torch.bfloat16, device=gpu)
    shadowkv.sparse_attn_decode(q.to(gpu), K.to(gpu), V.to(gpu), L, out, ws)
    torch.cuda.synchronize()
    mean = V.float().mean(dim=2).repeat_interleave(Hq // Hk, dim=1)
    torch.testing.assert_close(out.cpu().float(), mean, rtol=1e-2, atol=1e-2)


def test_attention_device_length_matches_host_length(gpu):
    """kv_len_dev (a device int32 read when the kernel runs) gives the host-length result bit for bit,
    including at split boundaries, and is clamped to [1, kv_len]."""
    B, Hq, Hk, Lmax = 2, 32, 8, 1100
    g = torch.Generator().manual_seed(3)
    K = torch.randn(B, Hk, Lmax, 128, generator=g).to(torch.bfloat16).to(gpu)
    V = torch.randn(B, Hk, Lmax, 128, generator=g).to(torch.bfloat16).to(gpu)
    q = torch.randn(B, Hq, 128, generator=g).to(torch.bfloat16).to(gpu)
    ws = shadowkv.sparse_attn_workspace(B, Hq, Lmax, gpu)
    ldev = torch.zeros(1, dtype=torch.int32, device=gpu)
    for L, eff in ((1, 1), (255, 255), (256, 256), (257, 257), (1024, 1024), (1100, 1100), (0, 1), (5000, 1100)):
        _say(f"attention device length {L}")
        ldev.fill_(L)
        got = torch.empty(B, Hq, 128, dtype=torch.bfloat16, device=gpu)
        shadowkv.sparse_attn_decode(q, K, V, Lmax, got, ws, kv_len_dev=ldev)
        want = torch.empty_like(got)
        ws2 = shadowkv.sparse_attn_workspace(B, Hq, eff, gpu)
        shadowkv.sparse_attn_decode(q, K, V, eff, want, ws2)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), want.cpu()), L
        ref = oracle.sparse_attention(q.cpu(), K.cpu(), V.cpu(), eff)
        torch.testing.assert_close(got.cpu().float(), ref.float(), rtol=RTOL, atol=ATOL)


def test_attention_device_length_long_rows(gpu, monkeypatch):
    """Rows long enough for several merge groups (more than 32 splits) of the two-launch merge: a
    device length below the maximum merges in the same order as the same host length (bit for
    bit). The split size and the merge are pinned (by default the shorter host lengths would take
    64-key splits and the one-launch merge, which sum in another order)."""
    monkeypatch.setenv("SKV_ATTN_SPLIT", "128")
    monkeypatch.setenv("SKV_ATTN_FUSED", "0")
    B, Hq, Hk, Lmax = 1, 32, 8, 12000
    g = torch.Generator().manual_seed(4)
    K = torch.randn(B, Hk, Lmax, 128, generator=g).to(torch.bfloat16).to(gpu)
    V = torch.randn(B, Hk, Lmax, 128, generator=g).to(torch.bfloat16).to(gpu)
    q = torch.randn(B, Hq, 128, generator=g).to(torch.bfloat16).to(gpu)
    ws = shadowkv.sparse_attn_workspace(B, Hq, Lmax, gpu)
    ldev = torch.zeros(1, dtype=torch.int32, device=gpu)
    for L in (3000, 4096, 4097, 8300, 12000):
        _say(f"attention long rows, device length {L}")
        ldev.fill_(L)
        got = torch.empty(B, Hq, 128, dtype=torch.bfloat16, device=gpu)
        shadowkv.sparse_attn_decode(q, K, V, Lmax, got, ws, kv_len_dev=ldev)
        want = torch.empty_like(got)
        ws2 = shadowkv.sparse_attn_workspace(B, Hq, L, gpu)
        shadowkv.sparse_attn_decode(q, K, V, L, want, ws2)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), want.cpu()), L
        ref = oracle.sparse_attention(q.cpu(), K.cpu(), V.cpu(), L)
        torch.testing.assert_close(got.cpu().float(), ref.float(), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("glm", [False, True])
def test_rebuild_tile_shapes_agree(gpu, glm, monkeypatch):
    """Workgroups of 256, 128 and 64 rows (chosen by the grid size, forced here), with the miss
    rows in whole tiles or dealt evenly over every tile (also chosen by the grid size), run the
    same per-row MFMA sequence: bit-identical keys, and within tolerance of the oracle."""
    B, H, ctx, R, S, c = 2, 8, 4096, 160, 256, 8
    _say(f"rebuild tile shapes glm={glm}")
    U, SV, ids, cnts = _rebuild_case(B, H, ctx, R, S, c, 21, True, False)
    cs = oracle.build_glm_cos_sin_cache(ctx, 5e6) if glm else oracle.build_cos_sin_cache(ctx, 5e5)
    start = 448
    cache = torch.randn(B, H, start + S * c + 32, 128).to(torch.bfloat16)
    outs = []
    for tile in (256, 128, 64, "w256"):
        for spread in ("0", "1"):  # whole tiles (hit tiles idle) or the miss rows dealt over every tile
            monkeypatch.setenv("SKV_REBUILD_TILE", str(tile))
            monkeypatch.setenv("SKV_REBUILD_SPREAD", spread)
            cg = cache.to(gpu)
            shadowkv.rebuild_k_rope(U.to(gpu), SV.to(gpu), ids.to(gpu), cnts.to(gpu), cs.to(gpu), cg, start, c)
            torch.cuda.synchronize()
            outs.append(cg.cpu())
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    want = oracle.rebuild_k_rope(U, SV, ids, cnts, cs, c, cache.clone(), start, glm=glm)
    torch.testing.assert_close(outs[0].float(), want.float(), rtol=RTOL, atol=ATOL)


def test_rope_two_tables_and_chunk_positions(gpu):
    """The reference's remaining rotary bindings: separate cos/sin tables (apply_rotary_pos_emb),
    chunk-id positions without hit rows (apply_rotary_pos_emb_new_v2), and push_cache (the _opt
    contract), bit-exact against the oracle."""
    _say("rope two tables / new_v2 / push_cache")
    g = torch.Generator().manual_seed(77)
    B, H, Ls, D, rows = 2, 4, 40, 128, 600
    x = torch.randn(B, H, Ls, D, generator=g).to(torch.bfloat16)
    cos = torch.randn(rows, D, generator=g).to(torch.bfloat16)
    sin = torch.randn(rows, D, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, rows, (B, H, Ls), generator=g)
    pos[0, 1, 3] = rows + 7  # outside the tables: row left unwritten
    out = torch.full_like(x, 5.0).to(gpu)
    xs = x.stride()
    shadowkv.apply_rotary_pos_emb(x.to(gpu), cos.to(gpu), sin.to(gpu), pos.to(gpu), out, B, H, Ls, D, *xs,
                                  cos.stride(0), sin.stride(0), *pos.stride(), D // 2)
    torch.cuda.synchronize()
    got = out.cpu()
    want = oracle.rope_two_tables(x, cos[pos.clamp_max(rows - 1)], sin[pos.clamp_max(rows - 1)])
    want[0, 1, 3] = 5.0
    assert torch.equal(got, want)
    # new_v2: every row at its chunk id's position
    c, S = 8, Ls // 8
    cs = oracle.build_cos_sin_cache(4096, 5e5)
    ids = torch.randint(0, 4000 // c, (B, H, S), generator=g, dtype=torch.int32)
    out2 = torch.zeros_like(x).to(gpu)
    shadowkv.apply_rotary_pos_emb_new_v2(x.to(gpu), cs.to(gpu), ids.to(gpu), out2, B, H, Ls, D, *xs, cs.stride(0),
                                         *ids.stride(), D // 2, c)
    torch.cuda.synchronize()
    want2 = oracle.rope_push(x, cs, ids, torch.zeros(B * H, dtype=torch.int32), c, torch.zeros_like(x), 0, Ls)
    assert torch.equal(out2.cpu(), want2)
    # push_cache == push_cache_opt
    cnts = torch.tensor([0, 1, 5, 2, 3, 0, 4, 1], dtype=torch.int32)
    buf = torch.randn(B, H, Ls + 20, D, generator=g).to(torch.bfloat16)
    outs = []
    for fn in (shadowkv.apply_rotary_pos_emb_push_cache, shadowkv.apply_rotary_pos_emb_push_cache_opt):
        o = buf.to(gpu)
        fn(x.to(gpu), cs.to(gpu), ids.to(gpu), o, cnts.to(gpu), B, H, Ls, D, *xs, cs.stride(0), *ids.stride(),
           *o.stride()[:3], 10, 10 + Ls - 4, D // 2, c)
        torch.cuda.synchronize()
        outs.append(o.cpu())
    assert torch.equal(outs[0], outs[1])
    want3 = oracle.rope_push(x, cs, ids, cnts, c, buf.clone(), 10, 10 + Ls - 4)
    assert torch.equal(outs[0], want3)



def test_rebuild_k_rope_random_shapes(gpu):
    """The rebuild + RoPE push on 10 seeded random shapes (batch 1-3, 1-8 heads, rank 8-192,
    1-300 chunks of 4, 8 or 16 rows, random hit counts, both rotations, per-head or shared U/SV)
    against the oracle: the rebuilt rows within tolerance, every other row untouched."""
    rng = np.random.default_rng(77)
    for case in range(10):
        B, H = int(rng.integers(1, 4)), int(rng.choice([1, 2, 3, 8]))
        R = 8 * int(rng.integers(1, 25))
        c = int(rng.choice([4, 8, 16]))
        S = int(rng.integers(1, 301))
        ctx = c * max(S + 16, int(rng.integers(S + 16, 1200)))
        glm, per_head_u, shared_sv = (bool(rng.integers(0, 2)) for _ in range(3))
        _say(f"rebuild random case {case}: B={B} H={H} R={R} c={c} S={S} ctx={ctx} glm={glm} "
             f"per_head_u={per_head_u} shared_sv={shared_sv}")
        U, SV, ids, cnts = _rebuild_case(B, H, ctx, R, S, c, 1000 + case, per_head_u, shared_sv)
        cs = oracle.build_glm_cos_sin_cache(ctx, 5e6) if glm else oracle.build_cos_sin_cache(ctx, 5e5)
        start = int(rng.integers(0, 64)) * 8
        buf = start + S * c + 24
        cache = torch.randn(B, H, buf, 128).to(torch.bfloat16)
        SVf = SV.unsqueeze(0).expand(B, -1, -1, -1) if shared_sv else SV
        want = oracle.rebuild_k_rope(U, SVf, ids, cnts, cs, c, cache.clone(), start, glm=glm)
        cg = cache.to(gpu)
        shadowkv.rebuild_k_rope(U.to(gpu), SV.to(gpu), ids.to(gpu), cnts.to(gpu), cs.to(gpu), cg, start, c)
        torch.cuda.synchronize()
        got = cg.cpu()
        assert torch.equal(got[:, :, :start], cache[:, :, :start])
        assert torch.equal(got[:, :, start + S * c:], cache[:, :, start + S * c:])
        for bh in range(B * H):
            b, h = divmod(bh, H)
            miss = start + int(cnts[bh]) * c
            assert torch.equal(got[b, h, start:miss], cache[b, h, start:miss])
            torch.testing.assert_close(got[b, h, miss:start + S * c].float(), want[b, h, miss:start + S * c].float(),
                                       rtol=RTOL, atol=ATOL)


def test_sparse_attention_random_shapes(gpu):
    """Sparse decode attention on 10 seeded random shapes (batch 1-6, 1-8 kv heads of 1-16 query
    heads, lengths 1-20000, buffers longer than the length) against the oracle."""
    rng = np.random.default_rng(78)
    for case in range(10):
        B, Hk, G = int(rng.integers(1, 7)), int(rng.choice([1, 2, 4, 8])), int(rng.choice([1, 2, 4, 8, 16]))
        L = int(rng.choice([1, 2, 127, 128, 129])) if case < 3 else int(rng.integers(1, 20001))
        Hq = Hk * G
        _say(f"attention random case {case}: B={B} Hq={Hq} Hk={Hk} L={L}")
        g = torch.Generator().manual_seed(500 + case)
        buf = L + int(rng.integers(0, 50))
        K = torch.randn(B, Hk, buf, 128, generator=g).to(torch.bfloat16)
        V = torch.randn(B, Hk, buf, 128, generator=g).to(torch.bfloat16)
        q = torch.randn(B, Hq, 128, generator=g).to(torch.bfloat16)
        want = oracle.sparse_attention(q, K, V, L)
        ws = shadowkv.sparse_attn_workspace(B, Hq, L, gpu)
        out = torch.empty(B, Hq, 128, dtype=torch.bfloat16, device=gpu)
        shadowkv.sparse_attn_decode(q.to(gpu), K.to(gpu), V.to(gpu), L, out, ws)
        torch.cuda.synchronize()
        torch.testing.assert_close(out.cpu().float(), want.float(), rtol=RTOL, atol=ATOL)
