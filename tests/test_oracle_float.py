"""Pins for the oracle's floating-point functions (RoPE, rebuild, scoring, attention) on the CPU.

Each check is independent of the oracle's own formula: numpy with explicit rounding,
float64 references, closed forms and special cases that a dropped term, a wrong sign or a
transposed operand would break.
"""
import math

import numpy as np
import torch

import oracle
from tests.golden import make_golden


def bf16_round_np(x: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 (nearest even), returned as float32."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


def to_np(t):
    return t.float().numpy()


def test_rope_half_split_bit_exact_vs_numpy():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(300, 128, generator=g).to(torch.bfloat16)
    ang = torch.rand(300, 64, generator=g) * 50
    c, s = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    got = to_np(oracle.rope_half_split(x, c, s))
    xn, cn, sn = to_np(x), to_np(c), to_np(s)
    x1, x2 = xn[:, :64], xn[:, 64:]
    y1 = bf16_round_np(bf16_round_np(x1 * cn) + bf16_round_np(-x2 * sn))
    y2 = bf16_round_np(bf16_round_np(x2 * cn) + bf16_round_np(x1 * sn))
    assert np.array_equal(got, np.concatenate([y1, y2], axis=1))


def test_rope_identity_at_position_zero_and_rotation():
    cs = oracle.build_cos_sin_cache(100, 500000.0)
    x = torch.randn(5, 128).to(torch.bfloat16)
    assert torch.equal(oracle.rope_half_split(x, cs[0, :64].expand(5, -1), cs[0, 64:].expand(5, -1)), x)
    # agreement with an exact complex rotation (x1 + i x2) * e^{i theta} within bf16 rounding
    pos = 37
    y = to_np(oracle.rope_half_split(x, cs[pos, :64].expand(5, -1), cs[pos, 64:].expand(5, -1))).astype(np.float64)
    inv = 1.0 / (500000.0 ** (np.arange(0, 128, 2) / 128.0))
    z = (to_np(x)[:, :64] + 1j * to_np(x)[:, 64:]).astype(np.complex128) * np.exp(1j * pos * inv)
    assert np.abs(y[:, :64] - z.real).max() < 0.05 and np.abs(y[:, 64:] - z.imag).max() < 0.05


def test_rope_push_skips_hits_and_uses_token_positions():
    B, H, S, c, D = 1, 2, 4, 8, 128
    cs = oracle.build_cos_sin_cache(512, 10000.0)
    x = torch.randn(B, H, S * c, D).to(torch.bfloat16)
    ids = torch.tensor([[[3, 10, 20, 40], [5, 6, 7, 50]]])
    cnts = torch.tensor([1, 3], dtype=torch.int32)
    cache = torch.zeros(B, H, 100, D, dtype=torch.bfloat16)
    oracle.rope_push(x, cs, ids, cnts, c, cache, 10, 10 + S * c)
    for h in range(H):
        hit_rows = int(cnts[h]) * c
        assert (cache[0, h, 10:10 + hit_rows] == 0).all()
        for r in range(hit_rows, S * c):
            p = int(ids[0, h, r // c]) * c + r % c
            want = oracle.rope_half_split(x[0, h, r], cs[p, :64], cs[p, 64:])
            assert torch.equal(cache[0, h, 10 + r], want)


def test_rope_glm_vs_numpy():
    cs = oracle.build_glm_cos_sin_cache(64, 10000.0 * 500)
    B, H, S, c, D = 1, 1, 2, 8, 128
    x = torch.randn(B, H, S * c, D).to(torch.bfloat16)
    ids = torch.tensor([[[2, 5]]])
    cache = torch.zeros(B, H, S * c, D, dtype=torch.bfloat16)
    oracle.rope_push_glm(x, cs, ids, torch.tensor([0], dtype=torch.int32), c, cache, 0, S * c)
    xn, csn = to_np(x[0, 0]), to_np(cs)
    for r in range(S * c):
        p = int(ids[0, 0, r // c]) * c + r % c
        co, si = csn[p, :32], csn[p, 32:]
        e, o = xn[r, 0:64:2], xn[r, 1:64:2]
        ye = bf16_round_np(bf16_round_np(e * co) + bf16_round_np(-o * si))
        yo = bf16_round_np(bf16_round_np(o * co) + bf16_round_np(e * si))
        got = to_np(cache[0, 0, r])
        assert np.array_equal(got[0:64:2], ye) and np.array_equal(got[1:64:2], yo)
        assert np.array_equal(got[64:], xn[r, 64:])


def test_rebuild_basis_rows_and_float64():
    B, H, ctx, R, D, c = 2, 3, 64, 32, 128, 8
    g = torch.Generator().manual_seed(5)
    SV = torch.randn(B, H, D, R, generator=g).to(torch.bfloat16)
    U = torch.zeros(B, ctx, R, dtype=torch.bfloat16)
    for p in range(ctx):
        U[:, p, p % R] = 1.0
    ids = torch.tensor([[[0, 3], [7, 1], [2, 2]], [[1, 0], [6, 4], [5, 7]]])
    k = oracle.rebuild_k(U, SV, ids, c)
    for b in range(B):
        for h in range(H):
            for r in range(2 * c):
                p = int(ids[b, h, r // c]) * c + r % c
                assert torch.equal(k[b, h, r], SV[b, h, :, p % R])  # basis row picks an SV column exactly
    U = torch.randn(B, ctx, R, generator=g).to(torch.bfloat16)
    k = oracle.rebuild_k(U, SV, ids, c).float().numpy()
    Un, SVn = U.double().numpy(), SV.double().numpy()
    for b in range(B):
        for h in range(H):
            pos = (ids[b, h].numpy()[:, None] * c + np.arange(c)).reshape(-1)
            want = Un[b, pos] @ SVn[b, h].T
            assert np.allclose(k[b, h], want, rtol=1e-2, atol=1e-2)


def test_score_softmax_special_cases_and_float64():
    alpha = 1.0 / math.sqrt(128)
    q = torch.randn(3, 4, 128).to(torch.bfloat16)
    same = torch.randn(1, 1, 128).to(torch.bfloat16).expand(3, 77, 128).contiguous()
    _, p = oracle.score_logits_softmax(q, same, alpha)
    assert torch.equal(p, torch.full_like(p, 1.0 / 77).to(torch.bfloat16))
    _, p1 = oracle.score_logits_softmax(q, same[:, :1], alpha)
    assert (p1 == 1.0).all()
    L = torch.randn(3, 500, 128).to(torch.bfloat16)
    D, P = oracle.score_logits_softmax(q, L, alpha)
    logits = np.einsum("zid,zjd->zij", q.double().numpy(), L.double().numpy()) * alpha
    assert np.abs(D.double().numpy() - logits).max() <= np.abs(logits).max() * 2 ** -8
    Dn = D.double().numpy()
    e = np.exp(Dn - Dn.max(-1, keepdims=True))
    want = e / e.sum(-1, keepdims=True)
    assert np.all(np.abs(P.double().numpy() - want) <= want * 2 ** -8 + 1e-30)
    m = oracle.score_gqa_max(q, L, alpha)
    assert torch.equal(m, P.max(dim=1).values)


def test_attention_special_cases_and_float64():
    B, Hq, Hk, D = 2, 8, 2, 128
    q = torch.randn(B, Hq, D).to(torch.bfloat16)
    K = torch.randn(B, Hk, 50, D).to(torch.bfloat16)
    V = torch.randn(B, Hk, 50, D).to(torch.bfloat16)
    out1 = oracle.sparse_attention(q, K, V, 1)
    for hq in range(Hq):
        assert torch.equal(out1[:, hq], V[:, hq // 4, 0])
    Ksame = K[:, :, :1].expand(-1, -1, 50, -1)
    outm = oracle.sparse_attention(q, Ksame, V, 50).float()
    mean = V.float().mean(dim=2).repeat_interleave(4, dim=1)
    assert torch.allclose(outm, mean, atol=1e-2, rtol=1e-2)
    out = oracle.sparse_attention(q, K, V, 37).double().numpy()
    qn, Kn, Vn = q.double().numpy(), K.double().numpy(), V.double().numpy()
    for b in range(B):
        for hq in range(Hq):
            s = Kn[b, hq // 4, :37] @ qn[b, hq] / math.sqrt(D)
            p = np.exp(s - s.max())
            p /= p.sum()
            assert np.allclose(out[b, hq], p @ Vn[b, hq // 4, :37], atol=1e-2, rtol=1e-2)


def test_decode_small_fixture_regression():
    d = np.load(make_golden.HERE / "decode_small.npz")
    case = make_golden.decode_small_case()
    st, res = case["st"], case["res"]
    assert [make_golden.digest(case["state_in"][k]) for k in sorted(case["state_in"])] == d["in_digests"].tolist()
    assert np.array_equal(res["scores"].view(torch.int16).numpy(), d["out_scores"])
    assert np.array_equal(res["selected"].numpy(), d["out_selected"])
    assert np.array_equal(res["cnts"], d["out_cnts"])
    assert np.array_equal(res["offsets"], d["out_offsets"])
    assert np.array_equal(st.position_ids.numpy(), d["out_position_ids"])
    assert np.array_equal(res["out"].view(torch.int16).numpy(), d["out_attn"])
    assert [make_golden.digest(st.kbuf), make_golden.digest(st.vbuf)] == d["out_digests"].tolist()


def test_decode_step_from_given_scores_matches_computed():
    """decode_layer_step(scores=...) with the oracle's own scores reproduces the committed fixture."""
    import numpy as np
    from tests.decode_harness import fresh_oracle_state
    from tests.golden import make_golden
    case = make_golden.decode_small_case()
    d = np.load(make_golden.HERE / "decode_small.npz")
    st = fresh_oracle_state(case)
    res = oracle.decode_layer_step(st, case["q"], case["k_new"], case["v_new"], case["cos_sin"],
                                   scores=case["res"]["scores"])
    assert np.array_equal(res["cnts"], d["out_cnts"])
    assert np.array_equal(res["offsets"], d["out_offsets"])
    assert np.array_equal(st.position_ids.numpy(), d["out_position_ids"])
    assert torch.equal(res["out"], case["res"]["out"])


def test_encode_layer_overrides_reproduce_the_default_path():
    """encode_layer(outliers=..., init_scores=...) given the default path's own outlier order and
    GQA-max scores builds the same state (the device encoder's tests continue from its decisions)."""
    import math
    import torch.nn.functional as F
    from oracle.shadowkv_oracle import _rope_tokens
    from tests.golden import make_golden

    case = make_golden.decode_small_case()
    d = case["dims"]
    st = oracle.LayerState(**case["state_in"], chunks=case["st"].chunks, sparse_start=case["st"].sparse_start)
    B, H, D, ctx, c = d["B"], d["H"], d["D"], d["ctx"], d["chunk"]
    k = _rope_tokens(case["k_pre"], case["cos_sin"], torch.arange(ctx))
    kc = k[:, :, :st.chunks * c].reshape(B, H, st.chunks, c, D)
    cand = kc.mean(dim=-2)
    cos = F.cosine_similarity(cand.unsqueeze(3).expand(-1, -1, -1, c, -1), kc, dim=-1)
    n_out = (d["budget"] // 1024) * 24
    outliers = cos.min(dim=-1).values.topk(n_out, largest=False).indices
    q = _rope_tokens(case["q_last"], case["cos_sin"], torch.tensor([ctx - 1]))
    n = st.landmarks.shape[-2]
    # the default path's own scores (bf16 einsum, fp32 softmax, bf16, max over the group)
    sc = torch.einsum("bhgd,bhcd->bhgc", q.reshape(B, H, -1, D), st.landmarks) / math.sqrt(128)
    sc = F.softmax(sc, dim=-1, dtype=torch.float32).to(torch.bfloat16).max(dim=-2).values
    st2 = oracle.encode_layer(case["k_pre"], case["v"], case["q_last"], case["cos_sin"], rank=d["rank"], chunk=c,
                              budget=d["budget"], outliers=outliers, init_scores=sc)
    for name in ("landmarks", "landmark_idx", "host_v", "U", "SV"):
        a, b = getattr(st, name), getattr(st2, name)
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b), name
    for buf in ("kbuf", "vbuf"):  # local + outlier regions identical
        assert torch.equal(getattr(st, buf)[:, :, :st.sparse_start].view(torch.int16),
                           getattr(st2, buf)[:, :, :st.sparse_start].view(torch.int16)), buf
    # the initial selection: the same chunks, up to ties at the top-S boundary (torch.topk breaks
    # them arbitrarily, topk_gather by the lowest landmark index)
    S = d["budget"] // c
    for r in range(B * H):
        b, h = divmod(r, H)
        vals = sc[b, h].float()
        kth = torch.sort(vals, descending=True).values[S - 1]
        score_of = {int(i): float(v) for i, v in zip(st.landmark_idx[b, h], vals)}
        a, bsel = set(st.position_ids[b, h].tolist()), set(st2.position_ids[b, h].tolist())
        assert all(score_of[i] == kth for i in a ^ bsel), r
        assert {i for i, v in score_of.items() if v > kth} <= a & bsel


def test_glm_token_rope_matches_glm_push():
    """The oracle's token RoPE with a GLM (width-64) table equals its GLM cache push (pinned against
    an independent numpy restatement above) row for row, and position 0 is the identity."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, 2, 16, 128, generator=g).to(torch.bfloat16)
    cs = oracle.build_glm_cos_sin_cache(64, 10000.0)
    from oracle import shadowkv_oracle
    got = shadowkv_oracle._rope_tokens(x, cs, torch.arange(16))
    cache = torch.zeros(1, 2, 16, 128, dtype=torch.bfloat16)
    ids = torch.arange(16).view(1, 1, 16).expand(1, 2, 16).contiguous()
    oracle.rope_push_glm(x, cs, ids, torch.zeros(2, dtype=torch.int32), 1, cache, 0, 16)
    assert torch.equal(got, cache)
    assert torch.equal(got[:, :, 0], x[:, :, 0])
    assert torch.equal(got[..., 64:], x[..., 64:])


def test_rope_two_tables_bit_exact_vs_numpy():
    """The separate-table rotation: numpy float32 with explicit rounding, second half with the
    tables' second halves; with equal halves it is the half-split rotation."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(200, 128, generator=g).to(torch.bfloat16)
    c = torch.randn(200, 128, generator=g).to(torch.bfloat16)
    s = torch.randn(200, 128, generator=g).to(torch.bfloat16)
    got = to_np(oracle.rope_two_tables(x, c, s))
    xn, cn, sn = to_np(x), to_np(c), to_np(s)
    y1 = bf16_round_np(bf16_round_np(xn[:, :64] * cn[:, :64]) + bf16_round_np(-xn[:, 64:] * sn[:, :64]))
    y2 = bf16_round_np(bf16_round_np(xn[:, 64:] * cn[:, 64:]) + bf16_round_np(xn[:, :64] * sn[:, 64:]))
    assert np.array_equal(got, np.concatenate([y1, y2], axis=1))
    ch = torch.cat((c[:, :64], c[:, :64]), dim=-1)
    sh = torch.cat((s[:, :64], s[:, :64]), dim=-1)
    assert torch.equal(oracle.rope_two_tables(x, ch, sh), oracle.rope_half_split(x, c[:, :64], s[:, :64]))


def test_encode_layer_sv_head_split():
    """encode_layer's per-head SV (shadow.py:437-442): for every head of both fixtures U @ SV[h]^T
    gives back that head's pre-RoPE keys down to the noise the rank-R truncation must leave; a
    transposed split and a head permutation of the same factors exceed the bound over twice."""
    from tests import svd_pins

    for case in (make_golden.decode_small_case(), make_golden.single_layer_case()):
        st, k_pre, R = case["st"], case["k_pre"], case["dims"]["rank"]
        err = svd_pins.head_errors(k_pre, st.U, st.SV)
        lim = svd_pins.bound(k_pre, R)
        floor = svd_pins.noise_floor(k_pre, R)
        assert (err <= lim).all(), (err, lim)
        assert (err >= 0.97 * floor).all(), (err, floor)  # not better than the noise allows
        wrong = svd_pins.head_errors(k_pre, st.U, svd_pins.transposed_split(st.SV))
        assert (wrong > 2 * lim).all(), (wrong, lim)
        swapped = svd_pins.head_errors(k_pre, st.U, st.SV.flip(1))
        assert (swapped > 2 * lim).all(), (swapped, lim)
