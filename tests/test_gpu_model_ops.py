"""The fused new-token operations around the path: residual add + RMSNorm, SiLU-and-mul, and
q/k RoPE + KV append, against fp32 torch references and the oracle's rotation."""
import pytest
import torch

import oracle
from shadowkv_amd.kernels import shadowkv
from tests.decode_harness import assert_bf16_close

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _rms_ref(h: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    hf = h.float()
    return (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).to(torch.bfloat16)


@pytest.mark.parametrize("rows,hidden", [(4, 4096), (8, 4096), (3, 1024), (2, 8192), (1, 520)])
def test_rmsnorm(gpu, rows, hidden):
    _say(f"rmsnorm rows={rows} hidden={hidden}")
    g = torch.Generator().manual_seed(hidden + rows)
    x = torch.randn(rows, 1, hidden, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16)
    out = torch.empty(rows, 1, hidden, dtype=torch.bfloat16, device=gpu)
    shadowkv.rmsnorm(x.to(gpu), w.to(gpu), 1e-5, out)
    torch.cuda.synchronize()
    assert_bf16_close(out.cpu(), _rms_ref(x, w, 1e-5), what="rmsnorm")


@pytest.mark.parametrize("inplace", [False, True])
def test_rmsnorm_with_residual(gpu, inplace):
    rows, hidden = 4, 4096
    _say(f"rmsnorm + residual inplace={inplace}")
    g = torch.Generator().manual_seed(5)
    x = torch.randn(rows, 1, hidden, generator=g).to(torch.bfloat16)
    r = (4 * torch.randn(rows, 1, hidden, generator=g)).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16)
    xg, rg = x.to(gpu), r.to(gpu)
    ro = rg if inplace else torch.empty_like(rg)
    out = torch.empty_like(xg)
    shadowkv.rmsnorm(xg, w.to(gpu), 1e-6, out, residual=rg, residual_out=ro)
    torch.cuda.synchronize()
    h = (r.float() + x.float()).to(torch.bfloat16)  # the bf16 residual add
    assert torch.equal(ro.cpu(), h)
    assert_bf16_close(out.cpu(), _rms_ref(h, w, 1e-6), what="rmsnorm(residual)")


@pytest.mark.parametrize("rows,d", [(4, 14336), (8, 13696), (1, 8)])
def test_silu_and_mul(gpu, rows, d):
    _say(f"silu_and_mul rows={rows} d={d}")
    g = torch.Generator().manual_seed(d)
    x = (3 * torch.randn(rows, 1, 2 * d, generator=g)).to(torch.bfloat16)
    out = torch.empty(rows, 1, d, dtype=torch.bfloat16, device=gpu)
    shadowkv.silu_and_mul(x.to(gpu), out)
    torch.cuda.synchronize()
    gt, up = x.float()[..., :d], x.float()[..., d:]
    # vLLM silu_and_mul (the reference's activation): silu in fp32 rounded to bf16, then the bf16 product
    want = ((gt / (1 + torch.exp(-gt))).to(torch.bfloat16).float() * up).to(torch.bfloat16)
    assert_bf16_close(out.cpu(), want, what="silu_and_mul")


@pytest.mark.parametrize("glm", [False, True])
def test_rope_qk_append(gpu, glm):
    B, Hq, Hk, D, buf = 3, 32, 8 if not glm else 2, 128, 40
    _say(f"rope_qk_append glm={glm}")
    g = torch.Generator().manual_seed(11)
    cs = oracle.build_glm_cos_sin_cache(3000, 5e6) if glm else oracle.build_cos_sin_cache(3000, 5e5)
    qkv = torch.randn(B, (Hq + 2 * Hk) * D, generator=g).to(torch.bfloat16)
    pos = torch.tensor([0, 1777, cs.shape[0] + 5])  # identity row, an ordinary row, beyond the table
    kc = torch.randn(B, Hk, buf, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(B, Hk, buf, D, generator=g).to(torch.bfloat16)
    row = torch.tensor([17])
    q_out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=gpu)
    kg, vg = kc.to(gpu), vc.to(gpu)
    shadowkv.rope_qk_append(qkv.to(gpu), Hq, Hk, pos.to(gpu), cs.to(gpu), q_out, kg, vg, row.to(gpu))
    torch.cuda.synchronize()
    q = qkv[:, :Hq * D].view(B, Hq, 1, D)
    k = qkv[:, Hq * D:(Hq + Hk) * D].view(B, Hk, 1, D)
    v = qkv[:, (Hq + Hk) * D:].view(B, Hk, D)

    def rot(x):
        H = x.shape[1]
        out = x.clone()
        for b in range(B):
            if int(pos[b]) >= cs.shape[0]:
                continue  # no rotation row: unrotated
            ids = torch.full((1, H, 1), int(pos[b]))
            if glm:
                oracle.rope_push_glm(x[b:b + 1], cs, ids, torch.zeros(H, dtype=torch.int32), 1, out[b:b + 1], 0, 1)
            else:
                oracle.rope_push(x[b:b + 1], cs, ids, torch.zeros(H, dtype=torch.int32), 1, out[b:b + 1], 0, 1)
        return out

    assert torch.equal(q_out.cpu(), rot(q).view(B, Hq, D))
    want_k, want_v = kc.clone(), vc.clone()
    want_k[:, :, 17] = rot(k).view(B, Hk, D)
    want_v[:, :, 17] = v
    assert torch.equal(kg.cpu(), want_k)
    assert torch.equal(vg.cpu(), want_v)
    assert torch.equal(q_out.cpu()[0], q.view(B, Hq, D)[0])  # position 0 is the identity rotation

    # an append row outside the buffer writes nothing
    shadowkv.rope_qk_append(qkv.to(gpu), Hq, Hk, pos.to(gpu), cs.to(gpu), q_out, kg, vg,
                            torch.tensor([buf], device=gpu))
    torch.cuda.synchronize()
    assert torch.equal(kg.cpu(), want_k) and torch.equal(vg.cpu(), want_v)


# (rows, q heads, kv heads, k, glm): the Llama-3 (32 / 8) and GLM-4 (32 / 2) shapes at 1-4 token
# rows, and a small shape whose k is not a multiple of the 512-element block.
# GLM's projection with its bias (models/glm.py:165), the half-split one with and without.
QKV_ROPE_CASES = [(4, 32, 8, 4096, False, False), (1, 32, 8, 4096, False, True), (3, 32, 8, 4096, False, False),
                  (4, 32, 2, 4096, True, True), (2, 32, 2, 4096, True, True), (3, 4, 2, 1032, False, True),
                  (3, 4, 2, 1032, True, False)]


@pytest.mark.parametrize("B,Hq,Hk,k,glm,bias", QKV_ROPE_CASES)
def test_linear_qkv_rope_append_equals_linear_then_rope(gpu, B, Hq, Hk, k, glm, bias):
    """The QKV projection with RoPE + append in its epilogue writes, bit for bit, what the skinny
    linear (with the bias) followed by rope_qk_append writes: rotated q, the appended rotated k and
    raw v rows; positions outside the table leave q/k unrotated, an append row outside the buffer
    writes no key/value row."""
    D, buf = 128, 40
    _say(f"linear_qkv_rope_append B={B} Hq={Hq} Hk={Hk} k={k} glm={glm} bias={bias}")
    g = torch.Generator().manual_seed(B * 31 + Hk + k + glm)
    cs = oracle.build_glm_cos_sin_cache(3000, 5e6) if glm else oracle.build_cos_sin_cache(3000, 5e5)
    n = (Hq + 2 * Hk) * D
    x = torch.randn(B, 1, k, generator=g).to(torch.bfloat16).to(gpu)
    w = (torch.randn(n, k, generator=g) / k ** 0.5 * 2).to(torch.bfloat16).to(gpu)
    bq = (torch.randn(n, generator=g) * 0.5).to(torch.bfloat16).to(gpu) if bias else None
    w_rope = shadowkv.qkv_rope_weight(w, Hq, Hk, glm)
    b_rope = shadowkv.qkv_rope_weight(bq, Hq, Hk, glm) if bias else None
    if bias and not glm:  # the bias in the weight's row order
        qk = (Hq + Hk) * D
        assert torch.equal(b_rope[:qk].view(Hq + Hk, 64, 2)[:, :, 1], bq[:qk].view(Hq + Hk, 2, 64)[:, 1])
    if glm:
        assert torch.equal(w_rope, w)
    else:  # rows (d, d + 64) of every q/k head adjacent, v rows in place
        qk = (Hq + Hk) * D
        wh, rh = w[:qk].view(Hq + Hk, 2, 64, k), w_rope[:qk].view(Hq + Hk, 64, 2, k)
        assert torch.equal(rh[:, :, 0], wh[:, 0]) and torch.equal(rh[:, :, 1], wh[:, 1])
        assert torch.equal(w_rope[qk:], w[qk:])
    pos = torch.tensor([1777, 0, cs.shape[0] + 5, 2999][:B], device=gpu)  # an ordinary row, identity, beyond the table
    row = torch.tensor([17], device=gpu)
    kc = torch.randn(B, Hk, buf, D, generator=g).to(torch.bfloat16).to(gpu)
    vc = torch.randn(B, Hk, buf, D, generator=g).to(torch.bfloat16).to(gpu)
    csg = cs.to(gpu)
    qkv = torch.empty(B, 1, n, dtype=torch.bfloat16, device=gpu)
    shadowkv.linear(x, w, qkv, bias=bq)
    q_want = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=gpu)
    k_want, v_want = kc.clone(), vc.clone()
    shadowkv.rope_qk_append(qkv.view(B, n), Hq, Hk, pos, csg, q_want, k_want, v_want, row)
    q_got = torch.full((B, Hq, D), 3.0, dtype=torch.bfloat16, device=gpu)
    k_got, v_got = kc.clone(), vc.clone()
    shadowkv.linear_qkv_rope_append(x.view(B, k), w_rope, Hq, Hk, pos, csg, q_got, k_got, v_got, row, b_rope)
    torch.cuda.synchronize()
    assert torch.equal(q_got.cpu(), q_want.cpu())
    assert torch.equal(k_got.cpu(), k_want.cpu())
    assert torch.equal(v_got.cpu(), v_want.cpu())
    assert not torch.equal(k_got.cpu(), kc.cpu())  # the row was appended
    # an append row outside the buffer: q written, no key/value row
    q2 = torch.zeros_like(q_got)
    k2, v2 = kc.clone(), vc.clone()
    shadowkv.linear_qkv_rope_append(x.view(B, k), w_rope, Hq, Hk, pos, csg, q2, k2, v2,
                                    torch.tensor([buf], device=gpu), b_rope)
    torch.cuda.synchronize()
    assert torch.equal(q2.cpu(), q_want.cpu())
    assert torch.equal(k2.cpu(), kc.cpu()) and torch.equal(v2.cpu(), vc.cpu())


def test_linear_qkv_rope_append_rejects(gpu):
    from shadowkv_amd import _lib
    Hq, Hk, k, D = 4, 2, 64, 128
    n = (Hq + 2 * Hk) * D
    w = torch.zeros(n, k, dtype=torch.bfloat16, device=gpu)
    cs = torch.zeros(10, 128, dtype=torch.bfloat16, device=gpu)
    row = torch.zeros(1, dtype=torch.int64, device=gpu)
    x9 = torch.zeros(9, k, dtype=torch.bfloat16, device=gpu)  # one row past the epilogue's limit
    kc = torch.zeros(9, Hk, 4, D, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="at most 8"):
        shadowkv.linear_qkv_rope_append(x9, w, Hq, Hk, torch.zeros(9, dtype=torch.int64, device=gpu), cs,
                                        torch.empty(9, Hq, D, dtype=torch.bfloat16, device=gpu), kc, kc.clone(), row)
    rc = _lib.lib().skv_linear_qkv_rope_append(x9.data_ptr(), k, w.data_ptr(), k, None, 9, k, Hq, Hk, row.data_ptr(),
                                               cs.data_ptr(), 128, 10, 0, kc.data_ptr(), Hq * D, kc.data_ptr(),
                                               kc.data_ptr(), Hk * 4 * D, 4 * D, D, row.data_ptr(), 4, None)
    assert rc == 2  # SKV_EUNSUPPORTED
    with pytest.raises(ValueError, match="shape mismatch"):  # weight rows for other head counts
        shadowkv.linear_qkv_rope_append(x9[:2], w[:-128], Hq, Hk, row.repeat(2), cs,
                                        torch.empty(2, Hq, D, dtype=torch.bfloat16, device=gpu), kc[:2],
                                        kc[:2].clone(), row)
