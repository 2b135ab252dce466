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
