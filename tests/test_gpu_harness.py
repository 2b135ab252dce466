"""The random-init decode harness: in-place q/k RoPE on the fused QKV rows and multi-lane decode
(regression for an output buffer smaller than the input's stride pattern)."""
from dataclasses import replace

import pytest
import torch

import oracle
from shadowkv_amd import decode_model

pytestmark = pytest.mark.gpu


def test_inplace_rope_on_qkv_rows(gpu):
    shape = replace(decode_model.LLAMA31_8B, layers=1)
    b, D, hq, hk = 3, 128, shape.heads, shape.kv_heads
    cos_sin = oracle.build_cos_sin_cache(4096, shape.rope_theta)
    qkv = torch.randn(b, 1, (hq + 2 * hk) * D).to(torch.bfloat16)
    pos = torch.tensor([17, 4000, 999])
    model = types_ns(cos_sin.to(gpu), shape)
    q, k, _ = qkv.to(gpu).split([hq * D, hk * D, hk * D], dim=-1)
    qr, kr = decode_model.SyntheticDecoder._rope_for(model, None)(q, k, pos.to(gpu))
    torch.cuda.synchronize()
    for x, got, h in ((qkv[..., :hq * D], qr, hq), (qkv[..., hq * D:(hq + hk) * D], kr, hk)):
        xv = x.reshape(b, h, D)
        cs = cos_sin[pos].unsqueeze(1)
        want = oracle.rope_half_split(xv, cs[..., :64].expand(-1, h, -1), cs[..., 64:].expand(-1, h, -1))
        assert torch.equal(got.reshape(b, h, D).cpu(), want)


def types_ns(cos_sin, shape):
    import types
    return types.SimpleNamespace(cos_sin=cos_sin, shape=shape)


@pytest.mark.parametrize("lanes", [1, 2, 4])
def test_multi_lane_decode_runs(gpu, lanes):
    print(f"harness lanes={lanes}", flush=True)
    shape = replace(decode_model.LLAMA31_8B, layers=2, vocab=1024)
    model = decode_model.SyntheticDecoder(shape, 4, 16384, decode_len=8, lanes=lanes)
    tok = torch.randint(0, shape.vocab, (4, 1), device=gpu)
    for _ in range(3):
        tok = model.decode_step(tok)
    torch.cuda.synchronize()
    assert tok.shape == (4, 1) and int(tok.min()) >= 0 and int(tok.max()) < shape.vocab
    for lane in model.lanes:
        assert lane.cache.gen_offset == 3
        assert int(lane.cache.cnts.min()) >= 0 and int(lane.cache.cnts.max()) <= lane.cache.select_sets
