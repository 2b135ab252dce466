"""The allocation-free attention entry point (skv_sparse_attn_decode_noalloc, split partials in
the library's per-GPU device array) against skv_sparse_attn_decode with a caller workspace: the
same kernels in the same order, so bit-identical outputs, on two calls in a row (the second with
a smaller input, so it runs over the first call's leftover partials), also with a device-resident
length; sizes beyond the array are refused."""
import pytest
import torch

import oracle
from shadowkv_amd import _lib

pytestmark = pytest.mark.gpu


def _case(gpu, B, Hq, Hkv, buf, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    q = torch.randn(B, Hq, 128, generator=g, device=gpu).to(torch.bfloat16)
    k = torch.randn(B, Hkv, buf, 128, generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn(B, Hkv, buf, 128, generator=g, device=gpu).to(torch.bfloat16)
    return q, k, v


def _run_ws(q, k, v, L, L_dev, out):
    B, Hq = q.shape[0], q.shape[1]
    lib = _lib.lib()
    nbytes = lib.skv_sparse_attn_workspace_bytes(B, Hq, L)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=q.device)  # zero-filled before first use
    rc = lib.skv_sparse_attn_decode(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(), k.stride(0),
                                    k.stride(1), k.stride(2), B, Hq, k.shape[1], 128, L,
                                    L_dev.data_ptr() if L_dev is not None else None, 128 ** -0.5, ws.data_ptr(),
                                    nbytes, out.data_ptr(), out.stride(0), out.stride(1),
                                    torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.last_error()
    return ws


def _run_noalloc(q, k, v, L, L_dev, out):
    B, Hq = q.shape[0], q.shape[1]
    return _lib.lib().skv_sparse_attn_decode_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), k.stride(2), B,
        Hq, k.shape[1], 128, L, L_dev.data_ptr() if L_dev is not None else None, 128 ** -0.5, out.data_ptr(),
        out.stride(0), out.stride(1), torch.cuda.current_stream().cuda_stream)


def test_noalloc_attention_matches_workspace_entry(gpu):
    # (batch, query heads, kv heads, buffer rows, length, device length): the decode step's shape
    # (batch 8, L = 2497 + 100), then a smaller one with a device-resident live length, then GLM's
    # 16 query heads per kv head
    cases = [(8, 32, 8, 2700, 2597, None), (2, 32, 8, 800, 800, 613), (4, 32, 2, 2600, 2498, None)]
    for i, (B, Hq, Hkv, buf, L, live) in enumerate(cases):
        print(f"noalloc attention call {i}: batch {B} heads {Hq}/{Hkv} L {L} live {live}", flush=True)
        q, k, v = _case(gpu, B, Hq, Hkv, buf, 40 + i)
        L_dev = torch.tensor([live], dtype=torch.int32, device=gpu) if live else None
        want = torch.full((B, Hq, 128), 9.0, dtype=torch.bfloat16, device=gpu)
        got = torch.full((B, Hq, 128), 7.0, dtype=torch.bfloat16, device=gpu)
        ws = _run_ws(q, k, v, L, L_dev, want)
        rc = _run_noalloc(q, k, v, L, L_dev, got)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), i
        n = live or L
        ref = oracle.sparse_attention(q.cpu(), k.cpu(), v.cpu(), n)
        torch.testing.assert_close(got.cpu().float(), ref.float(), rtol=2e-2, atol=2e-2)
        del ws


def test_noalloc_attention_refuses_more_than_its_scratch(gpu):
    lib = _lib.lib()
    cap = lib.skv_sparse_attn_noalloc_max_bytes()
    assert cap == 32 << 20
    B, Hq, L = 64, 32, 262144
    assert lib.skv_sparse_attn_workspace_bytes(B, Hq, L) > cap
    q = torch.zeros(B, Hq, 128, dtype=torch.bfloat16, device=gpu)
    kv = torch.zeros(1, 8, 8, 128, dtype=torch.bfloat16, device=gpu)
    out = torch.empty(B, Hq, 128, dtype=torch.bfloat16, device=gpu)
    rc = lib.skv_sparse_attn_decode_noalloc(q.data_ptr(), 0, 128, kv.data_ptr(), kv.data_ptr(), 0, 0, 128, B, Hq, 8,
                                            128, L, None, 0.1, out.data_ptr(), 4096, 128,
                                            torch.cuda.current_stream().cuda_stream)
    assert rc == 2 and "scratch" in _lib.last_error()
