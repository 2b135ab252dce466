"""The sparse attention's one-launch merge (SKV_ATTN_FUSED=1: the last split workgroup of each
(sequence, kv head) row merges the row's partials in its XCD's L2) against the default two-launch
merge and the oracle, over repeated calls, device lengths, graph replays and the paged (chunk
pool) form."""
import numpy as np
import pytest
import torch

import oracle
from shadowkv_amd.kernels import shadowkv
from shadowkv_amd.streams import capture_graph

pytestmark = pytest.mark.gpu

RTOL = 2e-2
ATOL = 2e-2
ARRIVAL_BYTES = 4096 * 4  # the arrival counters at the head of the workspace


def _say(msg):
    print(msg, flush=True)


def _qkv(gpu, B, Hq, Hk, buf, seed):
    g = torch.Generator().manual_seed(seed)
    K = torch.randn(B, Hk, buf, 128, generator=g).to(torch.bfloat16)
    V = torch.randn(B, Hk, buf, 128, generator=g).to(torch.bfloat16)
    q = torch.randn(B, Hq, 128, generator=g).to(torch.bfloat16)
    return q.to(gpu), K.to(gpu), V.to(gpu)


def _attn(q, K, V, L, ws, **kw):
    out = torch.full((q.shape[0], q.shape[1], 128), 5.0, dtype=torch.bfloat16, device=q.device)
    shadowkv.sparse_attn_decode(q, K, V, L, out, ws, **kw)
    return out


def _one_ulp_close(a: torch.Tensor, b: torch.Tensor):
    """Two fp32 merges of the same partials in different orders, each rounded to bf16 once."""
    x, y = a.float(), b.float()
    m = torch.maximum(x.abs(), y.abs()).clamp_min(2.0 ** -126)
    ulp = torch.exp2(torch.floor(torch.log2(m)) - 7)
    bad = (x - y).abs() > ulp + 1e-6
    assert not bad.any(), f"{int(bad.sum())} beyond one bf16 step, max diff {(x - y).abs().max():.3e}"


def _counters_zero(ws):
    assert int(ws[:ARRIVAL_BYTES].count_nonzero()) == 0, "arrival counters left nonzero"


# (batch, query heads, kv heads, length): the decode lane (32 rows x 4 heads), batch 8, GLM-4-9B
# (8 rows x 16 heads), two 16-row shapes of 8 query heads per kv head, one split per row, 64
# splits of 128 keys, and rows that are not a multiple of 8.
SHAPES = [(4, 32, 8, 2597), (8, 32, 8, 2600), (4, 32, 2, 2497), (2, 64, 8, 1000), (8, 16, 2, 700), (1, 8, 8, 1),
          (2, 32, 8, 100), (1, 64, 8, 8192), (8, 32, 8, 4096), (3, 12, 4, 1500), (5, 20, 2, 333)]


@pytest.mark.parametrize("B,Hq,Hk,L", SHAPES)
def test_fused_merge_matches_two_launch_and_oracle(gpu, monkeypatch, B, Hq, Hk, L):
    _say(f"fused attention B={B} Hq={Hq} Hk={Hk} L={L}")
    monkeypatch.setenv("SKV_ATTN_FUSED", "1")
    q, K, V = _qkv(gpu, B, Hq, Hk, L + 13, 900 + L)
    ws = shadowkv.sparse_attn_workspace(B, Hq, L, gpu)
    fused = _attn(q, K, V, L, ws)
    torch.cuda.synchronize()
    _counters_zero(ws)
    monkeypatch.setenv("SKV_ATTN_FUSED", "0")
    two = _attn(q, K, V, L, ws)
    torch.cuda.synchronize()
    _one_ulp_close(fused, two)
    want = oracle.sparse_attention(q.cpu(), K.cpu(), V.cpu(), L)
    torch.testing.assert_close(fused.cpu().float(), want.float(), rtol=RTOL, atol=ATOL)
    chk = shadowkv.sparse_attn_xcd_check()
    _say(f"xcd check {chk}")
    assert chk["state"] == 1 and chk["misplaced"] == 0


@pytest.mark.parametrize("split", ["64", "128"])
def test_fused_merge_repeated_calls_and_device_lengths(gpu, monkeypatch, split):
    """One workspace over many calls: a device length gives the host length's result bit for bit
    (both take the one-launch merge with the same split size) at split boundaries, and the arrival
    counters are back at zero after every call."""
    monkeypatch.setenv("SKV_ATTN_SPLIT", split)
    monkeypatch.setenv("SKV_ATTN_FUSED", "1")
    B, Hq, Hk = 2, 32, 8
    Lmax = 64 * int(split)  # 64 splits: the longest row the one-launch merge takes
    q, K, V = _qkv(gpu, B, Hq, Hk, Lmax, 31)
    ws = shadowkv.sparse_attn_workspace(B, Hq, Lmax, gpu)
    ldev = torch.zeros(1, dtype=torch.int32, device=gpu)
    k = int(split)
    for L in (1, k - 1, k, k + 1, 5 * k + 3, Lmax - 1, Lmax, 2 * k):
        _say(f"fused device length {L} split {split}")
        ldev.fill_(L)
        got = _attn(q, K, V, Lmax, ws, kv_len_dev=ldev)
        want = _attn(q, K, V, L, ws)
        torch.cuda.synchronize()
        _counters_zero(ws)
        assert torch.equal(got, want), L
        ref = oracle.sparse_attention(q.cpu(), K.cpu(), V.cpu(), L)
        torch.testing.assert_close(got.cpu().float(), ref.float(), rtol=RTOL, atol=ATOL)


def test_fused_merge_graph_replays(gpu, monkeypatch):
    """A captured fused attention replayed four times, with eager fused calls on the same workspace
    and a host synchronization between replays: every replay equals the eager result bit for bit."""
    monkeypatch.setenv("SKV_ATTN_FUSED", "1")
    B, Hq, Hk, L = 4, 32, 8, 2597
    q, K, V = _qkv(gpu, B, Hq, Hk, L, 77)
    ws = shadowkv.sparse_attn_workspace(B, Hq, L, gpu)
    ldev = torch.full((1,), L, dtype=torch.int32, device=gpu)
    eager = _attn(q, K, V, L, ws, kv_len_dev=ldev)
    torch.cuda.synchronize()
    out = torch.empty_like(eager)
    g = torch.cuda.CUDAGraph()
    with capture_graph(g, gpu):
        shadowkv.sparse_attn_decode(q, K, V, L, out, ws, kv_len_dev=ldev)
    for r in range(4):
        _say(f"fused graph replay {r}")
        out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), r
        _counters_zero(ws)
        other = _attn(q, K, V, L - 100 * r, ws)  # eager work on the same workspace between replays
        torch.cuda.synchronize()
        ref = oracle.sparse_attention(q.cpu(), K.cpu(), V.cpu(), L - 100 * r)
        torch.testing.assert_close(other.cpu().float(), ref.float(), rtol=RTOL, atol=ATOL)


def test_fused_merge_paged(gpu, monkeypatch):
    """The chunk-pool form (selected chunks read through a slot list) on the one-launch merge equals
    the two-launch merge to one bf16 step, and the oracle on the gathered keys."""
    monkeypatch.setenv("SKV_ATTN_FUSED", "1")
    B, Hq, Hk, c, S, P, sp0, gen = 2, 32, 8, 8, 64, 96, 40, 5
    rows = B * Hk
    buf = sp0 + P * c + gen
    L = sp0 + S * c + gen
    q, K, V = _qkv(gpu, B, Hq, Hk, buf, 55)
    rng = np.random.default_rng(3)
    slots = np.stack([rng.permutation(P)[:S] for _ in range(rows)]).astype(np.int32)
    slot_list = torch.from_numpy(slots).view(B, Hk, S).to(gpu)
    ws = shadowkv.sparse_attn_workspace(B, Hq, L, gpu)
    pool = (slot_list, sp0, S, c, P)
    fused = _attn(q, K, V, L, ws, pool=pool)
    torch.cuda.synchronize()
    _counters_zero(ws)
    monkeypatch.setenv("SKV_ATTN_FUSED", "0")
    two = _attn(q, K, V, L, ws, pool=pool)
    torch.cuda.synchronize()
    _one_ulp_close(fused, two)
    idx = torch.cat([torch.arange(sp0).expand(rows, -1),
                     (torch.from_numpy(slots).long()[:, :, None] * c + sp0 + torch.arange(c)).reshape(rows, -1),
                     torch.arange(sp0 + P * c, buf).expand(rows, -1)], dim=1).view(B, Hk, -1)
    Kg = torch.gather(K.cpu(), 2, idx[..., None].expand(-1, -1, -1, 128))
    Vg = torch.gather(V.cpu(), 2, idx[..., None].expand(-1, -1, -1, 128))
    ref = oracle.sparse_attention(q.cpu(), Kg, Vg, L)
    torch.testing.assert_close(fused.cpu().float(), ref.float(), rtol=RTOL, atol=ATOL)
