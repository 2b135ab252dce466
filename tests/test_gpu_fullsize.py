"""Parity at the benchmarked sizes (the decode workloads and the rebuild microbenchmark).

* The low-rank key rebuild + RoPE at U [B*8, 122880, 160] per head, B in {1, 8, 32, 48} (U up to
  15 GB, per-head offsets beyond 2^31 elements): every (b, h) row against a float32 torch
  reference of the same product on the device (one bf16 rounding, then torch's bf16 RoPE), and
  sampled rows, the first and the last among them, against the oracle on the CPU.
* One decode step of the Llama-3.1-8B shape at batch 8, ctx 122880 (two pipelined lanes of 4
  sequences), of the GLM-4-9B shape at batch 4, ctx 262144 and of the Llama-3-8B-1M shape at
  batch 1, ctx 1048576, budget 16384: the first, a middle and the last layer of every lane
  against oracle.decode_layer_step from the device's own scores (selection, offsets, hit
  counts, slot ids and value buffer bit-exact; keys and attention within rtol/atol 2e-2).
  The step checked is the second one, so the generated tail holds a token of the first.
* The same Llama-3.1-8B step from a prompt state built by the device encoder (two layers), with
  the value store in device memory (batch 8 and batch 24), and with a chunk pool of 2048 slots
  after 12 steps that fill it (against oracle.decode_layer_step_pooled from the recorded tables).
* The prefill's rank-160 factors at ctx 122880 against torch.linalg.svd on the device.
"""
import gc
import math

import pytest
import torch

import oracle
from shadowkv_amd import decode_model
from shadowkv_amd.kernels import shadowkv
from shadowkv_amd.models.kvcache.shadow import low_rank_factors
from shadowkv_amd.models.tensor_op import build_cos_sin_cache
from tests.decode_harness import LayerProbe, assert_bf16_close, check_layer_record, check_pooled_layer_record

pytestmark = pytest.mark.gpu

CTX = 122880


def _say(msg):
    print(msg, flush=True)


def _release():
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch._C._host_emptyCache()  # pinned host blocks of the value stores


# ------------------------------------------------------------------ rebuild microbenchmark sizes

@pytest.fixture(scope="module")
def u_per_head(gpu):
    """U [48*8, 122880, 160] bf16 ~ N(0, 1), the largest batch of the rebuild microbenchmark."""
    g = torch.Generator(device=gpu).manual_seed(2024)
    u = torch.empty(48 * 8, CTX, 160, dtype=torch.bfloat16, device=gpu)
    for i in range(0, u.shape[0], 32):
        u[i:i + 32].normal_(generator=g)
    yield u
    del u
    _release()


def _rope_half_torch(x, cs):
    """torch's bf16 (x*cos) + (rotate_half(x)*sin), each operation rounded to bf16."""
    h = x.shape[-1] // 2
    c = torch.cat((cs[..., :h], cs[..., :h]), dim=-1)
    s = torch.cat((cs[..., h:], cs[..., h:]), dim=-1)
    rot = torch.cat((-x[..., h:], x[..., :h]), dim=-1)
    return (x * c) + (rot * s)


@pytest.mark.parametrize("B", [1, 8, 32, 48])
def test_rebuild_microbench_sizes(gpu, u_per_head, B):
    """U and SV ~ N(0, 1) as the microbenchmark specifies, so rebuilt keys have standard deviation
    sqrt(rank) (~12.6): the pre-RoPE product (skv_batch_gather_gemm, per-head U as rows of a
    [B*8, ctx, R] batch) is checked within one bf16 rounding step of the float32 product, and the
    rotated keys within rtol 2e-2 / atol 2e-2 after scaling by 1/sqrt(rank) to unit variance (at
    |k| ~ 12 one bf16 step is 0.0625, above an unscaled atol)."""
    H, S, c, R, start = 8, 256, 8, 160, 448
    _say(f"rebuild at U [{B}*8, {CTX}, {R}] per head, S={S}")
    g = torch.Generator(device=gpu).manual_seed(B)
    U = u_per_head[:B * H].view(B, H, CTX, R)
    SV = torch.randn(H, 128, R, generator=g, device=gpu).to(torch.bfloat16)  # shared across the batch
    ids = torch.rand(B * H, CTX // c, generator=g, device=gpu).argsort(dim=-1)[:, :S].sort(dim=-1).values
    ids = ids.view(B, H, S).contiguous()
    # half the rows all misses, half with the reference's 60% hit setting (154 of 256 chunks in place)
    cnts = torch.where(torch.rand(B * H, generator=g, device=gpu) < 0.5, 0, 154).to(torch.int32)
    cs = build_cos_sin_cache(CTX, 500000.0, 128, device=gpu)
    buf = start + S * c + 96
    cache0 = torch.randn(B, H, buf, 128, generator=g, device=gpu).to(torch.bfloat16)
    cache = cache0.clone()
    shadowkv.rebuild_k_rope(U, SV, ids, cnts, cs, cache, start, c)
    # the plain rebuild (no RoPE) through the reference's batch_gather_gemm entry point
    plain = torch.full((B * H, S * c, 128), 3.0, dtype=torch.bfloat16, device=gpu)
    shadowkv.batch_gather_gemm(U.view(B * H, CTX, R), SV.repeat(B, 1, 1).contiguous(), None, None,
                               ids.view(B * H, S).to(torch.int32), plain, B * H, 1, CTX, 128, R, S * c, CTX, c, cnts)
    torch.cuda.synchronize()
    # every row: the float32 product on the device, one rounding, torch's bf16 RoPE
    pos = (ids.unsqueeze(-1) * c + torch.arange(c, device=gpu)).view(B * H, S * c)
    rows = torch.stack([U[b, h][pos[b * H + h]] for b in range(B) for h in range(H)])  # [BH, S*c, R]
    k = torch.matmul(rows.float(), SV.float().transpose(-1, -2).contiguous().repeat(B, 1, 1)).to(torch.bfloat16)
    del rows
    r_idx = torch.arange(S * c, device=gpu).view(1, -1)
    is_miss = (r_idx >= cnts.view(-1, 1) * c).unsqueeze(-1)  # [BH, S*c, 1]
    assert torch.equal(torch.where(is_miss, torch.full_like(plain, 3.0), plain), torch.full_like(plain, 3.0)), \
        "plain rebuild wrote hit rows"
    assert_bf16_close(torch.where(is_miss, plain, k), k, floor=1e-4, what=f"pre-RoPE rebuild B={B}")
    want = _rope_half_torch(k, cs[pos]).view(B, H, S * c, 128)
    del k, plain
    is_miss = is_miss.view(B, H, S * c, 1)
    got = cache[:, :, start:start + S * c]
    assert torch.equal(cache[:, :, :start], cache0[:, :, :start])
    assert torch.equal(cache[:, :, start + S * c:], cache0[:, :, start + S * c:])
    assert torch.equal(torch.where(is_miss, cache0[:, :, start:start + S * c], got), cache0[:, :, start:start + S * c]), \
        "hit rows were written"
    scale = 1.0 / math.sqrt(R)
    torch.testing.assert_close(torch.where(is_miss, got, want).float() * scale, want.float() * scale, rtol=2e-2,
                               atol=2e-2)
    # sampled rows against the oracle on the CPU (first, last, two more)
    cs_cpu = oracle.build_cos_sin_cache(CTX, 500000.0)
    assert torch.equal(cs_cpu, cs.cpu())
    for r in sorted({0, B * H - 1, (B * H) // 2, (7 * B * H) // 11}):
        b, h = divmod(r, H)
        u_row = torch.zeros(1, CTX, R, dtype=torch.bfloat16)
        u_row[0, pos[r].cpu()] = U[b, h][pos[r]].cpu()
        ref = cache0[b:b + 1, h:h + 1].cpu().clone()
        oracle.rebuild_k_rope(u_row, SV[h:h + 1].cpu().unsqueeze(0), ids[b:b + 1, h:h + 1].cpu(), cnts[r:r + 1].cpu(),
                              cs_cpu, c, ref, start)
        torch.testing.assert_close(cache[b, h].cpu().float() * scale, ref[0, 0].float() * scale, rtol=2e-2, atol=2e-2)
        m = start + int(cnts[r]) * c
        assert torch.equal(cache[b, h, :m].cpu(), ref[0, 0, :m])


# ------------------------------------------------------------------ decode workloads

def _decode_and_check(shape, batch, ctx, budget, layers_checked, gpu, state="synthetic", value_store="host"):
    # The value stores of these workloads would take 20-64 GiB of pinned host memory, close to what
    # one process may pin on the MI355X hosts (about 65 GiB): the layers share two host stores (the
    # oracle reads the same store the device fetched from), and blocks cached by earlier tests are
    # released first.
    _release()
    lanes = decode_model.auto_lanes(shape, batch, budget, value_store)
    _say(f"{shape.name} batch {batch} ctx {ctx} budget {budget}: building ({lanes} lane(s), {state} state, "
         f"{value_store} value store)")
    dec = decode_model.SyntheticDecoder(shape, batch, ctx, sparse_budget=budget, decode_len=8, lanes=lanes,
                                        seed=7, state=state, host_stores=2, value_store=value_store)
    tok = torch.randint(0, shape.vocab, (batch, 1), device=gpu, generator=torch.Generator(device=gpu).manual_seed(1))
    tok = dec.decode_step(tok)  # the first step; the checked one follows
    probe = LayerProbe(dec, layers_checked)
    dec.decode_step(tok)
    torch.cuda.synchronize()
    _say(f"{shape.name}: step done, checking {len(probe.records)} lane-layers against the oracle")
    cs = dec.cos_sin.cpu()
    for (i, layer), rec in sorted(probe.records.items()):
        res = check_layer_record(rec, dec.lanes[i].cache, layer, cs, what=f"{shape.name} lane {i} layer {layer}")
        _say(f"  lane {i} layer {layer}: hits {int(res['cnts'].sum())} of {res['cnts'].size * dec.cache.select_sets}, ok")
    assert len(probe.records) == len(dec.lanes) * len(set(layers_checked))
    del dec, probe
    _release()


def test_decode_llama31_8b_batch8_ctx122880(gpu):
    _decode_and_check(decode_model.LLAMA31_8B, 8, CTX, 2048, [0, 15, 31], gpu)


def test_decode_llama31_8b_batch8_ctx122880_device_store(gpu):
    """The same step with the value store in device memory: one lane, the attention reading the
    selected values in place from the store (checked through the buffer the gather would build)."""
    _decode_and_check(decode_model.LLAMA31_8B, 8, CTX, 2048, [0, 15, 31], gpu, value_store="device")


def test_decode_llama31_8b_batch24_ctx122880_device_store(gpu):
    """Batch 24 (the batch of the reference's published 122K figure) with the value store in device
    memory: one lane of 192 (b, h) rows, so the selection takes its one-workgroup-per-row path and
    the projections run on hipBLASLt; the first and last layer against the oracle."""
    _decode_and_check(decode_model.LLAMA31_8B, 24, CTX, 2048, [0, 31], gpu, value_store="device")


def test_decode_llama31_8b_batch8_ctx122880_pool(gpu):
    """The batch-8 ctx-122880 step with a chunk pool of 2048 slots per (b, h) and layer, after 12
    steps that fill it (about 13% of a step's chunks then hit): every lane's first and last layer
    against the oracle's pooled step from the recorded tables (two lanes, each lane's misses
    fetched and rebuilt into their slots by one launch on its own stream)."""
    shape, batch, ctx, budget, P = decode_model.LLAMA31_8B, 8, CTX, 2048, 2048
    _release()
    lanes = decode_model.auto_lanes(shape, batch, budget,
                                    miss_fraction=decode_model.pool_miss_fraction(P, ctx // 8))
    _say(f"{shape.name} batch {batch} ctx {ctx} budget {budget}: building ({lanes} lane(s), pool of {P} slots)")
    dec = decode_model.SyntheticDecoder(shape, batch, ctx, sparse_budget=budget, decode_len=16, lanes=lanes, seed=7,
                                        host_stores=2, chunk_cache=P)
    assert all(lane.cache.one_stream_active() for lane in dec.lanes)
    tok = torch.randint(0, shape.vocab, (batch, 1), device=gpu, generator=torch.Generator(device=gpu).manual_seed(1))
    for _ in range(12):
        tok = dec.decode_step(tok)
    probe = LayerProbe(dec, [0, 31])
    dec.decode_step(tok)
    torch.cuda.synchronize()
    _say(f"{shape.name}: pooled step done, checking {len(probe.records)} lane-layers against the oracle")
    cs = dec.cos_sin.cpu()
    for (i, layer), rec in sorted(probe.records.items()):
        res = check_pooled_layer_record(rec, dec.lanes[i].cache, layer, cs, what=f"pool lane {i} layer {layer}")
        hits = int(res["cnts"].sum())
        _say(f"  lane {i} layer {layer}: hits {hits} of {res['cnts'].size * dec.cache.select_sets}, ok")
        assert hits > 0
    assert len(probe.records) == len(dec.lanes) * 2
    del dec, probe
    _release()


def test_decode_glm4_9b_batch4_ctx262144(gpu):
    _decode_and_check(decode_model.GLM4_9B, 4, 262144, 2048, [0, 20, 39], gpu)


def test_decode_llama3_8b_1m_batch1_ctx1048576(gpu):
    _decode_and_check(decode_model.LLAMA3_8B_1M, 1, 1048576, 16384, [0, 15, 31], gpu)


def test_decode_llama31_8b_batch8_ctx122880_encoded_state(gpu):
    """The Llama-3.1-8B batch-8 ctx-122880 step from a prompt state built by the device encoder
    (decode_model.encode_state: rank-160 keys plus noise through get_svd, RoPE, prefill_kv_cache),
    two layers of every lane against the oracle."""
    from dataclasses import replace
    _decode_and_check(replace(decode_model.LLAMA31_8B, layers=2), 8, CTX, 2048, [0, 1], gpu, state="encoded")


# ------------------------------------------------------------------ prefill factors at size

def test_low_rank_factors_ctx122880_vs_svd(gpu):
    """The encoder's rank-160 factors of one layer's pre-RoPE keys [122880, 8*128] (the single-layer
    workload's recipe: A(ctx x 160).B(160 x 1024) + 0.05 N(0,1), A and B ~ N(0, 1/sqrt(160))) against
    the reference's method, a full float32 SVD (shadow.py:426), on the device: the rank-160
    reconstructions U.SV and the singular values."""
    g = torch.Generator(device=gpu).manual_seed(5)
    R = 160
    A = torch.randn(CTX, R, generator=g, device=gpu) / math.sqrt(math.sqrt(R))
    Bm = torch.randn(R, 1024, generator=g, device=gpu) / math.sqrt(math.sqrt(R))
    k = (A @ Bm + 0.05 * torch.randn(CTX, 1024, generator=g, device=gpu)).to(torch.bfloat16).unsqueeze(0)
    del A, Bm
    u, svt = low_rank_factors(k, R)
    rec = torch.matmul(u, svt)
    uu, s, vh = torch.linalg.svd(k.float(), full_matrices=False)
    ref = torch.matmul(uu[:, :, :R] * s[:, None, :R], vh[:, :R])
    rel = ((rec - ref).norm() / ref.norm()).item()
    _say(f"low-rank factors: relative difference of the reconstructions {rel:.2e}")
    assert rel < 1e-3
    s_gram = svt.norm(dim=-1)  # rows of diag(s) V^T have norm s
    torch.testing.assert_close(s_gram, s[:, :R], rtol=1e-3, atol=1e-3)
    del k, u, svt, rec, uu, s, vh, ref
    _release()
