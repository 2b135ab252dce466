"""The value fetch of the misses and the key rebuild as one launch (skv_fetch_misses_rebuild_k_rope)
against the two calls it replaces (gather_copy_with_offsets(..., misses_only=True) and
rebuild_k_rope): value and key buffers bit-identical, for every rebuild tile shape (64-, 128- and
256-row workgroups, so 2- and 4-wave fused grids), both rotary layouts, rows whose chunks are all
hits or all misses, and rebuild workgroups capped so that they loop over the tiles; and one-lane
decoders with the one-launch step against the two-stream one."""
from dataclasses import replace

import pytest
import torch

from shadowkv_amd import decode_model
from shadowkv_amd.kernels import shadowkv
from shadowkv_amd.models.tensor_op import build_cos_sin_cache, build_glm_cos_sin_cache

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,H,S,glm,R", [(1, 8, 256, False, 160), (4, 8, 256, False, 160), (8, 8, 256, False, 160),
                                         (4, 2, 256, True, 160), (1, 8, 2048, False, 160), (3, 2, 40, True, 160),
                                         (8, 8, 256, False, 192), (2, 2, 64, True, 96)])
def test_one_launch_equals_fetch_then_rebuild(gpu, B, H, S, glm, R):
    """(rank 192 at batch 8: the fused launch takes 128-row tiles where the rebuild alone takes 256)"""
    _one_launch_case(gpu, B, H, S, glm, R, 8, B * 100 + H * 10 + S)


def test_one_launch_random_shapes(gpu):
    """The same equality on 10 seeded random shapes: batch 1-4, 1-8 heads, 1-600 chunks of 4, 8 or
    16 rows, ranks 8-192, both rotary layouts."""
    import numpy as np
    rng = np.random.default_rng(79)
    for case in range(10):
        B, H = int(rng.integers(1, 5)), int(rng.choice([1, 2, 3, 8]))
        S, c = int(rng.integers(1, 601)), int(rng.choice([4, 8, 16]))
        R, glm = 8 * int(rng.integers(1, 25)), bool(rng.integers(0, 2))
        _one_launch_case(gpu, B, H, S, glm, R, c, 9000 + case)


def _one_launch_case(gpu, B, H, S, glm, R, c, seed):
    print(f"fetch+rebuild one launch B={B} H={H} S={S} glm={glm} rank={R} chunk={c}", flush=True)
    D = 128
    chunks = max(4 * S, 2048)
    ctx = chunks * c
    sparse_start, buf_len = 64, 64 + S * c + 32
    g = torch.Generator().manual_seed(seed)
    gd = torch.Generator(device=gpu).manual_seed(seed)
    values = torch.randn(B, H, chunks, c * D, generator=g).to(torch.bfloat16).pin_memory()
    U = torch.randn(B, H, ctx, R, generator=gd, device=gpu).to(torch.bfloat16)
    SV = (torch.randn(H, D, R, generator=gd, device=gpu) / R ** 0.5).to(torch.bfloat16)
    cos_sin = (build_glm_cos_sin_cache(ctx + 64, 10000.0, device=gpu) if glm
               else build_cos_sin_cache(ctx + 64, 500000.0, D, device=gpu))
    pos = torch.stack([torch.randperm(chunks, generator=g)[:S].sort().values for _ in range(B * H)]).view(B, H, S)
    cnts = torch.randint(0, S + 1, (B * H,), generator=g, dtype=torch.int32)
    cnts[0] = 0  # a row of misses only
    if B * H > 1:
        cnts[-1] = S  # and one of hits only
    offsets = pos.view(B * H, S).to(torch.int32).clone()  # misses: their chunk ids (hit entries unused here)
    v0 = torch.randn(B, H, buf_len, D, generator=gd, device=gpu).to(torch.bfloat16)
    k0 = torch.randn(B, H, buf_len, D, generator=gd, device=gpu).to(torch.bfloat16)
    pos_d, cnts_d, off_d = pos.to(gpu), cnts.to(gpu), offsets.view(-1).to(gpu)
    stride = buf_len * D
    va, ka = v0.clone(), k0.clone()
    shadowkv.gather_copy_with_offsets(values, va, None, off_d, cnts_d, None, B, H, chunks * c * D, S * c * D,
                                      sparse_start * D, stride, S, misses_only=True)
    shadowkv.rebuild_k_rope(U, SV, pos_d, cnts_d, cos_sin, ka, sparse_start, c)
    # rebuild workgroups: one per tile, or capped at 8 / 48 / 1000 (looping over the tiles where the
    # kernel instance supports it: the half-split rank-160 128-row tiles of 32 heads x 2048 rows)
    for cap in (0, 8, 48, 1000):
        vb, kb = v0.clone(), k0.clone()
        shadowkv.fetch_misses_rebuild_k_rope(values, vb, off_d, cnts_d, chunks * c * D, sparse_start * D, stride, U,
                                             SV, pos_d, cos_sin, kb, sparse_start, c, rebuild_workgroups=cap)
        torch.cuda.synchronize()
        assert torch.equal(vb.view(torch.int16), va.view(torch.int16)), cap
        assert torch.equal(kb.view(torch.int16), ka.view(torch.int16)), cap
    # the launch did write: every miss chunk of row 0 now holds its host chunk
    r0 = vb[0, 0, sparse_start:sparse_start + S * c].reshape(S, c * D).cpu()
    assert torch.equal(r0.view(torch.int16), values[0, 0, pos[0, 0]].view(torch.int16))
    assert not torch.equal(kb.view(torch.int16), k0.view(torch.int16))


@pytest.mark.parametrize("B,H,S,P,glm,R,c", [(4, 8, 256, 2048, False, 160, 8), (1, 8, 256, 512, False, 160, 8),
                                               (4, 2, 256, 384, True, 160, 8), (2, 3, 40, 40, False, 96, 16),
                                               (3, 2, 100, 333, True, 64, 4)])
def test_one_launch_slots_equals_gather_then_rebuild(gpu, B, H, S, P, glm, R, c):
    """The chunk pool's one-launch fetch + rebuild (fetch_misses_rebuild_k_rope_slots) against the
    two calls it replaces (gather_copy_misses_to_slots, rebuild_k_rope with miss_slot): value and
    key buffers bit-identical, pool rows of misses only and of hits only, rebuild workgroups
    capped or not; slots the miss list does not name are left untouched."""
    _one_launch_slots_case(gpu, B, H, S, P, glm, R, c, B * 1000 + H * 100 + S + P)


def test_one_launch_slots_random_shapes(gpu):
    """The same equality on 8 seeded random pools: batch 1-4, 1-8 heads, 1-300 selected chunks of
    4, 8 or 16 rows in pools of S to 4S slots, ranks 8-192, both rotary layouts."""
    import numpy as np
    rng = np.random.default_rng(97)
    for case in range(8):
        B, H = int(rng.integers(1, 5)), int(rng.choice([1, 2, 3, 8]))
        S, c = int(rng.integers(1, 301)), int(rng.choice([4, 8, 16]))
        P = int(rng.integers(S, 4 * S + 1))
        R, glm = 8 * int(rng.integers(1, 25)), bool(rng.integers(0, 2))
        _one_launch_slots_case(gpu, B, H, S, P, glm, R, c, 7000 + case)


def _one_launch_slots_case(gpu, B, H, S, P, glm, R, c, seed):
    print(f"pool fetch+rebuild one launch B={B} H={H} S={S} P={P} glm={glm} rank={R} chunk={c}", flush=True)
    D = 128
    chunks = max(4 * S, 2048)
    ctx = chunks * c
    sparse_start = 64
    buf_len = sparse_start + P * c + 24
    g = torch.Generator().manual_seed(seed)
    gd = torch.Generator(device=gpu).manual_seed(seed)
    values = torch.randn(B, H, chunks, c * D, generator=g).to(torch.bfloat16).pin_memory()
    U = torch.randn(B, ctx, R, generator=gd, device=gpu).to(torch.bfloat16)
    SV = (torch.randn(B, H, D, R, generator=gd, device=gpu) / R ** 0.5).to(torch.bfloat16)
    cos_sin = (build_glm_cos_sin_cache(ctx + 64, 10000.0, device=gpu) if glm
               else build_cos_sin_cache(ctx + 64, 500000.0, D, device=gpu))
    rows = B * H
    cnts = torch.randint(0, S + 1, (rows,), generator=g, dtype=torch.int32)
    cnts[0] = 0
    if rows > 1:
        cnts[-1] = S
    # miss list as pool_assign leaves it: entries [cnts, S) name distinct chunks and distinct slots
    miss_ids = torch.stack([torch.randperm(chunks, generator=g)[:S] for _ in range(rows)]).to(torch.int32)
    miss_slot = torch.stack([torch.randperm(P, generator=g)[:S] for _ in range(rows)]).to(torch.int32)
    v0 = torch.randn(B, H, buf_len, D, generator=gd, device=gpu).to(torch.bfloat16)
    k0 = torch.randn(B, H, buf_len, D, generator=gd, device=gpu).to(torch.bfloat16)
    ids_d, slot_d, cnts_d = miss_ids.view(B, H, S).to(gpu), miss_slot.view(B, H, S).to(gpu), cnts.to(gpu)
    va, ka = v0.clone(), k0.clone()
    shadowkv.gather_copy_misses_to_slots(values, va, ids_d, cnts_d, slot_d, B, H, chunks * c * D, sparse_start * D,
                                         buf_len * D, S, P, c * D)
    shadowkv.rebuild_k_rope(U, SV, ids_d, cnts_d, cos_sin, ka, sparse_start, c, miss_slot=slot_d, pool_slots=P)
    for cap in (0, 8, 48):
        vb, kb = v0.clone(), k0.clone()
        shadowkv.fetch_misses_rebuild_k_rope_slots(values, vb, ids_d, cnts_d, slot_d, chunks * c * D,
                                                   sparse_start * D, buf_len * D, U, SV, cos_sin, kb, sparse_start,
                                                   c, P, rebuild_workgroups=cap)
        torch.cuda.synchronize()
        assert torch.equal(vb.view(torch.int16), va.view(torch.int16)), cap
        assert torch.equal(kb.view(torch.int16), ka.view(torch.int16)), cap
    # the launch did write: row 0 (misses only) holds each miss chunk in its slot, in both buffers
    vr = vb[0, 0, sparse_start:sparse_start + P * c].reshape(P, c * D).cpu()
    assert torch.equal(vr[miss_slot[0].long()].view(torch.int16), values[0, 0, miss_ids[0].long()].view(torch.int16))
    untouched = torch.ones(P, dtype=torch.bool)
    untouched[miss_slot[0].long()] = False
    kr = kb[0, 0, sparse_start:sparse_start + P * c].reshape(P, c * D).cpu()
    k0r = k0[0, 0, sparse_start:sparse_start + P * c].reshape(P, c * D).cpu()
    assert torch.equal(kr[untouched].view(torch.int16), k0r[untouched].view(torch.int16))
    assert not torch.equal(kr[~untouched].view(torch.int16), k0r[~untouched].view(torch.int16))


def test_one_launch_rejects_inconsistent_buffers(gpu):
    B, H, S, c, D, R, chunks = 1, 2, 16, 8, 128, 160, 64
    values = torch.zeros(B, H, chunks, c * D, dtype=torch.bfloat16).pin_memory()
    U = torch.zeros(B, H, chunks * c, R, dtype=torch.bfloat16, device=gpu)
    SV = torch.zeros(H, D, R, dtype=torch.bfloat16, device=gpu)
    cos_sin = build_cos_sin_cache(chunks * c, 500000.0, D, device=gpu)
    pos = torch.zeros(B, H, S, dtype=torch.int64, device=gpu)
    cnts = torch.zeros(B * H, dtype=torch.int32, device=gpu)
    off = torch.zeros(B * H * S, dtype=torch.int32, device=gpu)
    buf = torch.zeros(B, H, 8 + S * c, D, dtype=torch.bfloat16, device=gpu)
    short = torch.zeros(B, H, 8 + S * c - 1, D, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="v_cache_buffer"):  # the value buffer is one row short
        shadowkv.fetch_misses_rebuild_k_rope(values, short, off, cnts, chunks * c * D, 8 * D, buf.shape[2] * D, U,
                                             SV, pos, cos_sin, buf, 8, c)
    with pytest.raises(ValueError, match="sparse region"):  # the key cache cannot hold the region
        shadowkv.fetch_misses_rebuild_k_rope(values, buf, off, cnts, chunks * c * D, 8 * D, buf.shape[2] * D, U, SV,
                                             pos, cos_sin, buf, 16, c)


def _state(model):
    out = []
    for lane in model.lanes:
        c = lane.cache
        out += [c.k_cache_buffer, c.v_cache_buffer, c.position_ids, c.offsets, c.cnts]
    return out


@pytest.mark.parametrize("shape,batch,ctx", [(replace(decode_model.LLAMA31_8B, layers=2, vocab=1000), 2, 16384),
                                              (replace(decode_model.GLM4_9B, layers=2, vocab=1000), 4, 16384)])
def test_one_lane_decoder_one_launch_matches_two_streams(gpu, shape, batch, ctx):
    """A one-lane decoder whose step issues the value fetch and key rebuild as one launch on the
    compute stream (the default for one lane) gives the same tokens and cache state, bit for bit,
    as the two-stream step (fetch on the copy stream, rebuild on the compute stream)."""
    print(f"one-launch vs two-stream step {shape.name} batch {batch}", flush=True)
    kw = dict(sparse_budget=2048, decode_len=8, lanes=1, seed=21)
    one = decode_model.SyntheticDecoder(shape, batch, ctx, **kw)
    two = decode_model.SyntheticDecoder(shape, batch, ctx, **kw, one_stream_fetch=False)
    assert one.cache.one_stream_active() and not two.cache.one_stream_active()
    t1 = t2 = torch.randint(0, shape.vocab, (batch, 1), device=gpu, generator=torch.Generator(device=gpu).manual_seed(7))
    hits = 0
    for t in range(4):
        t1 = one.decode_step(t1)
        t2 = two.decode_step(t2)
        torch.cuda.synchronize()
        assert torch.equal(t1, t2), t
        for a, b in zip(_state(one), _state(two)):
            assert torch.equal(a, b), t
        hits += int(one.cache.cnts.sum())
    assert hits > 0, "the steps moved no hit"
