"""Decoder-level equivalences of the bench model's kernel choices:
* the down projection forming SiLU-and-mul from the gate/up rows (two lanes of 4 sequences, the
  batch-8 decode's setting) gives the same tokens and cache state, bit for bit, as the
  SiLU-and-mul kernel followed by the linear kernel;
* the hit moves folded into the selection launch give the same tokens and cache state, bit for
  bit, as the separate in-buffer compaction launches (one lane and two lanes);
* the QKV projection with RoPE + append in its epilogue gives the same tokens and cache state, bit
  for bit, as the projection followed by the RoPE + append kernel;
* two lanes, each with its one-launch fetch + rebuild on its own side stream, give the same tokens
  and cache state, bit for bit, as the lanes sharing one fetch and one rebuild stream;
* the value store in device memory gives the same tokens and cache state, bit for bit, as the
  pinned host store;
* the fused new-token step (residual + RMSNorm, skinny linear, SiLU-and-mul, RoPE + append
  kernels) agrees with the reference call sequence on torch operations (F.rms_norm, F.linear,
  F.silu, apply_rotary_pos_emb_new + update_kv_cache) within bf16 tolerance."""
from dataclasses import replace

import pytest
import torch

from shadowkv_amd import decode_model

pytestmark = pytest.mark.gpu


def _state(model):
    out = [model.pos.clone()]
    for lane in model.lanes:
        c = lane.cache
        out += [c.position_ids.clone(), c.cnts.clone(), c.offsets.clone(), c.k_cache_buffer.clone(),
                c.v_cache_buffer.clone(), c.kv_len_dev.clone(), c.chunk_attn.clone()]
    return out


def test_gated_down_projection_matches_two_kernels(gpu):
    print("gated down projection vs silu_and_mul + linear, batch 8 in 2 lanes", flush=True)
    shape = replace(decode_model.LLAMA31_8B, layers=2, vocab=1000)
    kw = dict(sparse_budget=2048, decode_len=8, lanes=2, seed=13)
    gated = decode_model.SyntheticDecoder(shape, 8, 16384, **kw)
    plain = decode_model.SyntheticDecoder(shape, 8, 16384, **kw)
    assert gated.gated_down, "two lanes of 4 rows take the gated down projection"
    gated.act_epilogue = plain.act_epilogue = False  # (the epilogue form comes first where it runs)
    plain.gated_down = False
    tg = tp = torch.randint(0, shape.vocab, (8, 1), device=gpu, generator=torch.Generator(device=gpu).manual_seed(3))
    for t in range(3):
        tg = gated.decode_step(tg)
        tp = plain.decode_step(tp)
        torch.cuda.synchronize()
        assert torch.equal(tg, tp), t
        for a, b in zip(_state(gated), _state(plain)):
            assert torch.equal(a, b), t


@pytest.mark.parametrize("lanes", [1, 2])
def test_folded_hit_moves_match_separate_compaction(gpu, lanes):
    print(f"folded hit moves vs separate compaction, batch 8 in {lanes} lane(s)", flush=True)
    shape = replace(decode_model.LLAMA31_8B, layers=2, vocab=1000)
    kw = dict(sparse_budget=2048, decode_len=8, lanes=lanes, seed=15)
    folded = decode_model.SyntheticDecoder(shape, 8, 16384, **kw)
    separate = decode_model.SyntheticDecoder(shape, 8, 16384, **kw)
    for lane in separate.lanes:
        lane.cache.fold_hit_moves = False
    assert all(lane.cache.fold_hit_moves for lane in folded.lanes)
    tf = ts = torch.randint(0, shape.vocab, (8, 1), device=gpu, generator=torch.Generator(device=gpu).manual_seed(5))
    hits = 0
    for t in range(4):
        tf = folded.decode_step(tf)
        ts = separate.decode_step(ts)
        torch.cuda.synchronize()
        assert torch.equal(tf, ts), t
        for a, b in zip(_state(folded), _state(separate)):
            assert torch.equal(a, b), t
        hits += sum(int(lane.cache.cnts.sum()) for lane in folded.lanes)
    assert hits > 0, "the steps moved no hit"


@pytest.mark.parametrize("lanes", [1, 2])
def test_silu_epilogue_matches_two_kernels(gpu, lanes):
    """The gate/up projection with SiLU-and-mul in its epilogue (interleaved weight) gives the same
    tokens and cache state, bit for bit, as the projection followed by the SiLU-and-mul kernel."""
    print(f"SiLU epilogue vs two kernels, batch 8 in {lanes} lane(s)", flush=True)
    shape = replace(decode_model.LLAMA31_8B, layers=2, vocab=1000)
    kw = dict(sparse_budget=2048, decode_len=8, lanes=lanes, seed=16)
    epi = decode_model.SyntheticDecoder(shape, 8, 16384, **kw)
    two = decode_model.SyntheticDecoder(shape, 8, 16384, **kw)
    assert epi.act_epilogue == (lanes == 1)  # the decoder's own choice
    epi.act_epilogue = True  # (compared at both lane counts)
    two.act_epilogue = False
    two.gated_down = False
    te = tt = torch.randint(0, shape.vocab, (8, 1), device=gpu, generator=torch.Generator(device=gpu).manual_seed(6))
    for t in range(3):
        te = epi.decode_step(te)
        tt = two.decode_step(tt)
        torch.cuda.synchronize()
        assert torch.equal(te, tt), t
        for a, b in zip(_state(epi), _state(two)):
            assert torch.equal(a, b), t


@pytest.mark.parametrize("model,lanes,per_lane", [("llama", 1, 4), ("llama", 2, 4), ("glm", 1, 4), ("llama", 1, 8),
                                                   ("glm", 1, 6)])
def test_qkv_rope_epilogue_matches_two_kernels(gpu, model, lanes, per_lane):
    """The QKV projection with RoPE + append in its epilogue gives the same tokens and cache state,
    bit for bit, as the projection followed by the RoPE + append kernel (half-split and GLM
    rotations; one and two lanes of 4 rows, one lane of 6 and 8), eager and in captured graphs."""
    batch = per_lane * lanes
    print(f"QKV RoPE epilogue vs two kernels, {model} batch {batch} in {lanes} lane(s)", flush=True)
    base = decode_model.GLM4_9B if model == "glm" else decode_model.LLAMA31_8B
    shape = replace(base, layers=2, vocab=1000)
    kw = dict(sparse_budget=2048, decode_len=8, lanes=lanes, seed=18)
    epi = decode_model.SyntheticDecoder(shape, batch, 16384, **kw)
    two = decode_model.SyntheticDecoder(shape, batch, 16384, **kw)
    assert epi.qkv_rope_epilogue  # the decoder's own choice at 4 rows per lane
    two.qkv_rope_epilogue = False
    te = tt = torch.randint(0, shape.vocab, (batch, 1), device=gpu,
                            generator=torch.Generator(device=gpu).manual_seed(8))
    for t in range(3):
        te = epi.decode_step(te)
        tt = two.decode_step(tt)
        torch.cuda.synchronize()
        assert torch.equal(te, tt), t
        for a, b in zip(_state(epi), _state(two)):
            assert torch.equal(a, b), t
    epi.capture(te)
    two.capture(tt)
    for t in range(2):
        te, tt = epi.replay(), two.replay()
        torch.cuda.synchronize()
        assert torch.equal(te, tt), ("replay", t)
        for a, b in zip(_state(epi), _state(two)):
            assert torch.equal(a, b), ("replay", t)


@pytest.mark.parametrize("pool", [None, 512])
def test_lane_streams_match_shared_streams(gpu, pool):
    """Two lanes with each lane's one-launch value fetch + key rebuild on a side stream of its own
    (the decoder's default) give the same tokens and cache state, bit for bit, as the lanes sharing
    one fetch stream and one rebuild stream, eager and in captured graphs; also with a chunk pool
    (the one launch then fetches and rebuilds the pool's misses into their slots)."""
    print(f"lane streams vs shared fetch / rebuild streams, batch 8 in 2 lanes, pool {pool}", flush=True)
    shape = replace(decode_model.LLAMA31_8B, layers=2, vocab=1000)
    kw = dict(sparse_budget=2048, decode_len=12, lanes=2, seed=19, chunk_cache=pool)
    own = decode_model.SyntheticDecoder(shape, 8, 16384, **kw)
    shared = decode_model.SyntheticDecoder(shape, 8, 16384, lane_streams=False, **kw)
    assert own.lane_streams and not shared.lane_streams
    assert all(lane.cache.one_stream_active() and lane.cache.lane_stream is not None for lane in own.lanes)
    assert own.lanes[0].cache.lane_stream is not own.lanes[1].cache.lane_stream
    assert not any(lane.cache.one_stream_active() for lane in shared.lanes)
    to = ts = torch.randint(0, shape.vocab, (8, 1), device=gpu, generator=torch.Generator(device=gpu).manual_seed(9))
    for t in range(3):
        to = own.decode_step(to)
        ts = shared.decode_step(ts)
        torch.cuda.synchronize()
        assert torch.equal(to, ts), t
        for a, b in zip(_state(own), _state(shared)):
            assert torch.equal(a, b), t
    own.capture(to, steps=2)
    shared.capture(ts, steps=2)
    for t in range(2):
        to, ts = own.replay(), shared.replay()
        torch.cuda.synchronize()
        assert torch.equal(to, ts), ("replay", t)
        for a, b in zip(_state(own), _state(shared)):
            assert torch.equal(a, b), ("replay", t)


def _hidden_after_layers(dec, tok):
    """The residual stream after every layer of one decode step of a one-lane decoder."""
    lane = dec.lanes[0]
    h = dec._embed(tok)
    for idx in range(dec.shape.layers):
        pending = dec._layer_begin(idx, h, lane)
        h = dec._layer_end(idx, h, lane, pending)
    torch.cuda.synchronize()
    return h[0] if dec.fused else h


def test_fused_step_matches_reference_call_sequence(gpu):
    print("fused new-token step vs torch operations, batch 4, 2 layers", flush=True)
    shape = replace(decode_model.LLAMA31_8B, layers=2, vocab=1000)
    kw = dict(sparse_budget=2048, decode_len=8, lanes=1, seed=14)
    fused = decode_model.SyntheticDecoder(shape, 4, 16384, fused=True, **kw)
    ref = decode_model.SyntheticDecoder(shape, 4, 16384, fused=False, **kw)
    tok = torch.randint(0, shape.vocab, (4, 1), device=gpu, generator=torch.Generator(device=gpu).manual_seed(4))
    with torch.inference_mode():
        hf = _hidden_after_layers(fused, tok)
        hr = _hidden_after_layers(ref, tok)
    # Two decoder layers of different summation orders and roundings (skinny linear vs hipBLASLt,
    # single-rounding RMSNorm vs F.rms_norm): a few bf16 steps apart at |h| ~ 3-8, so the residual
    # streams are compared by their relative difference (a dropped term or a wrong operation is O(1)).
    rel = ((hf.float() - hr.float()).norm() / hr.float().norm()).item()
    print(f"residual stream relative difference {rel:.2e}, rms {hr.float().pow(2).mean().sqrt().item():.2f}",
          flush=True)
    assert rel < 1e-2, rel
    # the appended keys and values (rotated k and raw v of the new token) of every layer
    for l in range(shape.layers):
        cf, cr = fused.cache, ref.cache
        row = cf.sparse_end
        for bf, br in ((cf.k_cache_buffer[l][:, :, row], cr.k_cache_buffer[l][:, :, row]),
                       (cf.v_cache_buffer[l][:, :, row], cr.v_cache_buffer[l][:, :, row])):
            rel = ((bf.float() - br.float()).norm() / br.float().norm()).item()
            assert rel < 1e-2, (l, rel)


def _state_outside_selection(model):
    """_state with the value buffers' selected regions left out (values read in place never fill them)."""
    out = [model.pos.clone()]
    for lane in model.lanes:
        c = lane.cache
        v = c.v_cache_buffer.clone()
        v[:, :, :, c.sparse_start:c.sparse_start + c.select_sets * c.chunk_size] = 0
        out += [c.position_ids.clone(), c.cnts.clone(), c.offsets.clone(), c.k_cache_buffer.clone(), v,
                c.kv_len_dev.clone(), c.chunk_attn.clone()]
    return out


@pytest.mark.parametrize("lanes,in_place", [(1, True), (1, False), (2, True), (2, False)])
def test_device_value_store_matches_host_store(gpu, lanes, in_place):
    """The value store in device memory (value_store="device") gives the same tokens and cache
    state, bit for bit, as the pinned host store: the same kernels gather the same chunks, from HBM
    instead of over the host link, or (in_place, the device store's default) the attention reads the
    selected values in place from the store and the value buffer's selected region is never
    filled (compared outside it). Eager steps and captured graph replays, one and two lanes."""
    print(f"device value store (in place {in_place}) vs pinned host store, batch 8 in {lanes} lane(s)", flush=True)
    shape = replace(decode_model.LLAMA31_8B, layers=2, vocab=1000)
    kw = dict(sparse_budget=2048, decode_len=12, lanes=lanes, seed=29)
    host = decode_model.SyntheticDecoder(shape, 8, 16384, **kw)
    dev = decode_model.SyntheticDecoder(shape, 8, 16384, value_store="device", **kw)
    for hl, dl in zip(host.lanes, dev.lanes):
        assert hl.cache.v_cache_cpu[0].is_pinned() and dl.cache.v_cache_cpu[0].is_cuda
        assert not hl.cache.values_in_place and dl.cache.values_in_place
        dl.cache.values_in_place = in_place
        for a, b in zip(hl.cache.v_cache_cpu, dl.cache.v_cache_cpu):
            assert torch.equal(a, b.cpu())
    state = _state_outside_selection if in_place else _state
    th = td = torch.randint(0, shape.vocab, (8, 1), device=gpu, generator=torch.Generator(device=gpu).manual_seed(4))
    for t in range(3):
        th = host.decode_step(th)
        td = dev.decode_step(td)
        torch.cuda.synchronize()
        assert torch.equal(th, td), t
        for a, b in zip(state(host), state(dev)):
            assert torch.equal(a, b), t
    host.capture(th, steps=2)
    dev.capture(td, steps=2)
    for t in range(2):
        th, td = host.replay(), dev.replay()
        torch.cuda.synchronize()
        assert torch.equal(th, td), ("replay", t)
        for a, b in zip(state(host), state(dev)):
            assert torch.equal(a, b), ("replay", t)


def test_device_value_store_with_chunk_pool_matches_host_store(gpu):
    """A chunk pool over a value store in device memory (the pool's misses gathered from HBM by the
    slot-mapped one launch, no in-place reads) gives the same tokens and cache state, bit for bit,
    as the same pool over the pinned host store; eager steps and captured graph replays."""
    print("device value store vs pinned host store, both with a pool of 512 slots, batch 8 in 1 lane", flush=True)
    shape = replace(decode_model.LLAMA31_8B, layers=2, vocab=1000)
    kw = dict(sparse_budget=2048, decode_len=12, lanes=1, seed=31, chunk_cache=512)
    host = decode_model.SyntheticDecoder(shape, 8, 16384, **kw)
    dev = decode_model.SyntheticDecoder(shape, 8, 16384, value_store="device", **kw)
    for hl, dl in zip(host.lanes, dev.lanes):
        assert hl.cache.v_cache_cpu[0].is_pinned() and dl.cache.v_cache_cpu[0].is_cuda
        assert not dl.cache.values_in_place and dl.cache.one_stream_active() and hl.cache.one_stream_active()
    th = td = torch.randint(0, shape.vocab, (8, 1), device=gpu, generator=torch.Generator(device=gpu).manual_seed(5))
    for t in range(3):
        th = host.decode_step(th)
        td = dev.decode_step(td)
        torch.cuda.synchronize()
        assert torch.equal(th, td), t
        for a, b in zip(_state(host), _state(dev)):
            assert torch.equal(a, b), t
    host.capture(th, steps=2)
    dev.capture(td, steps=2)
    for t in range(2):
        th, td = host.replay(), dev.replay()
        torch.cuda.synchronize()
        assert torch.equal(th, td), ("replay", t)
        for a, b in zip(_state(host), _state(dev)):
            assert torch.equal(a, b), ("replay", t)
