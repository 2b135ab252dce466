"""A whole decode step captured in a HIP graph replays exactly like the eager step: same tokens,
same cache state (selected ids, slots, hit counts, assembled K/V buffers, device lengths), with
eager work and synchronizations between the replays."""
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
                c.v_cache_buffer.clone(), c.append_row_dev.clone(), c.kv_len_dev.clone(), c.chunk_attn.clone()]
        if c.pooled:
            out += [c.slot_of.clone(), c.slot_chunk.clone(), c.slot_used.clone(), c.pool_clock.clone(),
                    c.slot_list.clone()]
    return out


@pytest.mark.parametrize("lanes,chunk_cache", [(1, None), (2, None), (2, 384)])
def test_graph_replay_matches_eager(gpu, lanes, chunk_cache):
    print(f"graph replay vs eager, lanes={lanes}, chunk_cache={chunk_cache}", flush=True)
    shape = replace(decode_model.LLAMA31_8B, layers=2, vocab=1000)
    steps = 4
    kw = dict(sparse_budget=2048, decode_len=steps + 4, lanes=lanes, seed=11, chunk_cache=chunk_cache)
    eager = decode_model.SyntheticDecoder(shape, 4, 16384, **kw)
    graphed = decode_model.SyntheticDecoder(shape, 4, 16384, **kw)
    tok0 = torch.randint(0, shape.vocab, (4, 1), device=gpu, generator=torch.Generator(device=gpu).manual_seed(1))
    # one eager step on both (warms allocators and libraries), then capture on the second
    te = eager.decode_step(tok0)
    tg = graphed.decode_step(tok0)
    torch.cuda.synchronize()
    assert torch.equal(te, tg)
    graphed.capture(tg)
    torch.cuda.synchronize()
    for t in range(steps):
        te = eager.decode_step(te)
        tg = graphed.replay()
        torch.cuda.synchronize()
        noise = torch.randn(1 << 20, device=gpu)  # unrelated eager work between replays
        float(noise.sum())
        assert torch.equal(te, tg), t
        for a, b in zip(_state(eager), _state(graphed)):
            assert torch.equal(a, b), t
        for le, lg in zip(eager.lanes, graphed.lanes):
            assert le.cache.gen_offset == lg.cache.gen_offset == t + 2
    # eager steps after replays continue from the replayed state
    te = eager.decode_step(te)
    tg = graphed.decode_step(tg)
    torch.cuda.synchronize()
    assert torch.equal(te, tg)
    for a, b in zip(_state(eager), _state(graphed)):
        assert torch.equal(a, b)



@pytest.mark.parametrize("lanes,chunk_cache,glm", [(1, None, False), (2, None, False), (2, 384, False),
                                                  (2, None, True)])
def test_multi_step_graph_matches_eager(gpu, lanes, chunk_cache, glm):
    """A graph of 3 decode steps (one continuous lane pipeline across the step boundaries)
    replays like 3 eager steps, twice in a row; also the GLM-4-9B shape (2 kv heads of 16 query
    heads, GLM's interleaved RoPE table through the fused new-token kernel and the rebuild)."""
    print(f"3-step graph vs eager, lanes={lanes}, chunk_cache={chunk_cache}, glm={glm}", flush=True)
    shape = replace(decode_model.GLM4_9B if glm else decode_model.LLAMA31_8B, layers=2, vocab=1000)
    n = 3
    kw = dict(sparse_budget=2048, decode_len=2 * n + 4, lanes=lanes, seed=12, chunk_cache=chunk_cache)
    eager = decode_model.SyntheticDecoder(shape, 4, 16384, **kw)
    graphed = decode_model.SyntheticDecoder(shape, 4, 16384, **kw)
    tok0 = torch.randint(0, shape.vocab, (4, 1), device=gpu, generator=torch.Generator(device=gpu).manual_seed(2))
    te = eager.decode_step(tok0)
    tg = graphed.decode_step(tok0)
    torch.cuda.synchronize()
    assert torch.equal(te, tg)
    graphed.capture(tg, steps=n)
    torch.cuda.synchronize()
    for r in range(2):
        for _ in range(n):
            te = eager.decode_step(te)
        tg = graphed.replay()
        torch.cuda.synchronize()
        float(torch.randn(1 << 20, device=gpu).sum())  # unrelated eager work between replays
        assert torch.equal(te, tg), r
        for a, b in zip(_state(eager), _state(graphed)):
            assert torch.equal(a, b), r
        for le, lg in zip(eager.lanes, graphed.lanes):
            assert le.cache.gen_offset == lg.cache.gen_offset == 1 + n * (r + 1)
    # eager multi-step pipelining gives the same tokens and state as single steps
    te2 = eager.decode_steps(te, 2)
    tg2 = graphed.decode_step(graphed.decode_step(tg))
    torch.cuda.synchronize()
    assert torch.equal(te2, tg2)
    for a, b in zip(_state(eager), _state(graphed)):
        assert torch.equal(a, b)

def test_graph_replay_respects_capacity(gpu):
    shape = replace(decode_model.LLAMA31_8B, layers=1, vocab=1000)
    model = decode_model.SyntheticDecoder(shape, 2, 16384, decode_len=2)
    tok = model.decode_step(torch.zeros(2, 1, dtype=torch.int64, device=gpu))  # eager warm-up step
    cap = model.cache.buf_len - model.cache.sparse_end - 1
    model.capture(tok)
    for _ in range(cap):
        model.replay()
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="capacity"):
        model.replay()
    assert int(model.cache.kv_len_dev) == model.cache.buf_len



@pytest.mark.skip(reason="removed design: capturing a step whose lanes ran on their own streams (a lane stream "
                         "forking the value-fetch stream inside the capture) ended in a host segmentation fault at "
                         "end of capture, cause not found; lanes are now pipelined on the capture stream")
def test_lane_stream_capture():
    pass


@pytest.mark.skip(reason="removed design: eager decode with every lane on its own stream (five streams) hung in "
                         "its first full-size step (batch 8, ctx 122880, 2 lanes), cause not found")
def test_lane_stream_eager_full_size():
    pass
