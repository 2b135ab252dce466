"""The device chunk pool (f3): pool_assign against the oracle's policy, and decode steps through a
cache built with a pool against the oracle's pooled decode (from identical scores) and against the
reference-mode cache (P = S holds the same chunks)."""
import numpy as np
import pytest
import torch

import oracle
from shadowkv_amd.kernels import shadowkv
from shadowkv_amd.models.attention import ShadowAttention
from tests.decode_harness import build_cache, check_scoring, fresh_oracle_state, identity_rope
from tests.golden import make_golden
from tests.test_oracle_pool import _stream, _tables

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("rows,chunks,S,P,drift", [(16, 1000, 64, 64, 0.3), (16, 1000, 64, 96, 0.3),
                                                   (8, 4000, 256, 1024, 0.5), (4, 600, 100, 101, 1.0),
                                                   (2, 20000, 2048, 4096, 0.2), (2, 3000, 300, 1025, 0.4),
                                                   (1, 60000, 2048, 16384, 0.3)])
def test_pool_assign_matches_oracle(gpu, rows, chunks, S, P, drift):
    _say(f"pool_assign rows={rows} chunks={chunks} S={S} P={P} drift={drift}")
    rng = np.random.default_rng(rows + S + P)
    steps = 6
    stream = _stream(rng, rows, chunks, S, steps, drift)
    ref = _tables(rows, chunks, P, stream[0])
    dev = [torch.from_numpy(t.copy()).to(gpu) for t in ref]
    slot_list = torch.empty(rows, S, dtype=torch.int32, device=gpu)
    miss_ids = torch.empty(rows, S, dtype=torch.int32, device=gpu)
    miss_slot = torch.empty(rows, S, dtype=torch.int32, device=gpu)
    cnts = torch.empty(rows, dtype=torch.int32, device=gpu)
    for t in range(1, steps + 1):
        want = oracle.pool_assign(stream[t], *ref)
        shadowkv.pool_assign(torch.from_numpy(stream[t]).to(gpu), chunks, *dev, slot_list, miss_ids, miss_slot, cnts)
        torch.cuda.synchronize()
        assert np.array_equal(slot_list.cpu().numpy(), want[0]), t
        assert np.array_equal(cnts.cpu().numpy(), want[3]), t
        for r in range(rows):
            c = int(want[3][r])
            assert np.array_equal(miss_ids.cpu().numpy()[r, c:], want[1][r, c:])
            assert np.array_equal(miss_slot.cpu().numpy()[r, c:], want[2][r, c:])
        for d_t, r_t in zip(dev, ref):
            assert np.array_equal(d_t.cpu().numpy(), r_t), t


@pytest.mark.parametrize("span,empty", [(200, 0.0), (300, 0.1), (70000, 0.05), (1 << 25, 0.0)])
def test_pool_assign_after_long_decodes_matches_oracle(gpu, span, empty):
    """pool_assign from tables a long decode leaves behind: every slot's last use spread over the
    `span` steps before the clock (`empty` of the slots never used), so the victims' selection runs
    over one, two, three or four key bytes; against the oracle for 4 steps."""
    _say(f"pool_assign after a long decode: last uses over {span} steps, {empty:.0%} empty slots")
    rows, chunks, S, P = 4, 30000, 256, 4096
    rng = np.random.default_rng(span)
    clock0 = span + 1000
    slot_of = np.full((rows, chunks), -1, np.int32)
    slot_chunk = np.full((rows, P), -1, np.int32)
    slot_used = np.full((rows, P), -1, np.int32)
    for r in range(rows):
        held = rng.permutation(chunks)[:P]
        used = rng.random(P) >= empty
        slot_chunk[r, used] = held[used]
        slot_of[r, held[used]] = np.nonzero(used)[0]
        slot_used[r, used] = rng.integers(clock0 - span, clock0, size=int(used.sum()))
    ref = [slot_of, slot_chunk, slot_used, np.full(rows, clock0, np.int32)]
    dev = [torch.from_numpy(t.copy()).to(gpu) for t in ref]
    slot_list = torch.empty(rows, S, dtype=torch.int32, device=gpu)
    miss_ids = torch.empty(rows, S, dtype=torch.int32, device=gpu)
    miss_slot = torch.empty(rows, S, dtype=torch.int32, device=gpu)
    cnts = torch.empty(rows, dtype=torch.int32, device=gpu)
    for t in range(4):
        # half of each selection from the resident chunks, half from the others
        sel = np.stack([np.concatenate([rng.permutation(slot_chunk[r][slot_chunk[r] >= 0])[:S // 2],
                                        rng.permutation(np.setdiff1d(np.arange(chunks), slot_chunk[r]))[:S // 2]])
                        for r in range(rows)]).astype(np.int64)
        want = oracle.pool_assign(sel, *ref)
        shadowkv.pool_assign(torch.from_numpy(sel).to(gpu), chunks, *dev, slot_list, miss_ids, miss_slot, cnts)
        torch.cuda.synchronize()
        assert np.array_equal(slot_list.cpu().numpy(), want[0]), t
        assert np.array_equal(cnts.cpu().numpy(), want[3]), t
        assert (want[3] == S // 2).all()
        for r in range(rows):
            assert np.array_equal(miss_ids.cpu().numpy()[r, S // 2:], want[1][r, S // 2:])
            assert np.array_equal(miss_slot.cpu().numpy()[r, S // 2:], want[2][r, S // 2:])
        for d_t, r_t in zip(dev, ref):
            assert np.array_equal(d_t.cpu().numpy(), r_t), t


def _queries(B, H, G, D, steps, layers, seed, drift):
    """Per-(step, layer) queries that drift slowly, so consecutive selections overlap."""
    g = torch.Generator().manual_seed(seed)
    base = [torch.randn(B, H * G, D, generator=g) for _ in range(layers)]
    out = []
    for _ in range(steps):
        row = []
        for layer in range(layers):
            base[layer] = base[layer] + drift * torch.randn(B, H * G, D, generator=g)
            row.append((base[layer].to(torch.bfloat16), torch.randn(B, H, D, generator=g).to(torch.bfloat16),
                        torch.randn(B, H, D, generator=g).to(torch.bfloat16)))
        out.append(row)
    return out


@pytest.mark.parametrize("P,device_lengths,drift", [(256, True, 0.3), (160, False, 1.0), (128, True, 0.3)])
def test_pooled_decode_matches_oracle(gpu, P, device_lengths, drift):
    _say(f"pooled decode P={P} device_lengths={device_lengths} drift={drift}")
    _pooled_decode(gpu, make_golden.decode_small_case(), P, device_lengths, drift, steps=5, layers=2)


def test_pooled_decode_random_configurations(gpu):
    """Pooled decode steps on 5 seeded random configurations (batch 1-3, 1-4 kv heads of 1-16 query
    heads, chunks of 4/8/16 rows, budget 1024, pools of S to 3S slots) against the oracle's pooled
    step."""
    from tests.test_gpu_decode import _random_case
    rng = np.random.default_rng(83)
    for i in range(5):
        B, H = int(rng.integers(1, 4)), int(rng.choice([1, 2, 4]))
        G, chunk = int(rng.choice([1, 4, 16])), int(rng.choice([4, 8, 16]))
        S = 1024 // chunk
        P = int(rng.integers(S, 3 * S + 1))
        rank, glm, drift = int(rng.choice([16, 32])), bool(rng.integers(0, 2)), float(rng.choice([0.2, 0.5]))
        ctx = 64 * int(rng.integers(1024 * 2 // 64, 1024 * 4 // 64 + 1))
        _say(f"pooled random configuration {i}: B={B} H={H} G={G} chunk={chunk} P={P} rank={rank} ctx={ctx} "
             f"glm={glm} drift={drift}")
        case = _random_case(700 + i, B, H, G, ctx, rank, 1024, chunk, glm)
        _pooled_decode(gpu, case, P, bool(i % 2), drift, steps=4, layers=1)


@pytest.mark.parametrize("P,device_lengths", [(256, True), (160, False)])
def test_pooled_decode_one_launch_matches_oracle(gpu, P, device_lengths):
    """The pooled step with the misses' value fetch and key rebuild as one launch on the current
    stream (one_stream_fetch: fetch_misses_rebuild_k_rope_slots) against the oracle's pooled step."""
    _say(f"pooled decode, one-launch fetch + rebuild, P={P} device_lengths={device_lengths}")
    _pooled_decode(gpu, make_golden.decode_small_case(), P, device_lengths, 0.3, steps=5, layers=2, one_stream=True)


def _pooled_decode(gpu, case, P, device_lengths, drift, steps, layers, one_stream=False):
    d = case["dims"]
    B, H, G, D = d["B"], d["H"], d["G"], d["D"]
    cache = build_cache(case, gpu, max_decode_len=steps, num_layers=layers, chunk_cache=P)
    if device_lengths:
        cache.use_device_lengths()
    cache.one_stream_fetch = one_stream
    assert cache.one_stream_active() == one_stream
    cos_sin = case["cos_sin"]
    attn = ShadowAttention(cache, G, D, H * G * D, identity_rope(B, H * G, H, D), None, cos_sin.to(gpu))
    states = [fresh_oracle_state(case) for _ in range(layers)]
    pools = [oracle.pool_from_layer(st, P) for st in states]
    S, c, sp0 = cache.select_sets, cache.chunk_size, cache.sparse_start
    hits = []
    for t, row in enumerate(_queries(B, H, G, D, steps, layers, 5, drift)):
        for layer, (q, k, v) in enumerate(row):
            out = attn.decode(q.to(gpu).reshape(B, 1, -1), k.to(gpu).reshape(B, 1, -1), v.to(gpu).reshape(B, H, 1, D),
                              None, layer)
            torch.cuda.synchronize()
            check_scoring(cache, q, states[layer].landmarks)
            res = oracle.decode_layer_step_pooled(states[layer], pools[layer], q, k, v, cos_sin, gen_offset=t,
                                                  scores=cache.chunk_attn.cpu())
            assert np.array_equal(cache.cnts.cpu().numpy(), res["cnts"]), (t, layer)
            assert np.array_equal(cache.slot_list.cpu().numpy(), res["slot_list"]), (t, layer)
            pool = pools[layer]
            end = cache.sparse_end + cache.pool_delta + t + 1
            assert torch.equal(cache.v_cache_buffer[layer, :, :, :end].cpu(), pool["vbuf"][:, :, :end]), (t, layer)
            torch.testing.assert_close(cache.k_cache_buffer[layer, :, :, :end].cpu().float(),
                                       pool["kbuf"][:, :, :end].float(), rtol=2e-2, atol=2e-2)
            torch.testing.assert_close(out.view(B, H * G, D).cpu().float(), res["out"].float(), rtol=2e-2,
                                       atol=2e-2)
            for name in ("slot_of", "slot_chunk", "slot_used"):
                assert np.array_equal(getattr(cache, name)[layer].cpu().numpy(), pool[name]), name
            hits.append(int(res["cnts"].sum()))
    assert P == S or sum(hits[layers:]) > 0  # the drifting queries do reuse chunks


@pytest.mark.parametrize("mult", [1, 2, 4])
def test_pool_matches_reference_mode(gpu, mult):
    """A pool of P = mult * S slots selects the same chunks as a cache without a pool and gives the
    same attention outputs (to fp32 summation order: the slots are read in another order). P = S
    holds exactly the selected chunks, like the reference's slots, so the hit counts agree too;
    larger pools keep chunks across steps and hit at least as often."""
    _say(f"pool P = {mult} S vs reference mode")
    case = make_golden.decode_small_case()
    d = case["dims"]
    B, H, G, D = d["B"], d["H"], d["G"], d["D"]
    steps, layers = 4, 2
    S = case["dims"]["budget"] // case["dims"]["chunk"]
    caches = [build_cache(case, gpu, max_decode_len=steps, num_layers=layers, chunk_cache=P)
              for P in (None, mult * S)]
    for cch in caches:
        cch.keep_selected = True
    attns = [ShadowAttention(cch, G, D, H * G * D, identity_rope(B, H * G, H, D), None, case["cos_sin"].to(gpu))
             for cch in caches]
    for t, row in enumerate(_queries(B, H, G, D, steps, layers, 9, 0.3)):
        for layer, (q, k, v) in enumerate(row):
            outs, cnts, sels = [], [], []
            for cch, attn in zip(caches, attns):
                outs.append(attn.decode(q.to(gpu).reshape(B, 1, -1), k.to(gpu).reshape(B, 1, -1),
                                        v.to(gpu).reshape(B, H, 1, D), None, layer).cpu())
                cnts.append(cch.cnts.cpu().numpy().copy())
                sels.append(cch.selected_chunks.cpu().clone())
            assert torch.equal(sels[0], sels[1]), (t, layer)  # the same chunks, in top-k order
            if mult == 1:
                assert np.array_equal(cnts[0], cnts[1]), (t, layer)
            else:
                assert (cnts[1] >= cnts[0]).all(), (t, layer)
            torch.testing.assert_close(outs[0].float(), outs[1].float(), rtol=1e-2, atol=1e-2)
