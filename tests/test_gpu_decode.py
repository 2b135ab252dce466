"""End-to-end decode steps through the drop-in classes (ShadowKVCache_CPU + ShadowAttention)
against the oracle's composition of the same reference steps."""
import numpy as np
import pytest
import torch

import oracle
from tests.decode_harness import build_cache, check_scoring, fresh_oracle_state, run_decode_step_gpu
from tests.golden import make_golden

pytestmark = pytest.mark.gpu


def test_single_layer_decode_step(gpu):
    print("decode small fixture, one step", flush=True)
    case = make_golden.decode_small_case()
    d = np.load(make_golden.HERE / "decode_small.npz")
    got = run_decode_step_gpu(case, gpu)
    B, H = case["dims"]["B"], case["dims"]["H"]
    check_scoring(got["cache"], case["q"], case["state_in"]["landmarks"])
    # Selection, reorder and copies bit-exact from identical scores: the oracle step run on the
    # device's GQA-max scores.
    st = fresh_oracle_state(case)
    res = oracle.decode_layer_step(st, case["q"], case["k_new"], case["v_new"], case["cos_sin"],
                                   scores=got["scores"])
    assert torch.equal(got["selected"], res["selected"])
    assert np.array_equal(got["cnts"], res["cnts"])
    assert np.array_equal(got["offsets"], res["offsets"].reshape(B * H, -1))
    assert np.array_equal(got["position_ids"], st.position_ids.numpy())
    L = res["L"]
    assert torch.equal(got["vbuf"], st.vbuf[:, :, :L])
    torch.testing.assert_close(got["kbuf"].float(), st.kbuf[:, :, :L].float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(got["out"].float(), res["out"].float(), rtol=2e-2, atol=2e-2)
    # When the device scores equal the oracle's own (the usual case here), the committed fixture's
    # selection applies unchanged.
    if torch.equal(got["scores"], case["res"]["scores"]):
        assert np.array_equal(got["cnts"], d["out_cnts"])
        assert np.array_equal(got["offsets"], d["out_offsets"])
        assert np.array_equal(got["position_ids"], d["out_position_ids"])


def test_single_layer_step_at_workload_shape(gpu):
    """The composed single-layer step at the single-layer workload's own shape (8 kv heads, rank
    160, ctx 8192, budget 2048, 968 landmarks) through the drop-in classes, against the oracle."""
    print("single-layer workload shape: batch 1, 8 kv heads, ctx 8192, rank 160", flush=True)
    case = make_golden.single_layer_case()
    assert case["state_in"]["landmarks"].shape[-2] == 968 and case["st"].sparse_start == 448
    got = run_decode_step_gpu(case, gpu)
    B, H = case["dims"]["B"], case["dims"]["H"]
    check_scoring(got["cache"], case["q"], case["state_in"]["landmarks"])
    st = fresh_oracle_state(case)
    res = oracle.decode_layer_step(st, case["q"], case["k_new"], case["v_new"], case["cos_sin"],
                                   scores=got["scores"])
    assert torch.equal(got["selected"], res["selected"])
    assert np.array_equal(got["cnts"], res["cnts"])
    assert np.array_equal(got["offsets"], res["offsets"].reshape(B * H, -1))
    assert np.array_equal(got["position_ids"], st.position_ids.numpy())
    L = res["L"]
    assert L == 2497
    assert torch.equal(got["vbuf"], st.vbuf[:, :, :L])
    torch.testing.assert_close(got["kbuf"].float(), st.kbuf[:, :, :L].float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(got["out"].float(), res["out"].float(), rtol=2e-2, atol=2e-2)
    print(f"hits per head {got['cnts'].tolist()}", flush=True)


@pytest.mark.parametrize("device_lengths,chunk,split,glm", [(False, 8, None, False), (True, 8, None, False),
                                                           (True, 4, None, False), (True, 16, None, False),
                                                           (False, 16, None, False), (True, 8, "1", False),
                                                           (True, 8, None, True), (False, 16, "1", True),
                                                           (True, 8, "2", False), (True, 4, "2", True)])
def test_multi_layer_multi_step_decode(gpu, monkeypatch, device_lengths, chunk, split, glm):
    """Also chunk sizes other than 8 (budget 1024: 256 selected chunks of 4 rows, 64 of 16 rows)
    through every kernel of the step, the selection's few-row paths forced on (keys from the softmax
    kernel; also the radix passes over many workgroups per row), and the
    GLM-4-9B head layout (16 query heads per kv head) with GLM's interleaved RoPE table."""
    if split is not None:
        monkeypatch.setenv("SKV_SELECT_SPLIT", split)
    print(f"decode small fixture, 2 layers x 4 steps, device_lengths={device_lengths}, chunk={chunk}, split={split}, "
          f"glm={glm}", flush=True)
    case = make_golden.decode_small_case(chunk, glm=glm)
    _decode_and_check(gpu, case, device_lengths, steps=4, layers=2, seed=77)


def _random_case(seed, B, H, G, ctx, rank, budget, chunk, glm):
    """decode_small_case's construction (low-rank pre-RoPE keys plus noise, N(0,1) values and
    queries, encoded by the oracle) at other dimensions."""
    g = torch.Generator().manual_seed(seed)
    D = 128
    A = torch.randn(B, ctx, rank, generator=g) / rank ** 0.5
    Bm = torch.randn(B, rank, H * D, generator=g) / rank ** 0.5
    k_pre = (A @ Bm + 0.05 * torch.randn(B, ctx, H * D, generator=g)).view(B, ctx, H, D).transpose(1, 2)
    k_pre = k_pre.to(torch.bfloat16).contiguous()
    v = torch.randn(B, H, ctx, D, generator=g).to(torch.bfloat16)
    q_last = torch.randn(B, H * G, 1, D, generator=g).to(torch.bfloat16)
    cos_sin = oracle.build_glm_cos_sin_cache(ctx + 64, 10000.0) if glm else oracle.build_cos_sin_cache(ctx + 64, 500000.0)
    st = oracle.encode_layer(k_pre, v, q_last, cos_sin, rank=rank, chunk=chunk, budget=budget)
    state_in = dict(U=st.U.clone(), SV=st.SV.clone(), landmarks=st.landmarks.clone(),
                    landmark_idx=st.landmark_idx.clone(), host_v=st.host_v.clone(), kbuf=st.kbuf.clone(),
                    vbuf=st.vbuf.clone(), position_ids=st.position_ids.clone())
    return dict(state_in=state_in, st=st, cos_sin=cos_sin,
                dims=dict(B=B, H=H, G=G, D=D, ctx=ctx, rank=rank, chunk=chunk, budget=budget))


def test_decode_random_configurations(gpu):
    """Whole decode steps through the drop-in cache and attention classes on 6 seeded random
    configurations (batch 1-3, 1-4 kv heads of 1-16 query heads, chunks of 4/8/16 rows, budgets
    1024/2048, ranks 16-64, contexts 2-4x the budget, both rotary tables), 1 layer x 3 steps, checked
    against the oracle as in the fixture test."""
    rng = np.random.default_rng(82)
    for case_i in range(6):
        B, H = int(rng.integers(1, 4)), int(rng.choice([1, 2, 4]))
        G, chunk = int(rng.choice([1, 2, 4, 8, 16])), int(rng.choice([4, 8, 16]))
        budget, rank, glm = int(rng.choice([1024, 2048])), int(rng.choice([16, 32, 64])), bool(rng.integers(0, 2))
        ctx = 64 * int(rng.integers(budget * 2 // 64, budget * 4 // 64 + 1))
        print(f"decode random configuration {case_i}: B={B} H={H} G={G} chunk={chunk} budget={budget} rank={rank} "
              f"ctx={ctx} glm={glm}", flush=True)
        case = _random_case(600 + case_i, B, H, G, ctx, rank, budget, chunk, glm)
        _decode_and_check(gpu, case, device_lengths=bool(case_i % 2), steps=3, layers=1, seed=900 + case_i)


def _decode_and_check(gpu, case, device_lengths, steps, layers, seed):
    d = case["dims"]
    B, H, G, D = d["B"], d["H"], d["G"], d["D"]
    cache = build_cache(case, gpu, max_decode_len=steps, num_layers=layers)
    if device_lengths:
        cache.use_device_lengths()
    # oracle states: one per layer, fresh copies of the encoded state
    states = [fresh_oracle_state(case) for _ in range(layers)]
    from shadowkv_amd.models.attention import ShadowAttention
    from tests.decode_harness import identity_rope
    cos_sin = case["cos_sin"]
    attn = ShadowAttention(cache, G, D, H * G * D, identity_rope(B, H * G, H, D), None, cos_sin.to(gpu))
    g = torch.Generator().manual_seed(seed)
    for t in range(steps):
        for layer in range(layers):
            q = torch.randn(B, H * G, D, generator=g).to(torch.bfloat16)
            k = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
            v = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
            out = attn.decode(q.to(gpu).reshape(B, 1, -1), k.to(gpu).reshape(B, 1, -1), v.to(gpu).reshape(B, H, 1, D),
                              None, layer)
            torch.cuda.synchronize()
            check_scoring(cache, q, states[layer].landmarks)
            res = oracle.decode_layer_step(states[layer], q, k, v, cos_sin, gen_offset=t,
                                           scores=cache.chunk_attn.cpu())
            assert np.array_equal(cache.cnts.cpu().numpy(), res["cnts"]), (t, layer)
            assert np.array_equal(cache.position_ids[layer].cpu().numpy(), states[layer].position_ids.numpy())
            L = res["L"]
            assert torch.equal(cache.v_cache_buffer[layer, :, :, :L].cpu(), states[layer].vbuf[:, :, :L])
            torch.testing.assert_close(cache.k_cache_buffer[layer, :, :, :L].cpu().float(),
                                       states[layer].kbuf[:, :, :L].float(), rtol=2e-2, atol=2e-2)
            torch.testing.assert_close(out.view(B, H * G, D).cpu().float(), res["out"].float(), rtol=2e-2, atol=2e-2)
    assert cache.gen_offset == steps
    if device_lengths:
        assert int(cache.kv_len_dev) == cache.sparse_end + steps
        assert int(cache.append_row_dev) == cache.sparse_end + steps - 1


def test_decode_capacity_is_an_error(gpu):
    case = make_golden.decode_small_case()
    cache = build_cache(case, gpu)
    cap = cache.buf_len - cache.sparse_end
    d = case["dims"]
    k = torch.zeros(d["B"], d["H"], 1, d["D"], dtype=torch.bfloat16, device=gpu)
    for _ in range(cap):
        cache.update_kv_cache(k, k, 0)
    with pytest.raises(RuntimeError, match="decode capacity"):
        cache.update_kv_cache(k, k, 0)


@pytest.mark.parametrize("fold", [False, True])
def test_selection_moves_buffers_only_when_folding(gpu, fold):
    """The drop-in get_retrieval_position_ids leaves both buffers untouched, as the reference's
    does (ids, offsets and counts only); with fold_hit_moves it moves the value buffer's hits, and
    the cache's get_value_cache then moves nothing a second time (same buffer as the reference
    sequence of selection + gather_copy_with_offsets)."""
    print(f"selection buffer side effects, fold_hit_moves={fold}", flush=True)
    case = make_golden.decode_small_case()
    q = case["q"].to(gpu).view(1, -1, 1, case["dims"]["D"])
    caches = []
    for f in (False, fold):
        cache = build_cache(case, gpu)
        cache.fold_hit_moves = f
        caches.append(cache)
    ref, cache = caches
    assert ref.fold_hit_moves is False
    kb, vb = cache.k_cache_buffer[0].clone(), cache.v_cache_buffer[0].clone()
    ids = cache.get_retrieval_position_ids(0, q)
    ref_ids = ref.get_retrieval_position_ids(0, q)
    torch.cuda.synchronize()
    assert torch.equal(ids, ref_ids)
    assert torch.equal(cache.k_cache_buffer[0].view(torch.int16), kb.view(torch.int16))
    hits = int(cache.cnts.sum())
    assert hits > 0
    moved = not torch.equal(cache.v_cache_buffer[0].view(torch.int16), vb.view(torch.int16))
    assert moved == fold
    cache.get_value_cache(0, ids)
    ref.get_value_cache(0, ref_ids)
    torch.cuda.synchronize()
    assert torch.equal(cache.v_cache_buffer[0].view(torch.int16), ref.v_cache_buffer[0].view(torch.int16))
