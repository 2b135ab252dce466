"""Host-side extent checks of the shim (no GPU): every offset a kernel will address must lie in
the tensors passed, so a stride mismatch raises instead of reaching the device."""
import pytest
import torch

from shadowkv_amd.kernels import shadowkv


def test_max_offset():
    assert shadowkv.max_offset((2, 32, 1, 128), (6144, 128, 128, 1)) == 6144 + 31 * 128 + 127
    assert shadowkv.max_offset((0, 4), (1, 1)) == -1
    with pytest.raises(ValueError):
        shadowkv.max_offset((2,), (-1,))


def test_rope_output_with_smaller_extent_than_input_strides_is_rejected():
    # q of a fused QKV row (stride 6144 per batch row) written into a compact [2, 4096] buffer:
    # the kernel addresses the output with the input's strides, so the last row would run past it.
    qkv = torch.empty(2, 1, 6144, dtype=torch.bfloat16, device="meta")
    q = qkv[..., :4096].view(2, 32, 1, 128)
    out = torch.empty(2, 4096, dtype=torch.bfloat16, device="meta").view(2, 32, 1, 128)
    sizes, strides = (2, 32, 1, 128), q.stride()
    need = shadowkv.max_offset(sizes, strides) + 1
    assert need > out.numel()          # the shape that faulted
    assert need <= qkv.numel()         # in place, inside the QKV buffer: fine


def test_auto_lanes_follows_the_measured_choices():
    """Two pipelined lanes only where a layer's value fetch outlasts three passes over its dense
    weights: the faster setting measured on one MI355X for each of these shapes."""
    from shadowkv_amd import decode_model as dm
    assert dm.auto_lanes(dm.LLAMA31_8B, 8, 2048) == 2   # 383 vs 271 tokens/s
    assert dm.auto_lanes(dm.LLAMA31_8B, 4, 2048) == 2   # 271 vs 262
    assert dm.auto_lanes(dm.LLAMA31_8B, 2, 2048) == 1   # 197 vs 160
    assert dm.auto_lanes(dm.GLM4_9B, 4, 2048) == 1      # 393 vs 261
    assert dm.auto_lanes(dm.LLAMA3_8B_1M, 1, 16384) == 1  # one sequence: nothing to pipeline
    assert dm.auto_lanes(dm.LLAMA31_8B, 7, 2048) == 1   # odd batch
    assert dm.auto_lanes(dm.LLAMA31_8B, 8, 2048, value_store="device") == 1  # no host link to hide: 741 vs 641
    # a chunk pool takes misses away: 12288 of 15304 landmarks kept, 608.5 (one lane) vs 526.3
    assert dm.auto_lanes(dm.LLAMA31_8B, 8, 2048, miss_fraction=dm.pool_miss_fraction(12288, 15304)) == 1
    assert dm.auto_lanes(dm.LLAMA31_8B, 8, 2048, miss_fraction=dm.pool_miss_fraction(4096, 15304)) == 2  # 487 vs 392


def test_lane_fetch_workgroups_follow_the_pool():
    """A lane's fetch workgroups shrink with the square of the expected miss fraction (the nearest
    multiple of 8, at least 16): the full 64 without a pool, 48 / 32 / 16 with 2048 / 4096 / 8192
    of 15304 chunks pooled."""
    from shadowkv_amd import decode_model as dm
    assert dm.pool_miss_fraction(None, 15304) == 1.0
    assert dm.pool_miss_fraction(20000, 15304) == 0.0
    got = [dm.lane_fetch_workgroups(dm.pool_miss_fraction(p, 15304)) for p in (None, 256, 2048, 4096, 8192, 12288)]
    assert got == [64, 64, 48, 32, 16, 16]


def test_side_streams_are_limited_to_the_hardware_queues(monkeypatch):
    """Three side streams per device at most, one per role, reused by every caller (a stand-in
    stream class, no device): with the compute stream, 4 streams = the hardware queues."""
    from shadowkv_amd import streams

    class FakeStream:
        def __init__(self, device=None):
            self.device = device

    monkeypatch.setattr(streams.torch.cuda, "Stream", FakeStream)
    monkeypatch.setattr(streams, "_streams", {})
    got = [streams.side_stream("cuda:0", r) for r in streams.ROLES for _ in range(3)]
    assert streams.side_streams_created() == 3 and len({id(s) for s in got}) == 3
    assert streams.side_stream("cuda:0") is streams.side_stream("cuda:0", "fetch")
    assert streams.side_streams_created() + 1 <= streams.MAX_STREAMS
    with pytest.raises(ValueError):
        streams.side_stream("cuda:0", "lane2")


def test_decoder_capture_stays_on_the_fixed_streams(monkeypatch):
    """SyntheticDecoder.capture hands torch.cuda.graph the process's capture side stream (a
    stand-in graph context records it), so a capture creates no stream of its own."""
    from shadowkv_amd import decode_model, streams

    class FakeStream:
        def __init__(self, device=None):
            self.device = device

    seen = []

    class FakeGraphCtx:
        def __init__(self, graph, stream=None, **kw):
            seen.append(stream)

        def __enter__(self):
            return self

        def __exit__(self, *exc):
            return False

    monkeypatch.setattr(streams.torch.cuda, "Stream", FakeStream)
    monkeypatch.setattr(streams, "_streams", {})
    monkeypatch.setattr(decode_model.torch.cuda, "CUDAGraph", lambda: object())
    monkeypatch.setattr(decode_model.torch.cuda, "graph", FakeGraphCtx)
    dec = decode_model.SyntheticDecoder.__new__(decode_model.SyntheticDecoder)
    dec.device = "cuda:0"
    dec.lanes = []
    dec.decode_steps = lambda tokens, steps: tokens
    dec.capture(torch.zeros(2, 1, dtype=torch.long), steps=2)
    assert seen == [streams.side_stream("cuda:0", "capture")]
    assert streams.side_streams_created() + 1 <= streams.MAX_STREAMS


def test_capture_frees_dead_cycles_first_and_holds_the_collector_off(monkeypatch):
    """A dead reference cycle (like a decoder whose lanes' RoPE closures refer back to it) is
    freed before the capture starts, the cyclic collector stays off while the decode steps are
    traced, and it is on again afterwards, also when tracing raises (stand-in graph context)."""
    import gc
    import weakref

    from shadowkv_amd import decode_model, streams

    class FakeStream:
        def __init__(self, device=None):
            self.device = device

    class FakeGraphCtx:
        def __init__(self, graph, stream=None, **kw):
            pass

        def __enter__(self):
            return self

        def __exit__(self, *exc):
            return False

    class Cycle:
        pass

    monkeypatch.setattr(streams.torch.cuda, "Stream", FakeStream)
    monkeypatch.setattr(streams, "_streams", {})
    monkeypatch.setattr(decode_model.torch.cuda, "CUDAGraph", lambda: object())
    monkeypatch.setattr(decode_model.torch.cuda, "graph", FakeGraphCtx)
    dead = Cycle()
    dead.me = dead
    ref = weakref.ref(dead)
    del dead
    seen = []

    def steps(tokens, steps):
        seen.append((gc.isenabled(), ref() is None))
        return tokens

    dec = decode_model.SyntheticDecoder.__new__(decode_model.SyntheticDecoder)
    dec.device = "cuda:0"
    dec.lanes = []
    dec.decode_steps = steps
    assert gc.isenabled()
    dec.capture(torch.zeros(2, 1, dtype=torch.long), steps=2)
    assert seen == [(False, True)] and gc.isenabled()

    def failing(tokens, steps):
        raise RuntimeError("traced step failed")

    dec.decode_steps = failing
    with pytest.raises(RuntimeError):
        dec.capture(torch.zeros(2, 1, dtype=torch.long))
    assert gc.isenabled()


def test_qkv_rope_weight_row_order():
    """The QKV weight (and bias) row order of the RoPE epilogue, on the CPU: each q and k head's rows
    interleaved as (0, 64, 1, 65, ...) so that a rotation pair (d, d + 64) sits in adjacent rows, v
    rows in place; GLM's weight (pairs (2i, 2i + 1) already adjacent) unchanged."""
    Hq, Hk, D = 3, 2, 128
    n = (Hq + 2 * Hk) * D
    w = torch.arange(n, dtype=torch.float32)[:, None].repeat(1, 5)  # row r holds r
    got = shadowkv.qkv_rope_weight(w, Hq, Hk, glm=False)[:, 0].long()
    for head in range(Hq + Hk):
        for i in range(64):
            assert got[head * D + 2 * i] == head * D + i
            assert got[head * D + 2 * i + 1] == head * D + 64 + i
    assert torch.equal(got[(Hq + Hk) * D:], torch.arange((Hq + Hk) * D, n))
    assert sorted(got.tolist()) == list(range(n))  # a permutation
    b = torch.arange(n, dtype=torch.float32)
    assert torch.equal(shadowkv.qkv_rope_weight(b, Hq, Hk, glm=False).long(), got)  # the bias alike
    assert torch.equal(shadowkv.qkv_rope_weight(w, Hq, Hk, glm=True), w)
    with pytest.raises(ValueError):
        shadowkv.qkv_rope_weight(w[:-1], Hq, Hk, glm=False)
