"""Decode throughput of the ShadowKV sparse decode path on one MI355X.

Workload (default): Llama-3.1-8B shape (32 layers, hidden 4096, FFN 14336, GQA 32/8, head_dim
128, vocab 128256), random-init bf16 weights, batch 8, 122880-token context per sequence,
ShadowKV rank 160, chunk 8, sparse budget 2048 (256 chunks), 48 outlier chunks, values of every
layer offloaded to pinned host memory (64.4 GB). The post-prefill state is synthesized from
seeded random tensors of the exact shapes (no 122K-token prefill/SVD is run); timing covers
greedy decode steps only. A step = one new token for all 8 sequences through all 32 layers;
by default the step is captured once in a HIP graph and the timed steps are graph replays.

Prints one JSON line. `roofline` is measured on the landmark-scoring kernel (the largest HBM
stream of the path) with HIP events on its stream around back-to-back launches over every
layer's live landmarks, right after the timed steps;
`host_link` reports the value fetch from pinned host memory measured in a separate
instrumented step; `cpu_baseline` times the CPU oracle's restatement of one layer's
hot-path ops at the same shapes on this host (a reported baseline only).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK = 2.5e15  # dense bf16 FLOP/s


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=16)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--batch", type=int, default=8)
    p.add_argument("--ctx", type=int, default=122880)
    p.add_argument("--budget", type=int, default=2048)
    p.add_argument("--chunk", type=int, default=8, help="rows per chunk (the reference's default is 8)")
    p.add_argument("--chunk-cache", type=int, default=None,
                   help="device chunk pool of this many slots per (b, h) and layer (>= budget/chunk); "
                        "default: the reference's slot reuse")
    p.add_argument("--layers", type=int, default=None, help="override the layer count (debug only)")
    p.add_argument("--model", choices=["llama31_8b", "glm4_9b", "llama3_8b_1m"], default="llama31_8b",
                   help="model shape of the decode workload (random weights): Llama-3.1-8B (the headline), "
                        "GLM-4-9B (2 kv heads of 16 query heads, GLM RoPE), Llama-3-8B-1M (RoPE theta 3.58e6)")
    p.add_argument("--lanes", type=int, default=None,
                   help="independent batch slices pipelined per layer (default: 2 where the value fetch outweighs the dense layers, see decode_model.auto_lanes)")
    p.add_argument("--pool-variant", type=int, nargs="+", default=[2048, 8192, 12288],
                   help="after the main (reference-mode) measurement, time the same decode with a device chunk "
                        "pool of each of these many slots per (b, h) and layer and report them in detail.chunk_pool "
                        "(0: skip; only with the breakdown)")
    p.add_argument("--encoded-variant", type=int, default=1,
                   help="also time the decode from a prompt state built by the device encoder and report it in "
                        "detail.encoded_state (0: skip; only with the breakdown)")
    p.add_argument("--state", choices=["synthetic", "encoded"], default="synthetic",
                   help="prompt state of the main measurement: synthesized random contents of the exact shapes, "
                        "or built by the device encoder from low-rank keys")
    p.add_argument("--no-act-epilogue", action="store_true",
                   help="form SiLU-and-mul outside the gate/up projection (the down projection reading "
                        "[gate | up], or the SiLU-and-mul kernel) instead of in its epilogue, for comparison")
    p.add_argument("--no-qkv-rope-epilogue", action="store_true",
                   help="rotate q/k and append the new token's k/v in their own kernel after the QKV projection "
                        "instead of in its epilogue, for comparison")
    p.add_argument("--separate-hit-moves", action="store_true",
                   help="move the hits of the key and value buffers in their own launches instead of in the "
                        "selection's last launch (the same work, for comparison)")
    p.add_argument("--no-graph", action="store_true", help="time eager steps instead of HIP graph replays")
    p.add_argument("--graph-steps", type=int, default=8,
                   help="decode steps per captured graph (one continuous lane pipeline across steps); "
                        "reduced to a divisor of --steps")
    p.add_argument("--workload", choices=["decode", "rebuild", "attention", "select", "linear", "encode", "pool",
                                          "hostlink", "envelope"],
                   default="decode",
                   help="decode: the 32-layer decode step; rebuild: the low-rank key rebuild + RoPE kernel alone; "
                        "attention: the sparse decode attention alone; select: the fused chunk selection alone; "
                        "linear: the skinny decode projections alone (next to torch's GEMM); encode: the prefill "
                        "encoder (low-rank factors, chunk statistics, outliers, landmarks, initial selection); "
                        "pool: one layer's sparse step on drifting queries with and without a device chunk pool; "
                        "hostlink: pinned-host read rate of SDMA copies and of the value-fetch gather; "
                        "envelope: HBM streaming rate of the scoring kernel, a device copy and the read-only probe by "
                             "transfer size")
    p.add_argument("--rebuild-batches", type=int, nargs="+", default=[1, 8, 32, 48])
    p.add_argument("--linear-rows", type=int, nargs="+", default=[4, 8],
                   help="token rows of the linear workload (the skinny kernel takes at most 16)")
    p.add_argument("--cpu-runs", type=int, default=10)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-breakdown", action="store_true")
    p.add_argument("--summarize-trace", metavar="CSV",
                   help="summarise a rocprofv3 --kernel-trace CSV of a decode run of this script (made with the "
                        "same --model/--batch/--ctx/--budget/--steps/--warmup) into profiles/, then exit")
    p.add_argument("--value-store", choices=["host", "device"], default="host",
                   help="where the value store lives: pinned host memory (the workload as configured) or device "
                        "memory (HBM; the whole store fits MI355X's 288 GB)")
    p.add_argument("--device-store-variant", type=int, default=1,
                   help="also time the same decode with the value store in device memory, reported in detail "
                        "(0 to skip)")
    p.add_argument("--device-store-batch", type=int, default=-1,
                   help="and once more at this batch with the value store in device memory (default: 24, the "
                        "reference's published setting, for the Llama-3.1-8B shape at ctx 122880, else none; "
                        "0 to skip)")
    p.add_argument("--two-stream-fetch", action="store_true",
                   help="one-lane decoders: value fetch on the copy stream and key rebuild on the compute stream "
                        "(the reference's arrangement) instead of one fused launch on the compute stream; two-lane "
                        "decoders: the lanes' fetches on one shared fetch stream and their key rebuilds on one shared "
                        "rebuild stream instead of each lane's fused launch on a side stream of its own")
    return p.parse_args()


class KernelTimer:
    """Brackets every call of one shim function with HIP events on the current stream. The host
    first waits for that stream's earlier work (only that stream: the other streams' work keeps
    running beside the timed call), because a start event queued behind a cross-stream wait can be
    timestamped before the wait resolves and would then count the wait as the call's time; then a
    short device spin holds the stream while the start event and the call are queued, so the host's
    launch latency does not count either."""

    def __init__(self, module, name: str):
        import torch
        self.torch, self.module, self.name = torch, module, name
        self.orig = getattr(module, name)
        self.pairs = []
        self.active = False

        def wrapped(*a, **kw):
            if not self.active:
                return self.orig(*a, **kw)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.current_stream().synchronize()
            torch.cuda._sleep(100000)  # ~40 us of device spin: the call is queued before the stream resumes
            s.record()
            out = self.orig(*a, **kw)
            e.record()
            self.pairs.append((s, e))
            return out

        setattr(module, name, wrapped)

    def mean_ms(self) -> float:
        ms = [s.elapsed_time(e) for s, e in self.pairs]
        if not ms or min(ms) <= 0.0:
            raise RuntimeError(f"no usable event timings for {self.name}")
        return statistics.fmean(ms)


def logits_bytes(BH: int, G: int, n: int, D: int = 128) -> int:
    """Algorithmic HBM bytes of one score_logits launch: landmarks + queries read, logits and
    per-256-column (max, sum) partials written."""
    tiles = (n + 255) // 256
    return BH * (n * D * 2 + G * D * 2 + G * n * 2 + G * tiles * 8)


def scoring_launch_ms(model, rounds: int = 8, sweeps: int = 4):
    """Average duration of the landmark-scoring kernel on the live decode state: `sweeps` passes
    over the layers, one launch per layer over that layer's landmarks, captured in a HIP graph and
    replayed `rounds` times between HIP events (no host launch cost in the figure; the events
    bracket the replays on the stream the kernels run on). Runs right after the timed decode
    steps."""
    import torch
    from shadowkv_amd.kernels import shadowkv

    cache = model.cache
    B, H, G, D = cache.batch_size, cache.num_key_value_heads, cache.num_key_value_groups, cache.head_dim
    n = cache.k_landmark.shape[-2]
    q = torch.randn(B, H * G, 1, D, device=cache.device).to(torch.bfloat16)
    L = cache.num_layers

    def launch(i):
        layer = i % L
        shadowkv.score_logits(q, cache.k_landmark[layer], cache.gemm_o, cache.norm, cache.sum, B * H, G, n, D,
                              1.0 / math.sqrt(128))

    t = gpu_time_per_call(launch, sweeps * L, rounds)
    return (t * 1e3,
            f"HIP events around {rounds} replays of a HIP graph of {sweeps * L} back-to-back launches ({sweeps} "
            f"sweeps over the layers, each launch on its layer's live landmarks), after the timed steps")


def a1a2_bytes(BH: int, G: int, n: int, S: int, D: int = 128) -> int:
    """Algorithmic HBM bytes of the scoring + top-k unit per launch pair: landmarks and queries read,
    the GQA-max scores and the selected ids written."""
    return BH * (n * D * 2 + G * D * 2 + n * 2 + S * 8)


def a1a2_unit_ms(model, rounds: int = 8, sweeps: int = 2):
    """Average duration of the scoring + selection unit (score_logits, then select_chunks: softmax
    tail, GQA max, top-k, id gather, reorder) on lane 0's live decode state: `sweeps` passes over
    the layers, one pair per layer, captured in a HIP graph and replayed between HIP events. Runs
    after the timed decode steps (it re-selects on the layers' slots)."""
    import torch
    from shadowkv_amd.kernels import shadowkv

    cache = model.cache
    B, H, G, D = cache.batch_size, cache.num_key_value_heads, cache.num_key_value_groups, cache.head_dim
    BH, S, n = B * H, cache.select_sets, cache.k_landmark.shape[-2]
    q = torch.randn(B, H * G, 1, D, device=cache.device).to(torch.bfloat16)
    L = cache.num_layers

    def launch(i):
        layer = i % L
        shadowkv.score_logits(q, cache.k_landmark[layer], cache.gemm_o, cache.norm, cache.sum, BH, G, n, D,
                              1.0 / math.sqrt(128))
        shadowkv.select_chunks(cache.gemm_o, cache.norm, cache.sum, BH, G, n, cache.k_landmark_idx[layer].view(BH, n),
                               S, cache.chunks, cache.position_ids[layer].view(BH, -1), cache.offsets, cache.cnts,
                               out_scores=cache.chunk_attn, workspace=cache.select_workspace)

    t = gpu_time_per_call(launch, sweeps * L, rounds)
    return (t * 1e3,
            f"HIP events around {rounds} replays of a HIP graph of {sweeps * L} back-to-back scoring + selection "
            f"pairs ({sweeps} sweeps over the layers of one lane, each on its layer's live landmarks and slots), "
            f"after the timed steps")


# The kernels of each sparse-step operation, by kernel-name prefix (rocprofv3 kernel traces).
TRACE_OPS = {
    "score_logits": ("logits_kernel", "logits_rows_kernel"),
    "select_chunks": ("softmax_vec_kernel", "softmax_kernel", "select_kernel", "part_hist_kernel", "part_emit_kernel",
                      "select_finish_kernel"),
    "gather_copy_d2d_with_offsets": ("compact_hits_kernel",),
    "gather_copy_with_offsets": ("gather_chunks_kernel",),
    "rebuild_k_rope": ("rebuild_kernel",),
    "fetch_misses_rebuild_k_rope": ("fetch_rebuild_kernel",),
    "sparse_attn_decode": ("attn_split_kernel", "attn_combine_kernel"),
}


def summarize_trace(csv_path: str, layers: int, lanes: int, warmup: int, steps: int) -> dict:
    """Per-kernel durations inside the timed decode steps of a rocprofv3 kernel trace (CSV) of this
    script's decode run: the window is the logits launches of the timed steps (one per layer and
    lane per step, after `warmup` eager steps). Per operation of the sparse step, the device time
    per lane-layer (the sum of its kernels' durations per step / (layers x lanes))."""
    import collections
    import csv

    rows = sorted(csv.DictReader(open(csv_path)), key=lambda r: int(r["Start_Timestamp"]))
    li = [i for i, r in enumerate(rows) if any(k in r["Kernel_Name"] for k in TRACE_OPS["score_logits"])]
    per = layers * lanes
    a, b = li[warmup * per], li[(warmup + steps) * per]
    win = rows[a:b]
    span_ms = (int(rows[b]["Start_Timestamp"]) - int(win[0]["Start_Timestamp"])) / 1e6 / steps
    agg = collections.defaultdict(list)
    for r in win:
        name = r["Kernel_Name"].replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]
        agg[name].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    kernels = {k: {"launches_per_step": round(len(v) / steps, 2), "avg_us": round(sum(v) / len(v), 2),
                   "ms_per_step": round(sum(v) / steps / 1e3, 4)} for k, v in sorted(agg.items())}
    ops = {}
    for op, prefixes in TRACE_OPS.items():
        tot = sum(sum(v) for k, v in agg.items() if k.startswith(prefixes))
        if tot:
            ops[op] = round(tot / steps / per, 2)
    return {"trace_window_ms_per_step": round(span_ms, 3), "kernels": kernels, "op_us_per_lane_layer": ops}


def trace_summary_path(args) -> Path:
    """The committed kernel-trace summary of this decode workload's timed steps."""
    return ROOT / "profiles" / f"decode_{args.model}_b{args.batch}_ctx{args.ctx}_trace.json"


def trace_workload(args, lanes: int) -> dict:
    return {"model": args.model, "batch": args.batch, "ctx": args.ctx, "budget": args.budget, "chunk": args.chunk,
            "lanes": lanes}


def apply_trace_summary(kernels: list, args, lanes: int) -> None:
    """In-step figures of the kernel table from the committed kernel trace of this workload's timed
    graph replays (when one exists for it): the eager instrumented figure moves to
    eager_instrumented_us."""
    path = trace_summary_path(args)
    if not path.exists():
        return
    rec = json.loads(path.read_text())
    if rec.get("workload") != trace_workload(args, lanes):
        return
    ops = rec["op_us_per_lane_layer"]
    for k in kernels:
        if not k["trace_ops"] or not all(o in ops for o in k["trace_ops"]):
            continue
        us = sum(ops[o] for o in k["trace_ops"])
        k["eager_instrumented_us"] = k["in_step_us"]
        k["in_step_us"] = round(us, 2)
        k["in_step_frac"] = round(k["algorithmic_bytes"] / us / 1e3 / k["peak"], 4)
        k["in_step_source"] = (f"{path.relative_to(ROOT)}: rocprofv3 kernel trace of the timed graph replays of "
                               f"this workload (device time per lane-layer; not measured in this run)")


def host_cpu() -> tuple[int, str]:
    """(threads usable by this process, CPU model name from /proc/cpuinfo)."""
    try:
        threads = len(os.sched_getaffinity(0))
    except AttributeError:
        threads = os.cpu_count() or 1
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return max(1, threads), model


def cpu_baseline(model, runs: int) -> dict:
    """The CPU oracle on one layer's hot-path ops at the workload's shapes (layer 0 state), on every
    CPU this process may use."""
    import torch
    import oracle

    threads, cpu_model = host_cpu()
    torch.set_num_threads(threads)
    states = []
    for lane in model.lanes:  # layer-0 state of every batch slice: the whole batch
        c = lane.cache
        states.append(oracle.LayerState(
            U=c.U[0].cpu(), SV=c.SV[0].cpu(), landmarks=c.k_landmark[0].cpu(), landmark_idx=c.k_landmark_idx[0].cpu(),
            host_v=c.v_cache_cpu[0], kbuf=c.k_cache_buffer[0].cpu(), vbuf=c.v_cache_buffer[0].cpu(),
            position_ids=c.position_ids[0].cpu(), prefill_local=c.prefill_local, sparse_start=c.sparse_start,
            sparse_end=c.sparse_end, chunk=c.chunk_size, budget=c.sparse_budget, ctx=c.prefill, buf_len=c.buf_len))
    cache = model.cache
    B = model.batch
    H, D, Hq = cache.num_key_value_heads, cache.head_dim, cache.num_attention_heads
    cos_sin = model.cos_sin.cpu()
    g = torch.Generator().manual_seed(5)
    times = []
    for i in range(3 + runs):
        dt = 0.0
        for st, lane in zip(states, model.lanes):
            b = lane.cache.batch_size
            q = torch.randn(b, Hq, D, generator=g).to(torch.bfloat16)
            k = torch.randn(b, H, D, generator=g).to(torch.bfloat16)
            v = torch.randn(b, H, D, generator=g).to(torch.bfloat16)
            t0 = time.perf_counter()
            oracle.decode_layer_step(st, q, k, v, cos_sin, gen_offset=0)
            dt += time.perf_counter() - t0
        if i >= 3:
            times.append(dt)
    layer_s = statistics.median(times)
    return {"value": round(B / (layer_s * cache.num_layers), 3), "unit": "tokens/s", "cores": threads,
            "kind": "port", "cpu_model": cpu_model, "os_cpu_count": os.cpu_count(),
            "sample": (f"oracle (CPU torch/numpy) restatement of one layer's hot-path ops (scoring, GQA max, top-k, "
                       f"reorder, value fetch, key compaction, rebuild+RoPE, attention) at batch {B}, ctx "
                       f"{cache.prefill}, layer-0 state, torch threads {threads}; median of {runs} runs after 3 "
                       f"warmups = {layer_s * 1e3:.1f} ms/layer, scaled to {cache.num_layers} layers; dense layers "
                       f"excluded; reported baseline only")}


def single_layer_inputs(seed: int = 8192):
    """Seeded inputs of the single-layer decode workload: batch 1, 8 kv heads x 4 query heads,
    head_dim 128, ctx 8192; pre-RoPE keys A(8192 x 160).B(160 x 1024) + 0.05 N(0,1) with A, B of
    standard deviation 1/sqrt(160); values, the last prompt query and the decode token's q, k, v
    ~ N(0,1); bf16 CPU tensors."""
    import torch
    g = torch.Generator().manual_seed(seed)
    B, H, G, D, ctx, rank = 1, 8, 4, 128, 8192, 160
    A = torch.randn(ctx, rank, generator=g) / rank ** 0.5
    Bm = torch.randn(rank, H * D, generator=g) / rank ** 0.5
    k_pre = (A @ Bm + 0.05 * torch.randn(ctx, H * D, generator=g)).view(1, ctx, H, D).transpose(1, 2)
    k_pre = k_pre.to(torch.bfloat16).contiguous()
    v = torch.randn(B, H, ctx, D, generator=g).to(torch.bfloat16)
    q_last = torch.randn(B, H * G, 1, D, generator=g).to(torch.bfloat16)
    q = torch.randn(B, H * G, D, generator=g).to(torch.bfloat16)
    k_new = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    v_new = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    return dict(k_pre=k_pre, v=v, q_last=q_last, q=q, k_new=k_new, v_new=v_new, H=H, G=G, D=D, ctx=ctx, rank=rank)


def single_layer_gpu_ms(runs: int = 20) -> dict:
    """The single-layer workload on the product path: the device encoder builds the layer's state
    (get_svd + prefill_kv_cache), then one decode step of the layer through ShadowAttention.decode
    (scoring, selection, value fetch from pinned host memory, key rebuild, attention) is timed with
    HIP events, median over `runs` steps."""
    import types
    import torch
    from shadowkv_amd.models.attention import ShadowAttention
    from shadowkv_amd.models.kvcache import ShadowKVCache_CPU
    from shadowkv_amd.models.tensor_op import build_cos_sin_cache

    x = single_layer_inputs()
    H, G, D, ctx = x["H"], x["G"], x["D"], x["ctx"]
    dev = torch.device("cuda")
    cfg = types.SimpleNamespace(num_attention_heads=H * G, num_key_value_heads=H, hidden_size=H * G * D,
                                num_hidden_layers=1)
    cache = ShadowKVCache_CPU(cfg, batch_size=1, max_length=ctx, device="cuda", sparse_budget=2048, chunk_size=8,
                              rank=x["rank"], max_decode_len=runs + 8)
    cos_sin = build_cos_sin_cache(ctx + 64, 500000.0, D, device=dev)

    # the new token arrives rotated (the model's RoPE runs before the attention handler)
    attn = ShadowAttention(cache, G, D, H * G * D,
                           lambda q, k, p: (q.view(1, -1, H * G, D).transpose(1, 2), k.view(1, -1, H, D).transpose(1, 2)),
                           None, cos_sin)
    from shadowkv_amd.models.tensor_op import apply_rotary_pos_emb_cuda
    k_pre, v = x["k_pre"].to(dev), x["v"].to(dev)
    pos = torch.arange(ctx, device=dev).view(1, 1, ctx).expand(1, H, ctx)
    q_pos = torch.full((1, H * G, 1), ctx - 1, dtype=torch.int64, device=dev)
    q_last = apply_rotary_pos_emb_cuda(x["q_last"].to(dev), cos_sin, q_pos)
    cache.get_svd(k_pre, 0)
    cache.prefill_kv_cache(v, 0, apply_rotary_pos_emb_cuda(k_pre, cos_sin, pos), q_last)
    cache.H2D()
    q = x["q"].to(dev).reshape(1, 1, -1)
    k = x["k_new"].to(dev).reshape(1, 1, -1)
    vv = x["v_new"].to(dev).reshape(1, H, 1, D)
    ms = []
    for i in range(runs + 2):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        attn.decode(q, k, vv, None, 0)
        e.record()
        e.synchronize()
        if i >= 2:
            ms.append(s.elapsed_time(e))
    return {"gpu_ms_per_step": round(statistics.median(ms), 4), "n_landmarks": int(cache.k_landmark.shape[-2]),
            "hits_last_step": int(cache.cnts.sum())}


def single_layer_cpu_ms(runs: int) -> dict:
    """The CPU oracle's single-layer decode step at the single-layer workload's shape (state encoded
    by the oracle: full SVD, bf16 cosine outliers), median of `runs` steps after 3 warmups."""
    import copy
    import torch
    import oracle

    threads, _ = host_cpu()
    torch.set_num_threads(threads)
    x = single_layer_inputs()
    cs = oracle.build_cos_sin_cache(x["ctx"] + 64, 500000.0)
    st0 = oracle.encode_layer(x["k_pre"], x["v"], x["q_last"], cs, rank=x["rank"], chunk=8, budget=2048)
    times = []
    for i in range(3 + runs):
        st = copy.deepcopy(st0)
        t0 = time.perf_counter()
        oracle.decode_layer_step(st, x["q"], x["k_new"], x["v_new"], cs)
        if i >= 3:
            times.append(time.perf_counter() - t0)
    return {"cpu_ms_per_step": round(statistics.median(times) * 1e3, 3), "cores": threads, "kind": "port",
            "n_landmarks": int(st0.landmarks.shape[-2])}


def breakdown(model, tok) -> dict:
    """One instrumented step: per-op device time of the sparse path (HIP events on the stream each
    op runs on, in the pipelined eager step), the host-link rate, and each selection's offsets and
    hit counts (for replaying the layer's kernels alone)."""
    import torch
    from shadowkv_amd.kernels import shadowkv

    names = ["apply_rotary_pos_emb_new", "score_logits", "select_chunks", "softmax_gqa_max", "topk_gather",
             "pool_assign", "gather_copy_with_offsets", "gather_copy_misses_to_slots",
             "gather_copy_d2d_with_offsets", "rebuild_k_rope", "sparse_attn_decode"]
    timers = {n: KernelTimer(shadowkv, n) for n in names}
    cache = model.cache
    snaps = []  # (selected chunks, device copies of offsets and hit counts) per call, in call order
    pooled = cache.pooled
    sel_name = "pool_assign" if pooled else "select_chunks"
    orig_select = timers[sel_name].orig

    def select_and_snapshot(*a, **kw):
        out = orig_select(*a, **kw)
        if pooled:  # pool_assign(selected [rows, S], ..., cnts)
            snaps.append((a[0].numel(), None, a[9].clone()))
        else:  # select_chunks(..., rows, ..., select_sets, ..., position_ids, offsets, cnts)
            snaps.append((a[3] * a[7], a[10].clone(), a[11].clone()))
        return out

    timers[sel_name].orig = select_and_snapshot
    for t in timers.values():
        t.active = True
    # (the instrumented step times the value fetch and the key rebuild as separate calls, so
    # one-lane decoders take the two-stream arrangement for it)
    one_stream = [lane.cache.one_stream_fetch for lane in model.lanes]
    for lane in model.lanes:
        lane.cache.one_stream_fetch = False
    torch.cuda.synchronize()
    model.decode_step(tok)
    torch.cuda.synchronize()
    for lane, v in zip(model.lanes, one_stream):
        lane.cache.one_stream_fetch = v
    timers[sel_name].orig = orig_select
    for t in timers.values():
        t.active = False
        setattr(shadowkv, t.name, t.orig)
    ops = {n: round(t.mean_ms() * 1e3, 2) for n, t in timers.items() if t.pairs}
    chunk_bytes = cache.chunk_size * cache.head_dim * 2
    fetch_ms = timers["gather_copy_misses_to_slots" if pooled else "gather_copy_with_offsets"].mean_ms()
    total_sel = statistics.fmean(t for t, _, _ in snaps)
    miss_mean = statistics.fmean(t - int(c.sum()) for t, _, c in snaps)
    # calls run layer by layer, the lanes in order within a layer: call k = (layer k // lanes, lane k % lanes)
    nl = len(model.lanes)
    per_layer = {(k // nl, k % nl): (o, c) for k, (_, o, c) in enumerate(snaps)}
    return {"op_us_per_layer": ops, "hit_rate": round(1 - miss_mean / total_sel, 4),
            "host_link": {"bytes_per_layer": int(miss_mean * chunk_bytes),
                          "GBps": round(miss_mean * chunk_bytes / (fetch_ms * 1e-3) / 1e9, 2),
                          "note": "value fetch (zero-copy miss gather from pinned host memory) per lane-layer, "
                                  "HIP events on the fetch stream in one eager pipelined step"}}, per_layer


def host_link_peak_gbps(nbytes: int = 256 << 20, reps: int = 5) -> float:
    """Host-to-device rate of an SDMA copy (hipMemcpyAsync) of `nbytes` of pinned host memory."""
    import torch
    src = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        dst.copy_(src, non_blocking=True)
    e.record()
    e.synchronize()
    gbps = nbytes * reps / (s.elapsed_time(e) * 1e-3) / 1e9
    del src, dst
    return gbps


def measured_peaks() -> dict:
    """The nominal peaks (8 TB/s HBM, 2.5 PFLOP/s dense bf16 MFMA) checked on this GPU with the
    library's probes: a read-only stream of 1 GiB (contiguous non-temporal wave loads, four 64 KB
    tiles per workgroup, buffers rotated so reads come from HBM) and back-to-back bf16 MFMAs on
    register operands (2048 workgroups of 4 waves, 32x32x16 instructions). Reported beside the
    rooflines, which keep the published peaks."""
    import torch
    from shadowkv_amd.kernels import shadowkv

    nbytes = 1 << 30
    src = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(2)]
    for x in src:
        x.fill_(0x5a)
    sink = torch.empty(nbytes // shadowkv.HBM_PROBE_TILE_BYTES // 4 * 4096, dtype=torch.uint8, device="cuda")
    t = gpu_time_per_call(lambda i: shadowkv.hbm_read_probe(src[i % 2], 4, "contiguous", sink, True), 8)
    hbm = nbytes / t / 1e9
    del src, sink
    wgs, iters = 2048, 1024
    msink = torch.empty(wgs * 256, dtype=torch.float32, device="cuda")
    flops = shadowkv.mfma_peak_probe(wgs, iters, msink)
    t = gpu_time_per_call(lambda i: shadowkv.mfma_peak_probe(wgs, iters, msink), 8)
    mfma = flops / t / 1e12
    torch.cuda.empty_cache()
    return {"hbm_read_GBps": round(hbm, 1), "hbm_frac_of_nominal": round(hbm / HBM_PEAK_GBS, 4),
            "hbm_probe": "read-only stream of 1 GiB, contiguous non-temporal wave loads, 4 x 64 KB tiles per workgroup",
            "mfma_bf16_TFLOPs": round(mfma, 1), "mfma_frac_of_nominal": round(mfma * 1e12 / MFMA_BF16_PEAK, 4),
            "mfma_probe": "v_mfma_f32_32x32x16_bf16 back to back on register operands, 4 chains per wave, "
                          "2048 workgroups of 4 waves"}


def kernel_table(model, per_layer, ops_in_step, link_peak, sweeps: int = 2) -> list:
    """Every kernel of the sparse step at the workload's shapes, each alone: `sweeps` passes over
    the layers of lane 0 with that layer's live state (landmarks, U/SV, buffers, host store) and the
    offsets / hit counts its selection produced in the instrumented step, captured in a HIP graph
    and replayed between HIP events. Beside each, the in-step time (HIP events in the pipelined
    eager step), the algorithmic bytes of one launch and the fraction of the bounding roofline."""
    import torch
    from shadowkv_amd.kernels import shadowkv

    lane = model.lanes[0]
    c = lane.cache
    L = c.num_layers
    B, H, G, D = c.batch_size, c.num_key_value_heads, c.num_key_value_groups, c.head_dim
    BH, S, ch, R = B * H, c.select_sets, c.chunk_size, c.rank
    n = c.k_landmark.shape[-2]
    chunk_bytes = ch * D * 2
    offs = [per_layer[(l, 0)][0].clone() for l in range(L)]
    cnts = [per_layer[(l, 0)][1].clone() for l in range(L)]
    hits = [int(x.sum()) for x in cnts]
    mean_hits = statistics.fmean(hits)
    mean_miss = BH * S - mean_hits
    kv_len = c.sparse_end + c.gen_offset
    q = torch.randn(B, H * G, 1, D, device=c.device).to(torch.bfloat16)
    qa = q.view(B, H * G, D)
    out = torch.empty(B, H * G, D, dtype=torch.bfloat16, device=c.device)
    ws = shadowkv.sparse_attn_workspace(B, H * G, c.buf_len, c.device)
    reps = sweeps * L

    def t_us(fn):
        return gpu_time_per_call(fn, reps, rounds=4) * 1e6

    res = []

    def add(kernel, bound, nbytes, iso_us, step_us, peak, unit="GB/s", extra=None, ops=()):
        e = {"kernel": kernel, "bound": bound, "algorithmic_bytes": int(nbytes), "isolated_us": round(iso_us, 2),
             "in_step_us": round(step_us, 2) if step_us else None,
             "isolated_GBps": round(nbytes / iso_us / 1e3, 1), "peak": round(peak, 1), "unit": unit,
             "isolated_frac": round(nbytes / iso_us / 1e3 / peak, 4),
             "in_step_frac": round(nbytes / step_us / 1e3 / peak, 4) if step_us else None,
             "in_step_source": "eager instrumented step (HIP events around the call, its stream drained and held "
                               "by a device spin first; not the timed graph's schedule)",
             "trace_ops": list(ops)}
        if extra:
            e.update(extra)
        res.append(e)

    # a1: landmark scoring
    score_us = t_us(lambda i: shadowkv.score_logits(q, c.k_landmark[i % L], c.gemm_o, c.norm, c.sum, BH, G, n, D,
                                                    1.0 / math.sqrt(128)))
    lb = logits_bytes(BH, G, n)
    add("score_logits (a1 logits + per-tile softmax partials)", "hbm", lb, score_us, ops_in_step.get("score_logits"),
        HBM_PEAK_GBS, ops=("score_logits",))
    # a1 tail + a2 + a3: softmax normalisation, GQA max, top-k, id gather, reorder (the selection chain)
    sel_us = t_us(lambda i: shadowkv.select_chunks(
        c.gemm_o, c.norm, c.sum, BH, G, n, c.k_landmark_idx[i % L].view(BH, n), S, c.chunks,
        c.position_ids[i % L].view(BH, -1), c.offsets, c.cnts, out_scores=c.chunk_attn, workspace=c.select_workspace))
    sel_bytes = BH * (G * n * 2 + G * ((n + 255) // 256) * 8 + n * 8 + n * 2 + S * 8 * 2 + S * 4)
    add("select_chunks (softmax tail + GQA max + top-k + id gather + reorder)", "latency", sel_bytes, sel_us,
        ops_in_step.get("select_chunks"), HBM_PEAK_GBS, ops=("select_chunks",))
    # the survey's a1+a2 unit: landmarks + q read, scores and ids written, over scoring + selection
    unit_bytes = a1a2_bytes(BH, G, n, S)
    step_unit = (ops_in_step.get("score_logits", 0) + ops_in_step.get("select_chunks", 0)) or None
    add("a1+a2 unit (scoring + selection chain)", "hbm", unit_bytes, score_us + sel_us, step_unit, HBM_PEAK_GBS,
        ops=("score_logits", "select_chunks"))
    # a4/a5: in-buffer hit compaction (K and V: two launches of this per layer)
    comp_bytes = 2 * mean_hits * chunk_bytes
    comp_us = t_us(lambda i: shadowkv.gather_copy_d2d_with_offsets(
        c.v_cache_buffer[i % L], offs[i % L], cnts[i % L], B, H, int(c.sparse_budget * D), c.kernel_offset,
        c.kernel_stride, S))
    folded = getattr(c, "fold_hit_moves", False) and not c.pooled
    # the timed step's value fetch and key rebuild as one launch (fetch_rebuild_kernel), after a
    # selection that moved both buffers' hits
    fused_fetch = all(ln.cache.one_stream_active() for ln in model.lanes)
    add("gather_copy_d2d_with_offsets (hit compaction, per buffer)", "hbm", comp_bytes, comp_us,
        ops_in_step.get("gather_copy_d2d_with_offsets"), HBM_PEAK_GBS,
        ops=() if fused_fetch else ("gather_copy_d2d_with_offsets",),
        extra={"mean_hits": round(mean_hits, 1),
               "in_step": ("none in the timed step: both buffers' hits move inside the select_chunks launch"
                           if fused_fetch else
                           "key buffer only: the value buffer's hits move inside the select_chunks launch"
                           if folded else "both buffers")})
    # a4: value fetch of the misses from pinned host memory
    fetch_bytes = mean_miss * chunk_bytes
    fetch_us = t_us(lambda i: shadowkv.gather_copy_with_offsets(
        c.v_cache_cpu[i % L], c.v_cache_buffer[i % L], None, offs[i % L], cnts[i % L], None, B, H,
        int(c.max_ctx_chunks_len * D), int(c.sparse_budget * D), c.kernel_offset, c.kernel_stride, S,
        misses_only=True))
    add("gather_copy_with_offsets (value fetch of the misses, host link)", "host link", fetch_bytes, fetch_us,
        ops_in_step.get("gather_copy_with_offsets"), link_peak,
        ops=("fetch_misses_rebuild_k_rope",) if fused_fetch else ("gather_copy_with_offsets",),
        extra={"peak_source": "SDMA copy (hipMemcpyAsync) of 256 MiB pinned host memory, measured in this run",
               "nominal_link_GBps": 64.0,
               **({"in_step": "the timed step's one launch of the value fetch and the key rebuild "
                              "(fetch_misses_rebuild_k_rope), host-link bound"} if fused_fetch else {})})
    # a5-a7: low-rank key rebuild + RoPE of the miss rows
    rows = mean_miss * ch
    rb_bytes = rows * (R * 2 + D * 2 + D * 2) + BH * (R * D * 2 + S * 8)
    rb_us = t_us(lambda i: shadowkv.rebuild_k_rope(c.U[i % L], c.SV[i % L], c.position_ids[i % L], cnts[i % L],
                                                   model.cos_sin, c.k_cache_buffer[i % L], c.sparse_start, ch))
    flops = 2 * rows * R * D
    add("rebuild_k_rope (gather-GEMM on MFMA + RoPE epilogue)", "hbm", rb_bytes, rb_us,
        ops_in_step.get("rebuild_k_rope"), HBM_PEAK_GBS, ops=() if fused_fetch else ("rebuild_k_rope",),
        extra={"mfma_flops": int(flops), "isolated_mfma_util": round(flops / (rb_us * 1e-6) / MFMA_BF16_PEAK, 4),
               **({"in_step": "runs inside the value fetch's launch in the timed step (no separate "
                              "duration)"} if fused_fetch else {})})
    # a8: sparse attention (split + merge launches)
    at_bytes = BH * 2 * kv_len * D * 2 + 2 * B * H * G * D * 2
    at_us = t_us(lambda i: shadowkv.sparse_attn_decode(qa, c.k_cache_buffer[i % L][:, :, :kv_len],
                                                       c.v_cache_buffer[i % L][:, :, :kv_len], kv_len, out, ws))
    add("sparse_attn_decode (split + merge)", "hbm", at_bytes, at_us, ops_in_step.get("sparse_attn_decode"),
        HBM_PEAK_GBS, extra={"kv_len": kv_len}, ops=("sparse_attn_decode",))
    return res


# Footprint that the input sets of one timed loop must exceed, so that back-to-back launches read
# HBM and not the 256 MB last-level cache (MALL) that sits in front of it.
COLD_FOOTPRINT = 1 << 30


def cold_sets(bytes_per_launch: int) -> int:
    """Number of distinct input sets to rotate through so their total exceeds COLD_FOOTPRINT."""
    return max(1, -(-COLD_FOOTPRINT // max(1, bytes_per_launch)))


def gpu_time_per_call(fn, reps: int, rounds: int = 5) -> float:
    """Seconds per call of `fn` on the GPU: `reps` calls captured in one HIP graph, replayed
    `rounds` times between HIP events, so host launch cost does not enter the figure. `fn` takes
    the call's index, so a caller can rotate through several input sets."""
    import torch

    from shadowkv_amd.streams import capture_graph

    fn(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with capture_graph(g, torch.cuda.current_device()):
        for i in range(reps):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(rounds):
        g.replay()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) * 1e-3 / (rounds * reps)


def pool_variant(args, shape, P: int) -> dict:
    """The same decode workload with a device chunk pool (f3: P >= S chunk slots per (b, h) and
    layer kept across steps, least recently used replaced; the same chunks are selected and the
    attention outputs equal the reference mode's to bf16 summation order), timed as the main
    measurement. The reference-mode
    decoder is released first (its pinned host store is 64 GiB at batch 8)."""
    import gc
    import torch
    from shadowkv_amd import decode_model

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch._C._host_emptyCache()
    # Untimed steps until the pool is full: each step brings in the selection's misses, so a pool of
    # P slots fills in about P / S steps (a little more, as the hits grow); the timed steps then
    # see the steady-state hit rate.
    S = args.budget // args.chunk
    warm = max(args.warmup, math.ceil(1.25 * P / S) + 1)
    # lanes for the pool's share of the fetch (about ctx / chunk landmarks per row)
    lanes = decode_model.auto_lanes(shape, args.batch, args.budget,
                                    miss_fraction=decode_model.pool_miss_fraction(P, args.ctx // args.chunk))
    log(f"chunk pool variant: {P} slots per (b, h) and layer, {lanes} lane(s), {warm} untimed steps")
    try:
        pm = decode_model.SyntheticDecoder(shape, args.batch, args.ctx, sparse_budget=args.budget,
                                           chunk_size=args.chunk, decode_len=warm + args.steps + 8, lanes=lanes,
                                           chunk_cache=P)
    except torch.cuda.OutOfMemoryError as e:
        gc.collect()
        torch.cuda.empty_cache()
        torch._C._host_emptyCache()
        log(f"chunk pool variant: {P} slots do not fit: {e}")
        return {"slots": P, "skipped": f"the pool does not fit in device memory: {str(e).splitlines()[0]}"}
    tok = torch.randint(0, shape.vocab, (args.batch, 1), device="cuda")
    for _ in range(warm):
        tok = pm.decode_step(tok)
    per_call = math.gcd(args.steps, max(1, args.graph_steps))
    pm.capture(tok, steps=per_call)
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(args.steps // per_call):
        tok = pm.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    hits = [float(lane.cache.cnts.float().mean()) for lane in pm.lanes]  # last layer of the last step
    c = pm.cache
    extra = (P - c.select_sets) * c.chunk_size * c.head_dim * 2 * 2 * args.batch * shape.kv_heads * shape.layers
    res = {"slots": P, "lanes": lanes, "untimed_steps": warm,
           "tokens_per_s": round(args.batch * args.steps / elapsed, 3),
           "ms_per_step": round(elapsed * 1e3 / args.steps, 3),
           "hit_rate_last_layer": round(statistics.fmean(hits) / c.select_sets, 4),
           "extra_device_GB": round(extra / 1e9, 2),
           "note": "same workload with a device chunk pool (f3): the same chunks selected and attention outputs "
                   "equal to the reference mode's within bf16 summation order (tests/test_gpu_pool.py); hits are "
                   "chunks still resident from earlier steps (synthetic queries are independent from step to step, "
                   "so the hit rate is about slots / landmarks once the pool is full, which the untimed steps wait "
                   "for)"}
    log(f"chunk pool variant {res}")
    del pm
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch._C._host_emptyCache()
    return res


def device_store_variant(args, shape, batch: int) -> dict:
    """The decode workload at `batch` with the value store in device memory instead of pinned host
    memory (ShadowKVCache_CPU(value_store="device"); the Llama-3.1-8B ctx-122880 store is 8 GB per
    sequence, so MI355X's 288 GB of HBM holds it beside the rest of the state up to about batch 24):
    the attention reads the selected value chunks in place from the store and nothing crosses the
    host link, so one lane (auto_lanes) and the step is set by the compute. Timed as the main
    measurement; every other decoder is released first. A batch whose state does not fit reports
    the allocation failure instead."""
    import gc
    import torch
    from shadowkv_amd import decode_model

    def release():
        gc.collect()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()

    release()
    torch._C._host_emptyCache()
    lanes = decode_model.auto_lanes(shape, batch, args.budget, "device")
    log(f"device value store variant: batch {batch}, {lanes} lane(s)")
    try:
        dm = decode_model.SyntheticDecoder(shape, batch, args.ctx, sparse_budget=args.budget, chunk_size=args.chunk,
                                           decode_len=args.warmup + args.steps + 8, lanes=lanes, value_store="device")
    except torch.cuda.OutOfMemoryError as e:
        release()
        log(f"device value store variant: batch {batch} does not fit: {e}")
        return {"batch": batch, "skipped": f"state does not fit in device memory: {str(e).splitlines()[0]}"}
    try:
        tok = torch.randint(0, shape.vocab, (batch, 1), device="cuda")
        for _ in range(args.warmup):
            tok = dm.decode_step(tok)
        per_call = math.gcd(args.steps, max(1, args.graph_steps))
        dm.capture(tok, steps=per_call)
        torch.cuda.synchronize()
        start = time.perf_counter()
        for _ in range(args.steps // per_call):
            tok = dm.replay()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - start
    except torch.cuda.OutOfMemoryError as e:  # the step's own buffers (workspaces, graph pool) do not fit
        del dm
        release()
        log(f"device value store variant: batch {batch} steps do not fit: {e}")
        return {"batch": batch, "skipped": f"decode steps do not fit in device memory: {str(e).splitlines()[0]}"}
    store_gb = sum(t.numel() * t.element_size() for t in {id(t): t for t in dm.cache.v_cache_cpu}.values()) \
        * len(dm.lanes) / 1e9
    res = {"batch": batch, "tokens_per_s": round(batch * args.steps / elapsed, 3),
           "ms_per_step": round(elapsed * 1e3 / args.steps, 3), "lanes": lanes,
           "value_store_device_GB": round(store_gb, 1),
           "device_memory_used_GB": round(torch.cuda.memory_allocated() / 1e9, 1),
           "note": "same workload with the value store in device memory (HBM) instead of pinned host memory: the "
                   "attention reads the selected value chunks in place from the store, nothing crosses the host "
                   "link; the tokens and state equal the host-store decoder's bit for bit "
                   "(tests/test_gpu_decoder_variants.py)"}
    log(f"device value store variant {res}")
    del dm
    release()
    return res


def step_hit_rate(model, tok):
    """Fraction of the chunks selected by one eager decode step (every layer and lane) that the
    previous step had selected too (the cache hits), and the step's tokens."""
    import torch

    before = [lane.cache.position_ids.clone() for lane in model.lanes]
    tok = model.decode_step(tok)
    torch.cuda.synchronize()
    hits = total = 0
    for lane, b0 in zip(model.lanes, before):
        S = lane.cache.select_sets
        new = lane.cache.position_ids.reshape(-1, S)
        old = b0.reshape(-1, S).sort(dim=-1).values
        idx = torch.searchsorted(old, new).clamp_max(S - 1)
        hits += int((old.gather(-1, idx) == new).sum())
        total += new.numel()
    return hits / total, tok


def encoded_variant(args, shape, lanes) -> dict:
    """The same decode workload from a prompt state built by the device encoder (decode_model
    .encode_state: rank-160 keys plus noise, get_svd, RoPE, prefill_kv_cache) instead of the
    synthesized random state, timed as the main measurement; the per-step hit rate is measured on
    one eager step after the timed replays. The main decoder is released first."""
    import gc
    import torch
    from shadowkv_amd import decode_model

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch._C._host_emptyCache()
    log("encoded-state variant: building the prompt state with the device encoder")
    t0 = time.time()
    em = decode_model.SyntheticDecoder(shape, args.batch, args.ctx, sparse_budget=args.budget, chunk_size=args.chunk,
                                       decode_len=args.warmup + args.steps + 9, lanes=lanes, state="encoded")
    t_enc = time.time() - t0
    tok = torch.randint(0, shape.vocab, (args.batch, 1), device="cuda")
    for _ in range(args.warmup):
        tok = em.decode_step(tok)
    per_call = math.gcd(args.steps, max(1, args.graph_steps))
    em.capture(tok, steps=per_call)
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(args.steps // per_call):
        tok = em.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    hit_rate, tok = step_hit_rate(em, tok)
    res = {"tokens_per_s": round(args.batch * args.steps / elapsed, 3), "ms_per_step": round(elapsed * 1e3 / args.steps, 3),
           "hit_rate": round(hit_rate, 4), "encode_s": round(t_enc, 1),
           "state": "device encoder (get_svd, RoPE, prefill_kv_cache) over seeded prompts: pre-RoPE keys "
                    "A(ctx x 160).B(160 x H*128) + 0.05 N(0,1) with A, B of variance 1/sqrt(160), values and the "
                    "last prompt query ~ N(0,1); the initial selection from that query",
           "note": "decode queries come from the random-weight model, independent of the prompt, so hits are "
                   "chunks that consecutive queries both rank in their top S"}
    log(f"encoded-state variant {res}")
    del em
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch._C._host_emptyCache()
    return res


def envelope_microbench(args) -> int:
    """HBM streaming envelope of this GPU at decode-kernel sizes: the landmark scoring kernel (a
    pure stream of landmark rows with a little MFMA work, the bench line's roofline kernel),
    torch's device copy and the library's read-only probe (1 KB contiguous wave loads, or the
    MFMA-operand order of the scoring and attention loads; plain or non-temporal; one or four 64 KB
    tiles per workgroup), each over a range of transfer sizes, cold (every launch reads buffers that the
    previous ones did not touch, > 1 GiB in rotation). A least-squares fit time = t0 +
    bytes / rate over the sizes gives the marginal streaming rate and the fixed per-launch cost,
    which together bound the HBM fraction a kernel of a given size can reach."""
    import torch
    from shadowkv_amd.kernels import shadowkv

    n, m = 15304, 4
    row_bytes = n * 128 * 2 + m * 128 * 2 + m * n * 2 + m * ((n + 255) // 256) * 8
    sets = 8
    probes = (("read contiguous", "contiguous", 1, False), ("read contiguous nt", "contiguous", 1, True),
              ("read contiguous nt, 4 tiles per workgroup", "contiguous", 4, True),
              ("read operand order", "operand", 1, False), ("read operand order nt", "operand", 1, True),
              ("read operand order, 4 tiles per workgroup", "operand", 4, False))
    res = {"scoring": [], "copy": [], **{name: [] for name, *_ in probes}}
    for rows in (8, 16, 32, 48, 64, 96, 128):
        g = torch.Generator(device="cuda").manual_seed(rows)
        Ls = [torch.randn(rows, n, 128, generator=g, device="cuda").to(torch.bfloat16) for _ in range(sets)]
        q = torch.randn(rows, m, 128, generator=g, device="cuda").to(torch.bfloat16)
        tiles = (n + 255) // 256
        D = torch.empty(rows, m, n, dtype=torch.bfloat16, device="cuda")
        nm = torch.empty(rows, m, tiles, device="cuda")
        sm = torch.empty_like(nm)
        t = gpu_time_per_call(lambda i: shadowkv.score_logits(q, Ls[i % sets], D, nm, sm, rows, m, n, 128,
                                                              1.0 / math.sqrt(128)), 4 * sets)
        res["scoring"].append((rows * row_bytes, t))
        del Ls, D, nm, sm
        # a device copy moving the same bytes (half read, half written)
        half = rows * row_bytes // 2 // 2  # bf16 elements per side
        src = [torch.empty(half, dtype=torch.bfloat16, device="cuda") for _ in range(sets)]
        dst = [torch.empty(half, dtype=torch.bfloat16, device="cuda") for _ in range(sets)]
        t = gpu_time_per_call(lambda i: dst[i % sets].copy_(src[i % sets]), 4 * sets)
        res["copy"].append((4 * half, t))
        del src, dst
        # read-only probe over the same bytes (rounded down to 64 KB tiles)
        tiles = rows * row_bytes // shadowkv.HBM_PROBE_TILE_BYTES
        src = [torch.empty(tiles * shadowkv.HBM_PROBE_TILE_BYTES, dtype=torch.uint8, device="cuda") for _ in range(sets)]
        for x in src:
            x.random_(0, 256, generator=g)
        sink = torch.empty(tiles * 4096, dtype=torch.uint8, device="cuda")
        for name, pattern, per_wg, nt in probes:
            t = gpu_time_per_call(lambda i: shadowkv.hbm_read_probe(src[i % sets], per_wg, pattern, sink, nt), 4 * sets)
            res[name].append((tiles * shadowkv.HBM_PROBE_TILE_BYTES, t))
        del src, sink
        torch.cuda.empty_cache()
    peaks = measured_peaks()
    print(json.dumps({"metric": "measured peaks", **peaks}), flush=True)
    for kind, pts in res.items():
        xs = [b for b, _ in pts]
        ys = [t for _, t in pts]
        k = len(xs)
        mx, my = sum(xs) / k, sum(ys) / k
        slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
        t0 = my - slope * mx
        rate = 1.0 / slope / 1e9
        for b, t in pts:
            print(json.dumps({"metric": f"{kind} streaming rate", "value": round(b / t / 1e9, 1), "unit": "GB/s",
                              "bytes": int(b), "us": round(t * 1e6, 2), "hbm_frac": round(b / t / 1e9 / HBM_PEAK_GBS, 4),
                              "config": {"workload": f"{kind}: {b / 1e6:.1f} MB per launch, cold buffers"}}), flush=True)
        print(json.dumps({"metric": f"{kind} fit time = t0 + bytes / rate", "rate_GBps": round(rate, 1),
                          "rate_frac": round(rate / HBM_PEAK_GBS, 4), "t0_us": round(t0 * 1e6, 2),
                          "frac_at_100MB": round(100e6 / (t0 + 100e6 / (rate * 1e9)) / 1e9 / HBM_PEAK_GBS, 4)}),
              flush=True)
    return 0


def rebuild_bytes(rows_per_head: int, BH: int, S: int, R: int = 160, D: int = 128) -> int:
    """Algorithmic HBM bytes of one rebuild launch: per miss row a U row, a cos/sin row and the
    rotated K row; per (b,h) the SV block and the chunk ids."""
    return BH * (rows_per_head * (R * 2 + D * 2 + D * 2) + R * D * 2 + S * 8)


def rebuild_microbench(args) -> int:
    """Low-rank key rebuild + RoPE alone: per-head U [B*8, 122880, 160] and SV shared across the
    batch, 256 sorted unique chunk ids per head out of 15360 (2048 rows), hit counts 0 and 154,
    Llama RoPE (theta 5e5). One JSON line per (batch, hits)."""
    import torch
    from shadowkv_amd.kernels import shadowkv
    from shadowkv_amd.models.tensor_op import build_cos_sin_cache

    H, D, R, c, ctx, S = 8, 128, 160, 8, 122880, 256
    chunks, sparse_start = ctx // c, 448
    buf_len = sparse_start + S * c + 96
    dev = torch.device("cuda")
    cos_sin = build_cos_sin_cache(ctx + 1024, 500000.0, D, device=dev)
    reps = max(args.steps, 4)
    # A plain copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE counters of profiling runs.
    cal = torch.empty(64 * 2 ** 20, dtype=torch.float32, device=dev)
    torch.neg(cal, out=cal)
    del cal
    for B in args.rebuild_batches:
        g = torch.Generator(device=dev).manual_seed(1000 + B)
        U = torch.empty(B, H, ctx, R, dtype=torch.bfloat16, device=dev)
        for b in range(B):
            U[b].normal_(generator=g)
        SV = torch.empty(H, D, R, dtype=torch.bfloat16, device=dev).normal_(generator=g)
        # Distinct chunk-id sets and output buffers, rotated so that no launch finds its U rows
        # or its output lines in the last-level cache.
        sets = cold_sets(rebuild_bytes(S * c, B * H, S))
        set_reps = -(-reps // sets) * sets
        ids = [torch.stack([torch.randperm(chunks, generator=g, device=dev)[:S].sort().values
                            for _ in range(B * H)]).view(B, H, S) for _ in range(sets)]
        caches = [torch.zeros(B, H, buf_len, D, dtype=torch.bfloat16, device=dev) for _ in range(sets)]
        for hits in (0, 154):
            cnts = torch.full((B * H,), hits, dtype=torch.int32, device=dev)
            t = gpu_time_per_call(lambda i: shadowkv.rebuild_k_rope(U, SV, ids[i % sets], cnts, cos_sin,
                                                                    caches[i % sets], sparse_start, c),
                                  set_reps)
            rows = (S - hits) * c
            nbytes = rebuild_bytes(rows, B * H, S)
            flops = 2 * B * H * rows * R * D
            cpu = None
            if hits == 0 and B <= 8 and not args.no_cpu_baseline:
                cpu = rebuild_cpu_baseline(U, SV, ids[0], cnts, cos_sin, caches[0], sparse_start, c, args.cpu_runs)
            out = {"metric": "low-rank K rebuild + RoPE rows/s", "value": round(B * H * rows / t, 1),
                   "unit": "rows/s", "n_gpus": 1, "steps": set_reps, "warmup": 1,
                   "ms_per_step": round(t * 1e3, 4), "higher_is_better": True, "scaling": "strong",
                   "vs_baseline": None, "dtype": "bf16",
                   "data": "synthetic: U, SV ~ N(0,1) bf16, sorted unique random chunk ids; timed as HIP-graph "
                           f"replays of back-to-back launches rotating over {sets} id sets / output buffers "
                           "(> 1 GiB together, so reads come from HBM)",
                   "config": {"workload": f"rebuild microbench batch {B}, 8 kv heads, rank 160, ctx 122880, "
                                          f"256 chunks/head, {hits} hits", "batch": B, "hits": hits,
                              "rotated_sets": sets},
                   "roofline": {"kernel": "rebuild_kernel (gather-GEMM + RoPE epilogue)", "bound": "hbm",
                                "achieved": round(nbytes / t / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                                "algorithmic_bytes_per_launch": nbytes, "avg_launch_us": round(t * 1e6, 2),
                                "mfma_tflops": round(flops / t / 1e12, 2),
                                "mfma_util": round(flops / t / MFMA_BF16_PEAK, 5)},
                   "cpu_baseline": cpu}
            print(json.dumps(out), flush=True)
        del U, SV, ids, caches
        torch.cuda.empty_cache()
    return 0


def rebuild_cpu_baseline(U, SV, ids, cnts, cos_sin, cache, sparse_start, c, runs) -> dict:
    """The CPU oracle's rebuild + RoPE push at the same batch (a reported baseline only)."""
    import torch
    import oracle

    threads = max(1, min(os.cpu_count() or 1, 16))
    torch.set_num_threads(threads)
    B, H, S = ids.shape
    Uc, SVc = U.cpu(), SV.cpu().unsqueeze(0).expand(B, -1, -1, -1)
    idc, cc, csc, kc = ids.cpu(), cnts.cpu(), cos_sin.cpu(), cache.cpu()
    times = []
    for i in range(3 + runs):
        t0 = time.perf_counter()
        oracle.rebuild_k_rope(Uc, SVc, idc, cc, csc, c, kc, sparse_start)
        if i >= 3:
            times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    rows = B * H * S * c
    return {"value": round(rows / t, 1), "unit": "rows/s", "cores": threads, "kind": "port",
            "sample": f"oracle rebuild + RoPE push on CPU torch at batch {B} (all {rows} rows); median of {runs} "
                      f"runs after 3 warmups = {t * 1e3:.1f} ms"}


def attention_microbench(args) -> int:
    """Sparse decode attention alone at the decode shapes: one query token per sequence over the
    assembled K/V buffers (Llama-3-8B: 32/8 heads; GLM-4-9B: 32/2 heads), lengths around the
    sparse region's 2497 rows. One JSON line per shape."""
    import torch
    from shadowkv_amd.kernels import shadowkv

    D = 128
    reps = max(args.steps, 4)
    # A plain copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE counters of profiling runs.
    cal = torch.empty(64 * 2 ** 20, dtype=torch.float32, device="cuda")
    torch.neg(cal, out=cal)
    del cal
    for name, B, Hq, Hk, L in (("Llama-3-8B", 4, 32, 8, 2600), ("Llama-3-8B", 8, 32, 8, 2600),
                               ("Llama-3-8B", 24, 32, 8, 2600), ("GLM-4-9B", 4, 32, 2, 2600),
                               ("Llama-3-8B-1M", 1, 32, 8, 19616)):
        g = torch.Generator(device="cuda").manual_seed(L + B)
        buf = L + 32
        G = Hq // Hk
        nbytes = B * Hk * (2 * L * D * 2 + 2 * G * D * 2)  # K and V rows, q in, o out
        sets = cold_sets(nbytes)  # distinct K/V/q sets, rotated so reads come from HBM
        set_reps = -(-reps // sets) * sets
        K = [torch.randn(B, Hk, buf, D, generator=g, device="cuda").to(torch.bfloat16) for _ in range(sets)]
        V = [torch.randn(B, Hk, buf, D, generator=g, device="cuda").to(torch.bfloat16) for _ in range(sets)]
        q = [torch.randn(B, Hq, D, generator=g, device="cuda").to(torch.bfloat16) for _ in range(sets)]
        out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device="cuda")
        ws = shadowkv.sparse_attn_workspace(B, Hq, L, "cuda")
        t = gpu_time_per_call(lambda i: shadowkv.sparse_attn_decode(q[i % sets], K[i % sets], V[i % sets], L, out, ws),
                              set_reps)
        out_line = {"metric": "sparse decode attention (b,h) rows/s", "value": round(B * Hq / t, 1), "unit": "rows/s",
                    "n_gpus": 1, "steps": set_reps, "warmup": 1, "ms_per_step": round(t * 1e3, 4),
                    "higher_is_better": True, "scaling": "strong", "vs_baseline": None, "dtype": "bf16",
                    "data": "synthetic: q, K, V ~ N(0,1) bf16; timed as HIP-graph replays of back-to-back launches "
                            f"rotating over {sets} q/K/V sets (> 1 GiB together, so reads come from HBM)",
                    "config": {"workload": f"{name} shape attention: batch {B}, {Hq}/{Hk} heads, kv length {L}",
                               "batch": B, "q_heads": Hq, "kv_heads": Hk, "kv_len": L, "rotated_sets": sets},
                    "roofline": {"kernel": "attn_split_kernel + attn_combine_kernel", "bound": "hbm",
                                 "achieved": round(nbytes / t / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                                 "algorithmic_bytes_per_launch": nbytes, "avg_launch_us": round(t * 1e6, 2)},
                    "cpu_baseline": None}
        print(json.dumps(out_line), flush=True)
    return 0


def select_microbench(args) -> int:
    """Fused chunk selection alone (softmax normalisation, GQA max, top-k, id gather, cache-hit
    reorder) at the decode shapes, on logits produced by the scoring kernel. Latency-bound (few
    rows, a serial selection per row): reported in microseconds. One JSON line per shape."""
    import torch
    from shadowkv_amd.kernels import shadowkv

    reps = max(args.steps, 4)
    for name, B, H, G, n, S in (("Llama-3-8B 122K", 8, 8, 4, 15304, 256), ("Llama-3-8B 122K", 24, 8, 4, 15304, 256),
                                ("Llama-3-8B 122K", 4, 8, 4, 15304, 256), ("Llama-3-8B 122K", 1, 8, 4, 15304, 256),
                                ("GLM-4-9B 262K", 4, 2, 16, 32712, 256), ("Llama-3-8B-1M", 1, 8, 4, 130680, 2048)):
        g = torch.Generator(device="cuda").manual_seed(n + B)
        rows = B * H
        chunks = n + 48 + 8
        q = torch.randn(rows, G, 128, generator=g, device="cuda").to(torch.bfloat16)
        lm = torch.randn(rows, n, 128, generator=g, device="cuda").to(torch.bfloat16)
        tiles = (n + 255) // 256
        D = torch.empty(rows, G, n, dtype=torch.bfloat16, device="cuda")
        norm = torch.empty(rows, G, tiles, dtype=torch.float32, device="cuda")
        ssum = torch.empty_like(norm)
        shadowkv.score_logits(q, lm, D, norm, ssum, rows, G, n, 128, 1.0 / math.sqrt(128))
        del lm
        lidx = torch.stack([torch.randperm(chunks, generator=g, device="cuda")[:n].sort().values for _ in range(rows)])
        pos0 = torch.stack([lidx[r, torch.randperm(n, generator=g, device="cuda")[:S]] for r in range(rows)])
        pos = pos0.clone()
        offsets = torch.empty(rows * S, dtype=torch.int32, device="cuda")
        cnts = torch.empty(rows, dtype=torch.int32, device="cuda")
        scores = torch.empty(rows, n, dtype=torch.bfloat16, device="cuda")
        ws = torch.empty(shadowkv.select_workspace_bytes(rows, n, S), dtype=torch.uint8, device="cuda")

        def run(_):
            pos.copy_(pos0)
            shadowkv.select_chunks(D, norm, ssum, rows, G, n, lidx, S, chunks, pos, offsets, cnts, out_scores=scores,
                                   workspace=ws)

        t_all = gpu_time_per_call(run, reps)
        t_copy = gpu_time_per_call(lambda _: pos.copy_(pos0), reps)
        env = os.environ.get("SKV_SELECT_SPLIT")
        few = rows <= (64 if ws is not None else 32) and G * n >= 1 << 15  # the library's path rule
        path = {"0": "fused", "1": "split", "2": "parts"}.get(env, ("parts" if n >= 65536 else "split") if few else "fused")
        t = t_all - t_copy
        out_line = {"metric": "fused chunk selection latency", "value": round(t * 1e6, 2), "unit": "us",
                    "n_gpus": 1, "steps": reps, "warmup": 1, "ms_per_step": round(t * 1e3, 4),
                    "higher_is_better": False, "scaling": "strong", "vs_baseline": None, "dtype": "bf16",
                    "data": "synthetic: logits of random q / landmarks from the scoring kernel; timed as HIP-graph "
                            "replays (minus the replayed slot-restore copy)",
                    "config": {"workload": f"{name} selection: {rows} rows x {G} queries x {n} landmarks, top {S}",
                               "rows": rows, "m": G, "n": n, "select_sets": S},
                    "roofline": {"kernel": {"fused": "select_kernel",
                                            "split": "softmax_vec_kernel + select_kernel (keys and key histograms on "
                                                     "many workgroups, selection on a candidate list)",
                                            "parts": "softmax_kernel + part_*_kernel + select_finish_kernel "
                                                     "(many workgroups per row)"}[path],
                                 "bound": "latency", "achieved": None, "peak": None,
                                 "unit": "us", "frac": None, "traffic": None,
                                 "algorithmic_bytes_per_launch": rows * (G * n * 2 + n * 8 + S * 28),
                                 "avg_launch_us": round(t * 1e6, 2)},
                    "cpu_baseline": None}
        print(json.dumps(out_line), flush=True)
    return 0


def linear_microbench(args) -> int:
    """The skinny linear kernel on the Llama-3-8B decode projections (fused QKV, o, fused
    gate/up, down, lm head) at 4 and 8 token rows (--linear-rows), cold weights (distinct copies rotated past the
    last-level cache), next to torch's GEMM on the same operands. One JSON line per (shape, rows)."""
    import torch
    from shadowkv_amd.kernels import shadowkv

    shapes = (("qkv", 6144, 4096), ("o_proj", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336),
              ("lm_head", 128256, 4096))
    reps = max(args.steps, 4)
    for name, n, k in shapes:
        wbytes = n * k * 2
        sets = cold_sets(wbytes)
        g = torch.Generator(device="cuda").manual_seed(n + k)
        ws = [(torch.randn(n, k, generator=g, device="cuda") * 0.02).to(torch.bfloat16) for _ in range(sets)]
        set_reps = -(-reps // sets) * sets
        for rows in args.linear_rows:
            x = torch.randn(rows, k, generator=g, device="cuda").to(torch.bfloat16)
            y = torch.empty(rows, n, dtype=torch.bfloat16, device="cuda")
            t = gpu_time_per_call(lambda i: shadowkv.linear(x, ws[i % sets], y), set_reps)
            t_torch = gpu_time_per_call(lambda i: torch.matmul(x, ws[i % sets].t(), out=y), set_reps)
            nbytes = wbytes + rows * (k + n) * 2
            out_line = {"metric": "skinny decode linear weight stream GB/s", "value": round(nbytes / t / 1e9, 1),
                        "unit": "GB/s", "n_gpus": 1, "steps": set_reps, "warmup": 1, "ms_per_step": round(t * 1e3, 4),
                        "higher_is_better": True, "scaling": "strong", "vs_baseline": None, "dtype": "bf16",
                        "data": "synthetic: x ~ N(0,1), weights ~ N(0, 0.02) bf16; timed as HIP-graph replays of "
                                f"back-to-back launches rotating over {sets} weight copies (> 1 GiB together)",
                        "config": {"workload": f"Llama-3-8B {name} projection: {rows} rows x [{n}, {k}] weight",
                                   "rows": rows, "n": n, "k": k, "rotated_sets": sets},
                        "roofline": {"kernel": "linear_kernel", "bound": "hbm", "achieved": round(nbytes / t / 1e9, 1),
                                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                     "frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                                     "algorithmic_bytes_per_launch": nbytes, "avg_launch_us": round(t * 1e6, 2),
                                     "torch_matmul_us": round(t_torch * 1e6, 2)},
                        "cpu_baseline": None}
            if name == "down" and rows <= shadowkv.LINEAR_SILU_MUL_MAX_ROWS:
                # the same weight read through SiLU-and-mul of [gate | up] rows (offered up to 4 rows)
                gu = torch.randn(rows, 2 * k, generator=g, device="cuda").to(torch.bfloat16)
                act = torch.empty(rows, k, dtype=torch.bfloat16, device="cuda")
                t_gated = gpu_time_per_call(lambda i: shadowkv.linear_silu_mul(gu, ws[i % sets], y), set_reps)

                def two(i):
                    shadowkv.silu_and_mul(gu, act)
                    shadowkv.linear(act, ws[i % sets], y)
                t_two = gpu_time_per_call(two, set_reps)
                out_line["roofline"]["silu_mul_fused_us"] = round(t_gated * 1e6, 2)
                out_line["roofline"]["silu_mul_then_linear_us"] = round(t_two * 1e6, 2)
            print(json.dumps(out_line), flush=True)
        del ws
        torch.cuda.empty_cache()
    return 0


def pool_microbench(args) -> int:
    """One layer's sparse decode step (selection, value fetch, key rebuild, attention) at the
    Llama-3-8B shape, batch 8, ctx 122880, budget 2048, on queries that drift from step to step
    (q_t = q_{t-1} + drift * noise, so consecutive selections overlap as in real decoding), without
    and with a device chunk pool. Reports the hit rate, host-link bytes and time per step."""
    import types
    import torch
    from shadowkv_amd import decode_model
    from shadowkv_amd.models.attention import ShadowAttention
    from shadowkv_amd.models.kvcache import ShadowKVCache_CPU

    B, H, G, D, ctx, budget, c, steps, warm = 8, 8, 4, 128, args.ctx, 2048, 8, 24, 8
    S = budget // c
    cfg = types.SimpleNamespace(num_attention_heads=H * G, num_key_value_heads=H, hidden_size=H * G * D,
                                num_hidden_layers=1)
    cos_sin = decode_model.build_cos_sin_cache(ctx + 1024, 500000.0, D, device="cuda")
    for drift in (0.05, 0.2):
        for P in (None, 2 * S, 4 * S):
            cache = ShadowKVCache_CPU(cfg, batch_size=B, max_length=ctx, device="cuda", sparse_budget=budget,
                                      chunk_size=c, rank=160, max_decode_len=steps + warm + 4, zero_host_store=False,
                                      chunk_cache=P)
            decode_model.synthesize_state(cache, ctx, seed=3, cos_sin=cos_sin)
            attn = ShadowAttention(cache, G, D, H * G * D, None, None, cos_sin)
            g = torch.Generator(device="cuda").manual_seed(17)
            q = torch.randn(B, H * G, 1, D, generator=g, device="cuda")
            hits, times = [], []
            for t in range(warm + steps):
                q = q + drift * torch.randn(B, H * G, 1, D, generator=g, device="cuda")
                k = torch.randn(B, H, 1, D, generator=g, device="cuda").to(torch.bfloat16)
                v = torch.randn(B, H, 1, D, generator=g, device="cuda").to(torch.bfloat16)
                cache.update_kv_cache(k, v, 0)
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                attn.decode_end(attn.decode_begin_appended(q.to(torch.bfloat16), 0))
                e.record()
                e.synchronize()
                if t >= warm:
                    times.append(s.elapsed_time(e))
                    hits.append(int(cache.cnts.sum()))
            hit_rate = statistics.fmean(hits) / (B * H * S)
            ms = statistics.fmean(times)
            host = (1 - hit_rate) * B * H * S * c * D * 2
            out = {"metric": "sparse layer step ms with a device chunk pool", "value": round(ms, 4), "unit": "ms",
                   "n_gpus": 1, "steps": steps, "warmup": warm, "ms_per_step": round(ms, 4),
                   "higher_is_better": False, "scaling": "strong", "vs_baseline": None, "dtype": "bf16",
                   "data": f"synthetic ShadowKV state; queries drifting by {drift} x N(0,1) per step",
                   "config": {"workload": f"Llama-3-8B shape one-layer sparse step, batch {B}, ctx {ctx}, budget "
                                          f"{budget}, chunk {c}, " + (f"chunk pool of {P} slots" if P else
                                                                       "reference slot reuse"),
                              "drift": drift, "pool_slots": P},
                   "hit_rate": round(hit_rate, 4), "host_link_MB_per_step": round(host / 1e6, 2),
                   "roofline": None, "cpu_baseline": None}
            print(json.dumps(out), flush=True)
            del cache, attn
            torch.cuda.empty_cache()
    return 0


def encode_microbench(args) -> int:
    """The device prefill encoder per layer (ShadowKVCache_CPU.get_svd + prefill_kv_cache) at the
    Llama-3-8B shape (8 kv heads x 4 query heads), ctx 122880, rank 160, chunk 8, budget 2048, on
    random low-rank-plus-noise keys; components timed separately, the chunk-statistics kernel against
    its HBM roofline. One JSON line per batch size."""
    import types
    import torch
    from shadowkv_amd.kernels import shadowkv
    from shadowkv_amd.models.kvcache import ShadowKVCache_CPU
    from shadowkv_amd.models.kvcache.shadow import low_rank_factors

    H, G, D, R, c, budget, ctx = 8, 4, 128, 160, 8, 2048, args.ctx
    dev = torch.device("cuda")
    cal = torch.empty(64 * 2 ** 20, dtype=torch.float32, device=dev)
    torch.neg(cal, out=cal)
    del cal

    def timed(fn, reps=3):
        fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        e.synchronize()
        return s.elapsed_time(e) / reps

    for B in (1, 8):
        g = torch.Generator(device=dev).manual_seed(B)
        a = torch.randn(B, ctx, 128, generator=g, device=dev) @ torch.randn(B, 128, H * D, generator=g, device=dev)
        k_pre = (a / 12 + 0.1 * torch.randn(B, ctx, H * D, generator=g, device=dev)).to(torch.bfloat16)
        del a
        k_pre = k_pre.view(B, ctx, H, D).transpose(1, 2).contiguous()
        k_roped = k_pre.clone()  # the encoder's cost does not depend on the rotation
        v = torch.randn(B, H, ctx, D, generator=g, device=dev).to(torch.bfloat16)
        q = torch.randn(B, H * G, 1, D, generator=g, device=dev).to(torch.bfloat16)
        cfg = types.SimpleNamespace(num_attention_heads=H * G, num_key_value_heads=H, hidden_size=H * G * D,
                                    num_hidden_layers=1)
        cache = ShadowKVCache_CPU(cfg, batch_size=B, max_length=ctx, device="cuda", sparse_budget=budget,
                                  chunk_size=c, rank=R, zero_host_store=False)

        def encode():
            cache.prefilled_batch = 0
            cache.get_svd(k_pre, 0)
            cache.prefill_kv_cache(v, 0, k_roped, q)

        t_all = timed(encode)
        kf = k_pre.transpose(1, 2).reshape(B, ctx, H * D)
        t_svd = timed(lambda: low_rank_factors(kf, R))
        chunks = cache.chunks
        cand = torch.empty(B, H, chunks, D, dtype=torch.bfloat16, device=dev)
        mc = torch.empty(B, H, chunks, dtype=torch.float32, device=dev)
        t_stats = timed(lambda: shadowkv.chunk_stats(k_roped, chunks, c, cand, mc), reps=20)
        out_idx = torch.empty(B * H, cache.outlier_chunk, dtype=torch.int64, device=dev)
        rest = torch.empty(B * H, chunks - cache.outlier_chunk, dtype=torch.int64, device=dev)
        t_sel = timed(lambda: shadowkv.select_outliers(mc.view(B * H, chunks), cache.outlier_chunk, out_idx, rest),
                      reps=20)
        t_full = None
        if B == 1:
            t_full = timed(lambda: torch.linalg.svd(kf.float(), full_matrices=False), reps=1)
        stats_bytes = B * H * (chunks * c * D * 2 + chunks * D * 2 + chunks * 4)
        achieved = stats_bytes / (t_stats * 1e-3) / 1e9
        cpu = None
        if B == 1 and not args.no_cpu_baseline:
            cpu = encode_cpu_baseline(k_pre, v, q, R, c, budget)
        out = {"metric": "prefill encoder ms per layer", "value": round(t_all, 3), "unit": "ms", "n_gpus": 1,
               "steps": 3, "warmup": 1, "ms_per_step": round(t_all, 3), "higher_is_better": False,
               "scaling": "strong", "vs_baseline": None, "dtype": "bf16 (fp32 factors)",
               "data": "synthetic: rank-128 keys plus noise, random values and last query, bf16",
               "config": {"workload": f"prefill encoder, Llama-3-8B shape (8 kv heads), batch {B}, ctx {ctx}, "
                                      f"rank {R}, chunk {c}, budget {budget}", "batch": B, "ctx": ctx},
               "components_ms": {"low_rank_factors (Gram GEMM + eigh + GEMM)": round(t_svd, 3),
                                 "chunk_stats": round(t_stats, 4), "select_outliers": round(t_sel, 4),
                                 "reference full SVD on the GPU (torch.linalg.svd, fp32)":
                                     round(t_full, 1) if t_full else None},
               "roofline": {"kernel": "chunk_stats_kernel", "bound": "hbm", "achieved": round(achieved, 1),
                            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                            "traffic": None, "algorithmic_bytes_per_launch": stats_bytes,
                            "avg_launch_us": round(t_stats * 1e3, 2)},
               "cpu_baseline": cpu}
        print(json.dumps(out), flush=True)
        del cache, k_pre, k_roped, v, kf
        torch.cuda.empty_cache()
    return 0


def hostlink_microbench(args) -> int:
    """Host-link read rate from pinned host memory: SDMA copies (hipMemcpyAsync host-to-device) of
    16 MiB to 1 GiB, and the value-fetch kernel's zero-copy gather at the decode shape (one batch
    lane of the Llama-3-8B workload: 4 sequences x 8 kv heads, 256 random missing 2 KB chunks per
    (b, h) out of a 1 GiB store of 15360 chunks per row) and at 8x that many chunks. The gather's
    workgroup count follows SKV_FETCH_WGS (read once per process). One JSON line per case."""
    import torch
    from shadowkv_amd.kernels import shadowkv

    dev = torch.device("cuda")
    rounds = max(args.steps, 4)
    for mib in (16, 256, 1024):
        nbytes = mib << 20
        t = host_link_peak_gbps(nbytes, reps=rounds)
        print(json.dumps({"metric": "host-to-device GB/s", "value": round(t, 2), "unit": "GB/s", "n_gpus": 1,
                          "higher_is_better": True, "dtype": "u8", "data": "pinned host memory",
                          "config": {"workload": f"SDMA copy (hipMemcpyAsync) of {mib} MiB pinned -> device"}}),
              flush=True)
    B, H, S, chunks, E = 4, 8, 256, 15360, 8 * 128
    store = torch.empty(B, H, chunks, E, dtype=torch.bfloat16, pin_memory=True)
    store.view(torch.int16).copy_(torch.randint(-30000, 30000, (B, H, chunks, E), dtype=torch.int16))
    g = torch.Generator(device=dev).manual_seed(3)
    wgs = os.environ.get("SKV_FETCH_WGS", "default (48)")
    for mult in (1, 8):
        s_sets = S * mult
        buf = torch.empty(B, H, s_sets * 8, 128, dtype=torch.bfloat16, device=dev)
        sets = [torch.rand(B * H, chunks, generator=g, device=dev).argsort(dim=-1)[:, :s_sets].sort(dim=-1)
                .values.to(torch.int32).reshape(-1).contiguous() for _ in range(8)]
        cnts = torch.zeros(B * H, dtype=torch.int32, device=dev)
        t = gpu_time_per_call(lambda i: shadowkv.gather_copy_with_offsets(
            store, buf, None, sets[i % 8], cnts, None, B, H, chunks * E, s_sets * E, 0, s_sets * E, s_sets,
            misses_only=True), 16, rounds=rounds)
        nbytes = B * H * s_sets * E * 2
        print(json.dumps({"metric": "zero-copy gather GB/s", "value": round(nbytes / t / 1e9, 2), "unit": "GB/s",
                          "n_gpus": 1, "higher_is_better": True, "dtype": "bf16",
                          "data": "pinned host store of 1 GiB, random sorted chunk ids",
                          "config": {"workload": f"value-fetch kernel, {B * H} rows x {s_sets} chunks of 2 KB "
                                                 f"({nbytes / 2 ** 20:.0f} MiB per launch)", "fetch_wgs": wgs,
                                     "us_per_launch": round(t * 1e6, 2)}}), flush=True)
    return 0


def encode_cpu_baseline(k_pre, v, q, R, c, budget, sample_ctx: int = 16384) -> dict:
    """The CPU oracle's encode_layer on the first sample_ctx tokens of batch row 0 (a reported
    baseline only), scaled linearly to the full prompt."""
    import torch
    import oracle

    threads = max(1, min(os.cpu_count() or 1, 16))
    torch.set_num_threads(threads)
    ctx = k_pre.shape[2]
    cs = oracle.build_cos_sin_cache(sample_ctx + 64, 500000.0)
    kp, vv, qq = k_pre[:1, :, :sample_ctx].cpu(), v[:1, :, :sample_ctx].cpu(), q[:1].cpu()
    t0 = time.perf_counter()
    oracle.encode_layer(kp, vv, qq, cs, rank=R, chunk=c, budget=budget)
    t = time.perf_counter() - t0
    return {"value": round(t * 1e3 * ctx / sample_ctx, 1), "unit": "ms per layer (scaled)", "cores": threads,
            "kind": "port", "sample": f"oracle encode_layer (full fp32 SVD, bf16 cosine, torch.topk) on batch row 0, "
                                      f"first {sample_ctx} tokens: {t * 1e3:.0f} ms, scaled by {ctx}/{sample_ctx}"}


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the sparse decode path is not sharded "
              f"across GPUs in this build", file=sys.stderr)
        return 2
    if args.workload == "rebuild":
        return rebuild_microbench(args)
    if args.workload == "attention":
        return attention_microbench(args)
    if args.workload == "select":
        return select_microbench(args)
    if args.workload == "linear":
        return linear_microbench(args)
    if args.workload == "encode":
        return encode_microbench(args)
    if args.workload == "pool":
        return pool_microbench(args)
    if args.workload == "hostlink":
        return hostlink_microbench(args)
    if args.workload == "envelope":
        return envelope_microbench(args)
    import torch
    from shadowkv_amd import decode_model
    from shadowkv_amd.kernels import shadowkv
    from dataclasses import replace

    shape = {"llama31_8b": decode_model.LLAMA31_8B, "glm4_9b": decode_model.GLM4_9B,
             "llama3_8b_1m": decode_model.LLAMA3_8B_1M}[args.model]
    if args.layers:
        shape = replace(shape, layers=args.layers)
    if args.summarize_trace:
        lanes = args.lanes if args.lanes else decode_model.auto_lanes(shape, args.batch, args.budget)
        lanes = lanes if args.batch % lanes == 0 else 1
        rec = {"workload": trace_workload(args, lanes),
               "trace": f"rocprofv3 --kernel-trace of python bench.py --model {args.model} --batch {args.batch} "
                        f"--ctx {args.ctx} --budget {args.budget} --steps {args.steps} --warmup {args.warmup} "
                        f"--no-cpu-baseline --no-breakdown (timed steps as HIP graph replays)",
               **summarize_trace(args.summarize_trace, shape.layers, lanes, args.warmup, args.steps)}
        path = trace_summary_path(args)
        path.write_text(json.dumps(rec, indent=1) + "\n")
        print(f"wrote {path.relative_to(ROOT)}: {rec['op_us_per_lane_layer']}")
        return 0
    t0 = time.time()
    log(f"building {shape.name} batch {args.batch} ctx {args.ctx} (random weights, synthesized state)")
    lanes = args.lanes if args.lanes else decode_model.auto_lanes(
        shape, args.batch, args.budget, args.value_store,
        miss_fraction=decode_model.pool_miss_fraction(args.chunk_cache, args.ctx // args.chunk))
    lanes = lanes if args.batch % lanes == 0 else 1
    model = decode_model.SyntheticDecoder(shape, args.batch, args.ctx, sparse_budget=args.budget, chunk_size=args.chunk,
                                          decode_len=args.warmup + args.steps + 8, lanes=lanes,
                                          chunk_cache=args.chunk_cache, state=args.state,
                                          one_stream_fetch=False if args.two_stream_fetch else None,
                                          value_store=args.value_store)
    if args.separate_hit_moves:
        for lane in model.lanes:
            lane.cache.fold_hit_moves = False
    if args.no_act_epilogue:
        model.act_epilogue = False
    if args.no_qkv_rope_epilogue:
        model.qkv_rope_epilogue = False
    cache_one_stream = all(lane.cache.one_stream_active() for lane in model.lanes)
    lane_streams = model.lane_streams
    qkv_rope_epi = model.qkv_rope_epilogue
    cache = model.cache
    log(f"setup done in {time.time() - t0:.1f}s; sparse_start {cache.sparse_start} sparse_end {cache.sparse_end} "
        f"landmarks {cache.k_landmark.shape[-2]}")

    # A plain copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE counters of profiling runs.
    cal = torch.empty(64 * 2 ** 20, dtype=torch.float32, device="cuda")
    torch.neg(cal, out=cal)
    torch.cuda.synchronize()

    tok = torch.randint(0, shape.vocab, (args.batch, 1), device="cuda")
    for i in range(args.warmup):
        tok = model.decode_step(tok)
    torch.cuda.synchronize()
    log(f"warmup {args.warmup} steps done")

    graph = not args.no_graph
    per_call = 1
    if graph:
        per_call = math.gcd(args.steps, max(1, args.graph_steps))
        model.capture(tok, steps=per_call)
        torch.cuda.synchronize()
        log(f"{per_call} decode step(s) captured in a HIP graph")

        def step(_):
            return model.replay()
    else:
        step = model.decode_step
    torch.cuda.synchronize()
    start = time.perf_counter()
    for i in range(args.steps // per_call):
        tok = step(tok)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    log(f"timed {args.steps} steps as {args.steps // per_call} {'graph replays' if graph else 'eager steps'} "
        f"in {elapsed:.3f}s")

    n = cache.k_landmark.shape[-2]
    BH = cache.batch_size * shape.kv_heads  # one launch covers one lane's batch slice
    G = shape.heads // shape.kv_heads
    lb = logits_bytes(BH, G, n)
    k_ms, timing = scoring_launch_ms(model)
    achieved = lb / (k_ms * 1e-3) / 1e9
    traffic, traffic_source = None, None
    # HBM traffic per launch of this launch shape, from the committed FETCH_SIZE / WRITE_SIZE
    # counter runs (rocprofv3 --pmc cannot run inside this process)
    for tfile in sorted((ROOT / "profiles").glob("score_logits_*_traffic.json")):
        rec = json.loads(tfile.read_text())
        if rec.get("launch") == {"rows": BH, "m": G, "n": n, "k": 128}:
            traffic = rec.get("bytes_per_launch")
            traffic_source = (f"{tfile.relative_to(ROOT)}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of this "
                              f"launch shape, scaled by the counters' reading of a plain copy (not measured in this run)")

    S = cache.select_sets
    ub = a1a2_bytes(BH, G, n, S)
    u_ms, u_timing = a1a2_unit_ms(model)
    u_achieved = ub / (u_ms * 1e-3) / 1e9

    detail = None
    if not args.no_breakdown:
        detail, per_layer = breakdown(model, tok)
        log(f"breakdown {detail}")
        link_peak = host_link_peak_gbps()
        hl = detail["host_link"]
        hl.update(peak_GBps=round(link_peak, 1), frac_of_peak=round(hl["GBps"] / link_peak, 4),
                  peak_source="SDMA copy (hipMemcpyAsync) of 256 MiB of pinned host memory in this run; "
                              "profiles/hostlink_microbench.md has the zero-copy gather beside it",
                  nominal_GBps=64.0)
        if not cache.pooled:
            detail["kernels"] = kernel_table(model, per_layer, detail["op_us_per_layer"], link_peak)
            apply_trace_summary(detail["kernels"], args, lanes)
            for k in detail["kernels"]:
                log(f"kernel {k['kernel'][:40]:40s} isolated {k['isolated_us']:8.2f} us "
                    f"({k['isolated_frac'] * 100:5.1f}%), in step {k['in_step_us']} us")
        detail["measured_peaks"] = measured_peaks()
        log(f"measured peaks {detail['measured_peaks']}")
        detail["single_layer"] = {"workload": "single-layer decode step, batch 1, 8 kv heads x 4 query heads, ctx "
                                              "8192, rank 160, budget 2048, 968 landmarks, V in pinned host memory",
                                  **single_layer_gpu_ms()}
        log(f"single layer {detail['single_layer']}")
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU oracle baseline")
        cpu = cpu_baseline(model, args.cpu_runs)
        if detail is not None:
            sl = single_layer_cpu_ms(args.cpu_runs)
            detail["single_layer"].update(sl)
            log(f"single layer CPU {sl}")

    host_store = args.value_store == "host"
    if detail is not None and args.chunk_cache is None and host_store and \
            (any(p > 0 for p in args.pool_variant) or args.encoded_variant or args.device_store_variant or
             args.device_store_batch != 0):
        model = cache = step = None  # release the reference-mode decoder first
        pools = [p for p in args.pool_variant if p > 0]
        if pools:
            detail["chunk_pool"] = [pool_variant(args, shape, p) for p in pools]
        if args.encoded_variant and args.state == "synthetic":
            detail["encoded_state"] = encoded_variant(args, shape, lanes)
        if args.device_store_variant:
            detail["device_value_store"] = device_store_variant(args, shape, args.batch)
        if args.device_store_batch < 0:
            args.device_store_batch = 24 if args.model == "llama31_8b" and args.ctx == 122880 else 0
        if args.device_store_batch > 0:
            # The reference's project page quotes its 122K-context throughput at batch 24 (Llama-3.1-8B:
            # 245.90 tokens/s on one A100, values in host memory; index.html:211-213).
            detail["device_value_store_batch"] = device_store_variant(args, shape, args.device_store_batch)

    out = {
        "metric": ("decode tokens/sec @122K ctx, Llama-3-8B shape; per-kernel HBM GB/s / MFMA util"
                   if args.model == "llama31_8b" else f"decode tokens/sec, {shape.name} shape"),
        "value": round(args.batch * args.steps / elapsed, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": ("synthetic: random-init weights, seeded random ShadowKV state of the exact shapes, greedy tokens"
                 if args.state == "synthetic" else
                 "synthetic: random-init weights, ShadowKV state built by the device encoder from seeded low-rank "
                 "prompt keys, greedy tokens"),
        "config": {"workload": f"{shape.name}-shape {shape.layers}-layer decode, batch {args.batch}, ctx {args.ctx}, "
                               f"ShadowKV rank 160 chunk {args.chunk} budget {args.budget}, "
                               + ("V in pinned host memory, " if host_store else "V in device memory, ")
                               + (f"device chunk pool of {args.chunk_cache} slots, " if args.chunk_cache else "")
                               + f"{lanes} interleaved batch lane(s), "
                               + ("hit moves in their own launches, " if args.separate_hit_moves else
                                  "hit moves in the selection launch, ")
                               + (("value fetch and key rebuild in one launch on each lane's own stream, "
                                   if lane_streams else
                                   "value fetch and key rebuild in one launch on the compute stream, ")
                                  if cache_one_stream else "")
                               + ("RoPE + KV append in the QKV projection's epilogue, "
                                  if qkv_rope_epi else "")
                               + (f"HIP graphs of {per_call} step(s)" if graph else "eager steps"),
                   "global_batch": args.batch, "seq_len": args.ctx, "parallelism": "none (1 GPU)"},
        "roofline": {"kernel": "score_logits (landmark scoring)", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_source": traffic_source, "algorithmic_bytes_per_launch": lb,
                     "avg_launch_us": round(k_ms * 1e3, 2), "timing": timing},
        "roofline_a1a2": {"kernel": "scoring + selection unit (score_logits, then select_chunks: softmax tail, GQA "
                                    "max, top-k, id gather, reorder)", "bound": "hbm",
                          "achieved": round(u_achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(u_achieved / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_launch": ub,
                          "bytes": "per (b, h) row: landmarks n*D*2 + queries G*D*2 read, GQA-max scores n*2 and "
                                   "ids S*8 written", "avg_launch_us": round(u_ms * 1e3, 2), "timing": u_timing},
        "cpu_baseline": cpu,
    }
    if detail is not None:
        out["detail"] = detail
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
