"""Decode throughput of the ShadowKV sparse decode path on one MI355X.

Workload (default): Llama-3.1-8B shape (32 layers, hidden 4096, FFN 14336, GQA 32/8, head_dim
128, vocab 128256), random-init bf16 weights, batch 8, 122880-token context per sequence,
ShadowKV rank 160, chunk 8, sparse budget 2048 (256 chunks), 48 outlier chunks, values of every
layer offloaded to pinned host memory (64.4 GB). The post-prefill state is synthesized from
seeded random tensors of the exact shapes (no 122K-token prefill/SVD is run); timing covers
greedy decode steps only. A step = one new token for all 8 sequences through all 32 layers.

Prints one JSON line. `roofline` is measured live on the landmark-scoring kernel (the
largest HBM stream of the path) with HIP events on its stream during the timed steps;
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
    p.add_argument("--layers", type=int, default=None, help="override the layer count (debug only)")
    p.add_argument("--cpu-runs", type=int, default=10)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-breakdown", action="store_true")
    return p.parse_args()


class KernelTimer:
    """Brackets every call of one shim function with HIP events on the current stream."""

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
            s.record()
            out = self.orig(*a, **kw)
            e.record()
            self.pairs.append((s, e))
            return out

        setattr(module, name, wrapped)

    def mean_ms(self) -> float:
        return statistics.fmean(s.elapsed_time(e) for s, e in self.pairs)


def logits_bytes(BH: int, G: int, n: int, D: int = 128) -> int:
    """Algorithmic HBM bytes of one score_logits launch: landmarks + queries read, logits and
    per-256-column (max, sum) partials written."""
    tiles = (n + 255) // 256
    return BH * (n * D * 2 + G * D * 2 + G * n * 2 + G * tiles * 8)


def cpu_baseline(model, runs: int) -> dict:
    """The CPU oracle on one layer's hot-path ops at the workload's shapes (layer 0 state)."""
    import torch
    import oracle

    cache = model.cache
    threads = max(1, min(os.cpu_count() or 1, 16))
    torch.set_num_threads(threads)
    B, H, D = cache.batch_size, cache.num_key_value_heads, cache.head_dim
    Hq = cache.num_attention_heads
    st = oracle.LayerState(
        U=cache.U[0].cpu(), SV=cache.SV[0].cpu(), landmarks=cache.k_landmark[0].cpu(),
        landmark_idx=cache.k_landmark_idx[0].cpu(), host_v=cache.v_cache_cpu[0], kbuf=cache.k_cache_buffer[0].cpu(),
        vbuf=cache.v_cache_buffer[0].cpu(), position_ids=cache.position_ids[0].cpu(),
        prefill_local=cache.prefill_local, sparse_start=cache.sparse_start, sparse_end=cache.sparse_end,
        chunk=cache.chunk_size, budget=cache.sparse_budget, ctx=cache.prefill, buf_len=cache.buf_len)
    cos_sin = model.cos_sin.cpu()
    g = torch.Generator().manual_seed(5)
    times = []
    for i in range(3 + runs):
        q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
        k = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
        v = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
        t0 = time.perf_counter()
        oracle.decode_layer_step(st, q, k, v, cos_sin, gen_offset=0)
        dt = time.perf_counter() - t0
        if i >= 3:
            times.append(dt)
    layer_s = statistics.median(times)
    return {"value": round(B / (layer_s * cache.num_layers), 3), "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": (f"oracle (CPU torch/numpy) restatement of one layer's hot-path ops (scoring, GQA max, top-k, "
                       f"reorder, value fetch, key compaction, rebuild+RoPE, attention) at batch {B}, ctx "
                       f"{cache.prefill}, layer-0 state; median of {runs} runs after 3 warmups = "
                       f"{layer_s * 1e3:.1f} ms/layer, scaled to {cache.num_layers} layers; dense layers excluded; "
                       f"reported baseline only")}


def breakdown(model, tok) -> dict:
    """One instrumented step: per-op device time of the sparse path and the host-link rate."""
    import torch
    from shadowkv_amd.kernels import shadowkv

    names = ["apply_rotary_pos_emb_new", "score_logits", "select_chunks", "gather_copy_with_offsets",
             "gather_copy_d2d_with_offsets", "rebuild_k_rope", "sparse_attn_decode"]
    timers = {n: KernelTimer(shadowkv, n) for n in names}
    cache = model.cache
    snaps = []  # per-layer copies of the hit counts, taken on the device (no host sync in the step)
    orig_select = timers["select_chunks"].orig

    def select_and_snapshot(*a, **kw):
        out = orig_select(*a, **kw)
        snaps.append(cache.cnts.clone())
        return out

    timers["select_chunks"].orig = select_and_snapshot
    for t in timers.values():
        t.active = True
    torch.cuda.synchronize()
    model.decode_step(tok)
    torch.cuda.synchronize()
    timers["select_chunks"].orig = orig_select
    for t in timers.values():
        t.active = False
        setattr(shadowkv, t.name, t.orig)
    ops = {n: round(t.mean_ms() * 1e3, 2) for n, t in timers.items() if t.pairs}
    chunk_bytes = cache.chunk_size * cache.head_dim * 2
    fetch_ms = timers["gather_copy_with_offsets"].mean_ms()
    total_sel = cache.select_sets * cache.batch_size * cache.num_key_value_heads
    miss_mean = statistics.fmean(total_sel - int(c.sum()) for c in snaps)
    return {"op_us_per_layer": ops, "hit_rate": round(1 - miss_mean / total_sel, 4),
            "host_link": {"bytes_per_layer": int(miss_mean * chunk_bytes),
                          "GBps": round(miss_mean * chunk_bytes / (fetch_ms * 1e-3) / 1e9, 2),
                          "note": "value fetch (hit compaction + zero-copy miss gather) per layer"}}


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the sparse decode path is not sharded "
              f"across GPUs in this build", file=sys.stderr)
        return 2
    import torch
    from shadowkv_amd import decode_model
    from shadowkv_amd.kernels import shadowkv
    from dataclasses import replace

    shape = decode_model.LLAMA31_8B
    if args.layers:
        shape = replace(shape, layers=args.layers)
    t0 = time.time()
    log(f"building {shape.name} batch {args.batch} ctx {args.ctx} (random weights, synthesized state)")
    model = decode_model.SyntheticDecoder(shape, args.batch, args.ctx, sparse_budget=args.budget,
                                          decode_len=args.warmup + args.steps + 8)
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

    timer = KernelTimer(shadowkv, "score_logits")
    timer.active = True
    torch.cuda.synchronize()
    start = time.perf_counter()
    for i in range(args.steps):
        tok = model.decode_step(tok)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    timer.active = False
    setattr(shadowkv, "score_logits", timer.orig)
    log(f"timed {args.steps} steps in {elapsed:.3f}s")

    n = cache.k_landmark.shape[-2]
    BH = args.batch * shape.kv_heads
    G = shape.heads // shape.kv_heads
    lb = logits_bytes(BH, G, n)
    k_ms = timer.mean_ms()
    achieved = lb / (k_ms * 1e-3) / 1e9
    traffic = None
    tfile = ROOT / "profiles" / "score_logits_traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("bytes_per_launch")

    detail = None
    if not args.no_breakdown:
        detail = breakdown(model, tok)
        log(f"breakdown {detail}")
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU oracle baseline")
        cpu = cpu_baseline(model, args.cpu_runs)

    out = {
        "metric": "decode tokens/sec @122K ctx, Llama-3-8B shape; per-kernel HBM GB/s / MFMA util",
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
        "data": "synthetic: random-init weights, seeded random ShadowKV state of the exact shapes, greedy tokens",
        "config": {"workload": f"{shape.name}-shape {shape.layers}-layer decode, batch {args.batch}, ctx {args.ctx}, "
                               f"ShadowKV rank 160 chunk 8 budget {args.budget}, V in pinned host memory",
                   "global_batch": args.batch, "seq_len": args.ctx, "parallelism": "none (1 GPU)"},
        "roofline": {"kernel": "score_logits (landmark scoring)", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "algorithmic_bytes_per_launch": lb, "avg_launch_us": round(k_ms * 1e3, 2)},
        "cpu_baseline": cpu,
    }
    if detail is not None:
        out["detail"] = detail
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
