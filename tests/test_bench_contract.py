"""bench.py's command-line contract on a host without a GPU: more than one GPU is refused with a
message, before anything touches the device."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_multi_gpu_request_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_trace_summary_window_and_ops(tmp_path):
    """The kernel-trace summary takes the timed steps' window (after the warm-up steps' logits
    launches) and sums each operation's kernels per lane-layer; the kernel table then reads it."""
    import csv
    import importlib.util
    import types

    spec = importlib.util.spec_from_file_location("bench", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    layers, lanes, warmup, steps = 2, 2, 1, 2
    rows, t = [], 0

    def k(name, us):
        nonlocal t
        rows.append({"Kernel_Name": name, "Start_Timestamp": str(t), "End_Timestamp": str(t + int(us * 1000))})
        t += int(us * 1000) + 1000

    for step in range(warmup + steps + 1):  # the extra step marks the window's end
        slow = 1000 if step < warmup else 1  # warm-up kernels must not count
        for _ in range(layers * lanes):
            k("void (anonymous namespace)::logits_kernel<4>(Args)", 30 * slow)
            k("softmax_vec_kernel<false, true, 4, 2>(A)", 10)
            k("select_kernel<4>(A)", 20)
            k("attn_split_kernel<4, false, 128, false>(A)", 15)
            k("attn_combine_kernel(A)", 5)
        k("at::native::elementwise_kernel(x)", 3)
    path = tmp_path / "trace.csv"
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    out = bench.summarize_trace(str(path), layers, lanes, warmup, steps)
    ops = out["op_us_per_lane_layer"]
    assert ops == {"score_logits": 30.0, "select_chunks": 30.0, "sparse_attn_decode": 20.0}
    assert out["kernels"]["select_kernel<4>"]["launches_per_step"] == layers * lanes
    # applied to the kernel table of the same workload
    args = types.SimpleNamespace(model="tiny", batch=2, ctx=100, budget=64, chunk=8)
    summary = tmp_path / "s.json"
    import json
    summary.write_text(json.dumps({"workload": bench.trace_workload(args, lanes), **out}))
    bench.trace_summary_path = lambda a: summary
    bench.ROOT = tmp_path
    table = [{"kernel": "unit", "trace_ops": ["score_logits", "select_chunks"], "in_step_us": 99.0,
              "algorithmic_bytes": 480000, "peak": 8000.0},
             {"kernel": "fetch", "trace_ops": ["gather_copy_with_offsets"], "in_step_us": 7.0,
              "algorithmic_bytes": 1, "peak": 1.0}]
    bench.apply_trace_summary(table, args, lanes)
    assert table[0]["in_step_us"] == 60.0 and table[0]["eager_instrumented_us"] == 99.0
    assert table[0]["in_step_frac"] == round(480000 / 60.0 / 1e3 / 8000.0, 4)
    assert table[1]["in_step_us"] == 7.0 and "eager_instrumented_us" not in table[1]


def test_device_store_variant_reports_a_state_that_does_not_fit(monkeypatch):
    """The device-store variant at a batch whose state does not fit in device memory reports the
    allocation failure in its detail entry instead of ending the bench run (stand-in decoder and
    device calls, no GPU)."""
    import importlib.util
    import types

    import torch

    spec = importlib.util.spec_from_file_location("bench", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    from shadowkv_amd import decode_model

    def no_room(*a, **kw):
        raise torch.cuda.OutOfMemoryError("HIP out of memory. Tried to allocate 6.04 GiB\nmore text")

    monkeypatch.setattr(decode_model, "SyntheticDecoder", no_room)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **kw: None)
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: None)
    monkeypatch.setattr(torch._C, "_host_emptyCache", lambda: None)
    args = types.SimpleNamespace(budget=2048, ctx=122880, chunk=8, warmup=1, steps=2, graph_steps=2)
    res = bench.device_store_variant(args, decode_model.LLAMA31_8B, 64)
    assert res == {"batch": 64, "skipped": "state does not fit in device memory: HIP out of memory. Tried to "
                                          "allocate 6.04 GiB"}
