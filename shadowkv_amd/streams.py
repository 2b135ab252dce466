"""Side streams of the decode path, limited to what the hardware queues of a process hold.

HIP maps a process's streams onto at most GPU_MAX_HW_QUEUES hardware queues (4 by default, the
setting of the MI355X hosts this runs on). With more streams than queues, two streams share one
queue; a cross-stream wait queued in that shared queue ahead of the work it waits for can then
block the queue for good. The decode path therefore uses at most 4 streams: the caller's compute
stream and three side streams per device, one per role (the value fetch, the key rebuild, and
the stream a decoder captures its HIP graph on: torch.cuda.graph would otherwise create a capture
stream of its own), created once and shared by every cache and decoder of the process. Work of different
caches on one side stream runs in issue order. A two-lane decoder gives each lane one of the
first two (its one-launch value fetch + key rebuild runs there), so that the lanes' fetches can
overlap on the host link.
"""
from __future__ import annotations

import contextlib
import gc
import threading

import torch

MAX_STREAMS = 4  # compute stream + side streams, per process
ROLES = ("fetch", "rebuild", "capture")
assert len(ROLES) + 1 <= MAX_STREAMS

_lock = threading.Lock()
_streams: dict = {}  # (device index, role) -> torch.cuda.Stream


def side_stream(device, role: str = "fetch") -> torch.cuda.Stream:
    """The process's side stream of `role` on `device` (created on first use, default priority)."""
    if role not in ROLES:
        raise ValueError(f"side stream role {role!r} is not one of {ROLES}")
    dev = torch.device(device)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), role)
    with _lock:
        s = _streams.get(key)
        if s is None:
            s = torch.cuda.Stream(device=dev)
            _streams[key] = s
    return s


def side_streams_created() -> int:
    """Side streams created so far on all devices."""
    return len(_streams)


@contextlib.contextmanager
def capture_graph(graph: torch.cuda.CUDAGraph, device):
    """torch.cuda.graph(graph) on the process's capture side stream, with Python's cyclic garbage
    collector run to completion first and switched off until the capture ends.

    A collection that starts inside the traced code runs the destructors of whatever unreachable
    objects it finds there: dead decoders (their lanes' RoPE closures refer back to them, so only
    the collector frees them) with their HIP graphs, pinned host blocks and events. Freeing those
    while a stream captures in global mode is an illegal call that aborts the process; collecting
    before the capture frees them outside it."""
    enabled = gc.isenabled()
    gc.collect()
    gc.disable()
    try:
        with torch.cuda.graph(graph, stream=side_stream(device, "capture")):
            yield graph
    finally:
        if enabled:
            gc.enable()
