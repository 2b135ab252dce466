"""Side streams of the decode path, limited to what the hardware queues of a process hold.

HIP maps a process's streams onto at most GPU_MAX_HW_QUEUES hardware queues (4 by default, the
setting of the MI355X hosts this runs on). With more live streams than queues, two streams share
one queue; a cross-stream wait queued in that shared queue ahead of the work it waits for can then
block the queue for good. The decode path therefore uses at most 4 streams: the caller's compute
stream and up to 3 side streams (the value fetch, the key rebuild, and one spare), and every side
stream the package creates goes through side_stream(), which refuses a fourth live one.
"""
from __future__ import annotations

import weakref

import torch

MAX_STREAMS = 4  # compute stream + side streams, per process
_live: "weakref.WeakSet[torch.cuda.Stream]" = weakref.WeakSet()


def live_side_streams() -> int:
    """Distinct side streams created by side_stream() that are still referenced."""
    return len({s.cuda_stream for s in list(_live)})


def side_stream(device) -> torch.cuda.Stream:
    """A new side stream at the default priority; raises RuntimeError when the process would hold
    more than MAX_STREAMS streams with the compute stream counted."""
    if live_side_streams() + 1 >= MAX_STREAMS:
        import gc
        gc.collect()  # streams of dropped caches may still sit in reference cycles
        if live_side_streams() + 1 >= MAX_STREAMS:
            raise RuntimeError(f"the decode path would use more than {MAX_STREAMS} streams (the hardware queues "
                               f"of a process): {live_side_streams()} side streams are live; release caches or "
                               f"share their streams")
    s = torch.cuda.Stream(device=device)
    _live.add(s)
    return s
