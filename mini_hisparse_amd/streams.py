"""A side stream that the GPU runs beside the caller's stream.

HIP binds every new stream to one of a few hardware queues (``GPU_MAX_HW_QUEUES``, 4
by default) in turn, and a queue runs its packets in order: a side stream bound to the
queue of the stream it should overlap is serialised with it (a transfer stream's
gathers then wait behind the compute stream's dense layers).  Which queue a stream
gets depends on every stream the process created before it, so it is probed.
"""

from __future__ import annotations

import time

import torch

# spin of the probe: ~4 ms at 2.4 GHz, far above an idle queue's event latency
_PROBE_CYCLES = 10_000_000


def independent_stream(device, tries=8):
    """A new stream whose work runs beside the current stream's.  Each candidate is
    probed: a spin kernel on the current stream, then an event on the candidate; the
    candidate has its own hardware queue when that event completes while the spin is
    still running.  After ``tries`` candidates that share the queue (a process with a
    single hardware queue), the last one is returned: work on it is still correct, only
    not overlapped."""
    device = torch.device(device)
    current = torch.cuda.current_stream(device)
    candidate = None
    for _ in range(tries):
        candidate = torch.cuda.Stream(device)
        current.synchronize()
        with torch.cuda.stream(current):
            torch.cuda._sleep(_PROBE_CYCLES)
        spun = torch.cuda.Event()
        spun.record(current)
        marker = torch.cuda.Event()
        marker.record(candidate)
        deadline = time.perf_counter() + 0.5
        while not marker.query() and time.perf_counter() < deadline:
            time.sleep(0.0001)
        independent = marker.query() and not spun.query()
        current.synchronize()
        if independent:
            return candidate
    return candidate
