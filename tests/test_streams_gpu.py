"""The transfer streams overlap the compute stream: HIP binds streams to a few hardware
queues in turn, and a side stream on the compute stream's queue would run in its order."""

import time

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_independent_stream_runs_beside_the_current_stream(gpu):
    from mini_hisparse_amd.streams import independent_stream

    # streams created first shift the hardware queues the next ones get
    extra = [torch.cuda.Stream(gpu) for _ in range(5)]
    side = independent_stream(gpu)
    current = torch.cuda.current_stream(gpu)
    current.synchronize()
    torch.cuda._sleep(20_000_000)
    spun = torch.cuda.Event()
    spun.record(current)
    marker = torch.cuda.Event()
    marker.record(side)
    deadline = time.perf_counter() + 1.0
    while not marker.query() and time.perf_counter() < deadline:
        time.sleep(0.0001)
    assert marker.query() and not spun.query()
    current.synchronize()
    del extra


def test_engine_transfer_stream_is_independent(gpu):
    """The batched engine's transfer stream, after its projection choice created a capture
    stream, is probed to its own queue."""
    from mini_hisparse_amd.batched_engine import BatchedDecodeEngine, build_state, random_model
    from tests.test_batched_engine import tiny

    wl = tiny(selector="uniform")
    engine = BatchedDecodeEngine(random_model(wl, gpu, seed=1), build_state(wl, gpu, seed=2), wl.top_pages,
                                 selector="uniform")
    current = torch.cuda.current_stream(gpu)
    current.synchronize()
    torch.cuda._sleep(20_000_000)
    spun = torch.cuda.Event()
    spun.record(current)
    marker = torch.cuda.Event()
    marker.record(engine.transfer)
    deadline = time.perf_counter() + 1.0
    while not marker.query() and time.perf_counter() < deadline:
        time.sleep(0.0001)
    assert marker.query() and not spun.query()
    current.synchronize()
