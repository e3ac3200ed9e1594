"""End-to-end parity with the reference CLI ``demo`` (BASELINE configs[0] and friends).

The golden file holds the reference's generated tokens, row statistics and
policy counters (tests/golden/make_golden.py).  On CPU the product's engine,
model and cache run with the oracle kernels: every counter must match.  On
the GPU the HIP kernels run and mirror completion is asynchronous, so the
tokens and the total number of selected rows must match while the split
between resident / hot / miss may follow the device's event timing.  The split
is not a device-independent quantity of the reference either: a CPU cache has
no mirror events (host_ready is None), so under block pressure it finds no
mirror to wait for and raises CapacityError, where a device cache waits for a
completed-but-unpublished mirror and keeps the page (hybrid.py:369-378).  Even
with every device event waited for as it is recorded, the 65-token case keeps
26 resident / 16 hot rows on the GPU against the CPU golden's 10 / 32.  The
257-token case matches every row count and location on
the GPU too, and the test asserts that.
"""

import json
import os

import pytest
import torch

from mini_hisparse_amd.cli import build_parser, run
from tests.conftest import gpu_available
from tests.cpu_ops import CpuOracleOps

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "demo_outputs.json")
with open(GOLDEN) as f:
    CASES = json.load(f)["cases"]


def _args(argv, device):
    argv = list(argv)
    argv[argv.index("--device") + 1] = device
    return build_parser().parse_args(argv)


@pytest.mark.parametrize("case", CASES, ids=[" ".join(c["argv"][3:7]) for c in CASES])
def test_demo_matches_reference_on_cpu(case):
    torch.set_num_threads(1)
    report = run(_args(case["argv"], "cpu"), ops=CpuOracleOps())
    assert report["outputs"] == case["outputs"]
    assert report["requests"] == case["requests"]
    assert report["row_stats"] == case["row_stats"]
    assert report["stats"] == case["stats"]
    assert report["locations"] == case["locations"]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[" ".join(c["argv"][3:7]) for c in CASES])
def test_demo_matches_reference_on_gpu(case):
    if not gpu_available():
        pytest.skip("no ROCm GPU")
    report = run(_args(case["argv"], "cuda:0"))
    assert report["outputs"] == case["outputs"]
    assert report["requests"] == case["requests"]
    rows = report["row_stats"]
    expected = case["row_stats"]
    total = expected["resident_hits"] + expected["hot_hits"] + expected["misses"]
    assert rows["resident_hits"] + rows["hot_hits"] + rows["misses"] == total
    if case["argv"][case["argv"].index("--prompt-tokens") + 1] == "257":
        # no block pressure waits on a mirror, so the device's
        # event timing does not move any row: the full split and the final locations
        assert rows == expected
        assert report["locations"] == case["locations"]


PAGED = os.path.join(os.path.dirname(__file__), "golden", "paged_demo_outputs.json")
with open(PAGED) as f:
    PAGED_CASES = json.load(f)["cases"]
PAGED_IDS = [" ".join(c["argv"][9:]) for c in PAGED_CASES]


@pytest.mark.parametrize("case", PAGED_CASES, ids=PAGED_IDS)
def test_paged_demo_matches_reference_on_cpu(case):
    """The page layout end to end (eviction policy, window overlap, chunk width): tokens,
    every counter (misses, evictions, hits, windows, bytes) and the final page locations."""
    torch.set_num_threads(1)
    report = run(_args(case["argv"], "cpu"), ops=CpuOracleOps())
    assert report["outputs"] == case["outputs"]
    assert report["requests"] == case["requests"]
    assert report["stats"] == case["stats"]
    assert report["locations"] == case["locations"]
    assert report["timeline"][-1] == case["final_timeline"]


@pytest.mark.gpu
@pytest.mark.parametrize("case", PAGED_CASES, ids=PAGED_IDS)
def test_paged_demo_matches_reference_on_gpu(case):
    """On the GPU (hs_attend_window) the placement decisions are host logic, so the
    counters that follow them match too; only the reclamation of retired host slots
    follows the device's event timing."""
    if not gpu_available():
        pytest.skip("no ROCm GPU")
    report = run(_args(case["argv"], "cuda:0"))
    assert report["outputs"] == case["outputs"]
    assert report["requests"] == case["requests"]
    timing = {"reclaimed_requests"}
    assert {k: v for k, v in report["stats"].items() if k not in timing} == {
        k: v for k, v in case["stats"].items() if k not in timing
    }
