"""End-to-end parity with the reference CLI ``demo`` (BASELINE configs[0] and friends).

The golden file holds the reference's generated tokens, row statistics and
policy counters (tests/golden/make_golden.py).  On CPU the product's engine,
model and cache run with the oracle kernels: every counter must match.  On
the GPU the HIP kernels run and mirror completion is asynchronous, so the
tokens and the total number of selected rows must match while the split
between resident / hot / miss may follow the device's event timing.
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
