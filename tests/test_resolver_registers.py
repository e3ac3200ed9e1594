"""Per-thread register arrays of the resolver's front kernels stay inside their bounds.

The front kernel keeps per-thread state in small arrays (tag rows, packed LRU pairs,
page-bitmap words, early page-table entries, batches of probes and matches) indexed only
from fully unrolled loops, so every index is a constant after unrolling.  Compiled with
``HS_REG_CHECK=1`` every access to them carries a trap for an index outside the array;
a trap the compiler can prove unreachable (a constant index inside the range) is
folded away.  So the front's machine code, for the 16- and 32-slot-per-thread
instantiations and both page-size and LRU forms, must hold no ``s_trap``.  A kernel
with a planted out-of-range index, compiled the same way, must keep one: the check
can fail.  (Nothing here runs on a GPU: the code is compiled to gfx950 assembly only.)
"""

import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from mini_hisparse_amd import build

pytestmark = pytest.mark.skipif(shutil.which(build.HIPCC) is None, reason="hipcc is not installed")

PLANTED = r"""
#include "resolve.hip"
namespace hs {
__global__ void planted_kernel(const int* in, int* out) {
  Regs<int, 4> a;
#pragma unroll
  for (int k = 0; k <= 4; ++k) a[k] = in[k * 64 + threadIdx.x];  // k = 4 is outside a
  int s = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) s += a[k];
  out[threadIdx.x] = s;
}
}  // namespace hs
"""


def device_assembly(source, out):
    cmd = [build.HIPCC, *build.FLAGS, "-DHS_REG_CHECK=1", "--offload-device-only", "-S", "-o", str(out), str(source)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return out.read_text()


def functions(asm, prefix):
    """{mangled name: body} of the kernels whose names start with ``prefix``."""
    out = {}
    for m in re.finditer(rf"^({prefix}\w*):", asm, re.M):
        end = asm.index(".Lfunc_end", m.end())
        out[m.group(1)] = asm[m.end() : end]
    return out


@pytest.fixture(scope="module")
def assemblies(tmp_path_factory):
    tmp = tmp_path_factory.mktemp("regcheck")
    planted = tmp / "planted.hip"
    planted.write_text(PLANTED)
    jobs = [(build.CSRC / "resolve.hip", tmp / "resolve.s"), (planted, tmp / "planted.s")]
    with ThreadPoolExecutor(2) as pool:
        front, plant = pool.map(lambda job: device_assembly(*job), jobs)
    return front, plant


def test_front_register_indices_stay_in_range(assemblies):
    front, _ = assemblies
    kernels = functions(front, "_ZN2hs20resolve_front_kernel")
    # (power-of-two page, int16 LRU) x (16, 32 slots per thread)
    slots = sorted(int(re.search(r"ELi(\d+)EE", name).group(1)) for name in kernels)
    assert slots == [16] * 4 + [32] * 4, sorted(kernels)
    for name, body in kernels.items():
        assert "s_trap" not in body, f"{name}: a per-thread array index can leave its array"
    # the split front's three kernels (int16 and int64 LRU forms of the last two)
    split = functions(front, "_ZN2hs26resolve_split_")
    assert len(split) == 5, sorted(split)
    for name, body in split.items():
        assert "s_trap" not in body, f"{name}: a per-thread array index can leave its array"


def test_a_planted_out_of_range_index_is_caught(assemblies):
    _, plant = assemblies
    (body,) = functions(plant, "_ZN2hs14planted_kernel").values()
    assert "s_trap" in body
