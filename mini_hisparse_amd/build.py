"""Build libhisparse_hip.so (gfx950) in-tree with hipcc.

Usage: ``python -m mini_hisparse_amd.build`` (also called by ``__graft_entry__.build``).
Sources are compiled in parallel to objects under ``_build/`` and linked into
``mini_hisparse_amd/libhisparse_hip.so``.

Every kernel's register use is read from the compiler's resource-usage remarks and
written to ``_build/resource_usage.txt``.  A kernel that uses scratch memory or spills
VGPRs fails the build: a spilling build of the resolver's front kernel once returned
wrong tags for one register row, so no shipped kernel may spill.  (SGPR spills go to
VGPR lanes, not memory, and are only listed.)
"""

from __future__ import annotations

import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = ROOT / "include"
LIBRARY = PACKAGE / "libhisparse_hip.so"
ARCH = os.environ.get("HS_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # only the extern "C" API of include/hisparse.h is exported (the header sets default
    # visibility on it): kernel handles, device variables and hs:: helpers stay private, so
    # two copies of the library in one process cannot bind each other's symbols
    "-fvisibility=hidden",
    "-fvisibility-inlines-hidden",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # packed fp32 instructions are kept out of the device code
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def sources():
    return sorted(CSRC.glob("*.hip"))


REMARK = re.compile(r"remark:\s+(Function Name|ScratchSize \[bytes/lane\]|VGPRs|AGPRs|VGPRs Spill|"
                    r"SGPRs Spill|Occupancy \[waves/SIMD\]|LDS Size \[bytes/block\]):\s*(\S+)")


def resource_usage(stderr: str):
    """Per-kernel resource figures from ``-Rpass-analysis=kernel-resource-usage`` remarks:
    a list of dicts with the mangled name, VGPRs, AGPRs, scratch bytes per lane, VGPR and
    SGPR spills, occupancy and LDS bytes."""
    kernels, cur = [], None
    for line in stderr.splitlines():
        m = REMARK.search(line)
        if not m:
            continue
        key, value = m.group(1), m.group(2)
        if key == "Function Name":
            cur = {"name": value}
            kernels.append(cur)
        elif cur is not None:
            cur[key.split(" [")[0]] = int(value)
    return kernels


def spilling(kernels):
    """The kernels that use scratch memory or spill VGPRs."""
    return [k for k in kernels if k.get("ScratchSize", 0) or k.get("VGPRs Spill", 0)]


def _compile(src: Path, obj: Path):
    cmd = [HIPCC, *FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    lines = [line for line in proc.stderr.splitlines() if noise not in line]
    if proc.returncode:
        raise RuntimeError(f"hipcc failed for {src.name}:\n" + "\n".join(lines))
    kernels = resource_usage(proc.stderr)
    # the remarks (and the source lines clang echoes under them) are read, not printed
    warnings = [line for line in lines if "remark:" not in line and "Rpass-analysis" not in line
                and not re.match(r"^\s*(\d+ \||\|)", line)]
    return "\n".join(warnings), kernels


def build(verbose: bool = True) -> Path:
    out_dir = ROOT / "_build"
    out_dir.mkdir(exist_ok=True)
    srcs = sources()
    objs = [out_dir / (s.stem + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=min(len(srcs), 8)) as pool:
        results = list(pool.map(_compile, srcs, objs))
    if verbose:
        for src, (log, _) in zip(srcs, results):
            if log.strip():
                print(f"[{src.name}]\n{log}", file=sys.stderr)
    table = ["source kernel vgprs agprs scratch vgpr_spill sgpr_spill occupancy lds"]
    for src, (_, kernels) in zip(srcs, results):
        for k in kernels:
            table.append(f"{src.name} {k['name']} {k.get('VGPRs', '?')} {k.get('AGPRs', '?')} "
                         f"{k.get('ScratchSize', '?')} {k.get('VGPRs Spill', '?')} {k.get('SGPRs Spill', '?')} "
                         f"{k.get('Occupancy', '?')} {k.get('LDS Size', '?')}")
    (out_dir / "resource_usage.txt").write_text("\n".join(table) + "\n")
    bad = [(src.name, k) for src, (_, kernels) in zip(srcs, results) for k in spilling(kernels)]
    if bad:
        listing = "\n".join(f"  {name}: {k['name']} scratch {k.get('ScratchSize')} B/lane, "
                             f"{k.get('VGPRs Spill')} VGPRs spilled" for name, k in bad)
        raise RuntimeError("kernels use scratch memory or spill VGPRs (not allowed):\n" + listing)
    if not any(kernels for _, kernels in results):
        raise RuntimeError("no kernel resource-usage remarks were found; the spill check did not run")
    tmp = LIBRARY.with_suffix(".so.tmp")
    # the dynamic symbol table holds the hs_* C API only: kernel handles of
    # non-template kernels and the per-file offload ids keep default visibility
    # under -fvisibility=hidden, so a version script makes them local
    exports = out_dir / "exports.map"
    exports.write_text("{\n  global: hs_*;\n  local: *;\n};\n")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,--version-script={exports}",
           "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build()
