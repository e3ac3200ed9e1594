"""Build libhisparse_hip.so (gfx950) in-tree with hipcc.

Usage: ``python -m mini_hisparse_amd.build`` (also called by ``__graft_entry__.build``).
Sources are compiled in parallel to objects under ``_build/`` and linked into
``mini_hisparse_amd/libhisparse_hip.so``.
"""

from __future__ import annotations

import os
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


def _compile(src: Path, obj: Path):
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    return err


def build(verbose: bool = True) -> Path:
    out_dir = ROOT / "_build"
    out_dir.mkdir(exist_ok=True)
    srcs = sources()
    objs = [out_dir / (s.stem + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=min(len(srcs), 8)) as pool:
        logs = list(pool.map(_compile, srcs, objs))
    if verbose:
        for src, log in zip(srcs, logs):
            if log.strip():
                print(f"[{src.name}]\n{log}", file=sys.stderr)
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
