"""Build liboscar_amd.so for gfx950 with hipcc (in-tree, no torch headers).

``python -m oscar_amd.build`` compiles every source under ``oscar_amd/csrc`` into
``oscar_amd/liboscar_amd.so``.  All HIP code is compiled with packed FP32
instructions disabled (``-packed-fp32-ops``).
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "liboscar_amd.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["capi.cpp", "step.cpp", "store.hip", "rotate.hip", "attn_decode.hip", "attn_prefill.hip"]
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def sources() -> list[Path]:
    return [CSRC / s for s in SOURCES if (CSRC / s).exists()]


def build(verbose: bool = False) -> Path:
    """Compile each source to an object in oscar_amd/_build/, then link the .so."""
    out_dir = HERE / "_build"
    out_dir.mkdir(exist_ok=True)
    cmds, objs = [], []
    for src in sources():
        obj = out_dir / (src.stem + ".o")
        cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
        if src.suffix == ".cpp":
            cmd[1:1] = ["-x", "hip"]
        cmds.append(cmd)
        objs.append(str(obj))
    # the sources compile independently: at most one compiler process per source
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)], verbose)
    os.replace(tmp, LIB)
    return LIB


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


if __name__ == "__main__":
    print(build(verbose=True))
