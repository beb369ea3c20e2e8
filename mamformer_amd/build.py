"""Build libmamformer_hip.so (gfx950) in-tree from mamformer_amd/csrc/*.hip.

Usage: ``python -m mamformer_amd.build`` (or ``build()`` from Python).  Each
source is compiled separately with hipcc (in parallel), then linked into one
shared library next to this file.  Always rebuilds.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB_NAME = "libmamformer_hip.so"
LIB_PATH = HERE / LIB_NAME
OFFLOAD_ARCH = "gfx950"

SOURCES = ["ssd_decode.hip", "ssd_prefill.hip", "ssd_lookback.hip", "ssd_hstates.hip", "ssd_refform.hip", "ssd_backward.hip", "kda_scan.hip", "kda_backward.hip", "kda_precise.hip", "kda_step.hip", "conv1d.hip", "widen.hip", "capi.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # no packed fp32 instructions (v_pk_{add,mul,fma}_f32) anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{res.stderr}")
    return res


def build(verbose: bool = False) -> Path:
    hipcc = _hipcc()
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = objdir / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    with cf.ThreadPoolExecutor(max_workers=min(4, len(cmds))) as ex:
        for cmd, _ in zip(cmds, ex.map(_run, cmds)):
            if verbose:
                print(" ".join(cmd), file=sys.stderr)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose=True)
    print(path)
