"""Builds libmea.so, the gfx950 HIP library behind the C ABI in include/mea.h.

Every translation unit under csrc/ is compiled with hipcc for gfx950 only
and linked into one shared library next to this file. The library links the
HIP runtime by soname (libamdhip64.so.7); it is loaded after ``import torch``
so it binds to the runtime torch already mapped.

Usage: ``python -m memory_efficient_attn_layer_amd.build`` (or
``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libmea.so"
INCLUDE = PKG.parent / "include"

SOURCES = ["api.hip", "proj.hip", "attn_fwd.hip", "attn_bwd.hip", "gemm.hip", "decode.hip"]

# -packed-fp32-ops: keep hipcc from emitting v_pk_{add,mul,fma}_f32.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: cannot build the gfx950 library")


def _run(cmd: list[str]) -> str:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # The host pass does not know the packed-fp32 feature; that warning is noise.
    out = "\n".join(
        ln for ln in res.stdout.splitlines() if "packed-fp32-ops' is not a recognized feature" not in ln
    )
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compiles every csrc/ translation unit and links libmea.so. Returns its path."""
    hipcc = _hipcc()
    OBJ.mkdir(exist_ok=True)
    objs = [OBJ / (Path(s).stem + ".o") for s in SOURCES]
    cmds = [[hipcc, *HIPCC_FLAGS, "-c", str(CSRC / s), "-o", str(o)] for s, o in zip(SOURCES, objs)]
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 4) // 2), 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for cmd, out in zip(cmds, ex.map(_run, cmds)):
            if verbose or out.strip():
                print(" ".join(cmd[-3:]), "\n", out, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
