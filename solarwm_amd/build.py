"""Build libsolarkv.so (gfx950) in-tree with hipcc.

The library is compiled from ``solarwm_amd/csrc`` into ``solarwm_amd/libsolarkv.so``; nothing is
JIT-compiled at import time, so the built file travels with the source tree to the GPU host.
Usage: ``python -m solarwm_amd.build`` (also called by ``__graft_entry__.build()``).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "libsolarkv.so"
ARCH = "gfx950"

# Every HIP translation unit is built with packed-fp32 instruction selection disabled; the
# host pass prints a harmless "not a recognized feature" warning for it.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (looked at $HIPCC, /opt/rocm/bin/hipcc, PATH)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def build(verbose: bool = False) -> Path:
    """Compile every source under csrc/ and link libsolarkv.so; returns its path."""
    hipcc = _hipcc()
    with tempfile.TemporaryDirectory(prefix="skv_build_") as tmp:
        # the translation units compile side by side (one hipcc process each)
        jobs = []
        for src in sources():
            obj = Path(tmp) / (src.stem + ".o")
            cmd = [hipcc, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
            if verbose:
                print(" ".join(cmd), flush=True)
            jobs.append((src, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                    stderr=subprocess.PIPE, text=True)))
        objs, failed = [], []
        for src, obj, proc in jobs:
            out, err = proc.communicate()
            if proc.returncode != 0:
                failed.append(f"hipcc failed on {src.name}:\n{out}\n{err}")
            objs.append(str(obj))
        if failed:
            raise RuntimeError("\n".join(failed))
        tmp_lib = Path(tmp) / LIB_PATH.name
        cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp_lib)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
        # atomic replace so a process holding the old mapping keeps a consistent file
        staged = LIB_PATH.with_suffix(".so.tmp")
        shutil.copyfile(tmp_lib, staged)
        os.replace(staged, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
