"""Build libsolarkv.so (gfx950) in-tree with hipcc.

The library is compiled from ``solarwm_amd/csrc`` into ``solarwm_amd/libsolarkv.so``; nothing is
JIT-compiled at import time, so the built file travels with the source tree to the GPU host.
Usage: ``python -m solarwm_amd.build`` (also called by ``__graft_entry__.build()``).

Every translation unit that issues matrix-core products is also compiled to device assembly
(``--cuda-device-only -S``, side by side with the objects) and checked by ``isa_check``: a
library in which any path reads an MFMA result before its wait states have elapsed is not
linked.
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
    from . import isa_check

    hipcc = _hipcc()
    with tempfile.TemporaryDirectory(prefix="skv_build_") as tmp:
        # the translation units compile side by side (one hipcc process each), and so do the
        # device listings of those with MFMAs
        jobs, listings = [], []
        for src in sources():
            obj = Path(tmp) / (src.stem + ".o")
            cmds = [(obj, [hipcc, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])]
            if src.suffix == ".hip" and "__builtin_amdgcn_mfma" in src.read_text():
                asm = Path(tmp) / (src.stem + ".s")
                cmds.append((asm, [hipcc, *HIP_FLAGS, "--cuda-device-only", "-S", str(src), "-o", str(asm)]))
                listings.append(asm)
            for out_path, cmd in cmds:
                if verbose:
                    print(" ".join(cmd), flush=True)
                jobs.append((src, out_path, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                             stderr=subprocess.PIPE, text=True)))
        objs, failed = [], []
        for src, out_path, proc in jobs:
            out, err = proc.communicate()
            if proc.returncode != 0:
                failed.append(f"hipcc failed on {src.name}:\n{out}\n{err}")
            if out_path.suffix == ".o":
                objs.append(str(out_path))
        if failed:
            raise RuntimeError("\n".join(failed))
        short = []
        for asm in listings:
            for name, paths in isa_check.check_listing(asm.read_text()).items():
                short += [f"{asm.stem}: {name}: {p}" for p in paths]
        if short:
            raise RuntimeError("MFMA results read before their wait states (not linked):\n" +
                               "\n".join(short))
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
