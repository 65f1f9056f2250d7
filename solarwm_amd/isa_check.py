"""Static check of the gfx950 device assembly that hipcc writes for the library's kernels.

A matrix-core product (MFMA) writes its result registers several passes after it issues, and the
hardware does not hold back a later VALU, LDS or memory instruction that touches them: the
compiler must leave enough independent issue slots ("wait states") in between.  On gfx950 a VALU
read or write of an MFMA's result needs NumPasses + 4 of them (12 after an 8-pass product, 20
after a 16-pass one); a memory load that only overwrites the result needs one fewer.  hipcc's own
hazard pass has been seen to leave one such path short: a branch around a block put a VALU
compare 2 slots after the row-sum product it read, and the compare saw the previous tile's value.

``check_function`` walks every control-flow path forward from each MFMA (branches, fall-through)
and reports every instruction that touches the product's result registers before the wait
states have elapsed.  ``s_nop N`` counts N + 1, a later MFMA counts its own passes (it issues
only once the earlier product has left the pipeline) and anything else counts 1.  A later MFMA
that reads the result as its accumulator is left to the hardware's MFMA-to-MFMA rules.

``build.py`` runs it over every kernel of the translation units that hold MFMAs and refuses to
link a library that has a short path.
"""
from __future__ import annotations

import heapq
import re
from dataclasses import dataclass

# passes of each MFMA form the kernels use (gfx950, dense): 32x32x64 fp8 = 65536 MACs at 1024
# MACs per clock per SIMD = 64 clocks = 16 passes of 4 clocks; the others likewise.  Passes + 4
# is exactly the wait hipcc's hazard pass leaves before a VALU read in straight-line code (20,
# 12, 12, 12, 8 wait states; tests/test_isa_check.py compiles one product of each form).
PASSES = {
    "v_mfma_f32_32x32x64_f8f6f4": 16,
    "v_mfma_scale_f32_32x32x64_f8f6f4": 16,
    "v_mfma_f32_16x16x128_f8f6f4": 8,
    "v_mfma_scale_f32_16x16x128_f8f6f4": 8,
    "v_mfma_f32_32x32x16_bf16": 8,
    "v_mfma_f32_32x32x16_f16": 8,
    "v_mfma_f32_16x16x32_bf16": 4,
    "v_mfma_f32_16x16x32_f16": 4,
}
EXTRA_WAIT = 4  # wait states beyond the pass count before a VALU touches the result

_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")
_LOADS = ("ds_read", "buffer_load", "global_load", "flat_load", "scratch_load")


def _regs(text: str) -> set[str]:
    out: set[str] = set()
    for p, a, b, q, c in _REG.findall(text):
        if p:
            out |= {f"{p}{r}" for r in range(int(a), int(b) + 1)}
        else:
            out.add(f"{q}{c}")
    return out


@dataclass
class ShortPath:
    mfma: str       # the product
    reader: str     # the instruction that touches its result too early
    waited: int     # wait states on the shortest path
    needed: int

    def __str__(self) -> str:
        return f"{self.mfma!r} -> {self.reader!r}: {self.waited} wait states < {self.needed}"


def functions(asm: str):
    """(symbol, body lines) of every function in a hipcc -S listing."""
    lines = asm.split("\n")
    cur = None
    for i, line in enumerate(lines):
        m = re.match(r"^([^\s:;]+):\s*;\s*@(\S+)\s*$", line)  # "name: ; @name" opens a function
        if m and m.group(1) == m.group(2):
            cur = (m.group(1), i)
        elif cur and line.startswith(".Lfunc_end"):
            yield cur[0], lines[cur[1] + 1:i]
            cur = None


def check_function(body: list[str]) -> list[ShortPath]:
    """Short MFMA-result paths of one function body (assembly lines)."""
    ins: list[str] = []
    labels: dict[str, int] = {}
    for line in body:
        t = line.split(";")[0].strip()
        if not t:
            continue
        if t.endswith(":"):
            labels[t[:-1]] = len(ins)
            continue
        if t.startswith("."):
            continue
        ins.append(t)

    def succ(j: int) -> list[int]:
        op, *rest = ins[j].split()
        if op == "s_endpgm":
            return []
        if op == "s_branch":
            return [labels[rest[0]]]
        if op.startswith("s_cbranch"):
            return [labels[rest[0]], j + 1]
        return [j + 1] if j + 1 < len(ins) else []

    def cost(t: str) -> int:
        m = re.match(r"s_nop\s+(\d+)", t)
        if m:
            return int(m.group(1)) + 1
        return PASSES.get(t.split()[0], 1)

    found: list[ShortPath] = []
    for i, t in enumerate(ins):
        op = t.split()[0]
        if "mfma" not in op:
            continue
        if op not in PASSES:
            found.append(ShortPath(t, "(pass count of this MFMA form unknown)", 0, 0))
            continue
        need = PASSES[op] + EXTRA_WAIT
        dst = _regs(t.split(",")[0])
        best: dict[int, int] = {}
        heap = [(0, i + 1)]
        while heap:
            w, j = heapq.heappop(heap)
            if j >= len(ins) or w >= need or best.get(j, 1 << 30) <= w:
                continue
            best[j] = w
            tj = ins[j]
            opj = tj.split()[0]
            touched = _regs(tj) & dst
            if touched:
                if "mfma" not in opj:
                    load_waw = opj.startswith(_LOADS) and _regs(tj.split(",")[0]) >= touched
                    if w < need - (1 if load_waw else 0):
                        found.append(ShortPath(t, tj, w, need))
                continue  # past the first touch the product's hazard is the toucher's
            for s in succ(j):
                heapq.heappush(heap, (w + cost(tj), s))
    return found


def check_listing(asm: str) -> dict[str, list[ShortPath]]:
    """Every function of a listing with at least one short path (symbol -> paths)."""
    out = {}
    for name, body in functions(asm):
        bad = check_function(body)
        if bad:
            out[name] = bad
    return out
